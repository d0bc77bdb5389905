// Attribute model of the tb IR subset: constructors, MLIR-syntax printer and
// parser, typed accessors.
#include "attr.h"

#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <sstream>

namespace tb {

// ---- constructors ----------------------------------------------------------
static std::shared_ptr<Attr> make(AttrKind k) {
  auto a = std::make_shared<Attr>();
  a->kind = k;
  return a;
}
AttrP I64(int64_t v) {
  auto a = make(AttrKind::Int);
  a->i = v;
  return a;
}
AttrP IntU(int64_t v) {
  auto a = make(AttrKind::Int);
  a->i = v;
  a->itype = "";
  return a;
}
AttrP F32(double v) {
  auto a = make(AttrKind::Float);
  a->f = (double)(float)v;
  a->itype = "f32";
  return a;
}
AttrP Bool(bool v) {
  auto a = make(AttrKind::Bool);
  a->b = v;
  return a;
}
AttrP Str(const std::string &v) {
  auto a = make(AttrKind::String);
  a->s = v;
  return a;
}
AttrP Dense(const std::vector<int64_t> &v) {
  auto a = make(AttrKind::DenseI64);
  a->ints = v;
  return a;
}
AttrP Arr(const std::vector<AttrP> &v) {
  auto a = make(AttrKind::Array);
  a->elems = v;
  return a;
}
AttrP IntList(const std::vector<int64_t> &v) {
  std::vector<AttrP> e;
  for (int64_t x : v)
    e.push_back(IntU(x));
  return Arr(e);
}
AttrP Dict(const std::map<std::string, AttrP> &v) {
  auto a = make(AttrKind::Dict);
  a->dict = v;
  return a;
}
AttrP Dialect(const std::string &mnemonic, const Fields &params) {
  auto a = make(AttrKind::Dialect);
  a->s = mnemonic;
  a->params = params;
  return a;
}
AttrP TypeText(const std::string &text) {
  auto a = make(AttrKind::Type);
  a->s = text;
  return a;
}
AttrP Unit() { return make(AttrKind::Unit); }

// ---- printing --------------------------------------------------------------
static bool bareKey(const std::string &k) {
  if (k.empty() || !(std::isalpha((unsigned char)k[0]) || k[0] == '_'))
    return false;
  for (char ch : k)
    if (!(std::isalnum((unsigned char)ch) || ch == '_' || ch == '$' || ch == '.'))
      return false;
  return true;
}

static std::string quote(const std::string &s) {
  std::string o = "\"";
  for (char ch : s) {
    if (ch == '"' || ch == '\\') {
      o += '\\';
      o += ch;
    } else if (ch == '\n') {
      o += "\\0A";
    } else {
      o += ch;
    }
  }
  return o + "\"";
}

std::string printKey(const std::string &k) { return bareKey(k) ? k : quote(k); }

static void printTo(std::ostringstream &os, const AttrP &a);

// MLIR's float attribute text: scientific notation with six fraction digits
// when that reads back to the same value of the attribute's type, else as
// many digits as the type needs to round-trip.
static std::string printFloat(double v, const std::string &type) {
  char buf[64];
  snprintf(buf, sizeof buf, "%.6e", v);
  const double back = strtod(buf, nullptr);
  const bool same = type == "f32" ? (float)back == (float)v : back == v;
  if (!same)
    snprintf(buf, sizeof buf, type == "f32" ? "%.8e" : "%.16e", v);
  return buf;
}

static void printParams(std::ostringstream &os, const Fields &params) {
  os << "<";
  bool first = true;
  for (const auto &kv : params) {
    if (!first)
      os << ", ";
    first = false;
    os << kv.first << " = ";
    printTo(os, kv.second);
  }
  os << ">";
}

static void printTo(std::ostringstream &os, const AttrP &a) {
  switch (a->kind) {
  case AttrKind::Int:
    os << a->i;
    if (!a->itype.empty())
      os << " : " << a->itype;
    return;
  case AttrKind::Float:
    os << printFloat(a->f, a->itype) << " : " << a->itype;
    return;
  case AttrKind::Bool:
    os << (a->b ? "true" : "false");
    return;
  case AttrKind::String:
    os << quote(a->s);
    return;
  case AttrKind::DenseI64:
    os << "array<i64";
    for (size_t i = 0; i < a->ints.size(); ++i)
      os << (i == 0 ? ": " : ", ") << a->ints[i];
    os << ">";
    return;
  case AttrKind::Array:
    os << "[";
    for (size_t i = 0; i < a->elems.size(); ++i) {
      if (i)
        os << ", ";
      printTo(os, a->elems[i]);
    }
    os << "]";
    return;
  case AttrKind::Dict:
    os << printDictBody(a->dict);
    return;
  case AttrKind::Dialect:
    os << "#tb." << a->s;
    printParams(os, a->params);
    return;
  case AttrKind::Type:
    if (a->typeDialect == "memdesc") {
      os << "!tb.memdesc";
      printParams(os, a->params);
    } else {
      os << a->s;
    }
    return;
  case AttrKind::Unit:
    os << "unit";
    return;
  }
}

std::string printDictBody(const std::map<std::string, AttrP> &d) {
  std::ostringstream os;
  os << "{";
  bool first = true;
  for (const auto &kv : d) {
    if (!first)
      os << ", ";
    first = false;
    os << printKey(kv.first);
    if (kv.second->kind != AttrKind::Unit) {
      os << " = ";
      printTo(os, kv.second);
    }
  }
  os << "}";
  return os.str();
}

std::string print(const AttrP &a) {
  std::ostringstream os;
  printTo(os, a);
  return os.str();
}

// ---- parsing ---------------------------------------------------------------
void ParseCursor::skipWs() {
  while (pos < src.size()) {
    char ch = src[pos];
    if (std::isspace((unsigned char)ch)) {
      ++pos;
    } else if (ch == '/' && pos + 1 < src.size() && src[pos + 1] == '/') {
      while (pos < src.size() && src[pos] != '\n')
        ++pos;
    } else {
      break;
    }
  }
}
bool ParseCursor::eof() {
  skipWs();
  return pos >= src.size();
}
char ParseCursor::peek() {
  skipWs();
  return pos < src.size() ? src[pos] : '\0';
}
bool ParseCursor::consume(const std::string &tok) {
  skipWs();
  if (src.compare(pos, tok.size(), tok) == 0) {
    pos += tok.size();
    return true;
  }
  return false;
}
void ParseCursor::expect(const std::string &tok) {
  if (!consume(tok))
    fail("expected `" + tok + "`");
}
std::string ParseCursor::ident() {
  skipWs();
  size_t b = pos;
  if (pos < src.size() && (std::isalpha((unsigned char)src[pos]) || src[pos] == '_'))
    ++pos;
  else
    fail("expected identifier");
  while (pos < src.size() && (std::isalnum((unsigned char)src[pos]) ||
                              src[pos] == '_' || src[pos] == '$' ||
                              src[pos] == '.' || src[pos] == '-'))
    ++pos;
  return src.substr(b, pos - b);
}
std::string ParseCursor::stringLit() {
  skipWs();
  if (pos >= src.size() || src[pos] != '"')
    fail("expected string literal");
  ++pos;
  std::string out;
  while (pos < src.size() && src[pos] != '"') {
    if (src[pos] == '\\' && pos + 1 < src.size()) {
      char n = src[pos + 1];
      if (n == '"' || n == '\\') {
        out += n;
        pos += 2;
        continue;
      }
      if (pos + 2 < src.size() && std::isxdigit((unsigned char)n) &&
          std::isxdigit((unsigned char)src[pos + 2])) {
        out += (char)std::stoi(src.substr(pos + 1, 2), nullptr, 16);
        pos += 3;
        continue;
      }
    }
    out += src[pos++];
  }
  if (pos >= src.size())
    fail("unterminated string");
  ++pos;
  return out;
}
int64_t ParseCursor::integer() {
  skipWs();
  size_t b = pos;
  if (pos < src.size() && (src[pos] == '-' || src[pos] == '+'))
    ++pos;
  while (pos < src.size() && std::isdigit((unsigned char)src[pos]))
    ++pos;
  if (b == pos || (pos == b + 1 && !std::isdigit((unsigned char)src[b])))
    fail("expected integer");
  return std::stoll(src.substr(b, pos - b));
}
void ParseCursor::fail(const std::string &what) {
  size_t line = 1, col = 1;
  for (size_t i = 0; i < pos && i < src.size(); ++i) {
    if (src[i] == '\n') {
      ++line;
      col = 1;
    } else {
      ++col;
    }
  }
  throw Error("parse error at " + std::to_string(line) + ":" +
              std::to_string(col) + ": " + what);
}

static Fields parseParams(ParseCursor &c) {
  Fields f;
  c.expect("<");
  if (c.consume(">"))
    return f;
  while (true) {
    if (c.consume("struct(")) { // optional padding struct: skip balanced
      int depth = 1;
      while (depth > 0 && c.pos < c.src.size()) {
        char ch = c.src[c.pos++];
        if (ch == '(')
          ++depth;
        else if (ch == ')')
          --depth;
      }
    } else {
      std::string k = c.ident();
      c.expect("=");
      f.emplace_back(k, parseAttr(c));
    }
    if (c.consume(">"))
      return f;
    c.expect(",");
  }
}

// Balanced builtin type text such as memref<64x32xf16> or f16.
static std::string builtinTypeText(ParseCursor &c) {
  c.skipWs();
  size_t b = c.pos;
  while (c.pos < c.src.size() &&
         (std::isalnum((unsigned char)c.src[c.pos]) || c.src[c.pos] == '_'))
    ++c.pos;
  if (c.pos < c.src.size() && c.src[c.pos] == '<') {
    int depth = 0;
    do {
      char ch = c.src[c.pos++];
      if (ch == '<')
        ++depth;
      else if (ch == '>')
        --depth;
    } while (depth > 0 && c.pos < c.src.size());
  }
  if (b == c.pos)
    c.fail("expected type");
  return c.src.substr(b, c.pos - b);
}

AttrP parseType(ParseCursor &c) {
  if (c.consume("!tb.memdesc")) {
    auto a = std::make_shared<Attr>();
    a->kind = AttrKind::Type;
    a->typeDialect = "memdesc";
    a->params = parseParams(c);
    return a;
  }
  return TypeText(builtinTypeText(c));
}

std::map<std::string, AttrP> parseDictBody(ParseCursor &c) {
  std::map<std::string, AttrP> d;
  c.expect("{");
  if (c.consume("}"))
    return d;
  while (true) {
    std::string k = c.peek() == '"' ? c.stringLit() : c.ident();
    if (c.consume("=")) {
      d[k] = parseAttr(c);
    } else {
      d[k] = Unit();
    }
    if (c.consume("}"))
      return d;
    c.expect(",");
  }
}

AttrP parseAttr(ParseCursor &c) {
  char ch = c.peek();
  if (ch == '"')
    return Str(c.stringLit());
  if (ch == '{')
    return Dict(parseDictBody(c));
  if (ch == '[') {
    c.expect("[");
    std::vector<AttrP> e;
    if (!c.consume("]")) {
      while (true) {
        e.push_back(parseAttr(c));
        if (c.consume("]"))
          break;
        c.expect(",");
      }
    }
    return Arr(e);
  }
  if (ch == '#') {
    if (c.consume("#tb.")) {
      std::string mn = c.ident();
      return Dialect(mn, parseParams(c));
    }
    c.expect("#");
    std::string name = c.ident();
    if (!c.aliases || !c.aliases->count(name))
      c.fail("unknown attribute alias #" + name);
    return c.aliases->at(name);
  }
  if (ch == '!')
    return parseType(c);
  if (ch == '-' || std::isdigit((unsigned char)ch)) {
    // a float literal has a fraction or an exponent: `-1.5`, `6.000000e+00`
    size_t q = c.pos + (ch == '-' ? 1 : 0);
    while (q < c.src.size() && std::isdigit((unsigned char)c.src[q]))
      ++q;
    if (q < c.src.size() && (c.src[q] == '.' || c.src[q] == 'e' || c.src[q] == 'E')) {
      const char *begin = c.src.c_str() + c.pos;
      char *end = nullptr;
      const double v = strtod(begin, &end);
      if (end == begin)
        c.fail("expected a float literal");
      c.pos += (size_t)(end - begin);
      auto a = std::make_shared<Attr>();
      a->kind = AttrKind::Float;
      a->itype = "f64";
      size_t save = c.pos;
      if (c.consume(":")) {
        c.skipWs();
        if (c.consume("f32"))
          a->itype = "f32";
        else if (c.consume("f64"))
          a->itype = "f64";
        else
          c.pos = save;
      }
      a->f = a->itype == "f32" ? (double)(float)v : v;
      return a;
    }
    int64_t v = c.integer();
    size_t save = c.pos;
    if (c.consume(":")) {
      c.skipWs();
      size_t b = c.pos;
      while (c.pos < c.src.size() && std::isalnum((unsigned char)c.src[c.pos]))
        ++c.pos;
      std::string t = c.src.substr(b, c.pos - b);
      if (t == "i64" || t == "i32" || t == "index" || t == "i1" || t == "i8" ||
          t == "i16") {
        auto a = std::make_shared<Attr>();
        a->kind = AttrKind::Int;
        a->i = v;
        a->itype = t;
        return a;
      }
      c.pos = save;
    }
    return IntU(v);
  }
  if (c.consume("array<")) {
    c.expect("i64");
    std::vector<int64_t> v;
    if (c.consume(":")) {
      while (true) {
        v.push_back(c.integer());
        if (!c.consume(","))
          break;
      }
    }
    c.expect(">");
    return Dense(v);
  }
  size_t save = c.pos;
  std::string word = c.ident();
  if (word == "true")
    return Bool(true);
  if (word == "false")
    return Bool(false);
  if (word == "unit")
    return Unit();
  c.pos = save;
  return parseType(c); // f16, memref<...>, ...
}

// ---- typed access ------------------------------------------------------------
const Attr &field(const Attr &dict, const std::string &name) {
  if (dict.kind != AttrKind::Dict)
    throw Error("expected a dictionary attribute holding `" + name + "`");
  auto it = dict.dict.find(name);
  if (it == dict.dict.end())
    throw Error("missing field `" + name + "`");
  return *it->second;
}
bool has(const Attr &dict, const std::string &name) {
  return dict.kind == AttrKind::Dict && dict.dict.count(name);
}
int64_t getI64(const Attr &dict, const std::string &name) {
  const Attr &a = field(dict, name);
  if (a.kind != AttrKind::Int)
    throw Error("missing integer field `" + name + "`");
  return a.i;
}
bool getBool(const Attr &dict, const std::string &name) {
  const Attr &a = field(dict, name);
  if (a.kind != AttrKind::Bool)
    throw Error("missing bool field `" + name + "`");
  return a.b;
}
double getF64(const Attr &dict, const std::string &name) {
  const Attr &a = field(dict, name);
  if (a.kind == AttrKind::Float)
    return a.f;
  if (a.kind == AttrKind::Int)
    return (double)a.i;
  throw Error("missing float field `" + name + "`");
}
std::string getStr(const Attr &dict, const std::string &name) {
  const Attr &a = field(dict, name);
  if (a.kind != AttrKind::String)
    throw Error("missing string field `" + name + "`");
  return a.s;
}
std::vector<int64_t> getDense(const Attr &dict, const std::string &name) {
  const Attr &a = field(dict, name);
  if (a.kind != AttrKind::DenseI64)
    throw Error("missing dense i64 array field `" + name + "`");
  return a.ints;
}
const std::vector<AttrP> &getArr(const Attr &dict, const std::string &name) {
  const Attr &a = field(dict, name);
  if (a.kind != AttrKind::Array)
    throw Error("missing array field `" + name + "`");
  return a.elems;
}
const Attr &getDict(const Attr &dict, const std::string &name) {
  const Attr &a = field(dict, name);
  if (a.kind != AttrKind::Dict)
    throw Error("missing dictionary field `" + name + "`");
  return a;
}
const Attr &param(const Attr &d, const std::string &name) {
  for (const auto &kv : d.params)
    if (kv.first == name)
      return *kv.second;
  throw Error("#tb." + d.s + " is missing parameter `" + name + "`");
}
int64_t paramI64(const Attr &d, const std::string &name) {
  const Attr &a = param(d, name);
  if (a.kind != AttrKind::Int)
    throw Error("#tb." + d.s + " parameter `" + name + "` must be an integer");
  return a.i;
}
std::vector<int64_t> paramInts(const Attr &d, const std::string &name) {
  const Attr &a = param(d, name);
  std::vector<int64_t> v;
  if (a.kind == AttrKind::DenseI64)
    return a.ints;
  if (a.kind != AttrKind::Array)
    throw Error("#tb." + d.s + " parameter `" + name + "` must be an int list");
  for (const auto &e : a.elems) {
    if (e->kind != AttrKind::Int)
      throw Error("#tb." + d.s + " parameter `" + name + "` must be an int list");
    v.push_back(e->i);
  }
  return v;
}
bool paramBool(const Attr &d, const std::string &name) {
  const Attr &a = param(d, name);
  if (a.kind != AttrKind::Bool)
    throw Error("#tb." + d.s + " parameter `" + name + "` must be a bool");
  return a.b;
}
std::string paramStr(const Attr &d, const std::string &name) {
  const Attr &a = param(d, name);
  if (a.kind != AttrKind::String)
    throw Error("#tb." + d.s + " parameter `" + name + "` must be a string");
  return a.s;
}

bool equal(const AttrP &a, const AttrP &b) { return print(a) == print(b); }

} // namespace tb
