// Parser and printer of the tb IR subset.
#include "ir.h"
#include "verify.h"

#include <cctype>
#include <sstream>

namespace tb {

namespace {

std::string valueName(ParseCursor &c) {
  c.skipWs();
  if (c.peek() != '%')
    c.fail("expected SSA value");
  ++c.pos;
  size_t b = c.pos;
  while (c.pos < c.src.size() &&
         (std::isalnum((unsigned char)c.src[c.pos]) || c.src[c.pos] == '_'))
    ++c.pos;
  return "%" + c.src.substr(b, c.pos - b);
}

std::string opName(ParseCursor &c) {
  c.skipWs();
  size_t b = c.pos;
  while (c.pos < c.src.size() &&
         (std::isalnum((unsigned char)c.src[c.pos]) || c.src[c.pos] == '_' ||
          c.src[c.pos] == '.'))
    ++c.pos;
  if (b == c.pos)
    c.fail("expected operation name");
  return c.src.substr(b, c.pos - b);
}

std::vector<AttrP> typeList(ParseCursor &c) {
  std::vector<AttrP> t;
  while (true) {
    t.push_back(parseType(c));
    if (!c.consume(","))
      return t;
  }
}

Op parseOp(ParseCursor &c) {
  Op op;
  if (c.peek() == '%') {
    while (true) {
      op.results.push_back(valueName(c));
      if (!c.consume(","))
        break;
    }
    c.expect("=");
  }
  op.name = opName(c);
  if (op.name == "func.return" || op.name == "return") {
    op.name = "func.return";
    if (c.peek() == '%') {
      while (true) {
        op.operands.push_back(valueName(c));
        if (!c.consume(","))
          break;
      }
      c.expect(":");
      op.operandTypes = typeList(c);
    }
    return op;
  }
  if (c.peek() == '%') {
    while (true) {
      op.operands.push_back(valueName(c));
      if (!c.consume(","))
        break;
    }
  }
  if (c.peek() == '{')
    op.attrs = parseDictBody(c);
  if (c.consume(":")) {
    if (c.peek() == '(') {
      op.functionalType = true;
      c.expect("(");
      if (!c.consume(")")) {
        op.operandTypes = typeList(c);
        c.expect(")");
      }
      c.expect("->");
      if (c.consume("(")) {
        if (!c.consume(")")) {
          op.resultTypes = typeList(c);
          c.expect(")");
        }
      } else {
        op.resultTypes = typeList(c);
      }
    } else {
      op.operandTypes = typeList(c);
    }
  }
  if (c.peek() == '{') {
    op.hasRegion = true;
    c.expect("{");
    while (!c.consume("}"))
      op.region.push_back(parseOp(c));
  }
  return op;
}

Func parseFunc(ParseCursor &c) {
  Func f;
  c.expect("func.func");
  c.expect("@");
  f.name = c.ident();
  c.expect("(");
  if (!c.consume(")")) {
    while (true) {
      std::string n = valueName(c);
      c.expect(":");
      f.args.emplace_back(n, parseType(c));
      if (c.consume(")"))
        break;
      c.expect(",");
    }
  }
  if (c.consume("->")) {
    if (c.consume("(")) {
      if (!c.consume(")")) {
        f.resultTypes = typeList(c);
        c.expect(")");
      }
    } else {
      f.resultTypes.push_back(parseType(c));
    }
  }
  if (c.consume("attributes"))
    f.attrs = parseDictBody(c);
  c.expect("{");
  while (!c.consume("}"))
    f.body.push_back(parseOp(c));
  return f;
}

std::string typesText(const std::vector<AttrP> &t) {
  std::string s;
  for (size_t i = 0; i < t.size(); ++i)
    s += (i ? ", " : "") + print(t[i]);
  return s;
}

void printOp(std::ostringstream &os, const Op &op, int indent) {
  std::string pad(indent, ' ');
  os << pad;
  if (op.name == "func.return") {
    os << "return";
    if (!op.operands.empty()) {
      for (size_t i = 0; i < op.operands.size(); ++i)
        os << (i ? ", " : " ") << op.operands[i];
      os << " : " << typesText(op.operandTypes);
    }
    os << "\n";
    return;
  }
  for (size_t i = 0; i < op.results.size(); ++i)
    os << (i ? ", " : "") << op.results[i];
  if (!op.results.empty())
    os << " = ";
  os << op.name;
  for (size_t i = 0; i < op.operands.size(); ++i)
    os << (i ? ", " : " ") << op.operands[i];
  if (!op.attrs.empty())
    os << " " << printDictBody(op.attrs);
  if (op.functionalType) {
    os << " : (" << typesText(op.operandTypes) << ") -> ";
    if (op.resultTypes.size() == 1)
      os << print(op.resultTypes[0]);
    else
      os << "(" << typesText(op.resultTypes) << ")";
  } else if (!op.operandTypes.empty()) {
    os << " : " << typesText(op.operandTypes);
  }
  if (op.hasRegion) {
    os << " {\n";
    for (const Op &inner : op.region)
      printOp(os, inner, indent + 2);
    os << pad << "}";
  }
  os << "\n";
}

} // namespace

Module parseModule(const std::string &text) {
  Module m;
  ParseCursor c(text);
  c.aliases = &m.aliases;
  while (c.peek() == '#') {
    c.expect("#");
    std::string name = c.ident();
    c.expect("=");
    m.aliases[name] = parseAttr(c);
  }
  c.expect("module");
  if (c.consume("attributes"))
    m.attrs = parseDictBody(c);
  c.expect("{");
  while (!c.consume("}"))
    m.funcs.push_back(parseFunc(c));
  if (!c.eof())
    c.fail("trailing text after module");
  verifyModule(m); // as MLIR verifies a module after parsing it
  return m;
}

std::string printModule(const Module &m) {
  std::ostringstream os;
  os << "module";
  if (!m.attrs.empty())
    os << " attributes " << printDictBody(m.attrs);
  os << " {\n";
  for (const Func &f : m.funcs) {
    os << "  func.func @" << f.name << "(";
    for (size_t i = 0; i < f.args.size(); ++i)
      os << (i ? ", " : "") << f.args[i].first << ": " << print(f.args[i].second);
    os << ")";
    if (!f.resultTypes.empty()) {
      os << " -> ";
      if (f.resultTypes.size() == 1)
        os << print(f.resultTypes[0]);
      else
        os << "(" << typesText(f.resultTypes) << ")";
    }
    if (!f.attrs.empty())
      os << " attributes " << printDictBody(f.attrs);
    os << " {\n";
    for (const Op &op : f.body)
      printOp(os, op, 4);
    os << "  }\n";
  }
  os << "}\n";
  return os.str();
}

MemRefInfo parseMemRef(const AttrP &type) {
  if (!type || type->kind != AttrKind::Type || !type->typeDialect.empty())
    throw Error("expected a memref type");
  const std::string &t = type->s;
  if (t.rfind("memref<", 0) != 0 || t.back() != '>')
    throw Error("expected a memref type, got `" + t + "`");
  std::string body = t.substr(7, t.size() - 8);
  MemRefInfo info;
  size_t comma = body.find(',');
  if (comma != std::string::npos) {
    info.identityLayout = false; // strided / affine layout suffix
    body = body.substr(0, comma);
  }
  size_t p = 0;
  while (true) {
    size_t x = body.find('x', p);
    if (x == std::string::npos)
      break;
    std::string dim = body.substr(p, x - p);
    if (dim.empty() || dim == "?")
      throw Error("stage1 requires static memref shapes, got `" + t + "`");
    for (char ch : dim)
      if (!std::isdigit((unsigned char)ch))
        throw Error("stage1 requires static memref shapes, got `" + t + "`");
    info.shape.push_back(std::stoll(dim));
    p = x + 1;
  }
  info.elementType = body.substr(p);
  return info;
}

} // namespace tb
