// Attribute values of the tb IR subset, with MLIR-compatible text syntax.
//
// The reference keeps all plan state as MLIR attributes on the op (the IR
// text is the checkpoint: every plan has build/parse round trips, e.g.
// lib/Analysis/ProgramMappingPlan.cpp:460-581). MLIR is not available here,
// so this is a small self-contained value model that prints the same syntax
// MLIR prints for the attribute kinds the plans use:
//   integer      `5 : i64`      (untyped inside #tb.* parameter lists: `5`)
//   float        `6.000000e+00 : f32`
//   bool         `true`
//   string       `"x"`
//   dense i64    `array<i64: 1, 2>`
//   array        `[a, b]`
//   dictionary   `{a = 1 : i64, b = "x"}`, keys sorted like DictionaryAttr
//   dialect attr `#tb.shared<order = [1, 0], perPhase = 4, ...>`
//   type         `f16`, `memref<64x32xf16>`, `!tb.memdesc<...>`
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace tb {

// Thrown for every diagnostic (the reference's emitError + failure()).
struct Error : std::runtime_error {
  explicit Error(const std::string &m) : std::runtime_error(m) {}
};

struct Attr;
using AttrP = std::shared_ptr<const Attr>;
using Fields = std::vector<std::pair<std::string, AttrP>>;

enum class AttrKind { Int, Float, Bool, String, DenseI64, Array, Dict, Dialect, Type, Unit };

struct Attr {
  AttrKind kind = AttrKind::Unit;
  int64_t i = 0;
  std::string itype = "i64"; // Int: "i64", "i32", "index" or "" (untyped);
                             // Float: "f32" or "f64"
  double f = 0.0;
  bool b = false;
  std::string s; // String value, Type text, Dialect mnemonic ("shared")
  std::vector<int64_t> ints;   // DenseI64
  std::vector<AttrP> elems;    // Array
  std::map<std::string, AttrP> dict; // Dict (sorted, as MLIR prints it)
  Fields params;               // Dialect parameters in declaration order
  std::string typeDialect;     // Type: "" for builtin text, "memdesc" for !tb.memdesc
};

// ---- constructors --------------------------------------------------------
AttrP I64(int64_t v);
AttrP IntU(int64_t v); // untyped integer (dialect parameter / array element)
AttrP F32(double v); // float attribute of type f32 (value rounded to f32)
AttrP Bool(bool v);
AttrP Str(const std::string &v);
AttrP Dense(const std::vector<int64_t> &v);
AttrP Arr(const std::vector<AttrP> &v);
AttrP IntList(const std::vector<int64_t> &v); // `[1, 0]` inside #tb.* attrs
AttrP Dict(const std::map<std::string, AttrP> &v);
AttrP Dialect(const std::string &mnemonic, const Fields &params);
AttrP TypeText(const std::string &text);
AttrP Unit();

// ---- printing / parsing --------------------------------------------------
std::string print(const AttrP &a);
std::string printDictBody(const std::map<std::string, AttrP> &d); // `{...}`
std::string printKey(const std::string &k);

struct ParseCursor {
  const std::string &src;
  size_t pos = 0;
  // module-level `#name = value` aliases
  const std::map<std::string, AttrP> *aliases = nullptr;
  explicit ParseCursor(const std::string &s) : src(s) {}
  void skipWs();
  bool eof();
  char peek();
  bool consume(const std::string &tok);
  void expect(const std::string &tok);
  std::string ident(); // [A-Za-z_][A-Za-z0-9_$.-]*
  std::string stringLit();
  int64_t integer();
  [[noreturn]] void fail(const std::string &what);
};

AttrP parseAttr(ParseCursor &c);
// Parse a type at the cursor (builtin text up to a balanced end, or
// !tb.memdesc<...>).
AttrP parseType(ParseCursor &c);
std::map<std::string, AttrP> parseDictBody(ParseCursor &c); // expects `{`

// ---- typed access (throw tb::Error with the field name) -----------------
const Attr &field(const Attr &dict, const std::string &name);
bool has(const Attr &dict, const std::string &name);
int64_t getI64(const Attr &dict, const std::string &name);
bool getBool(const Attr &dict, const std::string &name);
double getF64(const Attr &dict, const std::string &name); // float or integer
std::string getStr(const Attr &dict, const std::string &name);
std::vector<int64_t> getDense(const Attr &dict, const std::string &name);
const std::vector<AttrP> &getArr(const Attr &dict, const std::string &name);
const Attr &getDict(const Attr &dict, const std::string &name);
// dialect attr parameter access
const Attr &param(const Attr &dialect, const std::string &name);
int64_t paramI64(const Attr &dialect, const std::string &name);
std::vector<int64_t> paramInts(const Attr &dialect, const std::string &name);
bool paramBool(const Attr &dialect, const std::string &name);
std::string paramStr(const Attr &dialect, const std::string &name);

bool equal(const AttrP &a, const AttrP &b);

} // namespace tb
