// The tb IR subset: a module of func.func bodies holding tb.matmul (before
// the plan pipeline), tb.pipeline_mainline with its cluster ops (after
// tb-cleanup-pipeline), tb.convert_layout, and tb.gfx950_launch (after the
// gfx950 lowering). Op forms follow the reference's assembly formats
// (include/tb/IR/TBOps.td): tb.matmul and tb.pipeline_mainline print
// `$a, $b, $c attr-dict : type($a), type($b), type($c)`; the cluster ops
// print `attr-dict`; tb.convert_layout prints
// `$source attr-dict : functional-type(operands, results)`.
#pragma once

#include "attr.h"

#include <map>
#include <string>
#include <vector>

namespace tb {

struct Op {
  std::string name;
  std::vector<std::string> results;  // "%0"
  std::vector<std::string> operands; // "%A"
  std::map<std::string, AttrP> attrs;
  std::vector<AttrP> operandTypes;
  std::vector<AttrP> resultTypes;
  bool functionalType = false; // `: (t) -> t` form
  bool hasRegion = false;
  std::vector<Op> region;
};

struct Func {
  std::string name;
  std::vector<std::pair<std::string, AttrP>> args; // (%name, type)
  std::vector<AttrP> resultTypes;
  std::map<std::string, AttrP> attrs;
  std::vector<Op> body;
};

struct Module {
  std::map<std::string, AttrP> attrs;
  std::map<std::string, AttrP> aliases;
  std::vector<Func> funcs;

  AttrP attr(const std::string &name) const {
    auto it = attrs.find(name);
    return it == attrs.end() ? nullptr : it->second;
  }
};

Module parseModule(const std::string &text);
std::string printModule(const Module &m);

// Static shape of a memref type text such as memref<64x32xf16>:
// {64, 32} and element type "f16". Throws for anything else.
struct MemRefInfo {
  std::vector<int64_t> shape;
  std::string elementType;
  bool identityLayout = true;
};
MemRefInfo parseMemRef(const AttrP &type);

} // namespace tb
