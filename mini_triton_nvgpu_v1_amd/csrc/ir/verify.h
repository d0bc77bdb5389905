// Verifiers of the tb IR subset: the #tb.* attributes, the !tb.memdesc type
// and the tb ops, run after parsing and after every pass (as MLIR verifies
// a module after parsing and after each pass). Each check restates the
// reference's verifier where one exists, with its diagnostic text:
//  * attributes: lib/IR/TBAttrs.cpp:47-195 (semantic_layout, cga, blocked,
//    shared, nvgpu_mma, dot_operand) plus the gfx950 amd_mfma parent
//    encoding and the parameter lists of include/tb/IR/TBAttrDefs.td;
//  * !tb.memdesc: lib/IR/TBTypes.cpp:16-56;
//  * ops: lib/IR/TBOps.cpp:34-60 and :128-304 (tb.matmul, tb.convert_layout,
//    tb.pipeline_mainline and its cluster ops) plus tb.gfx950_launch.
// Failures throw tb::Error.
#pragma once

#include "ir.h"

namespace tb {

void verifyAttr(const Attr &a);
void verifyModule(const Module &m);

} // namespace tb
