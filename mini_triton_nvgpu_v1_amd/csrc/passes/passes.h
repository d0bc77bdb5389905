// The tb-opt pass registry: the stage1 plan passes (same names, order and
// attribute contract as the reference's lib/Transforms/*.cpp) plus the
// gfx950 lowering that replaces tb-lower-pipeline-to-nvgpu.
#pragma once

#include "../ir/ir.h"
#include "tb_gfx950.h"

#include <map>
#include <string>
#include <vector>

namespace tb {

using PassOptions = std::map<std::string, std::string>;

struct PassSpec {
  std::string name;
  PassOptions options;
};

// `builtin.module(p1, p2{k=v k2=v2}, ...)` (the outer builtin.module(...)
// is optional).
std::vector<PassSpec> parsePassPipeline(const std::string &text);
// `key=value key2=value2` (a pass option string)
PassOptions parsePassOptions(const std::string &text);

void runPass(Module &m, const PassSpec &p);
void runPipeline(Module &m, const std::vector<PassSpec> &passes);

struct PassInfo {
  std::string name, summary;
};
std::vector<PassInfo> registeredPasses();

// The stage1 mainline for gfx950: verify-scope .. verify-pipeline-mainline-
// contract, optionally followed by tb-lower-pipeline-to-gfx950. Reference:
// Stage1Pipelines.cpp:15-40.
std::vector<PassSpec> stage1Pipeline(const std::string &gpuArch,
                                     const std::string &features, bool lower);

// The launch configuration of a tb.gfx950_launch op (written by
// tb-lower-pipeline-to-gfx950).
tb_gemm_config launchConfigOf(const Op &launch);
// Kernel instance name the runtime binds for a configuration.
std::string kernelInstanceName(const tb_gemm_config &c);

} // namespace tb
