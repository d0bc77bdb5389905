// tb_plan_from_mlir / tb_plan_from_file: run the stage1 plan pipeline (the
// same passes tb-opt runs) and flatten the sealed KernelContract into the
// tb_gemm_config the gfx950 kernels launch with.
//
// Reference boundary: tools/bench_stage1_fair.py:547-563 runs
// `tb-opt --pass-pipeline=builtin.module(tb-stage1-full-to-nvvm-pipeline{...})`
// on a tb.matmul module and loads the produced binary; here the same module
// text goes through the plan passes in-process and the contract selects a
// precompiled gfx950 instance.
#include "desc.h"

#include "../passes/passes.h"
#include "../plan/contract.h"

#include <fstream>
#include <sstream>

namespace {

int fail(const std::string &m) {
  tbrt::set_error(m);
  return -1;
}

// The single kernel op of a module (multi-kernel modules are rejected: one
// descriptor describes one launch).
tb::Op *singleOp(tb::Module &m, const char *name) {
  tb::Op *found = nullptr;
  for (tb::Func &f : m.funcs)
    for (tb::Op &op : f.body)
      if (op.name == name) {
        if (found)
          throw tb::Error(std::string("module holds more than one ") + name);
        found = &op;
      }
  return found;
}

tb_gemm_config configFromModule(tb::Module &m, const std::string &gpuArch) {
  if (tb::Op *launch = singleOp(m, "tb.gfx950_launch"))
    return tb::launchConfigOf(*launch);
  if (!singleOp(m, "tb.pipeline_mainline")) {
    if (!singleOp(m, "tb.matmul"))
      throw tb::Error("module holds no tb.matmul, tb.pipeline_mainline or "
                      "tb.gfx950_launch");
    tb::runPipeline(m, tb::stage1Pipeline(gpuArch, "", false));
  }
  tb::Op *mainline = singleOp(m, "tb.pipeline_mainline");
  tb::KernelContract k = tb::parseKernelContract(m, *mainline);
  tb::verifyMainlineContract(m, *mainline, k);
  return tb::lowerContractToConfig(k);
}

} // namespace

extern "C" int tb_plan_from_mlir(const char *mlir, size_t len, const char *gpu_arch,
                                 tb_gemm_desc **out) {
  if (!out)
    return fail("tb_plan_from_mlir: out is NULL");
  *out = nullptr;
  if (!mlir)
    return fail("tb_plan_from_mlir: mlir is NULL");
  try {
    tb::Module m = tb::parseModule(std::string(mlir, len));
    tb_gemm_config c = configFromModule(m, gpu_arch && *gpu_arch ? gpu_arch : "gfx950");
    return tbrt::create_desc(c, out);
  } catch (const tb::Error &e) {
    return fail(std::string("tb_plan_from_mlir: ") + e.what());
  } catch (const std::exception &e) {
    return fail(std::string("tb_plan_from_mlir: internal error: ") + e.what());
  }
}

extern "C" int tb_plan_from_file(const char *path, tb_gemm_desc **out) {
  if (!out)
    return fail("tb_plan_from_file: out is NULL");
  *out = nullptr;
  if (!path)
    return fail("tb_plan_from_file: path is NULL");
  std::ifstream in(path, std::ios::binary);
  if (!in)
    return fail(std::string("tb_plan_from_file: cannot open `") + path + "`");
  std::ostringstream ss;
  ss << in.rdbuf();
  std::string text = ss.str();
  try {
    tb::Module m = tb::parseModule(text);
    tb_gemm_config c = configFromModule(m, "gfx950");
    return tbrt::create_desc(c, out);
  } catch (const tb::Error &e) {
    return fail(std::string("tb_plan_from_file: ") + e.what());
  } catch (const std::exception &e) {
    return fail(std::string("tb_plan_from_file: internal error: ") + e.what());
  }
}
