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
#include "../plan/instances.h"

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

// The launch configuration of a module's one kernel, and the s_waitcnt
// depths its plan states: those of the lowered tb.gfx950_launch op, or of the
// AsyncPlan of a sealed tb.pipeline_mainline (which the lowering checked
// against the kernel instance it names).
struct Planned {
  tb_gemm_config config;
  std::vector<int64_t> waits; // {vm prologue, vm loop, lgkm loop}; empty: not stated
};

Planned configFromModule(tb::Module &m, const std::string &gpuArch) {
  if (tb::Op *launch = singleOp(m, "tb.gfx950_launch")) {
    Planned p{tb::launchConfigOf(*launch), {}};
    auto w = launch->attrs.find("waits");
    if (w != launch->attrs.end()) {
      if (w->second->kind != tb::AttrKind::DenseI64)
        throw tb::Error("tb.gfx950_launch `waits` must be array<i64: ...>");
      p.waits = w->second->ints;
    }
    return p;
  }
  if (!singleOp(m, "tb.pipeline_mainline")) {
    if (!singleOp(m, "tb.matmul"))
      throw tb::Error("module holds no tb.matmul, tb.pipeline_mainline or "
                      "tb.gfx950_launch");
    tb::runPipeline(m, tb::stage1Pipeline(gpuArch, "", false));
  }
  tb::Op *mainline = singleOp(m, "tb.pipeline_mainline");
  tb::KernelContract k = tb::parseKernelContract(m, *mainline);
  tb::verifyMainlineContract(m, *mainline, k);
  Planned p{tb::lowerContractToConfig(k), {}};
  const tb::InstanceSchedule s = tb::instanceSchedule(tb::instanceKeyOf(p.config));
  p.waits = {s.vmPrologue, s.vmLoop, s.lgkmLoop};
  return p;
}

// Bind the descriptor, then refuse it if the compiled kernel's waits are
// not the ones the plan states.
int bindPlanned(const Planned &p, tb_gemm_desc **out, const char *who) {
  if (int rc = tbrt::create_desc(p.config, out))
    return rc;
  if (p.waits.empty())
    return 0;
  int64_t have[3];
  tbrt::desc_waits(*out, have);
  if (p.waits.size() != 3 || p.waits[0] != have[0] || p.waits[1] != have[1] ||
      p.waits[2] != have[2]) {
    std::string msg = std::string(who) + ": the plan's waits (vmcnt prologue / loop, "
                      "lgkmcnt loop:";
    for (int64_t v : p.waits)
      msg += " " + std::to_string(v);
    msg += ") differ from the compiled kernel `" + std::string(tb_desc_kernel_name(*out)) +
           "` (" + std::to_string(have[0]) + " " + std::to_string(have[1]) + " " +
           std::to_string(have[2]) + ")";
    tb_desc_free(*out);
    *out = nullptr;
    return fail(msg);
  }
  return 0;
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
    Planned p = configFromModule(m, gpu_arch && *gpu_arch ? gpu_arch : "gfx950");
    return bindPlanned(p, out, "tb_plan_from_mlir");
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
    Planned p = configFromModule(m, "gfx950");
    return bindPlanned(p, out, "tb_plan_from_file");
  } catch (const tb::Error &e) {
    return fail(std::string("tb_plan_from_file: ") + e.what());
  } catch (const std::exception &e) {
    return fail(std::string("tb_plan_from_file: internal error: ") + e.what());
  }
}
