// tb_plan_from_mlir / tb_plan_from_file: run the plan pipeline and flatten
// the KernelContract into a tb_gemm_config.
#include "desc.h"

extern "C" int tb_plan_from_mlir(const char *mlir, size_t len,
                                 const char *gpu_arch, tb_gemm_desc **out) {
  (void)mlir;
  (void)len;
  (void)gpu_arch;
  (void)out;
  tbrt::set_error("tb_plan_from_mlir: plan pipeline not built yet");
  return -1;
}

extern "C" int tb_plan_from_file(const char *path, tb_gemm_desc **out) {
  (void)path;
  (void)out;
  tbrt::set_error("tb_plan_from_file: plan pipeline not built yet");
  return -1;
}
