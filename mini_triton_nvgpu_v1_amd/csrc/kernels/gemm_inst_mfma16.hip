// The v_mfma_f32_16x16x32_f16 instances of the 4-wave 256x256x64 2-stage
// f16 tile (any M, N and K; tile, grouped or persistent order), plain and
// with the fused epilogue steps.
#include "gemm_mfma16g.h"

namespace tbk {
static const KernelEntry kMfma16[] = {
    {{256, 256, 64, 2, 2, kOutF16, 2, 0, 1},
     reinterpret_cast<const void *>(&gemm_mfma16<false>),
     "tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32", kMfma16VmPrologue, kMfma16VmLoop,
     kMfma16LgkmLoop, reinterpret_cast<const void *>(
         &gemm_mfma16g<256, 256, 64, 2, 2, 2, kOutF16, false>)},
    {{256, 256, 64, 2, 2, kOutF16, 2, 1, 1},
     reinterpret_cast<const void *>(&gemm_mfma16<true>),
     "tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32_epi", kMfma16VmPrologue,
     kMfma16VmLoop, kMfma16LgkmLoop, reinterpret_cast<const void *>(
         &gemm_mfma16g<256, 256, 64, 2, 2, 2, kOutF16, true>)}};
const KernelEntry *entries_mfma16(int *n) {
  *n = sizeof(kMfma16) / sizeof(kMfma16[0]);
  return kMfma16;
}
} // namespace tbk
