// The v_mfma_f32_16x16x32_f16 instances of the 4-wave 256x256x64 2-stage
// tile with an f32 C: a plain f32 store (out1) and the reference's
// C += A*B (out2), each plain and with the fused epilogue steps (any M, N
// and K; tile, grouped or persistent order; never split-K).
#include "gemm_mfma16g.h"

namespace tbk {
#define TBK_MFMA16_F32(OUT, EPI, SUFFIX)                                               \
  {{256, 256, 64, 2, 2, OUT, 2, EPI, 1},                                               \
   reinterpret_cast<const void *>(&gemm_mfma16_f32<OUT, EPI>),                  \
   "tb_gemm_gfx950_256x256x64_w2x2_s2_out" #OUT "_16x16x32" SUFFIX, kMfma16VmPrologue, \
   kMfma16VmLoop, kMfma16LgkmLoop,                                                     \
   reinterpret_cast<const void *>(&gemm_mfma16g<256, 256, 64, 2, 2, 2, OUT, EPI>)}
static const KernelEntry kMfma16F32[] = {
    TBK_MFMA16_F32(1, false, ""), TBK_MFMA16_F32(1, true, "_epi"),
    TBK_MFMA16_F32(2, false, ""), TBK_MFMA16_F32(2, true, "_epi")};
#undef TBK_MFMA16_F32
const KernelEntry *entries_mfma16_f32(int *n) {
  *n = sizeof(kMfma16F32) / sizeof(kMfma16F32[0]);
  return kMfma16F32;
}
} // namespace tbk
