// gfx950 GEMM instances: the large tile list with the fused epilogue steps
// (bias, activation, clamp), for the output modes that write a whole result.
#include "gemm_gfx950_impl.h"
#include "gemm_tiles.h"

namespace tbk {
static const KernelEntry kLargeEpi[] = {
    TBK_TILES_LARGE(TBK_EPI_OUTS),
    {{256, 256, 64, 2, 2, kOutF16, 2, 1, 1},
     reinterpret_cast<const void *>(&gemm_mfma16<true>),
     "tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32_epi"}};
const KernelEntry *entries_large_epi(int *n) {
  *n = sizeof(kLargeEpi) / sizeof(kLargeEpi[0]);
  return kLargeEpi;
}
} // namespace tbk
