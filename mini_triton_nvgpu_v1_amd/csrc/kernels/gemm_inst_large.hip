// gfx950 GEMM instances: the large tile list, every output mode.
#include "gemm_gfx950_impl.h"
#include "gemm_tiles.h"

namespace tbk {
static const KernelEntry kLarge[] = {
    TBK_TILES_LARGE(TBK_OUTS),
    // the 16x16x32 instance of 256x256x64, 4 waves, 2 stages, f16 C
    {{256, 256, 64, 2, 2, kOutF16, 2, 0, 1},
     reinterpret_cast<const void *>(&gemm_mfma16<false>),
     "tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32"}};
const KernelEntry *entries_large(int *n) {
  *n = sizeof(kLarge) / sizeof(kLarge[0]);
  return kLarge;
}
} // namespace tbk
