// gfx950 GEMM instances: 256-wide macro-tiles (the MFMA-bound configs).
#include "gemm_gfx950_impl.h"

namespace tbk {
static const KernelEntry kLarge[] = {
    // 8 waves (2 per SIMD: one wave's MFMAs cover the other's waits), the
    // grid the plan derives for 8 waves on a 256x256 tile
    TBK_OUTS(256, 256, 64, 4, 2, 2),
    TBK_OUTS(256, 256, 32, 4, 2, 3),
    TBK_OUTS(256, 256, 32, 4, 2, 4),
    TBK_OUTS(256, 256, 64, 2, 2, 2),
    TBK_OUTS(256, 256, 32, 2, 2, 2),
    TBK_OUTS(256, 256, 32, 2, 2, 3),
    TBK_OUTS(256, 256, 32, 2, 2, 4),
    TBK_OUTS(256, 128, 64, 2, 2, 2),
    TBK_OUTS(256, 128, 64, 2, 2, 3),
    TBK_OUTS(128, 256, 64, 2, 2, 2),
    TBK_OUTS(128, 256, 64, 2, 2, 3),
};
const KernelEntry *entries_large(int *n) {
  *n = sizeof(kLarge) / sizeof(kLarge[0]);
  return kLarge;
}
} // namespace tbk
