// gfx950 GEMM instances: 128-wide macro-tiles (mid sizes, split-K partials).
#include "gemm_gfx950_impl.h"

namespace tbk {
static const KernelEntry kMid[] = {
    TBK_OUTS(128, 128, 32, 2, 2, 2),
    TBK_OUTS(128, 128, 32, 2, 2, 3),
    TBK_OUTS(128, 128, 32, 2, 2, 4),
    TBK_OUTS(128, 128, 64, 2, 2, 2),
    TBK_OUTS(128, 128, 64, 2, 2, 3),
    TBK_OUTS(128, 128, 64, 2, 2, 4),
    TBK_OUTS(128, 64, 64, 2, 2, 2),
    TBK_OUTS(128, 64, 64, 2, 2, 3),
    TBK_OUTS(64, 128, 64, 2, 2, 2),
    TBK_OUTS(64, 128, 64, 2, 2, 3),
    // the wave grids the plan derives for 4 waves on 128x64 / 64x128 tiles
    // (equal wave-tile imbalance; ties go to more waves along the long side)
    TBK_OUTS(128, 64, 64, 4, 1, 2),
    TBK_OUTS(128, 64, 64, 4, 1, 3),
    TBK_OUTS(64, 128, 64, 1, 4, 2),
    TBK_OUTS(64, 128, 64, 1, 4, 3),
};
const KernelEntry *entries_mid(int *n) {
  *n = sizeof(kMid) / sizeof(kMid[0]);
  return kMid;
}
} // namespace tbk
