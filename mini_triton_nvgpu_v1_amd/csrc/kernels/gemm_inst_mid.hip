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
};
const KernelEntry *entries_mid(int *n) {
  *n = sizeof(kMid) / sizeof(kMid[0]);
  return kMid;
}
} // namespace tbk
