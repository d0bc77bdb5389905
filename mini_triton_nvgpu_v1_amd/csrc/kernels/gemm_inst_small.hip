// gfx950 GEMM instances: 64x64 macro-tiles (launch-bound shapes).
#include "gemm_gfx950_impl.h"

namespace tbk {
static const KernelEntry kSmall[] = {
    TBK_OUTS(64, 64, 32, 1, 1, 2),
    TBK_OUTS(64, 64, 32, 1, 1, 3),
    TBK_OUTS(64, 64, 32, 2, 1, 2),
    TBK_OUTS(64, 64, 32, 2, 2, 2),
    TBK_OUTS(64, 64, 32, 2, 2, 3),
    TBK_OUTS(64, 64, 32, 2, 2, 4),
    TBK_OUTS(64, 64, 64, 1, 1, 2),
    TBK_OUTS(64, 64, 64, 2, 2, 2),
    TBK_OUTS(64, 64, 64, 2, 2, 3),
};
const KernelEntry *entries_small(int *n) {
  *n = sizeof(kSmall) / sizeof(kSmall[0]);
  return kSmall;
}
} // namespace tbk
