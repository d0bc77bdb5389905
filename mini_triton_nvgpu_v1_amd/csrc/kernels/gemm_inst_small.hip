// gfx950 GEMM instances: 64x64 macro-tiles (launch-bound shapes).
#include "gemm_gfx950_impl.h"

#define TBK_OUTS(BM, BN, BK, WGM, WGN)                                          \
  TBK_ENTRY(BM, BN, BK, WGM, WGN, 0), TBK_ENTRY(BM, BN, BK, WGM, WGN, 1),       \
      TBK_ENTRY(BM, BN, BK, WGM, WGN, 2), TBK_ENTRY(BM, BN, BK, WGM, WGN, 3)

namespace tbk {
static const KernelEntry kSmall[] = {
    TBK_OUTS(64, 64, 32, 1, 1), TBK_OUTS(64, 64, 32, 2, 1),
    TBK_OUTS(64, 64, 32, 2, 2), TBK_OUTS(64, 64, 64, 1, 1),
    TBK_OUTS(64, 64, 64, 2, 2),
};
const KernelEntry *entries_small(int *n) {
  *n = sizeof(kSmall) / sizeof(kSmall[0]);
  return kSmall;
}
} // namespace tbk
