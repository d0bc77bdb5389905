// gfx950 GEMM instances: 128-wide macro-tiles (mid sizes, split-K partials).
#include "gemm_gfx950_impl.h"

#define TBK_OUTS(BM, BN, BK, WGM, WGN)                                          \
  TBK_ENTRY(BM, BN, BK, WGM, WGN, 0), TBK_ENTRY(BM, BN, BK, WGM, WGN, 1),       \
      TBK_ENTRY(BM, BN, BK, WGM, WGN, 2), TBK_ENTRY(BM, BN, BK, WGM, WGN, 3)

namespace tbk {
static const KernelEntry kMid[] = {
    TBK_OUTS(128, 128, 32, 2, 2), TBK_OUTS(128, 128, 64, 2, 2),
    TBK_OUTS(128, 64, 64, 2, 2),  TBK_OUTS(64, 128, 64, 2, 2),
};
const KernelEntry *entries_mid(int *n) {
  *n = sizeof(kMid) / sizeof(kMid[0]);
  return kMid;
}
} // namespace tbk
