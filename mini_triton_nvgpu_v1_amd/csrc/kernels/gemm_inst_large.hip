// gfx950 GEMM instances: 256-wide macro-tiles (the MFMA-bound configs).
#include "gemm_gfx950_impl.h"

#define TBK_OUTS(BM, BN, BK, WGM, WGN)                                          \
  TBK_ENTRY(BM, BN, BK, WGM, WGN, 0), TBK_ENTRY(BM, BN, BK, WGM, WGN, 1),       \
      TBK_ENTRY(BM, BN, BK, WGM, WGN, 2), TBK_ENTRY(BM, BN, BK, WGM, WGN, 3)

namespace tbk {
static const KernelEntry kLarge[] = {
    TBK_OUTS(256, 256, 64, 2, 2),
    TBK_OUTS(256, 128, 64, 2, 2),
    TBK_OUTS(128, 256, 64, 2, 2),
};
const KernelEntry *entries_large(int *n) {
  *n = sizeof(kLarge) / sizeof(kLarge[0]);
  return kLarge;
}
} // namespace tbk
