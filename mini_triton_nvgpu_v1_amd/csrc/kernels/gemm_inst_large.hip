// gfx950 GEMM instances: 256-wide macro-tiles (the MFMA-bound configs).
#include "gemm_gfx950_impl.h"

namespace tbk {
static const KernelEntry kLarge[] = {
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
