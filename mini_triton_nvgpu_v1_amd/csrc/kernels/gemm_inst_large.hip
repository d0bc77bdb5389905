// gfx950 GEMM instances: the large tile list, every output mode.
#include "gemm_gfx950_impl.h"
#include "gemm_tiles.h"

namespace tbk {
static const KernelEntry kLarge[] = {TBK_TILES_LARGE(TBK_OUTS)};
const KernelEntry *entries_large(int *n) {
  *n = sizeof(kLarge) / sizeof(kLarge[0]);
  return kLarge;
}
} // namespace tbk
