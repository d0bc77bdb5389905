// gfx950 GEMM instances: the small tile list, every output mode.
#include "gemm_gfx950_impl.h"
#include "gemm_tiles.h"

namespace tbk {
static const KernelEntry kSmall[] = {TBK_TILES_SMALL(TBK_OUTS)};
const KernelEntry *entries_small(int *n) {
  *n = sizeof(kSmall) / sizeof(kSmall[0]);
  return kSmall;
}
} // namespace tbk
