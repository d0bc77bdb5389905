// gfx950 GEMM instances: the mid tile list, every output mode.
#include "gemm_gfx950_impl.h"
#include "gemm_tiles.h"

namespace tbk {
static const KernelEntry kMid[] = {TBK_TILES_MID(TBK_OUTS)};
const KernelEntry *entries_mid(int *n) {
  *n = sizeof(kMid) / sizeof(kMid[0]);
  return kMid;
}
} // namespace tbk
