// gfx950 GEMM instances: the small tile list with the fused epilogue steps
// (bias, activation, clamp), for the output modes that write a whole result.
#include "gemm_gfx950_impl.h"
#include "gemm_tiles.h"

namespace tbk {
static const KernelEntry kSmallEpi[] = {TBK_TILES_SMALL(TBK_EPI_OUTS)};
const KernelEntry *entries_small_epi(int *n) {
  *n = sizeof(kSmallEpi) / sizeof(kSmallEpi[0]);
  return kSmallEpi;
}
} // namespace tbk
