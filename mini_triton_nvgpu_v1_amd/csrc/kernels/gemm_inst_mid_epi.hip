// gfx950 GEMM instances: the mid tile list with the fused epilogue steps
// (bias, activation, clamp), for the output modes that write a whole result.
#include "gemm_gfx950_impl.h"
#include "gemm_tiles.h"

namespace tbk {
static const KernelEntry kMidEpi[] = {TBK_TILES_MID(TBK_EPI_OUTS)};
const KernelEntry *entries_mid_epi(int *n) {
  *n = sizeof(kMidEpi) / sizeof(kMidEpi[0]);
  return kMidEpi;
}
} // namespace tbk
