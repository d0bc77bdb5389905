// gfx950 GEMM instances: the large tile list with the fused epilogue steps
// (bias, activation, clamp), for the output modes that write a whole result.
#include "gemm_gfx950_impl.h"
#include "gemm_tiles.h"

namespace tbk {
static const KernelEntry kLargeEpi[] = {TBK_TILES_LARGE(TBK_EPI_OUTS)};
const KernelEntry *entries_large_epi(int *n) {
  *n = sizeof(kLargeEpi) / sizeof(kLargeEpi[0]);
  return kLargeEpi;
}
} // namespace tbk
