// The producer-wave builds of the f32-partial instances listed in
// TBK_PRODUCER_TILES (gemm_tiles.h). The registry (aux_kernels.hip) returns
// them in place of the general loop's entries of the same keys.
#include "gemm_gfx950_impl.h"
#include "gemm_tiles.h"

namespace tbk {
#define TBK_PW_ENTRY(BM, BN, BK, WGM, WGN, ST)                                    \
  {{BM, BN, BK, WGM, WGN, kOutF32Partial, ST, 0},                                 \
   reinterpret_cast<const void *>(&gemm_kernel_pw<BM, BN, BK, WGM, WGN, ST>),     \
   "tb_gemm_gfx950_" #BM "x" #BN "x" #BK "_w" #WGM "x" #WGN "_s" #ST "_out1",     \
   (ST - 1) * GemmTile<BM, BN, BK, WGM, WGN, ST>::LPT,                            \
   (ST - 2) * GemmTile<BM, BN, BK, WGM, WGN, ST>::LPT, -1, nullptr,               \
   2 * WGM * WGN * 64},
static const KernelEntry kProducer[] = {TBK_PRODUCER_TILES(TBK_PW_ENTRY)};
#undef TBK_PW_ENTRY
const KernelEntry *entries_producer(int *n) {
  *n = sizeof(kProducer) / sizeof(kProducer[0]);
  return kProducer;
}
} // namespace tbk
