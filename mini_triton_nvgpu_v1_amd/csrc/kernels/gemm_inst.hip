// gfx950 GEMM instances of one macro-tile shape: TBK_SHAPE names a list of
// gemm_tiles.h (e.g. 128x128); TBK_EPI=0 instantiates it in every output
// mode, TBK_EPI=1 with the fused epilogue steps. The Makefile compiles this
// file once per shape and flavour, so the instances build in parallel.
#include "gemm_gfx950_impl.h"
#include "gemm_tiles.h"

#if !defined(TBK_SHAPE) || !defined(TBK_EPI)
#error "compile with -DTBK_SHAPE=<shape of gemm_tiles.h> -DTBK_EPI=0|1"
#endif

#define TBK_CAT2(a, b) a##b
#define TBK_CAT(a, b) TBK_CAT2(a, b)
#if TBK_EPI
#define TBK_EACH TBK_EPI_OUTS
#define TBK_TABLE TBK_CAT(TBK_CAT(entries_, TBK_SHAPE), _epi)
#else
#define TBK_EACH TBK_OUTS
#define TBK_TABLE TBK_CAT(entries_, TBK_SHAPE)
#endif

namespace tbk {
static const KernelEntry kEntries[] = {TBK_CAT(TBK_TILES_, TBK_SHAPE)(TBK_EACH)};
const KernelEntry *TBK_TABLE(int *n) {
  *n = sizeof(kEntries) / sizeof(kEntries[0]);
  return kEntries;
}
} // namespace tbk
