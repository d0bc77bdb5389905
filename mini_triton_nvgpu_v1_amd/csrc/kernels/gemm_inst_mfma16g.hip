// 16x16x32 instances of one block shape of TBK_M16_SHAPES (gemm_tiles.h):
// TBK_SHAPE names the list, TBK_EPI=0 instantiates it plain and TBK_EPI=1
// with the fused epilogue steps, each with an f16 C, a plain f32 C and
// f32 C += A*B. The Makefile compiles this file once per shape and flavour.
#include "gemm_mfma16g.h"
#include "gemm_tiles.h"

#if !defined(TBK_SHAPE) || !defined(TBK_EPI)
#error "compile with -DTBK_SHAPE=<shape of TBK_M16_SHAPES> -DTBK_EPI=0|1"
#endif

#define TBK_CAT2(a, b) a##b
#define TBK_CAT(a, b) TBK_CAT2(a, b)
#define TBK_EPI_BOOL TBK_CAT(TBK_EPI_B, TBK_EPI)
#define TBK_EPI_B0 false
#define TBK_EPI_B1 true
#if TBK_EPI
#define TBK_M16_SUFFIX "_16x16x32_epi"
#define TBK_TABLE TBK_CAT(TBK_CAT(entries_m16_, TBK_SHAPE), _epi)
#else
#define TBK_M16_SUFFIX "_16x16x32"
#define TBK_TABLE TBK_CAT(entries_m16_, TBK_SHAPE)
#endif

#define TBK_M16_ENTRY(BM, BN, BK, WGM, WGN, ST, OUT)                                       \
  {{BM, BN, BK, WGM, WGN, OUT, ST, TBK_EPI, 1},                                           \
   reinterpret_cast<const void *>(                                                        \
       &gemm_mfma16g<BM, BN, BK, WGM, WGN, ST, OUT, TBK_EPI_BOOL>),                       \
   "tb_gemm_gfx950_" #BM "x" #BN "x" #BK "_w" #WGM "x" #WGN "_s" #ST "_out" #OUT          \
       TBK_M16_SUFFIX,                                                                    \
   Mfma16GTile<BM, BN, BK, WGM, WGN, ST>::VM_PROLOGUE,                                    \
   Mfma16GTile<BM, BN, BK, WGM, WGN, ST>::VM_LOOP, 0, nullptr, 0}
#define TBK_M16_OUTS(BM, BN, BK, WGM, WGN, ST)                                            \
  TBK_M16_ENTRY(BM, BN, BK, WGM, WGN, ST, 0), TBK_M16_ENTRY(BM, BN, BK, WGM, WGN, ST, 1), \
      TBK_M16_ENTRY(BM, BN, BK, WGM, WGN, ST, 2)

namespace tbk {
static const KernelEntry kEntries[] = {TBK_CAT(TBK_M16_TILES_, TBK_SHAPE)(TBK_M16_OUTS)};
const KernelEntry *TBK_TABLE(int *n) {
  *n = sizeof(kEntries) / sizeof(kEntries[0]);
  return kEntries;
}
} // namespace tbk
