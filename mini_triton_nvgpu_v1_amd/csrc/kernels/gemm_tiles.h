// The compiled gfx950 tile configurations, as X-macro lists of
// (BM, BN, BK, wave grid M, wave grid N, LDS stages), one list per macro-tile
// shape. Each list is instantiated twice (gemm_inst.hip, compiled once per
// shape and flavour by the Makefile): plain, in every output mode, and with
// the fused epilogue steps, in the modes that write a whole result.
//
// This file is plain preprocessor text, included by the kernels and by the
// host-side plan code: the plan's KernelConfig legality and the lowering
// refuse a configuration that has no entry here (csrc/plan/instances.cpp),
// so a plan never names a kernel that does not exist.
//
// The lists hold, for every shape, block_k in {32, 64}, 1 / 2 / 4 / 8 waves
// and 2 / 3 / 4 LDS stages, the wave grid the plan derives (minimal
// |wave_tile_m - wave_tile_n|, ties to more waves along the longer side),
// wherever the kernel template can run it:
//  * the LDS ring fits 160 KiB and the wave tile holds at most 256
//    accumulator registers per lane (16 tiles of 32x32);
//  * an operand's k-tile is whole wavefronts' rounds of 16-byte direct loads
//    (8 waves on a 32-deep k-tile of a 64- or 128-wide side leave whole
//    waves idle in the last round), and a lane's B swizzle phase is the same
//    in every load round (so 1 wave cannot load 256-wide B rows);
//  * the loads a thread may have in flight at a wait fit the 6-bit vmcnt
//    field (at most 63: 1 wave on 128x128x64 or 256x64x64 tiles stops at 3
//    stages);
// plus the 2x2 grids of 4 waves on 128x64, 64x128, 256x128 and 128x256 tiles
// (reachable through tb_desc_create). 192x128 tiles give persistent grids
// whose last row of tiles is ragged at 8192 rows.
#pragma once

// shapes with a list below (the Makefile reads these names)
#define TBK_SHAPES(S)                                                           \
  S(64x64) S(64x128) S(128x64) S(128x128) S(64x256) S(256x64) S(128x256)       \
      S(256x128) S(256x256) S(192x128) S(192x64) S(192x256) S(64x192) S(128x192)   \
          S(192x192) S(256x192)

// Tiles whose plain f32-partial instance (output mode 1: split-K partials and
// plain f32 C) is built with producer waves (gemm_kernel_pw: as many load-only
// waves as compute waves), in place of the general loop's build of the same
// key. The key serves split-K partials and plain f32 C alike, so a tile is
// listed where the build measured at least as fast in both (same box,
// bit-identical results):
//  * 128x64x64 on 8 waves, 3 stages, the split-K workload's tile: 512^2 x
//    16384 in 8 splits 18.9 -> 16.8 us per call; 2048^3 plain f32 C equal;
//  * 64x64x64 on 4 waves, 3 stages: 256^2 x 32768 in 16 splits 16.9 -> 15.0
//    us per call; 2048^3 plain f32 C 40.6 -> 35.6 us.
// Not listed: 64x128 (2x4, 2x2) and 128x64 (2x2) gain 5-10% on split-K but
// lose 12-23% on plain f32 C; 128x128 and 256x64 gain nothing.
// Entries are not separated: each X supplies its own separator.
#define TBK_PRODUCER_TILES(X) X(128, 64, 64, 4, 2, 3) X(64, 64, 64, 2, 2, 3)

#define TBK_TILES_64x64(X) \
  X(64, 64, 32, 1, 1, 2), X(64, 64, 32, 1, 1, 3), X(64, 64, 32, 1, 1, 4), \
  X(64, 64, 32, 2, 1, 2), X(64, 64, 32, 2, 1, 3), X(64, 64, 32, 2, 1, 4), \
  X(64, 64, 32, 2, 2, 2), X(64, 64, 32, 2, 2, 3), X(64, 64, 32, 2, 2, 4), \
  X(64, 64, 64, 1, 1, 2), X(64, 64, 64, 1, 1, 3), X(64, 64, 64, 1, 1, 4), \
  X(64, 64, 64, 2, 1, 2), X(64, 64, 64, 2, 1, 3), X(64, 64, 64, 2, 1, 4), \
  X(64, 64, 64, 2, 2, 2), X(64, 64, 64, 2, 2, 3), X(64, 64, 64, 2, 2, 4)

#define TBK_TILES_64x128(X) \
  X(64, 128, 32, 1, 1, 2), X(64, 128, 32, 1, 1, 3), \
  X(64, 128, 32, 1, 1, 4), X(64, 128, 32, 1, 2, 2), \
  X(64, 128, 32, 1, 2, 3), X(64, 128, 32, 1, 2, 4), \
  X(64, 128, 32, 1, 4, 2), X(64, 128, 32, 1, 4, 3), \
  X(64, 128, 32, 1, 4, 4), X(64, 128, 64, 1, 1, 2), \
  X(64, 128, 64, 1, 1, 3), X(64, 128, 64, 1, 1, 4), \
  X(64, 128, 64, 1, 2, 2), X(64, 128, 64, 1, 2, 3), \
  X(64, 128, 64, 1, 2, 4), X(64, 128, 64, 1, 4, 2), \
  X(64, 128, 64, 1, 4, 3), X(64, 128, 64, 1, 4, 4), \
  X(64, 128, 64, 2, 2, 2), X(64, 128, 64, 2, 2, 3), \
  X(64, 128, 64, 2, 4, 2), X(64, 128, 64, 2, 4, 3), \
  X(64, 128, 64, 2, 4, 4), X(64, 128, 32, 2, 4, 2), \
  X(64, 128, 32, 2, 4, 3), X(64, 128, 32, 2, 4, 4)

#define TBK_TILES_128x64(X) \
  X(128, 64, 32, 1, 1, 2), X(128, 64, 32, 1, 1, 3), \
  X(128, 64, 32, 1, 1, 4), X(128, 64, 32, 2, 1, 2), \
  X(128, 64, 32, 2, 1, 3), X(128, 64, 32, 2, 1, 4), \
  X(128, 64, 32, 4, 1, 2), X(128, 64, 32, 4, 1, 3), \
  X(128, 64, 32, 4, 1, 4), X(128, 64, 64, 1, 1, 2), \
  X(128, 64, 64, 1, 1, 3), X(128, 64, 64, 1, 1, 4), \
  X(128, 64, 64, 2, 1, 2), X(128, 64, 64, 2, 1, 3), \
  X(128, 64, 64, 2, 1, 4), X(128, 64, 64, 2, 2, 2), \
  X(128, 64, 64, 2, 2, 3), X(128, 64, 64, 4, 1, 2), \
  X(128, 64, 64, 4, 1, 3), X(128, 64, 64, 4, 1, 4), \
  X(128, 64, 64, 4, 2, 2), X(128, 64, 64, 4, 2, 3), \
  X(128, 64, 64, 4, 2, 4), X(128, 64, 32, 4, 2, 2), \
  X(128, 64, 32, 4, 2, 3), X(128, 64, 32, 4, 2, 4)

#define TBK_TILES_128x128(X) \
  X(128, 128, 32, 1, 1, 2), X(128, 128, 32, 1, 1, 3), \
  X(128, 128, 32, 1, 1, 4), X(128, 128, 32, 2, 1, 2), \
  X(128, 128, 32, 2, 1, 3), X(128, 128, 32, 2, 1, 4), \
  X(128, 128, 32, 2, 2, 2), X(128, 128, 32, 2, 2, 3), \
  X(128, 128, 32, 2, 2, 4), X(128, 128, 32, 4, 2, 2), \
  X(128, 128, 32, 4, 2, 3), X(128, 128, 32, 4, 2, 4), \
  X(128, 128, 64, 1, 1, 2), X(128, 128, 64, 1, 1, 3), \
  X(128, 128, 64, 2, 1, 2), X(128, 128, 64, 2, 1, 3), \
  X(128, 128, 64, 2, 1, 4), X(128, 128, 64, 2, 2, 2), \
  X(128, 128, 64, 2, 2, 3), X(128, 128, 64, 2, 2, 4), \
  X(128, 128, 64, 4, 2, 2), X(128, 128, 64, 4, 2, 3), \
  X(128, 128, 64, 4, 2, 4)

#define TBK_TILES_64x256(X) \
  X(64, 256, 32, 1, 2, 2), X(64, 256, 32, 1, 2, 3), \
  X(64, 256, 32, 1, 2, 4), X(64, 256, 32, 1, 4, 2), \
  X(64, 256, 32, 1, 4, 3), X(64, 256, 32, 1, 4, 4), \
  X(64, 256, 64, 1, 2, 2), X(64, 256, 64, 1, 2, 3), \
  X(64, 256, 64, 1, 2, 4), X(64, 256, 64, 1, 4, 2), \
  X(64, 256, 64, 1, 4, 3), X(64, 256, 64, 1, 4, 4), \
  X(64, 256, 64, 1, 8, 2), X(64, 256, 64, 1, 8, 3), \
  X(64, 256, 64, 1, 8, 4), X(64, 256, 32, 1, 8, 2), \
  X(64, 256, 32, 1, 8, 3), X(64, 256, 32, 1, 8, 4)

#define TBK_TILES_256x64(X) \
  X(256, 64, 32, 1, 1, 2), X(256, 64, 32, 1, 1, 3), \
  X(256, 64, 32, 1, 1, 4), X(256, 64, 32, 2, 1, 2), \
  X(256, 64, 32, 2, 1, 3), X(256, 64, 32, 2, 1, 4), \
  X(256, 64, 32, 4, 1, 2), X(256, 64, 32, 4, 1, 3), \
  X(256, 64, 32, 4, 1, 4), X(256, 64, 64, 1, 1, 2), \
  X(256, 64, 64, 1, 1, 3), X(256, 64, 64, 2, 1, 2), \
  X(256, 64, 64, 2, 1, 3), X(256, 64, 64, 2, 1, 4), \
  X(256, 64, 64, 4, 1, 2), X(256, 64, 64, 4, 1, 3), \
  X(256, 64, 64, 4, 1, 4), X(256, 64, 64, 8, 1, 2), \
  X(256, 64, 64, 8, 1, 3), X(256, 64, 64, 8, 1, 4), \
  X(256, 64, 32, 8, 1, 2), X(256, 64, 32, 8, 1, 3), \
  X(256, 64, 32, 8, 1, 4)

#define TBK_TILES_128x256(X) \
  X(128, 256, 32, 1, 2, 2), X(128, 256, 32, 1, 2, 3), \
  X(128, 256, 32, 1, 2, 4), X(128, 256, 32, 1, 4, 2), \
  X(128, 256, 32, 1, 4, 3), X(128, 256, 32, 1, 4, 4), \
  X(128, 256, 32, 2, 4, 2), X(128, 256, 32, 2, 4, 3), \
  X(128, 256, 32, 2, 4, 4), X(128, 256, 64, 1, 2, 2), \
  X(128, 256, 64, 1, 2, 3), X(128, 256, 64, 1, 4, 2), \
  X(128, 256, 64, 1, 4, 3), X(128, 256, 64, 2, 2, 2), \
  X(128, 256, 64, 2, 2, 3), X(128, 256, 64, 2, 4, 2), \
  X(128, 256, 64, 2, 4, 3)

#define TBK_TILES_256x128(X) \
  X(256, 128, 32, 2, 1, 2), X(256, 128, 32, 2, 1, 3), \
  X(256, 128, 32, 2, 1, 4), X(256, 128, 32, 4, 1, 2), \
  X(256, 128, 32, 4, 1, 3), X(256, 128, 32, 4, 1, 4), \
  X(256, 128, 32, 4, 2, 2), X(256, 128, 32, 4, 2, 3), \
  X(256, 128, 32, 4, 2, 4), X(256, 128, 64, 2, 1, 2), \
  X(256, 128, 64, 2, 1, 3), X(256, 128, 64, 2, 2, 2), \
  X(256, 128, 64, 2, 2, 3), X(256, 128, 64, 4, 1, 2), \
  X(256, 128, 64, 4, 1, 3), X(256, 128, 64, 4, 2, 2), \
  X(256, 128, 64, 4, 2, 3)

#define TBK_TILES_256x256(X) \
  X(256, 256, 32, 2, 2, 2), X(256, 256, 32, 2, 2, 3), \
  X(256, 256, 32, 2, 2, 4), X(256, 256, 32, 4, 2, 2), \
  X(256, 256, 32, 4, 2, 3), X(256, 256, 32, 4, 2, 4), \
  X(256, 256, 64, 2, 2, 2), X(256, 256, 64, 4, 2, 2)

#define TBK_TILES_192x128(X) \
  X(192, 128, 32, 2, 1, 2), X(192, 128, 32, 2, 1, 3), \
  X(192, 128, 32, 2, 1, 4), X(192, 128, 32, 2, 2, 2), \
  X(192, 128, 32, 2, 2, 3), X(192, 128, 32, 2, 2, 4), \
  X(192, 128, 32, 2, 4, 2), X(192, 128, 32, 2, 4, 3), \
  X(192, 128, 32, 2, 4, 4), X(192, 128, 64, 2, 1, 2), \
  X(192, 128, 64, 2, 1, 3), X(192, 128, 64, 2, 1, 4), \
  X(192, 128, 64, 2, 2, 2), X(192, 128, 64, 2, 2, 3), \
  X(192, 128, 64, 2, 2, 4), X(192, 128, 64, 2, 4, 2), \
  X(192, 128, 64, 2, 4, 3), X(192, 128, 64, 2, 4, 4)

// 192-row blocks on 64- and 256-wide B (96-row wave tiles: 3 MFMA tiles of
// 32 per wave column)
#define TBK_TILES_192x64(X) \
  X(192, 64, 32, 1, 1, 2), X(192, 64, 32, 1, 1, 3), X(192, 64, 32, 1, 1, 4), \
  X(192, 64, 32, 2, 1, 2), X(192, 64, 32, 2, 1, 3), X(192, 64, 32, 2, 1, 4), \
  X(192, 64, 32, 2, 2, 2), X(192, 64, 32, 2, 2, 3), X(192, 64, 32, 2, 2, 4), \
  X(192, 64, 64, 1, 1, 2), X(192, 64, 64, 1, 1, 3), \
  X(192, 64, 64, 2, 1, 2), X(192, 64, 64, 2, 1, 3), X(192, 64, 64, 2, 1, 4), \
  X(192, 64, 64, 2, 2, 2), X(192, 64, 64, 2, 2, 3), X(192, 64, 64, 2, 2, 4)

#define TBK_TILES_192x256(X) \
  X(192, 256, 32, 2, 2, 2), X(192, 256, 32, 2, 2, 3), X(192, 256, 32, 2, 2, 4), \
  X(192, 256, 32, 2, 4, 2), X(192, 256, 32, 2, 4, 3), X(192, 256, 32, 2, 4, 4), \
  X(192, 256, 64, 2, 2, 2), X(192, 256, 64, 2, 4, 2)

// 192-wide B (384-byte rows: a load round ends inside a row, so each round
// has its own lane offsets; B swizzle 2 rows per phase, 2 phases)
#define TBK_TILES_64x192(X) \
  X(64, 192, 32, 1, 1, 2), X(64, 192, 32, 1, 1, 3), X(64, 192, 32, 1, 1, 4), \
  X(64, 192, 32, 1, 2, 2), X(64, 192, 32, 1, 2, 3), X(64, 192, 32, 1, 2, 4), \
  X(64, 192, 32, 2, 2, 2), X(64, 192, 32, 2, 2, 3), X(64, 192, 32, 2, 2, 4), \
  X(64, 192, 64, 1, 1, 2), X(64, 192, 64, 1, 1, 3), X(64, 192, 64, 1, 2, 2), \
  X(64, 192, 64, 1, 2, 3), X(64, 192, 64, 1, 2, 4), X(64, 192, 64, 2, 2, 2), \
  X(64, 192, 64, 2, 2, 3), X(64, 192, 64, 2, 2, 4)

#define TBK_TILES_128x192(X) \
  X(128, 192, 32, 1, 2, 2), X(128, 192, 32, 1, 2, 3), X(128, 192, 32, 1, 2, 4), \
  X(128, 192, 32, 2, 2, 2), X(128, 192, 32, 2, 2, 3), X(128, 192, 32, 2, 2, 4), \
  X(128, 192, 32, 4, 2, 2), X(128, 192, 32, 4, 2, 3), X(128, 192, 32, 4, 2, 4), \
  X(128, 192, 64, 1, 2, 2), X(128, 192, 64, 1, 2, 3), X(128, 192, 64, 1, 2, 4), \
  X(128, 192, 64, 2, 2, 2), X(128, 192, 64, 2, 2, 3), X(128, 192, 64, 2, 2, 4), \
  X(128, 192, 64, 4, 2, 2), X(128, 192, 64, 4, 2, 3), X(128, 192, 64, 4, 2, 4)

#define TBK_TILES_192x192(X) \
  X(192, 192, 32, 2, 2, 2), X(192, 192, 32, 2, 2, 3), X(192, 192, 32, 2, 2, 4), \
  X(192, 192, 64, 2, 2, 2), X(192, 192, 64, 2, 2, 3)

#define TBK_TILES_256x192(X) \
  X(256, 192, 32, 2, 2, 2), X(256, 192, 32, 2, 2, 3), X(256, 192, 32, 2, 2, 4), \
  X(256, 192, 32, 4, 2, 2), X(256, 192, 32, 4, 2, 3), X(256, 192, 32, 4, 2, 4), \
  X(256, 192, 64, 2, 2, 2), X(256, 192, 64, 4, 2, 2)

// ---- the 16x16x32 loop (gemm_mfma16g.h) ------------------------------------
// Tiles built on v_mfma_f32_16x16x32_f16 besides the hand-scheduled 4-wave
// 256x256x64 2-stage instance, as (BM, BN, BK, wave grid M, wave grid N,
// LDS stages), one list per block shape (the Makefile compiles each list
// plain and with the fused epilogue steps, in the f16, plain f32 and
// f32 C += A*B modes). Wave tiles hold 16..64 MFMA tiles of 16x16 (at most
// 256 accumulator registers); the wave grid is the one the plan derives.
// (The hand-scheduled tile's partial-K build is this loop too, instantiated
// with its entries. 8 waves of 64x128 on 256x256 do not fit their 256
// registers per wave and are not listed.) The lists cover the 4- and 8-wave
// picks of the common blocks, and the wave tiles whose 32x32x16 builds
// spill: 128x128 (1 wave on 128x128, 2 on 256x128 / 128x256), 256x64 and
// 192x64 (1 wave) and 96x128 (2 waves on 192x128), at block_k 32 and 64
// wherever the prologue's loads (every stage's k-tile) fit the 6-bit vmcnt.
// 32-deep k-tiles run whole k-tile bodies with no tail, so their wave tiles
// of 48 or 64 MFMA tiles hold their accumulators without a merge.
#define TBK_M16_SHAPES(S)                                                              \
  S(128x128) S(256x128) S(128x256) S(256x64) S(192x128) S(256x256) S(192x64)

#define TBK_M16_TILES_128x128(X) \
  X(128, 128, 64, 2, 2, 2), X(128, 128, 64, 2, 2, 3), X(128, 128, 64, 2, 2, 4), \
  X(128, 128, 32, 2, 2, 2), X(128, 128, 32, 2, 2, 3), X(128, 128, 32, 2, 2, 4), \
  X(128, 128, 64, 1, 1, 2), \
  X(128, 128, 32, 1, 1, 2), X(128, 128, 32, 1, 1, 3), X(128, 128, 32, 1, 1, 4)

#define TBK_M16_TILES_256x128(X) \
  X(256, 128, 64, 4, 1, 2), X(256, 128, 64, 4, 1, 3), \
  X(256, 128, 32, 4, 1, 2), X(256, 128, 32, 4, 1, 3), X(256, 128, 32, 4, 1, 4), \
  X(256, 128, 64, 4, 2, 2), X(256, 128, 64, 4, 2, 3), \
  X(256, 128, 64, 2, 1, 2), X(256, 128, 64, 2, 1, 3), \
  X(256, 128, 32, 2, 1, 2), X(256, 128, 32, 2, 1, 3), X(256, 128, 32, 2, 1, 4)

#define TBK_M16_TILES_128x256(X) \
  X(128, 256, 64, 1, 4, 2), X(128, 256, 64, 1, 4, 3), \
  X(128, 256, 32, 1, 4, 2), X(128, 256, 32, 1, 4, 3), X(128, 256, 32, 1, 4, 4), \
  X(128, 256, 64, 2, 4, 2), X(128, 256, 64, 2, 4, 3), \
  X(128, 256, 64, 1, 2, 2), X(128, 256, 64, 1, 2, 3), \
  X(128, 256, 32, 1, 2, 2), X(128, 256, 32, 1, 2, 3), X(128, 256, 32, 1, 2, 4)


#define TBK_M16_TILES_256x64(X) \
  X(256, 64, 64, 1, 1, 2), X(256, 64, 32, 1, 1, 2), X(256, 64, 32, 1, 1, 3), \
  X(256, 64, 32, 1, 1, 4)

// one wave of 192x64 (its 32x32x16 build spills)
#define TBK_M16_TILES_192x64(X) X(192, 64, 64, 1, 1, 2)

// 4 waves of 128x128 on 256x256 with 32-deep k-tiles: in 3 or 4 LDS stages
// the same 128 KiB ring as the hand-scheduled 64-deep 2-stage tile, cut
// into k-tiles of half the depth (half the loads and reads per barrier); in
// 2 stages the key whose 32x32x16 build spills
#define TBK_M16_TILES_256x256(X) \
  X(256, 256, 32, 2, 2, 2), X(256, 256, 32, 2, 2, 3), X(256, 256, 32, 2, 2, 4)

#define TBK_M16_TILES_192x128(X) \
  X(192, 128, 64, 2, 1, 2), X(192, 128, 64, 2, 1, 3), X(192, 128, 64, 2, 1, 4), \
  X(192, 128, 64, 2, 2, 2), X(192, 128, 64, 2, 2, 3), X(192, 128, 64, 2, 2, 4), \
  X(192, 128, 32, 2, 2, 2), X(192, 128, 32, 2, 2, 3), X(192, 128, 32, 2, 2, 4)
