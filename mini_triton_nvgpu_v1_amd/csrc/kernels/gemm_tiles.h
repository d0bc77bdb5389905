// The compiled gfx950 tile configurations, as X-macro lists of
// (BM, BN, BK, wave grid M, wave grid N, LDS stages). Each list is
// instantiated twice: plain (every output mode) and with the fused epilogue
// steps (the modes that write a whole result).
#pragma once

// 64x64 macro-tiles (launch-bound shapes)
#define TBK_TILES_SMALL(X)                                                      \
  X(64, 64, 32, 1, 1, 2), X(64, 64, 32, 1, 1, 3), X(64, 64, 32, 2, 1, 2),       \
      X(64, 64, 32, 2, 2, 2), X(64, 64, 32, 2, 2, 3), X(64, 64, 32, 2, 2, 4),   \
      X(64, 64, 64, 1, 1, 2), X(64, 64, 64, 2, 2, 2), X(64, 64, 64, 2, 2, 3)

// 128-wide macro-tiles (mid sizes, split-K partials). The 4x1 / 1x4 grids
// are the ones the plan derives for 4 waves on 128x64 / 64x128 tiles (equal
// wave-tile imbalance; ties go to more waves along the long side).
#define TBK_TILES_MID(X)                                                        \
  X(128, 128, 32, 2, 2, 2), X(128, 128, 32, 2, 2, 3), X(128, 128, 32, 2, 2, 4), \
      X(128, 128, 64, 2, 2, 2), X(128, 128, 64, 2, 2, 3),                       \
      X(128, 128, 64, 2, 2, 4), X(128, 64, 64, 2, 2, 2), X(128, 64, 64, 2, 2, 3), \
      X(64, 128, 64, 2, 2, 2), X(64, 128, 64, 2, 2, 3), X(128, 64, 64, 4, 1, 2), \
      X(128, 64, 64, 4, 1, 3), X(64, 128, 64, 1, 4, 2), X(64, 128, 64, 1, 4, 3), \
      X(128, 64, 32, 4, 1, 2), X(64, 128, 32, 1, 4, 2)

// 256-wide macro-tiles (the MFMA-bound configs). 8 waves (2 per SIMD: one
// wave's MFMAs run while the other waits) in the 4x2 grid the plan derives
// for 8 waves on a 256x256 tile come first. The 4x1 / 1x4 grids are the ones
// the plan derives for 4 waves on 256x128 / 128x256 tiles.
#define TBK_TILES_LARGE(X)                                                      \
  X(256, 256, 64, 4, 2, 2), X(256, 256, 32, 4, 2, 3), X(256, 256, 32, 4, 2, 4), \
      X(256, 256, 64, 2, 2, 2), X(256, 256, 32, 2, 2, 2),                       \
      X(256, 256, 32, 2, 2, 3), X(256, 256, 32, 2, 2, 4),                       \
      X(256, 128, 64, 2, 2, 2), X(256, 128, 64, 2, 2, 3),                       \
      X(128, 256, 64, 2, 2, 2), X(128, 256, 64, 2, 2, 3),                       \
      X(256, 128, 64, 4, 1, 2), X(128, 256, 64, 1, 4, 2)
