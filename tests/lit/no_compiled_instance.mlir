// RUN: not %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})' 2>&1 | FileCheck %s
// RUN: %tb-opt %s --tb-verify-scope | FileCheck %s --check-prefix=SCOPE

// A configuration the reference's KernelConfig accepts (KernelConfig.cpp:
// 202-246: f16 inputs, block multiples of the MMA tile, 3 stages, 1 warp) and
// whose LDS ring fits gfx950's 160 KiB, but for which no gfx950 kernel
// instance is compiled: one wave cannot load a 256-wide B row ring with the
// 16-byte direct loads in whole rounds. The plan refuses it in the first
// plan pass that reads the gfx950 target, naming the block and the wave
// grids and stages that do exist, instead of lowering to a kernel name that
// would fail at launch.
module attributes {"tb.num-warps" = 1 : i64, "tb.requested-stages" = 3 : i64} {
  func.func @kernel(%A: memref<256x64xf16>, %B: memref<64x256xf16>,
                    %C: memref<256x256xf16>) {
    tb.matmul %A, %B, %C {block_m = 64 : i64, block_n = 256 : i64,
                          block_k = 32 : i64, exact_tile = true}
      : memref<256x64xf16>, memref<64x256xf16>, memref<256x256xf16>
    func.return
  }
}

// CHECK: error: tb-build-program-mapping-plan: no gfx950 kernel instance for block 64x256x32 on 1 waves (wave grid 1x1) with 3 LDS stages; compiled wave grids and stages for this block: 1x2 s2, 1x2 s3, 1x2 s4, 1x4 s2, 1x4 s3, 1x4 s4
// CHECK-NOT: tb.gfx950_launch

// tb-verify-scope has no target yet, so it does not know the kernels.
// SCOPE: tb.matmul
