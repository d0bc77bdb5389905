// RUN: not %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})' 2>&1 | FileCheck %s

// Register truth: the 4-wave 256x256x64 tile forced onto
// v_mfma_f32_32x32x16_f16 holds 256 accumulator registers per wave in 32x32
// tiles, and the compiler's report of that build (the instance resource
// table generated at build time) shows scratch. KernelConfig legality (the
// first pass that reads the gfx950 target) refuses it with the compiler's
// figures; without the forced instruction the plan binds the
// 16x16x32 instance of the same tile, which does not spill.
module attributes {"tb.num-warps" = 4 : i64, "tb.requested-stages" = 2 : i64} {
  func.func @kernel(%A: memref<512x256xf16>, %B: memref<256x768xf16>,
                    %C: memref<512x768xf16>) {
    tb.matmul %A, %B, %C {block_m = 256 : i64, block_n = 256 : i64,
                          block_k = 64 : i64, exact_tile = true,
                          mma = "mfma_f32_32x32x16_f16"}
      : memref<512x256xf16>, memref<256x768xf16>, memref<512x768xf16>
    func.return
  }
}

// CHECK: error: tb-build-program-mapping-plan: gfx950 kernel instance tb_gemm_gfx950_256x256x64_w2x2_s2_out0 spills {{[0-9]+}} bytes per lane to scratch
// CHECK-SAME: compiler report of gemm_kernel<256, 256, 64, 2, 2, 0, 2, -1, 0>
