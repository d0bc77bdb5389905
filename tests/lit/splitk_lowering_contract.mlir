// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})' | FileCheck %s

module attributes {"tb.num-warps" = 1 : i64, "tb.requested-stages" = 2 : i64,
                   "tb.split-k" = 2 : i64,
                   "tb.reduction-mode" = "split_k_parallel"} {
  func.func @kernel(%A: memref<64x64xf16>, %B: memref<64x64xf16>,
                    %C: memref<64x64xf32>) {
    tb.matmul %A, %B, %C {block_m = 64 : i64, block_n = 64 : i64,
                          block_k = 32 : i64, exact_tile = true}
      : memref<64x64xf16>, memref<64x64xf16>, memref<64x64xf32>
    func.return
  }
}

// split_k_parallel -> f32 global atomics (reduction 2 = TB_RED_ATOMIC,
// output mode 3), no workspace.
// CHECK: tb.gfx950_launch
// CHECK-SAME: mapping = 2 : i64
// CHECK-SAME: reduction = 2 : i64
// CHECK-SAME: split_k = 2 : i64
// CHECK-SAME: grid = array<i64: 2, 1, 1>
// CHECK-SAME: kernel = "tb_gemm_gfx950_64x64x32_w1x1_s2_out3"
// CHECK-SAME: workspace_bytes = 0 : i64
