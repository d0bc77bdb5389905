// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})' | FileCheck %s

// The split-k configuration of the benchmark: 512x512x16384, 8 splits,
// f16 C, deterministic f32 workspace reduction.
module attributes {"tb.num-warps" = 4 : i64, "tb.requested-stages" = 2 : i64,
                   "tb.split-k" = 8 : i64,
                   "tb.reduction-mode" = "split_k_serial"} {
  func.func @kernel(%A: memref<512x16384xf16>, %B: memref<16384x512xf16>,
                    %C: memref<512x512xf16>) {
    tb.matmul %A, %B, %C {block_m = 128 : i64, block_n = 128 : i64,
                          block_k = 64 : i64, exact_tile = true}
      : memref<512x16384xf16>, memref<16384x512xf16>, memref<512x512xf16>
    func.return
  }
}

// CHECK: tb.gfx950_launch
// CHECK-SAME: c_dtype = 0 : i64
// CHECK-SAME: mapping = 2 : i64
// CHECK-SAME: num_programs = 128 : i64
// CHECK-SAME: reduction = 1 : i64
// CHECK-SAME: split_k = 8 : i64
// CHECK-SAME: kernel = "tb_gemm_gfx950_128x128x64_w2x2_s2_out1"
// CHECK-SAME: workspace_bytes = 8388608 : i64
