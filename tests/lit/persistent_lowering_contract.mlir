// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})' | FileCheck %s

module attributes {"tb.num-warps" = 4 : i64, "tb.requested-stages" = 2 : i64,
                   "tb.persistent" = true, "tb.num-ctas" = 2 : i64} {
  func.func @kernel(%A: memref<192x32xf16>, %B: memref<32x128xf16>,
                    %C: memref<192x128xf32>) {
    tb.matmul %A, %B, %C {block_m = 64 : i64, block_n = 64 : i64,
                          block_k = 32 : i64, exact_tile = true}
      : memref<192x32xf16>, memref<32x128xf16>, memref<192x128xf32>
    func.return
  }
}

// Two resident workgroups of 4 waves loop over the 6 tiles in grouped order
// (mapping 4 = TB_MAP_PERSISTENT_GROUPED) and accumulate into f32 C (out2).
// CHECK: tb.gfx950_launch %A, %B, %C
// CHECK-SAME: block = array<i64: 256, 1, 1>
// CHECK-SAME: acc_init = 1 : i64
// CHECK-SAME: c_dtype = 1 : i64
// CHECK-SAME: mapping = 4 : i64
// CHECK-SAME: num_programs = 2 : i64
// CHECK-SAME: grid = array<i64: 2, 1, 1>
// CHECK-SAME: kernel = "tb_gemm_gfx950_64x64x32_w2x2_s2_out2"
// CHECK-SAME: lds_bytes = 16384 : i64
// CHECK-NOT: tb.pipeline_mainline
