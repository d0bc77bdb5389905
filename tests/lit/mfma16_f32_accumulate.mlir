// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})' | FileCheck %s

// The roofline configuration in the reference's own semantics: an f32 C, so
// C += A*B (the EpiloguePlan initialises from C). No `mma` attribute: the
// 4-wave 256x256x64 2-stage tile takes v_mfma_f32_16x16x32_f16 for an f32 C
// as well, and binds its C += A*B build (out2) with the same waits as the
// f16 build.
module attributes {"tb.num-warps" = 4 : i64, "tb.requested-stages" = 2 : i64} {
  func.func @kernel(%A: memref<4096x4096xf16>, %B: memref<4096x4096xf16>,
                    %C: memref<4096x4096xf32>) {
    tb.matmul %A, %B, %C {block_m = 256 : i64, block_n = 256 : i64,
                          block_k = 64 : i64, exact_tile = true,
                          group_m = 8 : i64}
      : memref<4096x4096xf16>, memref<4096x4096xf16>, memref<4096x4096xf32>
    func.return
  }
}

// CHECK: tb.gfx950_launch
// CHECK-SAME: acc_init = 1 : i64
// CHECK-SAME: c_dtype = 1 : i64
// CHECK-SAME: mfma = 1 : i64
// CHECK-SAME: kernel = "tb_gemm_gfx950_256x256x64_w2x2_s2_out2_16x16x32"
// CHECK-SAME: waits = array<i64: 16, 0, 0>
