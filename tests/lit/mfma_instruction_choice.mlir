// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})' | FileCheck %s

// An 8-wave 256x256x64 tile asking for v_mfma_f32_32x32x16_f16 by name: the
// plan keeps 32x32x16 (no `mfma` field in the launch config) and binds the
// general instance of its 4x2 wave grid (64x128 wave tiles, no scratch).
module attributes {"tb.num-warps" = 8 : i64, "tb.requested-stages" = 2 : i64} {
  func.func @kernel(%A: memref<512x256xf16>, %B: memref<256x768xf16>,
                    %C: memref<512x768xf16>) {
    tb.matmul %A, %B, %C {block_m = 256 : i64, block_n = 256 : i64,
                          block_k = 64 : i64, exact_tile = true,
                          mma = "mfma_f32_32x32x16_f16"}
      : memref<512x256xf16>, memref<256x768xf16>, memref<512x768xf16>
    func.return
  }
}

// CHECK: tb.gfx950_launch
// CHECK-SAME: mapping = 1 : i64
// CHECK-NOT: mfma =
// CHECK-SAME: kernel = "tb_gemm_gfx950_256x256x64_w4x2_s2_out0"
