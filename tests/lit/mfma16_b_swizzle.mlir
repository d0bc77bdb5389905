// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-mainline-pipeline)' | FileCheck %s

// The roofline tile on v_mfma_f32_16x16x32_f16: the B stage [64][256] f16 is
// read by ds_read_b64_tr_b16, whose 32-lane LDS cycle serves two 16-lane
// groups reading the same 16 columns of k rows 8 apart. The first XOR term
// (64-byte segments, phase k % 4, the reference's form from
// LowerPipelineToNVGPU.cpp:1589-1621) gives those rows the same phase; the
// gfx950 second term (32-byte units, phase (k / 8) % 2) separates them, so
// the read is conflict-free: chunk' = chunk ^ 4 (k % 4) ^ 2 ((k / 8) % 2).
// A keeps one term (16-byte chunks, phase (row / 2) % 8).
module attributes {"tb.num-warps" = 4 : i64, "tb.requested-stages" = 2 : i64} {
  func.func @kernel(%A: memref<512x256xf16>, %B: memref<256x512xf16>,
                    %C: memref<512x512xf16>) {
    tb.matmul %A, %B, %C {block_m = 256 : i64, block_n = 256 : i64,
                          block_k = 64 : i64, exact_tile = true}
      : memref<512x256xf16>, memref<256x512xf16>, memref<512x512xf16>
    func.return
  }
}

// CHECK: tb.encoding_plan = {
// CHECK-SAME: encoding = #tb.shared<order = [1, 0], perPhase = 2, maxPhase = 8, transposed = false, swizzlingByteWidth = 16, cga = #tb.cga<ctasPerCGA = [1, 1, 1], ctaSplitNum = [1, 1, 1], ctaOrder = [0, 1, 2]>>, name = "a_shared"
// CHECK-SAME: encoding = #tb.shared<order = [1, 0], perPhase = 1, maxPhase = 4, transposed = false, swizzlingByteWidth = 64, cga = #tb.cga<ctasPerCGA = [1, 1, 1], ctaSplitNum = [1, 1, 1], ctaOrder = [0, 1, 2]>, secondPerPhase = 8, secondMaxPhase = 2, secondSwizzlingByteWidth = 32>, name = "b_shared"
