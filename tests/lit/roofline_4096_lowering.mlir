// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})' | FileCheck %s

// The roofline configuration: 4096^3 f16 -> f16, 256x256x64 tiles,
// GROUP_M = 8, 4 waves (a 2x2 wave grid of 128x128 wave tiles): 256 programs,
// one per CU, in XCD-aware program order. No `mma` attribute: whole tiles of
// this configuration take v_mfma_f32_16x16x32_f16 (mfma = 1).
module attributes {"tb.num-warps" = 4 : i64, "tb.requested-stages" = 2 : i64} {
  func.func @kernel(%A: memref<4096x4096xf16>, %B: memref<4096x4096xf16>,
                    %C: memref<4096x4096xf16>) {
    tb.matmul %A, %B, %C {block_m = 256 : i64, block_n = 256 : i64,
                          block_k = 64 : i64, exact_tile = true,
                          group_m = 8 : i64}
      : memref<4096x4096xf16>, memref<4096x4096xf16>, memref<4096x4096xf16>
    func.return
  }
}

// CHECK: tb.target = {
// CHECK-SAME: gpu_arch = "gfx950"
// CHECK-SAME: max_shared_bytes_per_cta = 163840
// CHECK-SAME: mma_instr_shape = array<i64: 32, 32, 16>
// CHECK-SAME: num_sms = 256
// CHECK-SAME: threads_per_warp = 64
// CHECK: tb.gfx950_launch
// CHECK-SAME: block = array<i64: 256, 1, 1>
// CHECK-SAME: group_m = 8 : i64
// CHECK-SAME: mapping = 1 : i64
// CHECK-SAME: mfma = 1 : i64
// CHECK-SAME: num_programs = 256 : i64
// CHECK-SAME: xcd_remap = 8 : i64
// CHECK-SAME: kernel = "tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32"
// CHECK-SAME: lds_bytes = 131072 : i64
// The waits the AsyncPlan states and the lowering checked against this
// instance: vmcnt(16) in the prologue (k-tile 1's 16 loads per lane still in
// flight), vmcnt(0) lgkmcnt(0) at each k-tile's barrier.
// CHECK-SAME: waits = array<i64: 16, 0, 0>
