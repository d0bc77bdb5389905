// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})' | FileCheck %s
// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-mainline-pipeline)' | FileCheck %s --check-prefix=PLAN

// The benchmark's split-k workload on its tuned tile: 128x64x64 on a 4x2
// wave grid of 32x32 wave tiles, 3 LDS stages, 8 splits of 16384. Its f32
// partial instance is built with producer waves: 8 more waves that only
// issue the direct-to-LDS loads (3 per lane per k-tile). They issue k-tiles
// 0..2 in the prologue and wait for k-tile 0 only (vmcnt(6)); at each
// barrier the next k-tile has landed (vmcnt(3)) and the stage the barrier
// frees is refilled whole. The launch's block counts both halves: 16 waves
// of 64 lanes. The f16 instance of the same tile keeps the general loop,
// whose waits are the same ("burst") without loader waves.
module attributes {"tb.num-warps" = 8 : i64, "tb.requested-stages" = 3 : i64,
                   "tb.split-k" = 8 : i64,
                   "tb.reduction-mode" = "split_k_serial"} {
  func.func @kernel(%A: memref<512x16384xf16>, %B: memref<16384x512xf16>,
                    %C: memref<512x512xf16>) {
    tb.matmul %A, %B, %C {block_m = 128 : i64, block_n = 64 : i64,
                          block_k = 64 : i64, exact_tile = true}
      : memref<512x16384xf16>, memref<16384x512xf16>, memref<512x512xf16>
    func.return
  }
}

// CHECK: tb.gfx950_launch
// CHECK-SAME: block = array<i64: 1024, 1, 1>
// CHECK-SAME: mapping = 2 : i64
// CHECK-SAME: reduction = 1 : i64
// CHECK-SAME: split_k = 8 : i64
// CHECK-SAME: kernel = "tb_gemm_gfx950_128x64x64_w4x2_s3_out1"
// CHECK-SAME: waits = array<i64: 6, 3, -1>

// PLAN: tb.async_plan = {
// PLAN-SAME: issue_schedule = "producer_waves"
// PLAN-SAME: loader_waves = 8 : i64
// PLAN-SAME: loads_per_thread = 3 : i64
// PLAN-SAME: prologue_tail_loads = 3 : i64
// PLAN-SAME: waits = [{
// PLAN-SAME: group_id = 0 : i64, lgkmcnt_allowance = -1 : i64
// PLAN-SAME: vmcnt_allowance = 6 : i64
// PLAN-SAME: group_id = 1 : i64, lgkmcnt_allowance = -1 : i64
// PLAN-SAME: vmcnt_allowance = 3 : i64
