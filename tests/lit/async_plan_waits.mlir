// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})' | FileCheck %s
// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-mainline-pipeline)' | FileCheck %s --check-prefix=PLAN

// 8 waves on a 256x256x64 tile with 2 LDS stages: a 4x2 wave grid of 64x128
// wave tiles, 8 MFMAs per 16-deep k step, so the kernel cuts each k-tile into
// 32 MFMA slots and spreads a refill's 8 loads per lane over the 8 slots
// from the barrier on (one per slot), 4 of them before the next barrier's
// half k step. The prologue issues k-tile 0 whole and those first 4 loads of
// k-tile 1, so its wait leaves 4 in flight: vmcnt(4), not the 8 of a
// prologue that issued k-tile 1 whole. The reference derives the wait at the
// first use (AsyncPlan.cpp:776-780); the gfx950 depth is the bound kernel's.
module attributes {"tb.num-warps" = 8 : i64, "tb.requested-stages" = 2 : i64} {
  func.func @kernel(%A: memref<1024x512xf16>, %B: memref<512x1024xf16>,
                    %C: memref<1024x1024xf16>) {
    tb.matmul %A, %B, %C {block_m = 256 : i64, block_n = 256 : i64,
                          block_k = 64 : i64, exact_tile = true,
                          mma = "mfma_f32_32x32x16_f16"}
      : memref<1024x512xf16>, memref<512x1024xf16>, memref<1024x1024xf16>
    func.return
  }
}

// CHECK: tb.gfx950_launch
// CHECK-SAME: wave_grid_m = 4 : i64
// CHECK-SAME: wave_grid_n = 2 : i64
// CHECK-SAME: kernel = "tb_gemm_gfx950_256x256x64_w4x2_s2_out0"
// CHECK-SAME: waits = array<i64: 4, 0, -1>

// PLAN: tb.async_plan = {
// PLAN-SAME: issue_schedule = "slot_spread"
// PLAN-SAME: loads_per_thread = 8 : i64
// PLAN-SAME: prologue_tail_loads = 4 : i64
// PLAN-SAME: refill_spread_slots = 8 : i64
// PLAN-SAME: waits = [{
// PLAN-SAME: group_id = 0 : i64, lgkmcnt_allowance = -1 : i64
// PLAN-SAME: vmcnt_allowance = 4 : i64
// PLAN-SAME: group_id = 1 : i64, lgkmcnt_allowance = -1 : i64
// PLAN-SAME: vmcnt_allowance = 0 : i64
