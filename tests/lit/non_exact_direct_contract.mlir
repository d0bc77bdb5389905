// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-verify-scope,tb-attach-target-info{gpu-arch=gfx950},tb-semanticize-matmul,tb-build-program-mapping-plan,tb-build-layout-plan,tb-build-transport-plan,tb-build-c-register-plan,tb-rewrite-matmul-mainloop,tb-cleanup-layout-conversions,tb-build-mainloop-graph,tb-regularize-k-loop,tb-assign-latencies,tb-schedule-loops,tb-derive-waits,tb-expand-pipeline,tb-cleanup-pipeline,tb-verify-pipeline-mainline-contract)' | FileCheck %s

// gfx950 form of the reference's non-exact contract test. The reference
// routes a ragged tile through a workgroup-shared row reorder; on gfx950 an
// MFMA accumulator lane already owns 4 consecutive columns, so the 4-wide
// vectors land straight from registers and the buffer range check drops the
// ones outside 96x80.
module attributes {"tb.num-warps" = 1 : i64, "tb.requested-stages" = 2 : i64} {
  func.func @kernel(%A: memref<96x32xf16>, %B: memref<32x80xf16>,
                    %C: memref<96x80xf32>) {
    tb.matmul %A, %B, %C {block_m = 64 : i64, block_n = 64 : i64,
                          block_k = 32 : i64, exact_tile = false}
      : memref<96x32xf16>, memref<32x80xf16>, memref<96x80xf32>
    func.return
  }
}

// CHECK: tb.pipeline_mainline
// CHECK-SAME: zero_fill = true
// CHECK-SAME: #tb.shared<order = [1, 0], perPhase = 4, maxPhase = 4, transposed = false, swizzlingByteWidth = 16
// CHECK-SAME: boundary_aware = true
// CHECK-SAME: scalar_tail = false
// CHECK-SAME: kind = "register_pack_global_vector"
// CHECK-SAME: tb.epilogue_reorder_plan = {
// CHECK-SAME: kind = "none"
// CHECK-SAME: workspace_barrier_count = 0
// CHECK-SAME: selected_buffering_kind = "async_ab_plus_register_epilogue"
// CHECK-SAME: selected_c_landing_kind = "register_direct_vector"
// CHECK-SAME: selected_shared_workspace_policy = "single_cta_workspace_stage_ring"
// CHECK-SAME: boundary_m = true, boundary_n = true
// CHECK-SAME: landing_owner = "register_pack"
// CHECK-SAME: reorder_owner = "none"
