// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-verify-scope,tb-attach-target-info{gpu-arch=gfx950},tb-semanticize-matmul,tb-build-program-mapping-plan,tb-build-layout-plan,tb-build-transport-plan,tb-build-c-register-plan,tb-rewrite-matmul-mainloop,tb-cleanup-layout-conversions,tb-build-mainloop-graph,tb-regularize-k-loop,tb-assign-latencies,tb-schedule-loops,tb-derive-waits,tb-expand-pipeline,tb-cleanup-pipeline,tb-verify-pipeline-mainline-contract)' | FileCheck %s

// gfx950 form of the reference's exact-tile contract test: one wave, an
// exact 64x64x32 tile, f32 C accumulated in place.
module attributes {"tb.num-warps" = 1 : i64, "tb.requested-stages" = 2 : i64} {
  func.func @kernel(%A: memref<64x32xf16>, %B: memref<32x64xf16>,
                    %C: memref<64x64xf32>) {
    tb.matmul %A, %B, %C {block_m = 64 : i64, block_n = 64 : i64,
                          block_k = 32 : i64, exact_tile = true}
      : memref<64x32xf16>, memref<32x64xf16>, memref<64x64xf32>
    func.return
  }
}

// A stage [64][32] f16: 64-byte rows, 4 rows per 256-byte bank period,
// 4 chunks of 16 bytes to rotate; B stage [32][64]: 128-byte rows, two
// 64-byte segments.
// CHECK: tb.pipeline_mainline
// CHECK: #tb.shared<order = [1, 0], perPhase = 4, maxPhase = 4, transposed = false, swizzlingByteWidth = 16
// CHECK: #tb.shared<order = [1, 0], perPhase = 2, maxPhase = 2, transposed = false, swizzlingByteWidth = 64
// CHECK: init_mode = "direct_global_vector"
// CHECK: kind = "register_pack_global_vector"
// CHECK: required_sync_kind = "none"
