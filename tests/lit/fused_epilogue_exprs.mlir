// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-verify-scope,tb-attach-target-info{gpu-arch=gfx950},tb-semanticize-matmul,tb-build-program-mapping-plan,tb-build-layout-plan,tb-build-transport-plan,tb-build-c-register-plan)' | FileCheck %s --check-prefix=PLAN
// RUN: %tb-opt %s --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})' | FileCheck %s --check-prefix=LOWER

// Fused epilogue steps. The reference declares the EpiloguePlan expr kinds
// (include/tb/Analysis/EpiloguePlan.h:61-75) and serializes them
// (lib/Analysis/EpiloguePlan.cpp:423-459) but derives none; the gfx950 flow
// derives them from tb.matmul's epilogue_* attrs in the order bias,
// activation, clamp, then the f16 convert, and binds a kernel instance with
// the steps compiled in.
module attributes {"tb.num-warps" = 4 : i64, "tb.requested-stages" = 2 : i64} {
  func.func @kernel(%A: memref<96x32xf16>, %B: memref<32x80xf16>,
                    %C: memref<96x80xf16>) {
    tb.matmul %A, %B, %C {block_m = 64 : i64, block_n = 64 : i64,
                          block_k = 32 : i64, exact_tile = false,
                          epilogue_bias = "f16",
                          epilogue_activation = "gelu_tanh",
                          epilogue_clamp_min = -5.000000e-01 : f32,
                          epilogue_clamp_max = 6.0 : f32}
      : memref<96x32xf16>, memref<32x80xf16>, memref<96x80xf16>
    func.return
  }
}

// PLAN: epilogue_clamp_max = 6.000000e+00 : f32
// PLAN: tb.epilogue_plan
// PLAN-SAME: exprs = [{aux = "bias", input_scalar = "f16", kind = "load_bias", output_scalar = "f32", vector_width = 4 : i64}
// PLAN-SAME: {aux = "bias", input_scalar = "f32", kind = "add", output_scalar = "f32", vector_width = 4 : i64}
// PLAN-SAME: {aux = "gelu_tanh", input_scalar = "f32", kind = "activation", output_scalar = "f32", vector_width = 4 : i64}
// PLAN-SAME: {aux = "min=-0.5,max=6", input_scalar = "f32", kind = "clamp", output_scalar = "f32", vector_width = 4 : i64}
// PLAN-SAME: {aux = "round_to_nearest_even", input_scalar = "f32", kind = "convert", output_scalar = "f16", vector_width = 4 : i64}]

// LOWER: tb.gfx950_launch
// LOWER-SAME: clamp_max = 6.000000e+00 : f32
// LOWER-SAME: clamp_min = -5.000000e-01 : f32
// LOWER-SAME: epi_activation = 2 : i64
// LOWER-SAME: epi_bias = 1 : i64
// LOWER-SAME: epi_clamp = 3 : i64
// LOWER-SAME: kernel = "tb_gemm_gfx950_64x64x32_w2x2_s2_out0_epi"
// LOWER-NOT: epilogue_bias
