/*
 * tb_gfx950 -- C ABI of the MI355X (gfx950) backend for the tb.matmul GEMM
 * compiler path.
 *
 * The reference (zrqnwu/mini_triton_nvgpu_v1) hands a kernel from its
 * compiler to its launcher as process + text: `tb-opt` lowers the plan-
 * annotated module to PTX (lib/Transforms/Stage1Pipelines.cpp:101-120,
 * tools/tb-opt.cpp:11-24), an extractor pulls the binary out, and an external
 * driver calls cuModuleLoadData + cuLaunchKernel("kernel_tb_kernel_0",
 * grid, block = num_warps*32) (tools/bench_stage1_fair.py:547-563, :665-699).
 * This library replaces everything from tb-lower-pipeline-to-nvgpu
 * (lib/Transforms/LowerPipelineToNVGPU.cpp:2624-2732) downward: the plan
 * pipeline's finished KernelContract is flattened into a tb_gemm_config and
 * launched on hand-written gfx950 MFMA kernels.
 *
 * Conventions:
 *  - every int-returning function returns 0 on success, < 0 on error; the
 *    message is available from tb_last_error() (thread-local);
 *  - A, B, C and the workspace are caller-owned device pointers, row-major,
 *    A = M x K f16, B = K x N f16, C = M x N (f16 or f32) with leading
 *    dimensions from the descriptor;
 *  - `stream` is a hipStream_t (NULL = the null stream); launches are
 *    asynchronous and stream-ordered;
 *  - a tb_gemm_desc is immutable after creation and may be shared between
 *    threads.
 */
#ifndef TB_GFX950_H
#define TB_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TB_GFX950_ABI_VERSION 4

/* element types (reference ScalarKind, include/tb/Analysis/KernelConfig.h:13-16) */
#define TB_DTYPE_F16 0
#define TB_DTYPE_F32 1

/* accumulator initialisation (reference AccumulatorInitMode,
 * include/tb/Analysis/EpiloguePlan.h:16-20): Zero, or DirectGlobalVector =
 * load C first (the reference's C += A*B) */
#define TB_ACC_INIT_ZERO 0
#define TB_ACC_INIT_LOAD_C 1

/* program mapping (reference ProgramMappingKind,
 * include/tb/Analysis/ProgramMappingPlan.h:19-24, plus the grouped persistent
 * order this backend adds) */
#define TB_MAP_TILE 0
#define TB_MAP_GROUPED_TILE 1
#define TB_MAP_SPLIT_K 2
#define TB_MAP_PERSISTENT_TILE 3
#define TB_MAP_PERSISTENT_GROUPED 4

/* split-K reduction (reference ReductionPlanKind,
 * include/tb/Analysis/ReductionPlan.h:15-19): SplitKSerial is realised as a
 * global f32 workspace reduced in fixed split order (deterministic);
 * SplitKAtomic adds each split into f32 C with atomics */
#define TB_RED_NONE 0
#define TB_RED_WORKSPACE 1
#define TB_RED_ATOMIC 2

/* MFMA instruction of the instance (reference MmaKind,
 * include/tb/Analysis/KernelConfig.h:18-20, which names the mma.sync shape).
 * 16x16x32 exists for the 4-wave 256x256x64 2-stage tile with an f16 C, a
 * plain f32 C or f32 C += A*B, any M, N and K (tile, grouped or persistent
 * order; no split-K): the plan selects it there. */
#define TB_MFMA_32X32X16 0 /* v_mfma_f32_32x32x16_f16 */
#define TB_MFMA_16X16X32 1 /* v_mfma_f32_16x16x32_f16 */

/* fused epilogue steps (reference EpilogueExprKind LoadBias + Add,
 * Activation, Clamp; include/tb/Analysis/EpiloguePlan.h:61-75). They apply
 * to the f32 result in the order bias, activation, clamp, before C is
 * written (after C's prior value is added when acc_init is LOAD_C). The
 * reference declares these exprs but derives none; here tb.matmul's
 * `epilogue_*` attrs request them. */
#define TB_EPI_BIAS_NONE 0
#define TB_EPI_BIAS_F16 1 /* bias: N f16 values, C[r][c] += bias[c] */
#define TB_EPI_BIAS_F32 2 /* bias: N f32 values */
#define TB_ACT_NONE 0
#define TB_ACT_RELU 1      /* max(x, 0) */
#define TB_ACT_GELU_TANH 2 /* 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) */
#define TB_ACT_SILU 3      /* x / (1 + exp(-x)) */
#define TB_CLAMP_MIN 1     /* epi_clamp bits: x = max(x, clamp_min) */
#define TB_CLAMP_MAX 2     /*                 x = min(x, clamp_max) */

/* Flattened KernelContract: everything the gfx950 kernels consume. Mirrors
 * the fields the reference's lowering reads out of the plans
 * (LoweringContract, lib/Transforms/LowerPipelineToNVGPU.cpp:45-113). */
typedef struct tb_gemm_config {
  int64_t m, n, k;       /* problem shape (KernelConfig problemM/N/K) */
  int64_t lda, ldb, ldc; /* leading dimensions in elements */
  int32_t c_dtype;       /* TB_DTYPE_F16 | TB_DTYPE_F32 (A, B are f16) */
  int32_t acc_init;      /* TB_ACC_INIT_* */
  int64_t block_m, block_n, block_k; /* macro tile (tileM/N/K) */
  int64_t num_waves;     /* MFMA wavefronts per workgroup (tb.num-warps); an
                          * instance built with producer waves launches as many
                          * load-only waves again (the plan's loader_waves) */
  int64_t wave_grid_m, wave_grid_n; /* WarpDecompositionPlan warpGrid */
  int64_t stages;        /* LDS stages (requested stages) */
  int32_t mapping;       /* TB_MAP_* */
  int64_t group_m;       /* grouped order width (GROUP_M) */
  int64_t split_k;       /* split count (1 = none) */
  int32_t reduction;     /* TB_RED_* */
  int64_t num_programs;  /* workgroups launched (persistent: resident) */
  int32_t xcd_remap;     /* >1: remap program ids so neighbours share an XCD */
  int32_t epi_bias;      /* TB_EPI_BIAS_* */
  int32_t epi_activation; /* TB_ACT_* */
  int32_t epi_clamp;     /* TB_CLAMP_* bits */
  float clamp_min, clamp_max; /* finite, clamp_min <= clamp_max when both */
  int32_t mfma;          /* TB_MFMA_* (EncodingPlan instrShape) */
} tb_gemm_config;

typedef struct tb_gemm_desc tb_gemm_desc;

/* Thread-local message of the last failing call ("" if none). */
const char *tb_last_error(void);

/* Build a descriptor from a flattened config; selects the gfx950 kernel
 * instance. Replaces LowerPipelineToNVGPU.cpp:2624-2732 (contract
 * validation + gpu.func emission). A, C and the split-K workspace may be of
 * any size as long as one tile's rows of A and C (block_m rows) span less
 * than 1 GiB: the kernels address them through per-tile windows with 32-bit
 * offsets inside. B must span less than 2 GiB. */
int tb_desc_create(const tb_gemm_config *cfg, tb_gemm_desc **out);

/* Run the tb plan pipeline (tb-verify-scope ... tb-verify-pipeline-mainline-
 * contract, the pass list of lib/Transforms/Stage1Pipelines.cpp:14-36) on a
 * module holding one tb.matmul, with tb-attach-target-info{gpu-arch=
 * <gpu_arch>} (NULL or "" = "gfx950"), then flatten the KernelContract
 * (lib/Analysis/KernelContract.cpp:9-65) into a descriptor. A module that
 * already holds a sealed tb.pipeline_mainline or a lowered tb.gfx950_launch
 * is accepted as is. Operands are identity-layout memrefs, so the leading
 * dimensions are the memref row lengths. Errors carry the pass name and the
 * diagnostic (the reference's emitError text where the rule is shared). */
int tb_plan_from_mlir(const char *mlir, size_t len, const char *gpu_arch,
                      tb_gemm_desc **out);

/* Same, reading the module from a file: typically the output of
 * `tb-opt --pass-pipeline='builtin.module(tb-stage1-full-to-gfx950-pipeline
 * {cubin-chip=gfx950})'`, whose tb.gfx950_launch op replaces the gpu.binary
 * payload the reference's harness extracts (tools/bench_stage1_fair.py:
 * 531-564). */
int tb_plan_from_file(const char *path, tb_gemm_desc **out);

/* Copy the flattened config back out. */
int tb_desc_get_config(const tb_gemm_desc *desc, tb_gemm_config *out);
/* Name of the selected kernel instance (valid while desc lives). */
const char *tb_desc_kernel_name(const tb_gemm_desc *desc);
/* Static LDS bytes per workgroup of the selected instance. */
int64_t tb_desc_lds_bytes(const tb_gemm_desc *desc);

/* Bytes of caller-provided global workspace tb_gemm_launch needs (split-K
 * f32 partials: split_k * m * n * 4; 0 otherwise). Reference analogue:
 * ReductionPlan scratchBytes (lib/Analysis/ReductionPlan.cpp:158-177). */
size_t tb_workspace_bytes(const tb_gemm_desc *desc);

/* Enqueue C = A*B (or C += A*B for TB_ACC_INIT_LOAD_C) on `stream`, then
 * the fused epilogue steps of the config. Fails for a config with a bias
 * (use tb_gemm_launch_ex). A, B, C and the workspace must be 16-byte aligned
 * (hipMalloc and torch allocations are). Reference: the launcher of the
 * lowered kernel, tools/bench_stage1_fair.py:665-699 (A, B, C device
 * pointers). */
int tb_gemm_launch(const tb_gemm_desc *desc, const void *a, const void *b,
                   void *c, void *workspace, void *stream);

/* tb_gemm_launch plus the bias vector the epilogue reads (N elements of the
 * config's bias type; NULL when the config has no bias). No reference
 * counterpart: the reference's EpilogueExprKind::LoadBias
 * (include/tb/Analysis/EpiloguePlan.h:61-67) names a bias operand that its
 * tb.matmul never takes. */
int tb_gemm_launch_ex(const tb_gemm_desc *desc, const void *a, const void *b,
                      void *c, const void *bias, void *workspace, void *stream);

/* Bytes of the static split-K scratch tb_gemm_launch_noalloc uses on each
 * GPU (32 MiB: 8 splits of a 1024 x 1024 f32 result). */
#define TB_NOALLOC_SCRATCH_BYTES (32u * 1024u * 1024u)

/* tb_gemm_launch_ex without the workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): a split-K descriptor's f32 partials go to
 * a static scratch array of TB_NOALLOC_SCRATCH_BYTES in the library, one per
 * GPU, held until the process ends. It calls no hipMalloc, hipFree or other
 * allocating routine, and fails with a clear error when the descriptor needs
 * more workspace than the scratch holds (tb_workspace_bytes). Every call on
 * one GPU shares that GPU's scratch: calls that overlap on one GPU (other
 * streams, other threads) race. Nothing in the scratch needs clearing: each
 * call writes every partial its reduction reads. The scratch belongs to the
 * device of `stream` (the current device for the null stream). This entry
 * point has no counterpart in the reference; it is for callers that cannot
 * allocate. */
int tb_gemm_launch_noalloc(const tb_gemm_desc *desc, const void *a, const void *b,
                           void *c, const void *bias, void *stream);

void tb_desc_free(tb_gemm_desc *desc);

/* Harness helper (no reference counterpart: the reference's external driver
 * owns its inputs, tools/bench_stage1_fair.py:385-404). Fills a rows x cols
 * f16 matrix (leading dimension ld) on the device: element (r, c) is the
 * SplitMix64 draw r*cols + c of `seed`, uniform[-1,1) (dist 0) or
 * Box-Muller normal (dist 1), times `scale`, rounded to nearest even. */
int tb_fill_seeded_f16(void *dst, int64_t rows, int64_t cols, int64_t ld,
                       uint64_t seed, int32_t dist, double scale, void *stream);

/* Harness helper (no reference counterpart; the reference's harness reads
 * the GPU clock from nvidia-smi, tools/bench_stage1_fair.py:446-476). Launches
 * `workgroups` one-wave workgroups on `stream`; each measures the shader
 * clock of its CU over `window_ticks` ticks of the 100 MHz real-time counter
 * (s_memtime and s_memrealtime read by the same wave at both ends) and
 * writes three uint64 to out[3w..3w+2]: its XCC (XCD) id, the shader-clock
 * cycles and the 100 MHz ticks of the window (clock = cycles / ticks * 100
 * MHz). Workgroups are dealt to the XCDs round-robin, so 8 of them cover
 * every XCD of an MI355X. Launched right after some work on the same stream,
 * it reads the clock that work ran at. `out` is a device pointer. */
int tb_clock_probe(uint64_t *out, int32_t workgroups, int32_t window_ticks, void *stream);

/* Harness helper (no reference counterpart). Launches `workgroups` one-wave
 * workgroups on `stream`; each writes three uint64 to out[3w..3w+2]: where
 * it ran (XCC id << 8 | the SE, SH and CU fields of HW_ID) and the current
 * counts of its CU's shader clock (s_memtime) and of the 100 MHz real-time
 * counter (s_memrealtime). Both counters run on while other kernels execute,
 * so a stamp before and a stamp after some work on the same stream give, for
 * each CU both reached, the mean shader clock over that work: (cycles after
 * - cycles before) / (ticks after - ticks before) * 100 MHz. `out` is a
 * device pointer. */
int tb_clock_stamp(uint64_t *out, int32_t workgroups, void *stream);

/* Number of compiled kernel instances and the name of instance i. */
int tb_kernel_count(void);
const char *tb_kernel_name(int i);

/* The compiler's register report for kernel instance i (partial_k != 0: its
 * build for a partial last k-tile, K % block_k != 0): VGPRs and AGPRs per
 * wave and scratch bytes per lane, from the build-time table of hipcc's
 * kernel-resource-usage remarks. The plan pipeline and tb_desc_create refuse
 * an instance whose scratch is not zero. No counterpart in the reference:
 * here every instance is compiled ahead of time, so its register use is
 * known when the plan binds. */
int tb_kernel_resources(int i, int32_t partial_k, int32_t *vgprs, int32_t *agprs,
                        int32_t *scratch_bytes);

/* The s_waitcnt depths compiled into kernel instance i: vmcnt at the
 * prologue's wait, vmcnt at the per-k-tile barrier, and lgkmcnt at that
 * barrier (-1: none, the compiler orders the LDS reads). The plan's AsyncPlan
 * states the same numbers (the reference's lowering emits the waits its
 * AsyncPlan derives, LowerPipelineToNVGPU.cpp:2279-2294); tb_plan_from_mlir
 * and tb_plan_from_file refuse a plan whose waits differ from the kernel it
 * binds. */
int tb_kernel_waits(int i, int32_t *vm_prologue, int32_t *vm_loop, int32_t *lgkm_loop);

int tb_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* TB_GFX950_H */
