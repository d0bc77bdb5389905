// gfx950 (MI355X, CDNA4) MFMA GEMM kernels for the tb.matmul path.
//
// Replaces the reference's generated NVGPU kernel body
// (lib/Transforms/LowerPipelineToNVGPU.cpp:2019-2608) and its epilogue vector
// IO (lib/Transforms/LowerEpilogueVectorIO.cpp:22-385) with hand-written HIP
// for wave64 + MFMA + LDS:
//
//  * transport: buffer_load_dwordx4 ... lds (direct-to-LDS, 16 B per lane,
//    no register staging) from row-major A/B; bounds handled by the buffer
//    descriptor (an out-of-range offset loads zero); STAGES-deep ring of LDS
//    stages, tile it+STAGES-1 in flight while tile it is consumed;
//  * LDS layouts: A as [BM][BK] (K-contiguous, MFMA operand = one
//    ds_read_b128), B as [BK][BN] exactly as it lies in memory (N-contiguous,
//    MFMA operand = two ds_read_b64_tr_b16, the gfx950 transposing read);
//    XOR swizzles keep both reads bank-conflict free on the 64-bank
//    (256 B/cycle) LDS: A 16-byte chunk ^= (row / per_phase) % max_phase
//    (per_phase = max(1, 256 / row_bytes), max_phase = row_bytes / 16);
//    B 64-byte segment ^= (k / per_phase) % min(4, segments per row);
//  * compute: v_mfma_f32_32x32x16_f16 with the B fragment as srcA and the A
//    fragment as srcB, so each lane's 16 accumulators are 4 runs of 4
//    consecutive C columns of one row (4 x 8-byte f16 stores per tile);
//  * program order: row-major, grouped-M (Triton formula), split-K, and
//    persistent tile-stride loops in row-major or grouped order, optionally
//    remapped so consecutive tiles land on one XCD (shared L2).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace tbk {

enum MappingKind : int {
  kMapTile = 0,
  kMapGrouped = 1,
  kMapSplitK = 2,
  kMapPersistent = 3,        // reference order: row-major tile stride loop
  kMapPersistentGrouped = 4, // gfx950: grouped-M tile stride loop
};

enum OutMode : int {
  kOutF16 = 0,        // C(f16) = acc, accumulator starts at zero
  kOutF32Partial = 1, // ws[part*M*ws_ld + ...](f32) = acc (split-K partials,
                      // or a plain f32 store when ws aliases C)
  kOutF32Accum = 2,   // C(f32) = C + acc (reference C += A*B)
  kOutF32Atomic = 3,  // C(f32) += acc with f32 atomics (reference split_k_atomic)
};

struct GemmParams {
  const void *A;
  const void *B;
  void *C;
  float *ws;
  int M, N, K;
  int lda, ldb, ldc; // elements
  int tiles_m, tiles_n, tiles_k;
  int group_m;
  int split_k;
  int mapping;
  int total_work; // programs (non-persistent) or work items (persistent)
  int xcds;       // > 1: remap program ids so neighbours share an XCD
  int ws_ld;      // leading dimension of the f32 partial output (elements)
  // fused epilogue: bias (0 none, 1 f16, 2 f32; N values), activation
  // (0 none, 1 relu, 2 gelu_tanh, 3 silu), clamp bits (1 min, 2 max)
  const void *bias;
  int epi_bias, epi_act, epi_clamp;
  float clamp_lo, clamp_hi;
};

// The fused epilogue steps on 4 consecutive columns (col .. col+3) of one
// row, in order bias, activation, clamp. Callers only reach this when at
// least one step is set; every branch is on kernel arguments (wave-uniform).
struct EpiArgs {
  const void *bias;
  int bias_kind, act, clamp;
  float lo, hi;
};

// x / (1 + 2^t) with the hardware exp2 (v_exp_f32) and reciprocal
// (v_rcp_f32), each about 1 ulp; x sigmoid(z) is t = -z log2 e. For t ->
// +inf the denominator is +inf and the result 0; for t -> -inf it is x.
// The product is kept as an f32 value (an empty asm on it): otherwise a
// following f16 cast can be fused with it into one v_fma_mixlo_f16, which
// rounds the product once to f16, in kernels that cast right away and not in
// the others, and the kernels' results would differ in the last f16 bit.
__device__ __forceinline__ float epi_x_sigmoid2(float x, float t) {
  float y = x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(t));
  asm("" : "+v"(y));
  return y;
}

__device__ __forceinline__ float epi_activation(float x, int act) {
  if (act == 1)
    return x > 0.f ? x : 0.f;
  if (act == 2) { // tanh form of GELU (Hendrycks & Gimpel, 2016):
    // 0.5 x (1 + tanh(u)) = x sigmoid(2u), u = sqrt(2/pi) (x + 0.044715 x^3);
    // -2u log2 e = x (a + b x^2), a = -2 sqrt(2/pi) log2 e, b = 0.044715 a
    // (three operations before the exp2, not five)
    const float t = x * __builtin_fmaf(-0.1029432395800235f, x * x, -2.302208198144325f);
    return epi_x_sigmoid2(x, t);
  }
  if (act == 3) // SiLU: x sigmoid(x)
    return epi_x_sigmoid2(x, x * -1.4426950408889634f);
  return x;
}

typedef float epi_f32x4 __attribute__((ext_vector_type(4)));

// Bias values of columns col .. col+3 (zero past N: those columns are never
// stored). N % 4 == 0, so a group is wholly inside or outside. A buffer load
// whose records end at column N: columns past N read zeros without a
// per-lane branch (only the bias kind, a kernel argument, branches), so no
// divergent control flow lands in an epilogue that holds the accumulators.
__device__ __forceinline__ epi_f32x4 epi_load_bias(const EpiArgs &e, int col, int N) {
  epi_f32x4 b = {0.f, 0.f, 0.f, 0.f};
  if (e.bias_kind == 0)
    return b;
  const uint32_t off = col < N ? (uint32_t)col : 0x40000000u; // past N: out of range
  if (e.bias_kind == 1) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(e.bias), 0, N * 2, 0x00020000);
    const h4 h = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(r, off * 2u, 0, 0));
    b = (epi_f32x4){(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
  } else {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(e.bias), 0, N * 4, 0x00020000);
    b = __builtin_bit_cast(epi_f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off * 4u, 0, 0));
  }
  return b;
}

// The same steps with the activation fixed at compile time and, when CLAMP,
// the clamps as selects against bounds that are -inf / +inf for a clamp that
// is off (the same comparisons as epi_apply1, so the same results, NaN
// included): no branch per element in unrolled epilogue loops, and no
// compare / select pairs when neither clamp is set.
template <int ACT, bool CLAMP>
__device__ __forceinline__ float epi_apply_t(float x, float bias, float lo, float hi) {
  x += bias;
  x = epi_activation(x, ACT);
  if constexpr (CLAMP) {
    x = x < lo ? lo : x;
    x = x > hi ? hi : x;
  }
  return x;
}

// Calls f(integral_constant<int, ACT>, integral_constant<bool, CLAMP>) once
// for the activation and clamp a launch carries: the per-tile dispatch of
// code unrolled over a tile's elements.
template <typename F>
__device__ __forceinline__ void epi_dispatch(int act, int clamp, F &&f) {
  using C0 = std::integral_constant<bool, false>;
  using C1 = std::integral_constant<bool, true>;
  if (clamp) {
    switch (act) {
    case 1: f(std::integral_constant<int, 1>{}, C1{}); break;
    case 2: f(std::integral_constant<int, 2>{}, C1{}); break;
    case 3: f(std::integral_constant<int, 3>{}, C1{}); break;
    default: f(std::integral_constant<int, 0>{}, C1{}); break;
    }
  } else {
    switch (act) {
    case 1: f(std::integral_constant<int, 1>{}, C0{}); break;
    case 2: f(std::integral_constant<int, 2>{}, C0{}); break;
    case 3: f(std::integral_constant<int, 3>{}, C0{}); break;
    default: f(std::integral_constant<int, 0>{}, C0{}); break;
    }
  }
}

// The same with the clamp always applied as selects (bounds -inf / +inf for
// a clamp that is off: the same comparisons, so the same results): four
// variants of the unrolled code instead of eight, for the many general-loop
// instances, whose build time this halves.
template <typename F>
__device__ __forceinline__ void epi_dispatch_act(int act, F &&f) {
  using C1 = std::integral_constant<bool, true>;
  switch (act) {
  case 1: f(std::integral_constant<int, 1>{}, C1{}); break;
  case 2: f(std::integral_constant<int, 2>{}, C1{}); break;
  case 3: f(std::integral_constant<int, 3>{}, C1{}); break;
  default: f(std::integral_constant<int, 0>{}, C1{}); break;
  }
}

__device__ __forceinline__ float epi_apply1(float x, float bias, const EpiArgs &e) {
  x += bias;
  x = epi_activation(x, e.act);
  if (e.clamp & 1)
    x = x < e.lo ? e.lo : x;
  if (e.clamp & 2)
    x = x > e.hi ? e.hi : x;
  return x;
}

struct KernelKey {
  int bm, bn, bk, wgm, wgn, out, stages;
  int epi;  // 1: the fused epilogue steps are compiled in
  int mfma; // 0: v_mfma_f32_32x32x16_f16, 1: v_mfma_f32_16x16x32_f16
};

struct KernelEntry {
  KernelKey key;
  const void *fn;
  const char *name;
  // s_waitcnt depths compiled into the instance: vmcnt at the prologue's
  // wait, vmcnt at the per-k-tile barrier, lgkmcnt at that barrier (-1: none;
  // the compiler orders the LDS reads). The plan's AsyncPlan must state them.
  int vm_prologue, vm_loop, lgkm_loop;
  // the same instance built for a partial last k-tile (K % block_k != 0),
  // where its whole-K build carries no masking: the launcher picks it then
  // (null: fn handles every K)
  const void *fn_partial_k;
  // threads per workgroup when the build adds waves of its own (producer
  // waves); 0: num_waves * 64
  int threads;
};

// Registry of compiled instances (defined in the instance files).
const KernelEntry *find_kernel(const KernelKey &k);
int kernel_count();
const KernelEntry *kernel_at(int i);

// C = epilogue([C +] sum_{p < split_k} ws[p]) in fixed p order, cast to C's type.
hipError_t launch_reduce_ex(const float *ws, void *C, int M, int N, int ldc,
                            int split_k, int c_f16, int load_c, const EpiArgs &epi,
                            hipStream_t s);
hipError_t launch_fill(void *dst, int64_t rows, int64_t cols, int64_t ld,
                       uint64_t seed, int dist, double scale, hipStream_t s);
// `workgroups` one-wave probes of (XCC id, shader-clock cycles, 100 MHz
// ticks) over a window of `window` ticks.
hipError_t launch_clock_probe(unsigned long long *out, int workgroups, unsigned window,
                              hipStream_t s);
// `workgroups` one-wave stamps of (XCC id, shader-clock count, 100 MHz count).
hipError_t launch_clock_stamp(unsigned long long *out, int workgroups, hipStream_t s);

} // namespace tbk
