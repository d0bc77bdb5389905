// Auxiliary gfx950 kernels of the tb.matmul path:
//  * the deterministic split-K reduction (global f32 workspace summed in
//    fixed split order, then the fused epilogue steps, then cast) that realises the reference's
//    SplitKSerial reduction plan (lib/Analysis/ReductionPlan.cpp:136-193),
//    which the reference itself never lowers (LowerPipelineToNVGPU.cpp:803-810);
//  * the seeded f16 input generator used by the benchmark harness.
// Also aggregates the GEMM instance registry.
#include "gemm_gfx950.h"
#include "gemm_tiles.h"

#include <math.h>

namespace tbk {

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct ReduceArgs {
  const float *ws;
  void *C;
  int M, N, ldc, split_k;
  int c_f16;
  int load_c;
  EpiArgs epi;
};

// One thread per 4 consecutive columns (N % 4 == 0 is required by the host).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(ReduceArgs a) {
  const int cols4 = a.N / 4;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)a.M * cols4)
    return;
  const int row = (int)(idx / cols4), col = (int)(idx % cols4) * 4;
  const size_t plane = (size_t)a.M * (size_t)a.N;
  const f32x4 *src =
      reinterpret_cast<const f32x4 *>(a.ws + (size_t)row * a.N + col);
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  if (a.load_c && !a.c_f16)
    s = *reinterpret_cast<const f32x4 *>(reinterpret_cast<float *>(a.C) +
                                          (size_t)row * a.ldc + col);
  // fixed order p = 0, 1, ...: deterministic result. The planes are loaded 8
  // at a time before they are added, so a thread waits for memory once per 8
  // planes, not once per plane. Each partial is read once: non-temporal loads
  // (512^2 x 16384 in 8 splits: 0.5 us less per call).
  for (int p0 = 0; p0 < a.split_k; p0 += 8) {
    f32x4 v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (p0 + q < a.split_k)
        v[q] = __builtin_nontemporal_load(src + (p0 + q) * (plane / 4));
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (p0 + q < a.split_k)
        s += v[q];
  }
  if (a.epi.bias_kind | a.epi.act | a.epi.clamp) { // fused steps on the whole sum
    const f32x4 b = epi_load_bias(a.epi, col, a.N);
    for (int r = 0; r < 4; ++r)
      s[r] = epi_apply1(s[r], b[r], a.epi);
  }
  if (a.c_f16) {
    _Float16 *c = reinterpret_cast<_Float16 *>(a.C) + (size_t)row * a.ldc + col;
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 h = {(_Float16)s[0], (_Float16)s[1], (_Float16)s[2], (_Float16)s[3]};
    *reinterpret_cast<h4 *>(c) = h;
  } else {
    *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(a.C) +
                               (size_t)row * a.ldc + col) = s;
  }
}

// ---- seeded inputs -------------------------------------------------------
__device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// binary64 -> binary16, round to nearest even, from the bit pattern.
__device__ uint16_t f64_to_f16_bits(double x) {
  const uint64_t b = __double_as_longlong(x);
  const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
  const int exp = (int)((b >> 52) & 0x7ff);
  const uint64_t frac = b & 0xFFFFFFFFFFFFFull;
  if (exp == 0x7ff)
    return frac ? (uint16_t)(sign | 0x7e00u) : (uint16_t)(sign | 0x7c00u);
  if (exp == 0)
    return sign;
  int e = exp - 1023;
  const uint64_t m = frac | (1ull << 52);
  if (e >= 16)
    return (uint16_t)(sign | 0x7c00u);
  if (e >= -14) {
    uint64_t q = m >> 42;
    const uint64_t rem = m & ((1ull << 42) - 1), half = 1ull << 41;
    if (rem > half || (rem == half && (q & 1)))
      q++;
    if (q == 0x800) {
      q = 0x400;
      e++;
    }
    if (e >= 16)
      return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint16_t)(e + 15) << 10) | (uint16_t)(q & 0x3ff));
  }
  const int shift = 28 - e;
  if (shift > 54)
    return sign;
  uint64_t q = m >> shift;
  const uint64_t rem = m & ((1ull << shift) - 1), half = 1ull << (shift - 1);
  if (rem > half || (rem == half && (q & 1)))
    q++;
  return (uint16_t)(sign | (uint16_t)q);
}

__global__ __launch_bounds__(256) void fill_kernel(uint16_t *dst, int64_t rows,
                                                   int64_t cols, int64_t ld,
                                                   uint64_t seed, int dist,
                                                   double scale) {
  const int64_t n = rows * cols;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = idx / cols, c = idx % cols;
    double v;
    if (dist == 1) {
      const uint64_t x1 = splitmix64_at(seed, 2 * (uint64_t)idx);
      const uint64_t x2 = splitmix64_at(seed, 2 * (uint64_t)idx + 1);
      const double u1 = (double)((x1 >> 11) + 1) * (1.0 / 9007199254740992.0);
      const double u2 = (double)(x2 >> 11) * (1.0 / 9007199254740992.0);
      v = sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
    } else {
      const uint64_t x = splitmix64_at(seed, (uint64_t)idx);
      v = (double)(x >> 40) * (1.0 / 16777216.0) * 2.0 - 1.0;
    }
    dst[r * ld + c] = f64_to_f16_bits(v * scale);
  }
}

// ---- clock probe ---------------------------------------------------------
// Workgroup b (one wave) measures the shader clock of the CU it runs on:
// it reads the shader-clock counter (s_memtime) and the constant 100 MHz
// counter (s_memrealtime), spins until `window` ticks of the latter have
// passed (at most 2^20 reads: every wave exits), and reads both again. Both
// readings of a pair come from the same wave, so the counters' per-CU
// offsets cancel. out[3b] = the XCC (XCD) id, out[3b+1] = shader-clock
// cycles, out[3b+2] = 100 MHz ticks of the window; cycles / ticks * 100 MHz
// is the clock. Launched right after a stretch of work, it reads the clock
// that work ran at (the power manager reacts on a millisecond scale). Only
// lane 0 stores (vector stores).
__device__ __forceinline__ unsigned long long read_shader_clock() {
  unsigned long long t;
  asm volatile("s_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t)::"memory");
  return t;
}
__device__ __forceinline__ unsigned long long read_real_clock() {
  unsigned long long t;
  asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t)::"memory");
  return t;
}

__global__ __launch_bounds__(64) void clock_probe_kernel(unsigned long long *out,
                                                         unsigned window) {
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 16)" : "=s"(xcc));
  const unsigned long long t0 = read_shader_clock(), r0 = read_real_clock();
  for (int i = 0; i < (1 << 20); ++i)
    if (read_real_clock() - r0 >= window)
      break;
  const unsigned long long t1 = read_shader_clock(), r1 = read_real_clock();
  if (threadIdx.x == 0) {
    out[3 * blockIdx.x + 0] = xcc & 0xfu;
    out[3 * blockIdx.x + 1] = t1 - t0;
    out[3 * blockIdx.x + 2] = r1 - r0;
  }
}

// One reading per workgroup, no window: (where, shader-clock count, 100 MHz
// count), `where` = XCC id << 8 | the SE, SH and CU fields of HW_ID (bits
// 8..15). The shader-clock counter is not common to the CUs of an XCD, so
// two stamps on a stream around some work give the mean clock over that work
// per CU that both stamps reached: cycles between them / ticks between them.
__global__ __launch_bounds__(64) void clock_stamp_kernel(unsigned long long *out) {
  unsigned xcc, hwid;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 16)" : "=s"(xcc));
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID, 8, 8)" : "=s"(hwid));
  const unsigned long long t = read_shader_clock(), r = read_real_clock();
  if (threadIdx.x == 0) {
    out[3 * blockIdx.x + 0] = ((xcc & 0xfu) << 8) | (hwid & 0xffu);
    out[3 * blockIdx.x + 1] = t;
    out[3 * blockIdx.x + 2] = r;
  }
}

hipError_t launch_clock_stamp(unsigned long long *out, int workgroups, hipStream_t s) {
  hipLaunchKernelGGL(clock_stamp_kernel, dim3(workgroups), dim3(64), 0, s, out);
  return hipGetLastError();
}

hipError_t launch_clock_probe(unsigned long long *out, int workgroups, unsigned window,
                              hipStream_t s) {
  hipLaunchKernelGGL(clock_probe_kernel, dim3(workgroups), dim3(64), 0, s, out, window);
  return hipGetLastError();
}

hipError_t launch_reduce_ex(const float *ws, void *C, int M, int N, int ldc,
                            int split_k, int c_f16, int load_c, const EpiArgs &epi,
                            hipStream_t s) {
  ReduceArgs a{ws, C, M, N, ldc, split_k, c_f16, load_c, epi};
  const int64_t threads = (int64_t)M * (N / 4);
  const int blocks = (int)((threads + 255) / 256);
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_fill(void *dst, int64_t rows, int64_t cols, int64_t ld,
                       uint64_t seed, int dist, double scale, hipStream_t s) {
  const int64_t n = rows * cols;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536)
    blocks = 65536;
  if (blocks < 1)
    blocks = 1;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                     reinterpret_cast<uint16_t *>(dst), rows, cols, ld, seed,
                     dist, scale);
  return hipGetLastError();
}

// ---- instance registry ----------------------------------------------------
// One table per shape and flavour (gemm_inst.hip), the hand-scheduled
// 16x16x32 tables (f16 C; f32 C) and one 16x16x32 table per shape and
// flavour of TBK_M16_SHAPES (gemm_inst_mfma16g.hip).
#define TBK_DECLARE(SHAPE)                                                      \
  const KernelEntry *entries_##SHAPE(int *n);                                  \
  const KernelEntry *entries_##SHAPE##_epi(int *n);
TBK_SHAPES(TBK_DECLARE)
#undef TBK_DECLARE
#define TBK_DECLARE_M16(SHAPE)                                                  \
  const KernelEntry *entries_m16_##SHAPE(int *n);                              \
  const KernelEntry *entries_m16_##SHAPE##_epi(int *n);
TBK_M16_SHAPES(TBK_DECLARE_M16)
#undef TBK_DECLARE_M16
const KernelEntry *entries_mfma16(int *n);
const KernelEntry *entries_mfma16_f32(int *n);
const KernelEntry *entries_producer(int *n);

static bool same_key(const KernelKey &a, const KernelKey &b) {
  return a.bm == b.bm && a.bn == b.bn && a.bk == b.bk && a.wgm == b.wgm &&
         a.wgn == b.wgn && a.out == b.out && a.stages == b.stages && a.epi == b.epi &&
         a.mfma == b.mfma;
}

// the producer-wave build of a key, where one exists, in place of the
// general loop's entry
static const KernelEntry *preferred(const KernelEntry *e) {
  int n = 0;
  const KernelEntry *pw = entries_producer(&n);
  for (int i = 0; i < n; ++i)
    if (same_key(pw[i].key, e->key))
      return pw + i;
  return e;
}

#define TBK_TABLES(SHAPE) entries_##SHAPE, entries_##SHAPE##_epi,
#define TBK_M16_TABLES(SHAPE) entries_m16_##SHAPE, entries_m16_##SHAPE##_epi,
static const KernelEntry *(*const kTables[])(int *) = {
    TBK_SHAPES(TBK_TABLES) entries_mfma16, entries_mfma16_f32,
    TBK_M16_SHAPES(TBK_M16_TABLES)};
#undef TBK_TABLES
#undef TBK_M16_TABLES

int kernel_count() {
  int total = 0;
  for (auto t : kTables) {
    int n = 0;
    t(&n);
    total += n;
  }
  return total;
}

const KernelEntry *kernel_at(int i) {
  if (i < 0)
    return nullptr;
  for (auto t : kTables) {
    int n = 0;
    const KernelEntry *e = t(&n);
    if (i < n)
      return preferred(e + i);
    i -= n;
  }
  return nullptr;
}

const KernelEntry *find_kernel(const KernelKey &k) {
  const int n = kernel_count();
  for (int i = 0; i < n; ++i) {
    const KernelEntry *e = kernel_at(i);
    if (same_key(e->key, k))
      return e;
  }
  return nullptr;
}

} // namespace tbk
