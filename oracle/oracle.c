/*
 * CPU oracle for the tb.matmul GEMM path — TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker for the gfx950 kernels in libtb_gfx950.so and the
 * reported host fp32 baseline. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it. Nothing in the product path may
 * link, load or fall back to it.
 *
 * Reference citations are relative to the zrqnwu/mini_triton_nvgpu_v1 root.
 * The reference cannot be built here (it needs an MLIR/LLVM development tree,
 * CMakeLists.txt:10, and NVIDIA's toolchain for its generated kernel), so each
 * function restates the reference's algorithm and is pinned by the checks in
 * tests/test_oracle.py (known-answer vectors, numpy cross-checks, closed
 * forms, brute-force invariants).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* Seeded inputs. The reference's external driver (un-vendored, see
 * tools/bench_stage1_fair.py:385-404) owns its input pattern; these
 * generators are this build's own harness inputs: SplitMix64 (Steele, Lea &
 * Flood 2014; Vigna's public-domain finaliser constants).                    */
/* ------------------------------------------------------------------------ */
#define SM64_GAMMA 0x9E3779B97F4A7C15ULL

uint64_t tbo_splitmix64_at(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * SM64_GAMMA;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

double tbo_uniform_at(uint64_t seed, uint64_t i) {
  uint64_t x = tbo_splitmix64_at(seed, i);
  return (double)(x >> 40) * (1.0 / 16777216.0) * 2.0 - 1.0;
}

double tbo_normal_at(uint64_t seed, uint64_t i) {
  uint64_t x1 = tbo_splitmix64_at(seed, 2 * i);
  uint64_t x2 = tbo_splitmix64_at(seed, 2 * i + 1);
  double u1 = (double)((x1 >> 11) + 1) * (1.0 / 9007199254740992.0); /* (0,1] */
  double u2 = (double)(x2 >> 11) * (1.0 / 9007199254740992.0);       /* [0,1) */
  return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
}

/* IEEE-754 binary64 -> binary16, round to nearest, ties to even, computed
 * from the bit pattern (no intermediate binary32 rounding). */
uint16_t tbo_f64_to_f16(double x) {
  uint64_t b;
  memcpy(&b, &x, sizeof b);
  uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
  int exp = (int)((b >> 52) & 0x7ff);
  uint64_t frac = b & 0xFFFFFFFFFFFFFULL;
  if (exp == 0x7ff)
    return frac ? (uint16_t)(sign | 0x7e00u) : (uint16_t)(sign | 0x7c00u);
  if (exp == 0) /* binary64 zero or subnormal: far below half the f16 ulp */
    return sign;
  int e = exp - 1023;
  uint64_t m = frac | (1ULL << 52); /* 53 significant bits */
  if (e >= 16)
    return (uint16_t)(sign | 0x7c00u);
  if (e >= -14) {
    uint64_t q = m >> 42;
    uint64_t rem = m & ((1ULL << 42) - 1);
    uint64_t half = 1ULL << 41;
    if (rem > half || (rem == half && (q & 1)))
      q++;
    if (q == 0x800) { /* mantissa carried into the next binade */
      q = 0x400;
      e++;
    }
    if (e >= 16)
      return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint16_t)(e + 15) << 10) | (uint16_t)(q & 0x3ff));
  }
  /* subnormal result: units of 2^-24, value = m * 2^(e-52) */
  int shift = 28 - e; /* >= 43 */
  if (shift > 54)
    return sign;
  uint64_t q = m >> shift;
  uint64_t rem = m & ((1ULL << shift) - 1);
  uint64_t half = 1ULL << (shift - 1);
  if (rem > half || (rem == half && (q & 1)))
    q++;
  return (uint16_t)(sign | (uint16_t)q); /* q == 0x400 encodes the min normal */
}

double tbo_f16_to_f64(uint16_t h) {
  int sign = (h >> 15) & 1;
  int exp = (h >> 10) & 0x1f;
  int frac = h & 0x3ff;
  double v;
  if (exp == 0)
    v = ldexp((double)frac, -24);
  else if (exp == 31)
    v = frac ? NAN : INFINITY;
  else
    v = ldexp((double)(frac | 0x400), exp - 25);
  return sign ? -v : v;
}

void tbo_fill_f16(uint16_t *out, int64_t rows, int64_t cols, int64_t ld,
                  uint64_t seed, int dist, double scale) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      uint64_t idx = (uint64_t)(r * cols + c);
      double v = dist == 1 ? tbo_normal_at(seed, idx) : tbo_uniform_at(seed, idx);
      out[r * ld + c] = tbo_f64_to_f16(v * scale);
    }
  }
}

/* ------------------------------------------------------------------------ */
/* GEMM oracle. The reference's kernel computes C <- C + A*B with f16 A/B and
 * f32 C (accumulator initialised from C: lib/Transforms/
 * LowerPipelineToNVGPU.cpp:994-995, :2246-2263; the Triton comparator has the
 * same acc = load(C); acc += dot(a, b); store(C) body,
 * tools/build_triton_stage1_kernel.py:50-74). With init == NULL this is the
 * C = A*B form the f16-output configs use.                                  */
/* ------------------------------------------------------------------------ */
void tbo_gemm_f64(const uint16_t *A, const uint16_t *B, const float *init,
                  double *ref, int64_t M, int64_t N, int64_t K, int64_t lda,
                  int64_t ldb, int64_t ldi, int64_t ldr, int64_t row_begin,
                  int64_t row_end, int threads) {
  (void)M;
  double *Bd = (double *)malloc(sizeof(double) * (size_t)(K * N));
  if (!Bd)
    abort();
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : tbo_max_threads())
  for (int64_t k = 0; k < K; ++k)
    for (int64_t j = 0; j < N; ++j)
      Bd[k * N + j] = tbo_f16_to_f64(B[k * ldb + j]);

  const int64_t IB = 16, JB = 512, KB = 8;
  int64_t rows = row_end - row_begin;
  int64_t nib = (rows + IB - 1) / IB, njb = (N + JB - 1) / JB;
#pragma omp parallel num_threads(threads > 0 ? threads : tbo_max_threads())
  {
    double *acc = (double *)malloc(sizeof(double) * (size_t)(IB * JB));
    double *arow = (double *)malloc(sizeof(double) * (size_t)(IB * K));
#pragma omp for schedule(dynamic, 1)
    for (int64_t t = 0; t < nib * njb; ++t) {
      int64_t i0 = row_begin + (t / njb) * IB, j0 = (t % njb) * JB;
      int64_t ni = i0 + IB <= row_end ? IB : row_end - i0;
      int64_t nj = j0 + JB <= N ? JB : N - j0;
      for (int64_t i = 0; i < ni; ++i) {
        for (int64_t k = 0; k < K; ++k)
          arow[i * K + k] = tbo_f16_to_f64(A[(i0 + i) * lda + k]);
        for (int64_t j = 0; j < nj; ++j)
          acc[i * JB + j] = init ? (double)init[(i0 + i) * ldi + j0 + j] : 0.0;
      }
      for (int64_t k0 = 0; k0 < K; k0 += KB) {
        int64_t nk = k0 + KB <= K ? KB : K - k0;
        for (int64_t i = 0; i < ni; ++i) {
          const double *a = arow + i * K + k0;
          double *c = acc + i * JB;
          for (int64_t kk = 0; kk < nk; ++kk) {
            const double av = a[kk];
            const double *b = Bd + (k0 + kk) * N + j0;
            for (int64_t j = 0; j < nj; ++j)
              c[j] += av * b[j];
          }
        }
      }
      for (int64_t i = 0; i < ni; ++i)
        memcpy(ref + (i0 - row_begin + i) * ldr + j0, acc + i * JB,
               sizeof(double) * (size_t)nj);
    }
    free(acc);
    free(arow);
  }
  free(Bd);
}

/* ------------------------------------------------------------------------ */
/* Fused epilogue steps on an f64 result, in place: ref[r][c] += bias[c],
 * then the activation, then the clamp (the order the backend derives; the
 * reference declares these expr kinds, include/tb/Analysis/EpiloguePlan.h:
 * 61-75, but implements none, so the formulas are the textbook ones:
 * relu max(x, 0); GELU in its tanh form, Hendrycks & Gimpel 2016,
 * 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))); SiLU x / (1 + e^-x)).
 * act: 0 none, 1 relu, 2 gelu_tanh, 3 silu. clamp_bits: 1 min, 2 max.      */
/* ------------------------------------------------------------------------ */
void tbo_epilogue_f64(double *ref, int64_t rows, int64_t N, int64_t ldr,
                      const double *bias, int act, int clamp_bits, double lo,
                      double hi) {
  const double k0 = sqrt(2.0 / 3.14159265358979323846);
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t j = 0; j < N; ++j) {
      double x = ref[r * ldr + j];
      if (bias)
        x += bias[j];
      if (act == 1)
        x = x > 0.0 ? x : 0.0;
      else if (act == 2)
        x = 0.5 * x * (1.0 + tanh(k0 * (x + 0.044715 * x * x * x)));
      else if (act == 3)
        x = x / (1.0 + exp(-x));
      if ((clamp_bits & 1) && x < lo)
        x = lo;
      if ((clamp_bits & 2) && x > hi)
        x = hi;
      ref[r * ldr + j] = x;
    }
}

int64_t tbo_check_tolerance(const void *got, int got_is_f32, int64_t ldg,
                            const double *ref, int64_t ldr, int64_t N,
                            int64_t row_begin, int64_t row_end, double rtol,
                            double *max_abs_err, int64_t *worst_row,
                            int64_t *worst_col) {
  int64_t bad = 0;
  double worst = -1.0;
  int64_t wr = -1, wc = -1;
  for (int64_t i = row_begin; i < row_end; ++i) {
    for (int64_t j = 0; j < N; ++j) {
      double g = got_is_f32 ? (double)((const float *)got)[i * ldg + j]
                            : tbo_f16_to_f64(((const uint16_t *)got)[i * ldg + j]);
      double r = ref[(i - row_begin) * ldr + j];
      double err = fabs(g - r);
      if (!(err <= rtol * (fabs(r) + 1.0)))
        ++bad; /* also counts NaN */
      if (!(err <= worst)) {
        worst = err;
        wr = i;
        wc = j;
      }
    }
  }
  if (max_abs_err)
    *max_abs_err = worst;
  if (worst_row)
    *worst_row = wr;
  if (worst_col)
    *worst_col = wc;
  return bad;
}

/* ------------------------------------------------------------------------ */
/* Host fp32 GEMM baseline: packed B panels (KC x 16), packed A panels
 * (MC x KC in 6-row slivers), 6x16 register micro-kernel written with GCC
 * vector extensions (AVX2 width), OpenMP over MC blocks.                    */
/* ------------------------------------------------------------------------ */
typedef float v8f __attribute__((vector_size(32)));
#define MR 6
#define NR 16
#define MC 120
#define KC 256
#define NC 2048

int tbo_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

static void micro_6x16(int64_t kc, const float *ap, const float *bp, float *c,
                       int64_t ldc, int64_t mr, int64_t nr) {
  v8f acc[MR][2];
  for (int i = 0; i < MR; ++i)
    acc[i][0] = acc[i][1] = (v8f){0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t k = 0; k < kc; ++k) {
    v8f b0, b1;
    memcpy(&b0, bp + k * NR, 32);
    memcpy(&b1, bp + k * NR + 8, 32);
    for (int i = 0; i < MR; ++i) {
      float a = ap[k * MR + i];
      v8f av = {a, a, a, a, a, a, a, a};
      acc[i][0] += av * b0;
      acc[i][1] += av * b1;
    }
  }
  float tmp[NR];
  for (int64_t i = 0; i < mr; ++i) {
    memcpy(tmp, &acc[i][0], 32);
    memcpy(tmp + 8, &acc[i][1], 32);
    for (int64_t j = 0; j < nr; ++j)
      c[i * ldc + j] += tmp[j];
  }
}

void tbo_gemm_f32(const float *A, const float *B, float *C, int64_t M,
                  int64_t N, int64_t K, int threads) {
  int nt = threads > 0 ? threads : tbo_max_threads();
  memset(C, 0, sizeof(float) * (size_t)(M * N));
  float *Bp = (float *)aligned_alloc(64, sizeof(float) * (size_t)(KC * (NC + NR)));
  for (int64_t jc = 0; jc < N; jc += NC) {
    int64_t nc = jc + NC <= N ? NC : N - jc;
    for (int64_t pc = 0; pc < K; pc += KC) {
      int64_t kc = pc + KC <= K ? KC : K - pc;
      int64_t npanels = (nc + NR - 1) / NR;
#pragma omp parallel for num_threads(nt) schedule(static)
      for (int64_t jp = 0; jp < npanels; ++jp) {
        float *dst = Bp + jp * KC * NR;
        for (int64_t k = 0; k < kc; ++k)
          for (int64_t j = 0; j < NR; ++j) {
            int64_t col = jc + jp * NR + j;
            dst[k * NR + j] = col < jc + nc ? B[(pc + k) * N + col] : 0.0f;
          }
      }
      int64_t nblocks = (M + MC - 1) / MC;
#pragma omp parallel num_threads(nt)
      {
        float *Ap = (float *)aligned_alloc(64, sizeof(float) * (size_t)(KC * (MC + MR)));
#pragma omp for schedule(dynamic, 1)
        for (int64_t ib = 0; ib < nblocks; ++ib) {
          int64_t ic = ib * MC;
          int64_t mc = ic + MC <= M ? MC : M - ic;
          int64_t nsl = (mc + MR - 1) / MR;
          for (int64_t s = 0; s < nsl; ++s)
            for (int64_t k = 0; k < kc; ++k)
              for (int64_t i = 0; i < MR; ++i) {
                int64_t row = ic + s * MR + i;
                Ap[s * KC * MR + k * MR + i] =
                    row < ic + mc ? A[row * K + pc + k] : 0.0f;
              }
          for (int64_t jp = 0; jp < npanels; ++jp) {
            int64_t nr = jc + jp * NR + NR <= jc + nc ? NR : jc + nc - (jc + jp * NR);
            for (int64_t s = 0; s < nsl; ++s) {
              int64_t mr = s * MR + MR <= mc ? MR : mc - s * MR;
              micro_6x16(kc, Ap + s * KC * MR, Bp + jp * KC * NR,
                         C + (ic + s * MR) * N + jc + jp * NR, N, mr, nr);
            }
          }
        }
        free(Ap);
      }
    }
  }
  free(Bp);
}

/* ------------------------------------------------------------------------ */
/* Program -> tile index math.                                               */
/* ------------------------------------------------------------------------ */
/* Tile / grouped / persistent: lib/Transforms/LowerPipelineToNVGPU.cpp:286-305
 * (group = pid / (gM*tilesN), first = group*gM, gsz = min(gM, tilesM-first),
 * m = first + (pid % ppg) % gsz, n = (pid % ppg) / gsz); the launch-group
 * fields come from lib/Analysis/ProgramMappingPlan.cpp:389-443 (row-major
 * tile order is the gM = 1 case). Split-K: LowerPipelineToNVGPU.cpp:306-317
 * (m = pid / (tilesN*S), n = (pid % (tilesN*S)) / S, part = pid % S). The
 * reference forces gM = 1 for persistent (ProgramMappingPlan.cpp:389-401);
 * mapping 4 is this build's grouped persistent order, the same formula.     */
void tbo_program_to_tile(int mapping, int64_t pid, int64_t tiles_m,
                         int64_t tiles_n, int64_t group_m, int64_t split_k,
                         int64_t *tile_m, int64_t *tile_n, int64_t *part) {
  if (mapping == 2) {
    int64_t ppg = tiles_n * split_k;
    int64_t in_group = pid % ppg;
    *tile_m = pid / ppg;
    *tile_n = in_group / split_k;
    *part = in_group % split_k;
    return;
  }
  int64_t gm = (mapping == 1 || mapping == 4) ? group_m : 1;
  int64_t ppg = gm * tiles_n;
  int64_t group = pid / ppg;
  int64_t first = group * gm;
  int64_t gsz = tiles_m - first < gm ? tiles_m - first : gm;
  int64_t in_group = pid % ppg;
  *tile_m = first + in_group % gsz;
  *tile_n = in_group / gsz;
  *part = 0;
}

/* LowerPipelineToNVGPU.cpp:331-356: base = tilesK / S, extra = tilesK % S,
 * start = part*base + min(part, extra), count = base + (part < extra).      */
void tbo_split_k_range(int64_t tiles_k, int64_t split_k, int64_t part,
                       int64_t *start, int64_t *count) {
  int64_t base = tiles_k / split_k, extra = tiles_k % split_k;
  *start = part * base + (part < extra ? part : extra);
  *count = base + (part < extra ? 1 : 0);
}

/* LowerPipelineToNVGPU.cpp:1589-1621: phase = (major / perPhase) % maxPhase,
 * chunk' = ((minor / span) ^ phase) % (minorExtent / span).                 */
int64_t tbo_swizzle_minor(int64_t major, int64_t minor, int64_t per_phase,
                          int64_t max_phase, int64_t span_elems,
                          int64_t minor_extent) {
  if (max_phase <= 1 || span_elems <= 0)
    return minor;
  int64_t pp = per_phase > 1 ? per_phase : 1;
  int64_t phase = (major / pp) % max_phase;
  int64_t chunks = minor_extent / span_elems > 1 ? minor_extent / span_elems : 1;
  int64_t chunk = minor / span_elems, in_chunk = minor % span_elems;
  return ((chunk ^ phase) % chunks) * span_elems + in_chunk;
}

/* The gfx950 shared encoding with a second XOR term: the reference's swizzle
 * above, then the unit of span2_elems elements inside it XORed with
 * (major / per_phase2) % max_phase2 (span2 * max_phase2 <= span, so the term
 * permutes units inside one first-term span). max_phase2 <= 1 = no second
 * term. */
int64_t tbo_swizzle_minor2(int64_t major, int64_t minor, int64_t per_phase,
                           int64_t max_phase, int64_t span_elems, int64_t per_phase2,
                           int64_t max_phase2, int64_t span2_elems,
                           int64_t minor_extent) {
  int64_t m1 = tbo_swizzle_minor(major, minor, per_phase, max_phase, span_elems,
                                 minor_extent);
  if (max_phase2 <= 1 || span2_elems <= 0)
    return m1;
  int64_t pp2 = per_phase2 > 1 ? per_phase2 : 1;
  int64_t phase2 = (major / pp2) % max_phase2;
  return ((m1 / span2_elems) ^ phase2) * span2_elems + m1 % span2_elems;
}
