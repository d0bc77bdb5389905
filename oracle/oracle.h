/*
 * CPU oracle for the tb.matmul GEMM path — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker / reported CPU baseline. The
 * product path (libtb_gfx950.so) never links or calls it.
 *
 * Every function restates a piece of the reference's behaviour and cites the
 * reference file:line it follows (paths relative to the reference root).
 */
#ifndef TB_ORACLE_H
#define TB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- seeded input generation (harness inputs, not reference code) ------ */
/* i-th output of the SplitMix64 stream started at `seed` (i = 0 is the first
 * output). Counter form: state_i = seed + (i+1)*golden, then the finaliser. */
uint64_t tbo_splitmix64_at(uint64_t seed, uint64_t i);
/* U[-1,1): (x >> 40) * 2^-24 * 2 - 1, x = tbo_splitmix64_at(seed, i). */
double tbo_uniform_at(uint64_t seed, uint64_t i);
/* N(0,1) by Box-Muller in f64 from draws 2i and 2i+1 of the stream. */
double tbo_normal_at(uint64_t seed, uint64_t i);

/* IEEE binary16 round-to-nearest-even from binary64 (one rounding). */
uint16_t tbo_f64_to_f16(double x);
double tbo_f16_to_f64(uint16_t h);

/* dist: 0 = uniform[-1,1), 1 = normal(0,1). Element (r, c) uses stream
 * index r*cols + c; the value is dist_value * scale rounded to f16. */
void tbo_fill_f16(uint16_t *out, int64_t rows, int64_t cols, int64_t ld,
                  uint64_t seed, int dist, double scale);

/* ---- GEMM oracle -------------------------------------------------------- */
/* ref[i][j] = init[i][j] + sum_k A[i][k]*B[k][j] in f64, f16 operands widened
 * exactly; rows [row_begin, row_end) only (row-sample mode). `init` may be
 * NULL (then 0), else an f32 matrix with leading dimension ldi (the
 * reference's C += A*B form). ref has leading dimension ldr and holds
 * row_end-row_begin rows. OpenMP over rows with `threads` threads (<=0: all). */
void tbo_gemm_f64(const uint16_t *A, const uint16_t *B, const float *init,
                  double *ref, int64_t M, int64_t N, int64_t K, int64_t lda,
                  int64_t ldb, int64_t ldi, int64_t ldr, int64_t row_begin,
                  int64_t row_end, int threads);

/* Per-element tolerance |got - ref| <= rtol*(|ref| + 1). got is f16
 * (got_is_f32 = 0) or f32 (got_is_f32 = 1) with leading dimension ldg; ref as
 * produced by tbo_gemm_f64 for rows [row_begin, row_end). Returns the number
 * of violations; writes the largest |got-ref| and its (row, col). */
/* Fused epilogue steps in place on an f64 result (rows x N, leading
 * dimension ldr): += bias[c] (bias may be NULL), activation (0 none, 1 relu,
 * 2 gelu_tanh, 3 silu), clamp (bit 1: max(x, lo), bit 2: min(x, hi)). */
void tbo_epilogue_f64(double *ref, int64_t rows, int64_t N, int64_t ldr,
                      const double *bias, int act, int clamp_bits, double lo,
                      double hi);
int64_t tbo_check_tolerance(const void *got, int got_is_f32, int64_t ldg,
                            const double *ref, int64_t ldr, int64_t N,
                            int64_t row_begin, int64_t row_end, double rtol,
                            double *max_abs_err, int64_t *worst_row,
                            int64_t *worst_col);

/* Host fp32 GEMM C = A*B (row-major, packed-B cache blocking, OpenMP over
 * M panels). This is the reported CPU baseline, not a correctness oracle. */
void tbo_gemm_f32(const float *A, const float *B, float *C, int64_t M,
                  int64_t N, int64_t K, int threads);
int tbo_max_threads(void);

/* ---- program-mapping index math ---------------------------------------- */
/* mapping: 0 tile (row-major), 1 grouped_tile, 2 split_k, 3 persistent_tile
 * in the reference's row-major order, 4 persistent_tile in grouped order.
 * For the persistent kinds `pid` is the work item the stride loop visits. */
void tbo_program_to_tile(int mapping, int64_t pid, int64_t tiles_m,
                         int64_t tiles_n, int64_t group_m, int64_t split_k,
                         int64_t *tile_m, int64_t *tile_n, int64_t *part);
/* contiguous k-tile range of split `part` among `split_k` splits */
void tbo_split_k_range(int64_t tiles_k, int64_t split_k, int64_t part,
                       int64_t *start, int64_t *count);
/* swizzled minor coordinate of the shared physical layout */
int64_t tbo_swizzle_minor(int64_t major, int64_t minor, int64_t per_phase,
                          int64_t max_phase, int64_t span_elems,
                          int64_t minor_extent);
/* the same plus the gfx950 second XOR term on span2-element units */
int64_t tbo_swizzle_minor2(int64_t major, int64_t minor, int64_t per_phase,
                           int64_t max_phase, int64_t span_elems, int64_t per_phase2,
                           int64_t max_phase2, int64_t span2_elems,
                           int64_t minor_extent);

#ifdef __cplusplus
}
#endif
#endif /* TB_ORACLE_H */
