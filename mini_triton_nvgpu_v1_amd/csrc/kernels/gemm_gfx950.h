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
};

struct KernelKey {
  int bm, bn, bk, wgm, wgn, out, stages;
};

struct KernelEntry {
  KernelKey key;
  const void *fn;
  const char *name;
};

// Registry of compiled instances (defined in the instance files).
const KernelEntry *find_kernel(const KernelKey &k);
int kernel_count();
const KernelEntry *kernel_at(int i);

// C = [C +] sum_{p < split_k} ws[p] in fixed p order, cast to C's type.
hipError_t launch_reduce_ex(const float *ws, void *C, int M, int N, int ldc,
                            int split_k, int c_f16, int load_c, hipStream_t s);
hipError_t launch_fill(void *dst, int64_t rows, int64_t cols, int64_t ld,
                       uint64_t seed, int dist, double scale, hipStream_t s);

} // namespace tbk
