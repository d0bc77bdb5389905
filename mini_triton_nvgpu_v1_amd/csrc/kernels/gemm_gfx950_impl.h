// Template body of the gfx950 MFMA GEMM kernel. Included by the instance
// translation units (gemm_inst_*.hip); see gemm_gfx950.h for the design.
#pragma once

#include "gemm_gfx950.h"

namespace tbk {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Buffer descriptor dword3 for gfx9-family raw buffers (stride 0, untyped,
// bounds checked against num_records).
static constexpr int kBufferFlags = 0x00020000;
// Any offset at or above num_records reads zero / drops the store; the host
// guarantees every operand spans fewer than 2^31 bytes.
static constexpr uint32_t kOob = 0x80000000u;

// sched_group_barrier instruction classes (LLVM AMDGPU)
static constexpr int kSchedMfma = 0x008;
static constexpr int kSchedVmemRead = 0x020;
static constexpr int kSchedDsRead = 0x100;
static constexpr int kSchedDsWrite = 0x200;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p,
                                                            uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0,
                                           (int)bytes, kBufferFlags);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r,
                                            uint32_t voff, int soff) {
  return __builtin_bit_cast(
      u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Physical 16-byte chunk of (row, chunk) in a K-contiguous LDS tile with
// KCH chunks per row.
template <int KCH>
__device__ __forceinline__ int swz(int row, int chunk) {
  constexpr int PP = KCH >= 8 ? 1 : 8 / KCH; // rows per phase
  const int phase = ((row / PP) ^ (row / (8 * PP))) & (KCH - 1);
  return chunk ^ phase;
}

// Program id -> (tile_m, tile_n, split part).
// tile / grouped / persistent: lib/Transforms/LowerPipelineToNVGPU.cpp:286-305
// split-K: LowerPipelineToNVGPU.cpp:306-317
__device__ __forceinline__ void map_program(const GemmParams &p, int pid,
                                            int &tm, int &tn, int &part) {
  if (p.mapping == kMapSplitK) {
    const int ppg = p.tiles_n * p.split_k;
    const int in_group = pid % ppg;
    tm = pid / ppg;
    tn = in_group / p.split_k;
    part = in_group % p.split_k;
    return;
  }
  const int gm =
      (p.mapping == kMapGrouped || p.mapping == kMapPersistentGrouped) ? p.group_m
                                                                        : 1;
  const int ppg = gm * p.tiles_n;
  const int group = pid / ppg;
  const int first = group * gm;
  const int rem = p.tiles_m - first;
  const int gsz = rem < gm ? rem : gm;
  const int in_group = pid % ppg;
  tm = first + in_group % gsz;
  tn = in_group / gsz;
  part = 0;
}

template <int BM, int BN, int BK, int WGM, int WGN, int OUT>
struct GemmTile {
  static constexpr int NT = WGM * WGN * 64;
  static constexpr int WTM = BM / WGM;
  static constexpr int WTN = BN / WGN;
  static constexpr int TM = WTM / 32;
  static constexpr int TN = WTN / 32;
  static constexpr int NMFMA = TM * TN; // MFMAs per 16-deep k step per wave
  static constexpr int KCH = BK / 8;    // 16-byte chunks per LDS row
  static constexpr int KSTEPS = BK / 16;
  // A: BM*KCH chunks; thread t owns rows t/KCH + i*RS, chunk t%KCH
  static constexpr int NA = BM * KCH / NT;
  static constexpr int RS = NT / KCH;
  // B: blocks of KB rows x 8 columns, transposed in registers
  static constexpr int KB = ((BK / 8) * (BN / 8) >= NT)   ? 8
                            : ((BK / 4) * (BN / 8) >= NT) ? 4
                            : ((BK / 2) * (BN / 8) >= NT) ? 2
                                                          : 1;
  static constexpr int NBB = (BK / KB) * (BN / 8) / NT;
  static constexpr int A_STAGE = BM * KCH; // in 16-byte chunks
  static constexpr int B_STAGE = BN * KCH;
  static constexpr int STAGE = A_STAGE + B_STAGE;
  static constexpr int LDS_BYTES = 2 * STAGE * 16;
  // k step (within a k-tile) at which the next tile's A / B are written to
  // LDS and the tile after that is requested from global memory
  static constexpr int STEP_A = 0;
  static constexpr int STEP_B = KSTEPS >= 4 ? 1 : 0;

  static_assert(BM % (WGM * 32) == 0 && BN % (WGN * 32) == 0, "wave tile");
  static_assert(KSTEPS == 2 || KSTEPS == 4, "BK must be 32 or 64");
  static_assert(NT % KCH == 0, "threads per A row chunk");
  static_assert(NA >= 1 && NA * NT == BM * KCH, "A chunks per thread");
  static_assert(NBB >= 1 && NBB * NT == (BK / KB) * (BN / 8), "B blocks");
};

// Interleave one k step's MFMAs with its memory traffic so the matrix pipe
// never waits behind a burst of LDS or global instructions.
template <int NMFMA, int NREAD, int NWRITE, int NVMEM>
__device__ __forceinline__ void sched_step() {
#pragma unroll
  for (int i = 0; i < NMFMA; ++i) {
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
    if (i < NREAD)
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    if (i < NWRITE)
      __builtin_amdgcn_sched_group_barrier(kSchedDsWrite, 1, 0);
    if (i < NVMEM)
      __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
  }
}

template <int BM, int BN, int BK, int WGM, int WGN, int OUT>
__global__ __launch_bounds__(WGM *WGN * 64, 1) void gemm_kernel(GemmParams p) {
  using T = GemmTile<BM, BN, BK, WGM, WGN, OUT>;
  constexpr int NT = T::NT, KCH = T::KCH, NA = T::NA, KB = T::KB,
                NBB = T::NBB, TM = T::TM, TN = T::TN, RS = T::RS,
                KSTEPS = T::KSTEPS, NMFMA = T::NMFMA;
  __shared__ u32x4 lds[2 * T::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;

  const __amdgpu_buffer_rsrc_t ra =
      make_rsrc(p.A, (uint32_t)p.M * (uint32_t)p.lda * 2u);
  const __amdgpu_buffer_rsrc_t rb =
      make_rsrc(p.B, (uint32_t)p.K * (uint32_t)p.ldb * 2u);

  const bool persistent =
      p.mapping == kMapPersistent || p.mapping == kMapPersistentGrouped;
  int prog = blockIdx.x;
  const int nprog = gridDim.x;
  if (p.xcds > 1 && (nprog % p.xcds) == 0)
    prog = (prog % p.xcds) * (nprog / p.xcds) + prog / p.xcds;

  // per-thread constants of the global -> LDS transport
  const int a_row0 = tid / KCH, a_c = tid % KCH;
  const int a_soff_step = RS * p.lda * 2; // bytes between this thread's A rows
  const int fr_a = wm * T::WTM + (lane & 31); // fragment rows in the A tile
  const int fr_b = wn * T::WTN + (lane & 31); // fragment rows in the B^T tile
  const int khalf = lane >> 5;

  for (int work = prog; work < p.total_work;
       work += (persistent ? nprog : p.total_work)) {
    int tile_m, tile_n, part;
    map_program(p, work, tile_m, tile_n, part);
    int kt0 = 0, nk = p.tiles_k;
    if (p.mapping == kMapSplitK) {
      // LowerPipelineToNVGPU.cpp:331-356 (contiguous k-tile range per split)
      const int base = p.tiles_k / p.split_k, extra = p.tiles_k % p.split_k;
      kt0 = part * base + (part < extra ? part : extra);
      nk = base + (part < extra ? 1 : 0);
    }
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int kt_end = kt0 + nk;

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = (f32x16){};

    // The k-dependent part of every global address is wave-uniform and rides
    // in the buffer instruction's scalar offset. A row, column or k-tile
    // outside the problem gets the vector offset kOob: the load returns 0.
    const uint32_t a_voff =
        ((uint32_t)(m0 + a_row0) * (uint32_t)p.lda + (uint32_t)(a_c * 8)) * 2u;
    const int a_rows_left = p.M - m0 - a_row0; // row i valid iff i*RS < left
    uint32_t b_voff[NBB];
    int b_k[NBB];
#pragma unroll
    for (int j = 0; j < NBB; ++j) {
      const int b = tid + j * NT;
      const int kb = b / (BN / 8), nb = b % (BN / 8);
      b_k[j] = kb * KB;
      b_voff[j] = (n0 + nb * 8) < p.N
                      ? ((uint32_t)(kb * KB) * (uint32_t)p.ldb +
                         (uint32_t)(n0 + nb * 8)) * 2u
                      : kOob;
    }

    u32x4 ra_reg[NA];
    u32x4 rb_reg[NBB][KB];

    auto gload_a = [&](int kt) {
      const int k0 = kt * BK;
      const bool kt_ok = kt < kt_end && (k0 + a_c * 8) < p.K;
#pragma unroll
      for (int i = 0; i < NA; ++i)
        ra_reg[i] = buf_load16(ra, (kt_ok && i * RS < a_rows_left) ? a_voff : kOob,
                               k0 * 2 + i * a_soff_step);
    };
    auto gload_b = [&](int kt) {
      const int k0 = kt * BK;
#pragma unroll
      for (int j = 0; j < NBB; ++j)
#pragma unroll
        for (int r = 0; r < KB; ++r) {
          const bool ok = kt < kt_end && (k0 + b_k[j] + r) < p.K;
          rb_reg[j][r] = buf_load16(rb, ok ? b_voff[j] : kOob, (k0 + r) * p.ldb * 2);
        }
    };
    auto lds_store_a = [&](int stage) {
      u32x4 *As = lds + stage * T::STAGE;
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int row = a_row0 + i * RS;
        As[row * KCH + swz<KCH>(row, a_c)] = ra_reg[i];
      }
    };
    auto lds_store_b = [&](int stage) {
      u32x4 *Bs = lds + stage * T::STAGE + T::A_STAGE;
#pragma unroll
      for (int j = 0; j < NBB; ++j) {
        const int b = tid + j * NT;
        const int kb = b / (BN / 8), nb = b % (BN / 8);
        const int kk = kb * KB; // first k of the block inside the tile
        const int c = kk / 8, within = kk % 8;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const int n = nb * 8 + t;
          const int dw = t >> 1; // dword holding column t in each row
          const bool hi = (t & 1) != 0;
          char *rowp = reinterpret_cast<char *>(Bs + n * KCH + swz<KCH>(n, c)) +
                       within * 2;
          if constexpr (KB == 8) {
            u32x4 v;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const uint32_t lo = rb_reg[j][2 * q][dw], up = rb_reg[j][2 * q + 1][dw];
              v[q] = hi ? ((lo >> 16) | (up & 0xffff0000u))
                        : ((lo & 0xffffu) | (up << 16));
            }
            *reinterpret_cast<u32x4 *>(rowp) = v;
          } else if constexpr (KB == 4) {
            u32x2 v;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              const uint32_t lo = rb_reg[j][2 * q][dw], up = rb_reg[j][2 * q + 1][dw];
              v[q] = hi ? ((lo >> 16) | (up & 0xffff0000u))
                        : ((lo & 0xffffu) | (up << 16));
            }
            *reinterpret_cast<u32x2 *>(rowp) = v;
          } else if constexpr (KB == 2) {
            const uint32_t lo = rb_reg[j][0][dw], up = rb_reg[j][1][dw];
            *reinterpret_cast<uint32_t *>(rowp) =
                hi ? ((lo >> 16) | (up & 0xffff0000u)) : ((lo & 0xffffu) | (up << 16));
          } else {
            const uint32_t w = rb_reg[j][0][dw];
            *reinterpret_cast<uint16_t *>(rowp) = (uint16_t)(hi ? (w >> 16) : w);
          }
        }
      }
    };

    half8 fa[2][TM], fb[2][TN];
    auto read_frags = [&](int buf, int stage, int ks) {
      const u32x4 *As = lds + stage * T::STAGE;
      const u32x4 *Bs = As + T::A_STAGE;
      const int c = ks * 2 + khalf;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = fr_a + i * 32;
        fa[buf][i] = __builtin_bit_cast(half8, As[row * KCH + swz<KCH>(row, c)]);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = fr_b + j * 32;
        fb[buf][j] = __builtin_bit_cast(half8, Bs[row * KCH + swz<KCH>(row, c)]);
      }
    };
    // C^T tile += B^T-fragment x A-fragment, i.e. C += A*B for this k step
    auto mfma_range = [&](int buf, int lo, int hi) {
#pragma unroll
      for (int q = 0; q < NMFMA; ++q) {
        if (q >= lo && q < hi) {
          const int i = q / TN, j = q % TN;
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[buf][j], fa[buf][i],
                                                             acc[i][j], 0, 0, 0);
        }
      }
    };

    // ---- prologue: tile kt0 -> LDS stage 0, tile kt0+1 -> registers -------
    if (persistent)
      __syncthreads(); // the previous tile's last fragment reads are done
    gload_a(kt0);
    gload_b(kt0);
    lds_store_a(0);
    lds_store_b(0);
    gload_a(kt0 + 1);
    gload_b(kt0 + 1);
    __syncthreads();
    read_frags(0, 0, 0);

    // ---- main loop --------------------------------------------------------
    // k-tile `it` is consumed from LDS stage it&1 while tile it+1 moves from
    // registers into the other stage and tile it+2 is requested from global
    // memory. Fragments are double-buffered across the 16-deep k steps. The
    // single barrier per k-tile sits in the middle of the last k step, after
    // the next stage is complete and before its first fragments are read.
    // Every step is unconditional (out-of-range tiles load zeros), so one
    // iteration is one basic block the scheduler can interleave freely.
    for (int it = 0; it < nk; ++it) {
      const int s = it & 1;
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const int cur = ks & 1;
        if (ks + 1 < KSTEPS) {
          read_frags(cur ^ 1, s, ks + 1);
          if (ks == T::STEP_A) {
            lds_store_a(s ^ 1);
            gload_a(kt0 + it + 2);
          }
          if (ks == T::STEP_B) {
            lds_store_b(s ^ 1);
            gload_b(kt0 + it + 2);
          }
          mfma_range(cur, 0, NMFMA);
          constexpr int NW = (T::STEP_A == T::STEP_B) ? NA + NBB * 8 : NA;
          if (ks == T::STEP_A && T::STEP_A == T::STEP_B)
            sched_step<NMFMA, TM + TN, NA + NBB * 8, NA + NBB * KB>();
          else if (ks == T::STEP_A)
            sched_step<NMFMA, TM + TN, NW, NA>();
          else if (ks == T::STEP_B)
            sched_step<NMFMA, TM + TN, NBB * 8, NBB * KB>();
          else
            sched_step<NMFMA, TM + TN, 0, 0>();
          __builtin_amdgcn_sched_barrier(0); // k steps do not mix
        } else {
          mfma_range(cur, 0, NMFMA / 2);
          __builtin_amdgcn_sched_barrier(0);
          __syncthreads();
          read_frags(cur ^ 1, s ^ 1, 0);
          mfma_range(cur, NMFMA / 2, NMFMA);
          sched_step<NMFMA - NMFMA / 2, TM + TN, 0, 0>();
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }

    // ---- epilogue ---------------------------------------------------------
    // lane holds C[m0 + wm*WTM + i*32 + lane%32][n0 + wn*WTN + j*32 + 8g + 4h + r]
    // in acc[i][j][4g + r], h = lane / 32.
    const int crow_base = m0 + wm * T::WTM + (lane & 31);
    const int ccol_base = n0 + wn * T::WTN + 4 * khalf;
    if constexpr (OUT == kOutF16) {
      const __amdgpu_buffer_rsrc_t rc =
          make_rsrc(p.C, (uint32_t)p.M * (uint32_t)p.ldc * 2u);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = crow_base + i * 32;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int col = ccol_base + j * 32 + 8 * g;
            const bool ok = row < p.M && col < p.N;
            const uint32_t off =
                ok ? ((uint32_t)row * (uint32_t)p.ldc + (uint32_t)col) * 2u : kOob;
            const _Float16 h0 = (_Float16)acc[i][j][4 * g + 0];
            const _Float16 h1 = (_Float16)acc[i][j][4 * g + 1];
            const _Float16 h2 = (_Float16)acc[i][j][4 * g + 2];
            const _Float16 h3 = (_Float16)acc[i][j][4 * g + 3];
            u32x2 v;
            v[0] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            v[1] = (uint32_t)__builtin_bit_cast(uint16_t, h2) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16);
            __builtin_amdgcn_raw_buffer_store_b64(v, rc, off, 0, 0);
          }
      }
    } else if constexpr (OUT == kOutF32Partial || OUT == kOutF32Accum) {
      float *base = OUT == kOutF32Partial
                        ? p.ws + (size_t)part * (size_t)p.M * (size_t)p.ws_ld
                        : reinterpret_cast<float *>(p.C);
      const int ld = OUT == kOutF32Partial ? p.ws_ld : p.ldc;
      const __amdgpu_buffer_rsrc_t rc =
          make_rsrc(base, (uint32_t)p.M * (uint32_t)ld * 4u);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = crow_base + i * 32;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int col = ccol_base + j * 32 + 8 * g;
            const bool ok = row < p.M && col < p.N;
            const uint32_t off =
                ok ? ((uint32_t)row * (uint32_t)ld + (uint32_t)col) * 4u : kOob;
            f32x4 v = {acc[i][j][4 * g + 0], acc[i][j][4 * g + 1],
                       acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
            if constexpr (OUT == kOutF32Accum) {
              const f32x4 old = __builtin_bit_cast(
                  f32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, off, 0, 0));
              v += old;
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v),
                                                   rc, off, 0, 0);
          }
      }
    } else { // kOutF32Atomic
      float *C = reinterpret_cast<float *>(p.C);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = crow_base + i * 32;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int col = ccol_base + j * 32 + 8 * g;
            if (row < p.M && col < p.N) {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                unsafeAtomicAdd(C + (size_t)row * p.ldc + col + r,
                                acc[i][j][4 * g + r]);
            }
          }
      }
    }
    if (!persistent)
      break;
  }
}

} // namespace tbk

// One registry entry per instance.
#define TBK_ENTRY(BM, BN, BK, WGM, WGN, OUT)                                     \
  {{BM, BN, BK, WGM, WGN, OUT},                                                  \
   reinterpret_cast<const void *>(&tbk::gemm_kernel<BM, BN, BK, WGM, WGN, OUT>), \
   "tb_gemm_gfx950_" #BM "x" #BN "x" #BK "_w" #WGM "x" #WGN "_out" #OUT}
