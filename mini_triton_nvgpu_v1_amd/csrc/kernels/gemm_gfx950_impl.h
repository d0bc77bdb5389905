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

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p,
                                                            uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0,
                                           (int)bytes, kBufferFlags);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r,
                                            uint32_t off) {
  return __builtin_bit_cast(u32x4,
                            __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
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
  static constexpr int KCH = BK / 8; // 16-byte chunks per LDS row
  static constexpr int KSTEPS = BK / 16;
  // A: BM*KCH chunks
  static constexpr int NA = BM * KCH / NT;
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

  static_assert(BM % (WGM * 32) == 0 && BN % (WGN * 32) == 0, "wave tile");
  static_assert(BK % 16 == 0 && KCH <= 8, "BK must be 16, 32 or 64");
  static_assert(NA >= 1 && NA * NT == BM * KCH, "A chunks per thread");
  static_assert(NBB >= 1 && NBB * NT == (BK / KB) * (BN / 8), "B blocks");
};

template <int BM, int BN, int BK, int WGM, int WGN, int OUT>
__global__ __launch_bounds__(WGM *WGN * 64, 1) void gemm_kernel(GemmParams p) {
  using T = GemmTile<BM, BN, BK, WGM, WGN, OUT>;
  constexpr int NT = T::NT, KCH = T::KCH, NA = T::NA, KB = T::KB,
                NBB = T::NBB, TM = T::TM, TN = T::TN;
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

  for (int work = prog; work < p.total_work; work += (persistent ? nprog : p.total_work)) {
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

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = (f32x16){};

    // ---- per-thread global coordinates (fixed across the K loop) --------
    // The k-dependent part of every address is wave-uniform and travels in
    // the buffer instruction's scalar offset; a row or column outside the
    // problem gets a vector offset of kOob so the load returns zeros.
    const int a_kc = (tid % KCH) * 8; // same k chunk for all of this thread's A rows
    uint32_t a_voff[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int row = (tid + i * NT) / KCH;
      a_voff[i] = (m0 + row) < p.M
                      ? ((uint32_t)(m0 + row) * (uint32_t)p.lda + (uint32_t)a_kc) * 2u
                      : kOob;
    }
    uint32_t b_voff[NBB];
    int b_k[NBB];
#pragma unroll
    for (int j = 0; j < NBB; ++j) {
      const int b = tid + j * NT;
      const int kb = b / (BN / 8), nb = b % (BN / 8);
      b_k[j] = kb * KB;
      b_voff[j] = (n0 + nb * 8) < p.N
                      ? ((uint32_t)(kb * KB) * (uint32_t)p.ldb + (uint32_t)(n0 + nb * 8)) * 2u
                      : kOob;
    }

    u32x4 ra_reg[NA];
    u32x4 rb_reg[NBB][KB];

    auto gload = [&](int kt) {
      const int k0 = kt * BK;
      const bool kedge = k0 + BK > p.K; // only the last k-tile of a ragged K
      const bool a_ok = !kedge || (k0 + a_kc) < p.K;
#pragma unroll
      for (int i = 0; i < NA; ++i)
        ra_reg[i] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       ra, a_ok ? a_voff[i] : kOob, k0 * 2, 0));
#pragma unroll
      for (int j = 0; j < NBB; ++j)
#pragma unroll
        for (int r = 0; r < KB; ++r) {
          const bool ok = !kedge || (k0 + b_k[j] + r) < p.K;
          rb_reg[j][r] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         rb, ok ? b_voff[j] : kOob, (k0 + r) * p.ldb * 2, 0));
        }
    };

    auto lds_store = [&](int stage) {
      u32x4 *As = lds + stage * T::STAGE;
      u32x4 *Bs = As + T::A_STAGE;
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int q = tid + i * NT;
        const int row = q / KCH, c = q % KCH;
        As[row * KCH + swz<KCH>(row, c)] = ra_reg[i];
      }
#pragma unroll
      for (int j = 0; j < NBB; ++j) {
        const int b = tid + j * NT;
        const int kb = b / (BN / 8), nb = b % (BN / 8);
        const int kk = kb * KB; // first k of the block inside the tile
        const int c = kk / 8, within = kk % 8;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const int n = nb * 8 + t;
          const int dw = t >> 1;      // dword holding column t in each row
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

    // ---- main loop: 2 LDS stages + one k-tile of register prefetch -------
    gload(kt0);
    lds_store(0);
    if (nk > 1)
      gload(kt0 + 1);
    __syncthreads();

    const int a_row0 = wm * T::WTM + (lane & 31);
    const int b_row0 = wn * T::WTN + (lane & 31);
    const int khalf = lane >> 5;

    for (int it = 0; it < nk; ++it) {
      const int s = it & 1;
      if (it + 1 < nk) {
        lds_store(s ^ 1);
        if (it + 2 < nk)
          gload(kt0 + it + 2);
      }
      const u32x4 *As = lds + s * T::STAGE;
      const u32x4 *Bs = As + T::A_STAGE;
#pragma unroll
      for (int ks = 0; ks < T::KSTEPS; ++ks) {
        const int c = ks * 2 + khalf;
        half8 af[TM], bf[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int row = a_row0 + i * 32;
          af[i] = __builtin_bit_cast(half8, As[row * KCH + swz<KCH>(row, c)]);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int row = b_row0 + j * 32;
          bf[j] = __builtin_bit_cast(half8, Bs[row * KCH + swz<KCH>(row, c)]);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[j], af[i],
                                                               acc[i][j], 0, 0, 0);
      }
      __syncthreads();
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
            const uint32_t off = ok ? ((uint32_t)row * (uint32_t)p.ldc + (uint32_t)col) * 2u : kOob;
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
            const uint32_t off = ok ? ((uint32_t)row * (uint32_t)ld + (uint32_t)col) * 4u : kOob;
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
