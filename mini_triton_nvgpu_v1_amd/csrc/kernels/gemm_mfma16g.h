// The v_mfma_f32_16x16x32_f16 loop for the tile shapes of TBK_MFMA16_TILES
// (gemm_tiles.h): any block of BM x BN x BK (BK 32 or 64) on a WGM x WGN
// wave grid with 2..4 LDS stages, whose wave tiles hold at least 16
// MFMA tiles of 16 x 16. The 4-wave 256x256x64 2-stage tile keeps its own
// hand-scheduled build (mfma16_tile in gemm_gfx950_impl.h); this template
// carries the same design to the other shapes:
//  * the LDS ring, swizzles and direct-to-LDS loads of the plan's encoding
//    (A: 16-byte chunks, chunk ^ ((row / A_PP) % A_MAXPH); B: the first term
//    over 64-byte segments plus the 16x16x32 second term over 32-byte units,
//    chunk ^ 4 ((k / B_PP) % B_MAXPH) ^ 2 ((k / 8) % 2));
//  * fragment reads: A tile ii one ds_read_b128 (lane l: row 16 ii + l % 16,
//    k 8 (l / 16) .. +7 of the 32-deep k step), B tile jj two
//    ds_read_b64_tr_b16 (k rows 8 (l / 16) + (l % 16) / 4 (+4), columns
//    16 jj + 4 (l % 4) .. +3); the product is C^T += B^T A^T, so lane l ends
//    with C[16 ii + l % 16][16 jj + 4 (l / 16) + r];
//  * the MFMA is inline asm with the accumulator tied in place (no register
//    rotation through copies), so the hazard rules are the schedule's:
//    (a) each accumulator's first MFMA takes srcC = 0, (b) 24 wait states
//    between the last MFMA and the first accumulator read, (c) a fragment
//    register is rewritten at least 8 MFMA slots after its last MFMA read
//    (static_assert-ed in Mfma16GTile);
//  * one barrier per k-tile, before slot BQ of its last k step, after
//    vmcnt((STAGES-2) loads per thread) lgkmcnt(0): the next k-tile has
//    landed and this wave's reads of the stage the barrier frees are done.
//    After it: the next k-tile's first reads and the refill of the freed
//    stage, spread over the MFMA slots;
//  * every loop body runs from one barrier to the next with its ring stage
//    and fragment buffers fixed at compile time (the loop is unrolled by the
//    stage count, and by 2 for 32-deep k-tiles); the lookahead loads past
//    the last k-tile use a descriptor of zero records (zeros);
//  * ragged edges: A rows past M lie outside the tile's window (zeros), B
//    columns past N load from kOob, and neither is stored; in a partial last
//    k-tile the A chunks and B rows at or past K load from kOob (selects on
//    a wave-uniform condition, no second build);
//  * the C tile leaves through LDS in 16-row blocks of each wave tile, as
//    whole rows (f16: 8-byte writes with the chunk ^ row and half-swap
//    placement; f32: 16-byte writes with chunk ^ row), and C += A*B reads the
//    prior C as the same whole rows, a few blocks ahead.
#pragma once

#include "gemm_gfx950_impl.h"

namespace tbk {

constexpr int cgcd(int a, int b) { return b == 0 ? a : cgcd(b, a % b); }
constexpr int cmin(int a, int b) { return a < b ? a : b; }
constexpr int cmax(int a, int b) { return a > b ? a : b; }

template <int BM, int BN, int BK, int WGM, int WGN, int STAGES>
struct Mfma16GTile {
  static constexpr int NW = WGM * WGN, NT = NW * 64;
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;
  static constexpr int TI = WTM / 16, TJ = WTN / 16; // 16x16 tiles per wave tile
  static constexpr int KS = BK / 32;                  // 32-deep k steps per k-tile
  static constexpr int NM = TI * TJ;                  // MFMAs per k step
  static constexpr int NSLOT = KS * NM;               // MFMA slots per k-tile
  static constexpr int NR = TI + 2 * TJ;              // fragment read ops per k step
  // LDS stage: A [BM][BK] then B [BK][BN], f16, row-major
  static constexpr int RBA = BK * 2, RBB = BN * 2;       // row bytes
  static constexpr int CPRA = RBA / 16, CPRB = RBB / 16; // 16-byte chunks per row
  static constexpr int A_BYTES = BM * RBA, B_BYTES = BK * RBB;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int LDS_BYTES = STAGES * STAGE;
  // swizzles (the plan's #tb.shared encodings; 256-byte bank period)
  static constexpr int A_PP = 256 / RBA, A_MAXPH = CPRA;
  static constexpr int B_PP = RBB >= 256 ? 1 : 256 / RBB;
  static constexpr int B_MAXPH = cmin(CPRB / 4, 4);
  static constexpr int xa(int row) { return (row / A_PP) % A_MAXPH; }
  static constexpr int xb(int k) { return (4 * ((k / B_PP) % B_MAXPH)) ^ (2 * ((k / 8) % 2)); }
  // direct loads: a round moves NT x 16 bytes, RPR whole rows; the swizzle
  // phase repeats every 16 rows, so a lane's logical chunk repeats every P
  // rounds
  static constexpr int LA = A_BYTES / (NT * 16), LB = B_BYTES / (NT * 16);
  static constexpr int LPT = LA + LB;
  static constexpr int RPRA = NT * 16 / RBA, RPRB = NT * 16 / RBB;
  static constexpr int PA = 16 / cgcd(RPRA, 16), PB = 16 / cgcd(RPRB, 16);

  // ---- slot schedule ----------------------------------------------------
  // MFMA m of a k step: tile (m / TJ, m % TJ). Read op o of a k step: A0,
  // B0 (halves 0, 1), .., B(TJ-1), A1 .. A(TI-1): the order of first use.
  // the barrier sits before slot BQ of a k-tile's last k step; with 32-deep
  // k-tiles at the k-tile's start (BQ = 0), so that a loop body is exactly
  // one k-tile and the loop needs no tail whose fragment buffer depends on
  // the k-tile count's parity
  static constexpr int BQ = KS == 1 ? 0 : (NM >= 64 ? 8 : (NM >= 32 ? 4 : 2));
  static constexpr bool op_is_a(int o) { return o == 0 || o > 2 * TJ; }
  static constexpr int op_index(int o) {
    return o == 0 ? 0 : (o > 2 * TJ ? o - 2 * TJ : (o - 1) / 2);
  }
  static constexpr int op_half(int o) { return (o - 1) & 1; }
  // read op o of the next k step of the same k-tile (every k step but the
  // last), and of the next k-tile's first k step (the last k step, after
  // the barrier)
  static constexpr int last_use(int o) {
    return op_is_a(o) ? op_index(o) * TJ + TJ - 1 : (TI - 1) * TJ + op_index(o);
  }
  // reads spread evenly over slots [s0, NM), s0 the first start at or after
  // `lo` that keeps rule (c) for every op (a fragment's register is rewritten
  // at least 8 slots after its last MFMA read in the k step before)
  static constexpr int spread_slot(int s0, int o) { return s0 + o * (NM - s0) / NR; }
  static constexpr int first_start(int lo) {
    for (int s0 = lo; s0 < NM; ++s0) {
      bool ok = true;
      for (int o = 0; o < NR; ++o)
        ok = ok && NM - last_use(o) + spread_slot(s0, o) >= 8;
      if (ok)
        return s0;
    }
    return NM;
  }
  static constexpr int S0_MID = first_start(0), S0_LAST = first_start(BQ);
  static constexpr int slot_mid(int o) { return spread_slot(S0_MID, o); }
  static constexpr int slot_last(int o) { return spread_slot(S0_LAST, o); }
  // refill load l goes body slot load_slot(l) (a body runs NSLOT slots from
  // one barrier to the next); with 2 stages the refill is due at the next
  // barrier, so it goes out in the first 5/8 of the body
  static constexpr int SPREAD = STAGES == 2 ? NSLOT * 5 / 8 : NSLOT - NSLOT / 8;
  static constexpr int load_slot(int l) { return l * SPREAD / LPT; }
  // the k-th read op (or load) placed in slot m, -1 if none: per-slot
  // tables, so the unrolled slots instantiate only what they issue
  static constexpr int RPS = NR / NM + 2; // bound on read ops per slot
  static constexpr int LPS = LPT / SPREAD + 2; // bound on loads per body slot
  static constexpr int mid_op(int m, int k) {
    for (int o = 0, c = 0; o < NR; ++o)
      if (slot_mid(o) == m && c++ == k)
        return o;
    return -1;
  }
  static constexpr int last_op(int m, int k) {
    for (int o = 0, c = 0; o < NR; ++o)
      if (slot_last(o) == m && c++ == k)
        return o;
    return -1;
  }
  static constexpr int load_at(int s, int k) {
    for (int l = 0, c = 0; l < LPT; ++l)
      if (load_slot(l) == s && c++ == k)
        return l;
    return -1;
  }
  // s_waitcnt depths: the prologue issues STAGES k-tiles and waits for the
  // first; the barrier of k-tile it waits for k-tile it+1
  static constexpr int VM_PROLOGUE = (STAGES - 1) * LPT;
  static constexpr int VM_LOOP = (STAGES - 2) * LPT;
  // loop unrolling: stage (and, for 32-deep k-tiles, the fragment buffer)
  // fixed at compile time in every body
  static constexpr int U = KS == 2 ? STAGES : (STAGES % 2 ? 2 * STAGES : STAGES);

  // rule (c): slots between a fragment's last MFMA read and the read op that
  // rewrites its register
  static constexpr int min_rewrite_distance() {
    int d = 1 << 30;
    for (int o = 0; o < NR; ++o) {
      if (KS == 2)
        d = cmin(d, NM - last_use(o) + slot_mid(o));
      d = cmin(d, NM - last_use(o) + slot_last(o));
    }
    return d;
  }
  static constexpr bool reads_fit() {
    for (int o = 0; o < NR; ++o)
      if (slot_mid(o) >= NM || slot_last(o) < BQ || slot_last(o) >= NM)
        return false;
    return true;
  }

  // ---- epilogue staging (16-row blocks of the wave tile) ------------------
  static constexpr int E16_ROWB = WTN * 2, E16_CPR = E16_ROWB / 16;
  static constexpr int E16_RPW = cmax(1, 128 / E16_ROWB); // rows per 128-byte window
  static constexpr int E16_XM = cmin(8, E16_CPR);
  static constexpr int E16_RPI = 64 / E16_CPR;             // rows per 64-lane read
  static constexpr int E32_ROWB = WTN * 4, E32_CPR = E32_ROWB / 16;
  static constexpr int E32_RPW = cmax(1, 256 / E32_ROWB);  // rows per 256-byte period
  static constexpr int E32_XM = cmin(16, E32_CPR);
  static constexpr int E32_RPI = 64 / E32_CPR;
  static constexpr int EPI_REGION = 16 * E32_ROWB; // bytes per wave (f32 needs most)

  static_assert(BK == 32 || BK == 64, "k-tiles of one or two 32-deep k steps");
  static_assert(WTM % 16 == 0 && WTN % 16 == 0 && BM % WGM == 0 && BN % WGN == 0,
                "16x16 MFMA tiles");
  static_assert(NM >= 16 && NM <= 64, "16..64 MFMA tiles per wave (at most 256 AGPRs)");
  static_assert(BN >= 64 && WTN >= 32, "B rows of 128+ bytes, 32+ columns per wave");
  static_assert(LA >= 1 && LA * NT * 16 == A_BYTES, "whole A load rounds");
  static_assert(LB >= 1 && LB * NT * 16 == B_BYTES, "whole B load rounds");
  static_assert(RPRA >= 1 && RPRB >= 1, "a load round covers whole rows");
  static_assert(STAGES >= 2 && STAGES <= 4, "2..4 LDS stages");
  static_assert(LDS_BYTES <= 160 * 1024, "gfx950 LDS is 160 KiB per workgroup");
  static_assert(NW * EPI_REGION <= LDS_BYTES, "epilogue staging fits the ring");
  static_assert(VM_PROLOGUE < 64, "vmcnt range");
  static_assert(reads_fit(), "fragment reads fall inside their k step");
  static_assert(min_rewrite_distance() >= 8,
                "(c) a fragment register rewritten too soon after its last MFMA read");
  static_assert(SPREAD >= 1 && SPREAD <= NSLOT, "refill within one body");
  static constexpr bool tables_cover() {
    for (int m = 0; m < NM; ++m)
      if (mid_op(m, RPS - 1) >= 0 || last_op(m, RPS - 1) >= 0)
        return false;
    for (int s2 = 0; s2 < NSLOT; ++s2)
      if (load_at(s2, LPS - 1) >= 0)
        return false;
    return true;
  }
  static_assert(tables_cover(), "per-slot tables hold every read and load");
};

template <int BM, int BN, int BK, int WGM, int WGN, int STAGES, int OUT, bool EPI>
__device__ __forceinline__ void mfma16g_tile(const GemmParams &p, int m0, int n0, u32x4 *lds) {
  using T = Mfma16GTile<BM, BN, BK, WGM, WGN, STAGES>;
  constexpr int TI = T::TI, TJ = T::TJ, KS = T::KS, NM = T::NM, NR = T::NR, BQ = T::BQ;
  constexpr int LA = T::LA, LPT = T::LPT, U = T::U;
  static_assert(OUT == kOutF16 || OUT == kOutF32Partial || OUT == kOutF32Accum,
                "no atomic or split-K output on the 16x16x32 loop");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(TBK_LDS void *)lds;
  const int nk = (p.K + BK - 1) / BK;
  const int kfull = p.K / BK;
  const int krem = p.K - kfull * BK; // k values of the partial k-tile

  // ---- direct-load geometry ----------------------------------------------
  // Round R of thread t = 64 wave + lane fills 16 bytes at R * NT * 16 + 16 t
  // of the operand's stage area: row R * RPR + t / CPR, physical chunk t %
  // CPR, holding logical chunk (t % CPR) ^ swizzle(row).
  const int t = wave * 64 + lane;
  const int a_r0 = t / T::CPRA, a_pc = t % T::CPRA;
  const int b_r0 = t / T::CPRB, b_pc = t % T::CPRB;
  const void *a_tile = rows_at(p.A, m0, p.lda, 2); // A's window starts at row m0
  // A rows past M fall outside the window's records (it ends at row M) and
  // load zeros; B columns past N get the offset kOob
  const uint32_t a_bytes = rows_bytes(m0, p.M, p.lda, 2);
  const uint32_t b_bytes = (uint32_t)p.K * (uint32_t)p.ldb * 2u;
  // per swizzle phase (round mod PA / PB): the vector offset; for the A
  // rounds also the same offset with the partial k-tile's mask (chunks at
  // or past K load from kOob)
  uint32_t va[T::PA], vak[T::PA], vb[T::PB];
#pragma unroll
  for (int ph = 0; ph < T::PA; ++ph) {
    const int lc = a_pc ^ T::xa(a_r0 + ph * T::RPRA);
    va[ph] = ((uint32_t)a_r0 * (uint32_t)p.lda + (uint32_t)(lc * 8)) * 2u;
    vak[ph] = lc * 8 < krem ? va[ph] : kOob;
  }
#pragma unroll
  for (int ph = 0; ph < T::PB; ++ph) {
    const int col = n0 + 8 * (b_pc ^ T::xb(b_r0 + ph * T::RPRB));
    vb[ph] = col < p.N ? ((uint32_t)b_r0 * (uint32_t)p.ldb + (uint32_t)col) * 2u : kOob;
  }
  const uint32_t wlds = lds0 + wave * 1024u;
  // load l of k-tile kt into stage ST (A rounds first, then B rounds). In
  // the partial last k-tile (kt == kfull, K % BK != 0) A chunks and B rows at
  // or past K load zeros; the selects are on a wave-uniform condition.
  auto load = [&](const u32x4 &ra, const u32x4 &rb, int kt, auto st_c, auto l_c) {
    constexpr int ST = decltype(st_c)::value, L = decltype(l_c)::value;
    const bool kpart = kt == kfull;
    if constexpr (L < LA) {
      const uint32_t v = kpart ? vak[L % T::PA] : va[L % T::PA];
      load_lds16_at<ST * T::STAGE + L * T::NW * 1024>(
          ra, wlds, v, (uint32_t)kt * (BK * 2u) + (uint32_t)(L * T::RPRA) * (uint32_t)p.lda * 2u);
    } else {
      constexpr int R = L - LA;
      const int lim = kpart ? krem - R * T::RPRB : (1 << 30); // k rows of the round
      const uint32_t v = b_r0 >= lim ? kOob : vb[R % T::PB];
      load_lds16_at<ST * T::STAGE + T::A_BYTES + R * T::NW * 1024>(
          rb, wlds, v, ((uint32_t)kt * BK + (uint32_t)(R * T::RPRB)) * (uint32_t)p.ldb * 2u);
    }
  };
  // descriptors of k-tile kt: zero records past the last k-tile
  auto rsrc_a = [&](int kt) { return rsrc_dwords(a_tile, kt < nk ? a_bytes : 0u); };
  auto rsrc_b = [&](int kt) { return rsrc_dwords(p.B, kt < nk ? b_bytes : 0u); };

  // ---- fragment reads ----------------------------------------------------
  const int g = lane >> 4, ta = (lane >> 2) & 3, tb = lane & 3;
  uint32_t a_base[STAGES][KS], b_base[STAGES][TJ];
#pragma unroll
  for (int st = 0; st < STAGES; ++st) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int row = wm * T::WTM + (lane & 15);
      a_base[st][ks] = lds0 + st * T::STAGE + row * T::RBA +
                       (((4 * ks + g) ^ T::xa(row)) * 16);
    }
#pragma unroll
    for (int jj = 0; jj < TJ; ++jj) {
      const int k = 8 * g + ta; // + 32 ks + 4 half: the same swizzle phase
      const int c = (wn * T::WTN + 16 * jj) / 8 + (tb >> 1);
      b_base[st][jj] = lds0 + st * T::STAGE + T::A_BYTES + k * T::RBB +
                       ((c ^ T::xb(k)) * 16) + 8 * (tb & 1);
    }
  }
  f32x4 acc[TI][TJ];
  half8 fa[2][TI], fb[2][TJ];
  // read op o of k step ks of stage st into buffer buf
  auto rd = [&](auto buf_c, auto st_c, auto ks_c, auto o_c) {
    constexpr int BUF = decltype(buf_c)::value, ST = decltype(st_c)::value;
    constexpr int KSI = decltype(ks_c)::value, O = decltype(o_c)::value;
    if constexpr (T::op_is_a(O)) {
      constexpr int I = T::op_index(O);
      fa[BUF][I] = __builtin_bit_cast(
          half8, *(const TBK_LDS u32x4 *)(uintptr_t)(a_base[ST][KSI] + I * 16 * T::RBA));
    } else {
      constexpr int J = T::op_index(O), H = T::op_half(O);
      const half4 h = __builtin_bit_cast(
          half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((TBK_LDS short4 *)(uintptr_t)(
                     b_base[ST][J] + KSI * 32 * T::RBB + H * 4 * T::RBB)));
      if constexpr (H == 0)
        fb[BUF][J].lo = h;
      else
        fb[BUF][J].hi = h;
    }
  };
  // MFMA m of buffer buf (always inlined with constant arguments); `first`:
  // srcC = 0
  auto mfma = [&](int buf, int m, bool first) {
    const int i = m / TJ, j = m % TJ;
    if (first)
      asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0"
                   : "=a"(acc[i][j])
                   : "v"(fb[buf][j]), "v"(fa[buf][i]));
    else
      asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0"
                   : "+a"(acc[i][j])
                   : "v"(fb[buf][j]), "v"(fa[buf][i]));
  };
  auto barrier = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  using F = std::integral_constant<bool, false>;
  // buffer of k step ks of k-tile phase q (q = k-tile index mod U)
  auto buf_of = [](auto q_c, auto ks_c) {
    constexpr int Q = decltype(q_c)::value, KSI = decltype(ks_c)::value;
    return std::integral_constant<int, KS == 2 ? KSI : Q % 2>{};
  };

  // slots [LO, HI) of k step ks (k-tile phase q, stage st): the MFMAs, the
  // reads of the next k step of the same k-tile (all but the last k step),
  // and `extra(slot)`
  auto kstep = [&](auto q_c, auto ks_c, auto lo_c, auto hi_c, auto first_c, auto &&extra) {
    constexpr int Q = decltype(q_c)::value, KSI = decltype(ks_c)::value;
    constexpr int ST = Q % STAGES;
    using BUF = decltype(buf_of(q_c, ks_c));
    static_for<NM>([&](auto m_c) {
      constexpr int M = decltype(m_c)::value;
      if constexpr (M >= decltype(lo_c)::value && M < decltype(hi_c)::value) {
        mfma(BUF::value, M, decltype(first_c)::value);
        if constexpr (KSI + 1 < KS)
          static_for<T::RPS>([&](auto k_c) {
            constexpr int O = T::mid_op(M, decltype(k_c)::value);
            if constexpr (O >= 0)
              rd(std::integral_constant<int, 1>{}, std::integral_constant<int, ST>{},
                 std::integral_constant<int, KSI + 1>{}, std::integral_constant<int, O>{});
          });
        extra(m_c);
        __builtin_amdgcn_sched_barrier(0);
      }
    });
  };
  using Z = std::integral_constant<int, 0>;
  using LAST = std::integral_constant<int, KS - 1>;
  using QB = std::integral_constant<int, BQ>;
  using ENDS = std::integral_constant<int, NM>;
  auto nothing = [](auto) {};

  // body(it) with it = Q mod U: from the barrier of k-tile it to just before
  // the barrier of k-tile it+1. Stage Q % STAGES (k-tile it) is refilled with
  // k-tile it+STAGES. FIRST: the MFMAs before the first barrier of a 32-deep
  // k-tile's only k step are its first.
  auto body = [&](int it, auto q_c, auto first_c) {
    constexpr int Q = decltype(q_c)::value;
    constexpr int SC = Q % STAGES, SN = (Q + 1) % STAGES;
    using QN = std::integral_constant<int, (Q + 1) % U>;
    const u32x4 ra = rsrc_a(it + STAGES), rb = rsrc_b(it + STAGES);
    wait_vmcnt_lgkm0<T::VM_LOOP>();
    barrier();
    // body slot s: s = m - BQ in the last k step of k-tile it, then
    // NM - BQ + ks NM + m in k-tile it+1
    auto refill_at = [&](auto s_c) {
      static_for<T::LPS>([&](auto k_c) {
        constexpr int L = T::load_at(decltype(s_c)::value, decltype(k_c)::value);
        if constexpr (L >= 0)
          load(ra, rb, it + STAGES, std::integral_constant<int, SC>{},
               std::integral_constant<int, L>{});
      });
    };
    using BN0 = decltype(buf_of(QN{}, Z{}));
    kstep(q_c, LAST{}, QB{}, ENDS{}, first_c, [&](auto m_c) {
      constexpr int M = decltype(m_c)::value;
      static_for<T::RPS>([&](auto k_c) {
        constexpr int O = T::last_op(M, decltype(k_c)::value);
        if constexpr (O >= 0)
          rd(BN0{}, std::integral_constant<int, SN>{}, Z{}, std::integral_constant<int, O>{});
      });
      refill_at(std::integral_constant<int, M - BQ>{});
    });
    static_for<KS>([&](auto ks_c) {
      constexpr int KSI = decltype(ks_c)::value;
      using HI = std::integral_constant<int, KSI + 1 < KS ? NM : BQ>;
      kstep(QN{}, ks_c, Z{}, HI{}, F{}, [&](auto m_c) {
        refill_at(std::integral_constant<int, NM - BQ + KSI * NM + decltype(m_c)::value>{});
      });
    });
  };

  // ---- prologue: k-tiles 0 .. STAGES-1 in flight, wait for k-tile 0 -------
  static_for<STAGES>([&](auto st_c) {
    constexpr int ST = decltype(st_c)::value;
    const u32x4 ra = rsrc_a(ST), rb = rsrc_b(ST);
    static_for<LPT>([&](auto l_c) { load(ra, rb, ST, st_c, l_c); });
  });
  wait_vmcnt<T::VM_PROLOGUE>();
  barrier();
  if constexpr (KS == 1) {
    // 32-deep k-tiles: k-tile 0 runs in the loop's first body, whose code
    // serves every k-tile; the accumulators start from a zero product
    // instead (srcC = 0, rule (a))
    const half8 zf = {};
    auto zero = [&](int m) {
      asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %1, 0"
                   : "=a"(acc[m / TJ][m % TJ])
                   : "v"(zf));
    };
#pragma unroll
    for (int m = 0; m < NM; ++m)
      zero(m);
  }
  static_for<NR>([&](auto o_c) { rd(Z{}, Z{}, Z{}, o_c); });
  // k-tile 0 up to its barrier (with 64-deep k-tiles its first k step's
  // MFMAs are the first)
  static_for<KS>([&](auto ks_c) {
    constexpr int KSI = decltype(ks_c)::value;
    using HI = std::integral_constant<int, KSI + 1 < KS ? NM : BQ>;
    kstep(Z{}, ks_c, Z{}, HI{}, std::integral_constant<bool, KSI == 0 && KS == 2>{}, nothing);
  });
  // The loop: U bodies per trip, body q of a trip at phase q (k-tile it = 0
  // mod U at the trip's start). With 64-deep k-tiles it leaves after the
  // body of k-tile nk - 2, whichever body of the trip that is, and the tail
  // runs the last k-tile after its barrier point (buffer 1 whatever the
  // phase; no refill, no barrier). With 32-deep k-tiles a body is a whole
  // k-tile and the loop leaves after the body of k-tile nk - 1, whose reads
  // of k-tile nk land zeros and are not used: no tail, so no code path
  // after the loop depends on the parity of nk (at such a merge the
  // compiler would copy accumulators the last MFMAs are still writing: the
  // asm hides their latency).
  const int last_body = KS == 2 ? nk - 1 : nk;
  int it = 0;
  if (it < last_body) {
    for (;;) {
      bool done = false;
      static_for<U>([&](auto q_c) {
        if (!done) {
          body(it, q_c, F{});
          ++it;
          done = it >= last_body;
        }
      });
      if (done)
        break;
    }
  }
  if constexpr (KS == 2)
    kstep(Z{}, LAST{}, QB{}, ENDS{}, F{}, nothing);
  // (b) 24 wait states between the last MFMA and the first accumulator read
  acc_read_fence(acc);
  wait_vmcnt<0>(); // the zero loads past the end have landed too

  // ---- epilogue: 16-row blocks of the wave tile through this wave's LDS ----
  const int el = lane_id_fresh();
  const GemmParams pe = params_fresh();
  const EpiArgs ea{pe.bias, pe.epi_bias, pe.epi_act, pe.epi_clamp, pe.clamp_lo, pe.clamp_hi};
  const float lo = (pe.epi_clamp & 1) ? pe.clamp_lo : -__builtin_inff();
  const float hi = (pe.epi_clamp & 2) ? pe.clamp_hi : __builtin_inff();
  TBK_LDS char *wl = (TBK_LDS char *)(TBK_LDS void *)lds + wave * T::EPI_REGION;
  if constexpr (OUT == kOutF16) {
    // lane l holds row r = l % 16 of block i, columns 16 j + 4 (l / 16) .. +3:
    // 8 bytes at chunk c = 2 j + (l / 16) / 2, half (l / 16) % 2 of the row;
    // placed at chunk c ^ ((r / E16_RPW) % E16_XM), halves swapped when r / 8
    // is odd: the 16 rows a quarter wave writes land in 16 different 8-byte
    // slots of a 128-byte window, and whole-row reads cover the banks once
    epi_f32x4 bv[EPI ? TJ : 1];
    if constexpr (EPI) {
      const int ccol = n0 + wn * T::WTN + 4 * (el >> 4);
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        bv[j] = epi_load_bias(ea, ccol + 16 * j, pe.N);
    }
    barrier(); // every wave is past its last fragment read and load
    const __amdgpu_buffer_rsrc_t rc =
        make_rsrc(rows_at(pe.C, m0, pe.ldc, 2), rows_bytes(m0, pe.M, pe.ldc, 2));
    const int r = el & 15, gg = el >> 4;
    const int xr = (r / T::E16_RPW) % T::E16_XM, hs = (r >> 3) & 1;
    const int q = el % T::E16_CPR, rr0 = el / T::E16_CPR;
    const int col = n0 + wn * T::WTN + 8 * q;
    auto block = [&](auto i_c, auto act_c, auto clamp_c) {
      constexpr int i = decltype(i_c)::value;
      constexpr int ACT = decltype(act_c)::value;
      constexpr bool CLAMP = decltype(clamp_c)::value;
      epi_variant_fence<ACT, CLAMP>();
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[e] = acc[i][j][e];
          if constexpr (EPI)
            x[e] = epi_apply_t<ACT, CLAMP>(x[e], bv[j][e], lo, hi);
        }
        u32x2 v;
        v[0] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x[0]) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x[1]) << 16);
        v[1] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x[2]) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x[3]) << 16);
        const int chunk = (2 * j + (gg >> 1)) ^ xr;
        const int half = (gg & 1) ^ hs;
        *(TBK_LDS u32x2 *)(wl + r * T::E16_ROWB + chunk * 16 + half * 8) = v;
        if (j & 1)
          __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int s = 0; s < 16 / T::E16_RPI; ++s) {
        const int rr = s * T::E16_RPI + rr0; // row of the block
        u32x4 v = *(const TBK_LDS u32x4 *)(wl + rr * T::E16_ROWB +
                                           ((q ^ ((rr / T::E16_RPW) % T::E16_XM)) * 16));
        if ((rr >> 3) & 1)
          v = (u32x4){v[2], v[3], v[0], v[1]};
        const int trow = wm * T::WTM + 16 * i + rr; // row of the tile
        const uint32_t off =
            m0 + trow < pe.M && col < pe.N
                ? ((uint32_t)trow * (uint32_t)pe.ldc + (uint32_t)col) * 2u
                : kOob;
        __builtin_amdgcn_raw_buffer_store_b128(v, rc, off, 0, kStoreNT);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    epi_for_blocks<TI, EPI>(pe, block);
  } else {
    // f32: lane l holds row r = l % 16 of block i, columns 16 j + 4 (l / 16)
    // .. +3, 16 bytes at chunk 4 j + l / 16, placed at chunk ^ ((r /
    // E32_RPW) % E32_XM): a quarter wave's 16 rows land in 16 different
    // 16-byte slots of the 256-byte bank period. C += A*B loads the prior C
    // as the same whole rows, PF blocks ahead, and adds it before the fused
    // steps (epilogue(C + acc)).
    constexpr int NLD = 16 / T::E32_RPI; // row pieces per lane per block
    constexpr int PF = OUT == kOutF32Accum ? cmin(TI, EPI ? 2 : 4) : 1;
    const int q = el % T::E32_CPR, rr0 = el / T::E32_CPR;
    const int col = n0 + wn * T::WTN + 4 * q;
    const __amdgpu_buffer_rsrc_t rc =
        make_rsrc(rows_at(pe.C, m0, pe.ldc, 4), rows_bytes(m0, pe.M, pe.ldc, 4));
    auto c_off = [&](int i, int s) -> uint32_t {
      const int trow = wm * T::WTM + 16 * i + s * T::E32_RPI + rr0;
      return m0 + trow < pe.M && col < pe.N
                 ? ((uint32_t)trow * (uint32_t)pe.ldc + (uint32_t)col) * 4u
                 : kOob;
    };
    f32x4 old[OUT == kOutF32Accum ? PF : 1][NLD];
    auto load_old = [&](int i) {
      if constexpr (OUT == kOutF32Accum) {
#pragma unroll
        for (int s = 0; s < NLD; ++s)
          old[i % PF][s] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, c_off(i, s), 0, 0));
      }
    };
#pragma unroll
    for (int i = 0; i < PF; ++i)
      load_old(i);
    const epi_f32x4 bias = EPI ? epi_load_bias(ea, col, pe.N) : epi_f32x4{};
    barrier(); // every wave is past its last fragment read and load
    const int r = el & 15, gg = el >> 4;
    const int xr = (r / T::E32_RPW) % T::E32_XM;
    auto block = [&](auto i_c, auto act_c, auto clamp_c) {
      constexpr int i = decltype(i_c)::value;
      constexpr int ACT = decltype(act_c)::value;
      constexpr bool CLAMP = decltype(clamp_c)::value;
      epi_variant_fence<ACT, CLAMP>();
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        *(TBK_LDS f32x4 *)(wl + r * T::E32_ROWB + (((4 * j + gg) ^ xr) * 16)) = acc[i][j];
        if (j & 1)
          __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int s = 0; s < NLD; ++s) {
        const int rr = s * T::E32_RPI + rr0;
        f32x4 v = *(const TBK_LDS f32x4 *)(wl + rr * T::E32_ROWB +
                                           ((q ^ ((rr / T::E32_RPW) % T::E32_XM)) * 16));
        if constexpr (OUT == kOutF32Accum)
          v += old[i % PF][s];
        if constexpr (EPI) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] = epi_apply_t<ACT, CLAMP>(v[e], bias[e], lo, hi);
        }
        // a plain f32 C is written once (non-temporal); C += A*B keeps the
        // default policy
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rc, c_off(i, s),
                                               0, OUT == kOutF32Partial ? kStoreNT : 0);
      }
      if (i + PF < TI)
        load_old(i + PF);
      __builtin_amdgcn_sched_barrier(0);
    };
    epi_for_blocks<TI, EPI>(pe, block);
  }
}

// The programs of a 16x16x32 instance (tile, grouped or persistent order).
template <int BM, int BN, int BK, int WGM, int WGN, int STAGES, int OUT, bool EPI>
__global__ __launch_bounds__(WGM *WGN * 64, 1) void gemm_mfma16g(GemmParams p) {
  using T = Mfma16GTile<BM, BN, BK, WGM, WGN, STAGES>;
  __shared__ u32x4 lds[T::LDS_BYTES / 16];
  const bool persistent =
      p.mapping == kMapPersistent || p.mapping == kMapPersistentGrouped;
  int prog = blockIdx.x;
  const int nprog = gridDim.x;
  if (p.xcds > 1 && (nprog % p.xcds) == 0)
    prog = (prog % p.xcds) * (nprog / p.xcds) + prog / p.xcds;
  for (int work = prog; work < p.total_work;
       work += (persistent ? nprog : p.total_work)) {
    int tile_m, tile_n, part;
    map_program(p, work, tile_m, tile_n, part);
    if (work != prog)
      __syncthreads(); // every wave read its staged epilogue back
    mfma16g_tile<BM, BN, BK, WGM, WGN, STAGES, OUT, EPI>(p, tile_m * BM, tile_n * BN, lds);
  }
}

} // namespace tbk
