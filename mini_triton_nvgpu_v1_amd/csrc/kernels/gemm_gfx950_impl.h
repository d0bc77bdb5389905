// Template body of the gfx950 MFMA GEMM kernel. Included by the instance
// translation units (gemm_inst_*.hip); see gemm_gfx950.h for the design.
#pragma once

#include "gemm_gfx950.h"
#include "mfma16_schedule.h"

#include <type_traits>
#include <utility>

namespace tbk {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef short short4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define TBK_LDS __attribute__((address_space(3)))

// Buffer descriptor dword3 for gfx9-family raw buffers (stride 0, untyped,
// bounds checked against num_records).
static constexpr int kBufferFlags = 0x00020000;
// Any offset at or above num_records reads zero / drops the store. A, C and
// the split-K partials are addressed through windows that start at the
// tile's first row (rows_at), so only a tile's rows must span fewer than
// 2^31 bytes; B is addressed whole (the host checks both).
static constexpr uint32_t kOob = 0x80000000u;
// Cache-policy operand of a buffer store that sets nt (non-temporal) on gfx950.
static constexpr int kStoreNT = 2;

// sched_group_barrier instruction classes (LLVM AMDGPU)
static constexpr int kSchedMfma = 0x008;
static constexpr int kSchedVmemRead = 0x020;
static constexpr int kSchedDsRead = 0x100;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p,
                                                            uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0,
                                           (int)bytes, kBufferFlags);
}

// 16 bytes per lane from global memory straight into LDS at
// lds_base + 16 * lane (lds_base is wave-uniform), i.e.
// buffer_load_dwordx4 ... offen lds with M0 = lds_base.
// Issued as inline asm on purpose: the compiler then does not treat it as an
// LDS write, so it does not put vmcnt(0) in front of every later LDS read
// (it cannot tell that those reads hit a different stage). Ordering is the
// kernel's job: wait_vmcnt<N>() + barrier before a stage is read.
__device__ __forceinline__ void load_lds16(u32x4 rsrc, uint32_t lds_base,
                                           uint32_t voff, int soff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_base);
  const int so = __builtin_amdgcn_readfirstlane(soff);
  asm volatile("s_mov_b32 m0, %0\n\t"
               "buffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(rsrc), "s"(so)
               : "memory");
}

// The same with M0 = lds_base + OFF, OFF a constant: the sum is formed in
// M0 itself, so a kernel with many load rounds and stages keeps one LDS base
// in an SGPR instead of one per (stage, round).
template <uint32_t OFF>
__device__ __forceinline__ void load_lds16_at(u32x4 rsrc, uint32_t lds_base, uint32_t voff,
                                              uint32_t soff) {
  asm volatile("s_add_u32 m0, %0, %4\n\t"
               "buffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff), "i"(OFF)
               : "memory", "scc");
}

// The lane index computed afresh (mbcnt) behind an empty asm, for code
// after a main loop: the compiler can neither reuse a lane-derived value
// that the loop would have to keep live nor hoist the epilogue's addresses
// (derived from it) into the loop, where they would hold registers the loop
// needs.
__device__ __forceinline__ int lane_id_fresh() {
  int l = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  asm volatile("" : "+v"(l));
  return l;
}

// The kernel's GemmParams argument read again from the kernel-argument
// segment (its only argument, at offset 0) through an opaque pointer, for
// code after a main loop: the fields it uses are then loaded there (scalar
// loads) instead of being held in scalar registers across the loop (the
// fused epilogue's arguments would otherwise push the loop's scalar
// registers into spills).
typedef const __attribute__((address_space(4))) GemmParams *kernarg_params_ptr;
__device__ __forceinline__ GemmParams params_fresh() {
  kernarg_params_ptr q = (kernarg_params_ptr)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(q));
  GemmParams r;
  r.A = q->A, r.B = q->B, r.C = q->C, r.ws = q->ws;
  r.M = q->M, r.N = q->N, r.K = q->K, r.lda = q->lda, r.ldb = q->ldb, r.ldc = q->ldc;
  r.tiles_m = q->tiles_m, r.tiles_n = q->tiles_n, r.tiles_k = q->tiles_k;
  r.group_m = q->group_m, r.split_k = q->split_k, r.mapping = q->mapping;
  r.total_work = q->total_work, r.xcds = q->xcds, r.ws_ld = q->ws_ld;
  r.bias = q->bias, r.epi_bias = q->epi_bias, r.epi_act = q->epi_act;
  r.epi_clamp = q->epi_clamp, r.clamp_lo = q->clamp_lo, r.clamp_hi = q->clamp_hi;
  return r;
}

// First statement of each variant of a dispatched epilogue: an empty asm
// that differs per (activation, clamp), so the variants no longer begin with
// the same code, and a scheduling barrier that keeps the variant's own code
// below it. Otherwise the compiler hoists their common start (the
// accumulator reads of every element) above the dispatch, holding the whole
// tile in VGPRs at once (the fused 16x16x32 build spilled).
template <int ACT, bool CLAMP>
__device__ __forceinline__ void epi_variant_fence() {
  asm volatile("; fused epilogue variant %0 %1" ::"i"(ACT), "i"(CLAMP ? 1 : 0));
  __builtin_amdgcn_sched_barrier(0); // nothing scheduled above it
}



// f(std::integral_constant<int, i>{}) for i = 0 .. N-1, in order.
template <class F, int... I>
__device__ __forceinline__ void static_for_seq(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// The wait between the last inline-asm MFMA and the first read of the
// accumulators. The compiler does not see the latency of an asm MFMA: it
// places a read of a finished tile (the epilogue's, or a copy at a merge)
// anywhere after that tile's last asm, even two instructions after it,
// ahead of the MFMAs still running on the other tiles. Here 24 wait states
// (three s_nop 7) are followed by an empty asm per tile that takes the tile
// as an in-out AGPR operand: every later use reads that asm's result, so no
// read can move above the waits.
template <int TI, int TJ>
__device__ __forceinline__ void acc_read_fence(f32x4 (&acc)[TI][TJ]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
      asm volatile("" : "+a"(acc[i][j]));
}

// Runs block(i, act, clamp) for the epilogue's 16-row blocks i = 0 .. NB-1,
// with EPI the activation and clamp of the launch dispatched once per block
// (a block's code is specialised to them); without, the plain block.
// Dispatched per block rather than once for the whole tile, a variant reads
// only one block's accumulators, whatever the compiler hoists above it.
template <int NB, bool EPI, class F>
__device__ __forceinline__ void epi_for_blocks(const GemmParams &pe, F &&block) {
  static_for<NB>([&](auto i_c) {
    if constexpr (EPI)
      epi_dispatch(pe.epi_act, pe.epi_clamp, [&](auto a, auto c) { block(i_c, a, c); });
    else
      block(i_c, std::integral_constant<int, 0>{}, std::integral_constant<bool, false>{});
  });
}

// Raw buffer descriptor as four dwords for inline asm operands ("s"): the
// address and size are wave-uniform, and readfirstlane says so to the
// compiler, which otherwise keeps a base computed from the tile index in
// vector registers.
__device__ __forceinline__ u32x4 rsrc_dwords(const void *p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  return (u32x4){(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a),
                 (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu),
                 (uint32_t)__builtin_amdgcn_readfirstlane(bytes), (uint32_t)kBufferFlags};
}

// Row row0 of a row-major matrix of `ld` elements of `esize` bytes per row:
// the base of a tile's buffer window (a 64-bit address), so the 32-bit
// offsets a tile forms inside it stay small however large the matrix is.
__device__ __forceinline__ const void *rows_at(const void *p, int row0, int ld, int esize) {
  return static_cast<const char *>(p) + (size_t)row0 * (size_t)ld * (size_t)esize;
}
// num_records of that window: the rows from row0 to the matrix end, capped
// below kOob (the masks keep a tile inside its own rows).
__device__ __forceinline__ uint32_t rows_bytes(int row0, int rows, int ld, int esize) {
  const uint64_t b = (uint64_t)(rows - row0) * (uint64_t)ld * (uint64_t)esize;
  return b < (uint64_t)kOob ? (uint32_t)b : kOob - 16u;
}

// s_waitcnt vmcnt(N) (expcnt / lgkmcnt untouched), gfx9 encoding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// s_waitcnt vmcnt(N) lgkmcnt(0): also every LDS read of this wave is done.
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
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

constexpr int cgcd_(int a, int b) { return b == 0 ? a : cgcd_(b, a % b); }
// XOR phases over `units` swizzle units per row: the largest power of two
// dividing `units` (so a unit XOR-ed with the phase stays inside its row),
// at most `cap`
constexpr int swizzle_phases(int units, int cap) {
  return (units & -units) < cap ? (units & -units) : cap;
}

template <int BM, int BN, int BK, int WGM, int WGN, int STAGES, int SPREAD_REQ = -1>
struct GemmTile {
  static constexpr int NW = WGM * WGN; // waves
  static constexpr int NT = NW * 64;
  static constexpr int WTM = BM / WGM;
  static constexpr int WTN = BN / WGN;
  static constexpr int TM = WTM / 32;
  static constexpr int TN = WTN / 32;
  static constexpr int NMFMA = TM * TN; // MFMAs per 16-deep k step per wave
  static constexpr int KSTEPS = BK / 16;
  static constexpr int KCH = BK / 8;  // 16-byte chunks per A row
  static constexpr int BNC = BN / 8;  // 16-byte chunks per B row
  // LDS swizzles, both of the form chunk' = chunk ^ ((row / PP) % MAXPH)
  // with the bank period of gfx950 LDS (64 banks x 4 B = 256 B per cycle:
  // 16 lanes of ds_read_b128 or 32 lanes of ds_read_b64_tr_b16 at a time).
  // A: 16-byte chunks, PP = rows per 256 B, MAXPH = chunks per row.
  static constexpr int A_PP = 256 / (BK * 2) >= 1 ? 256 / (BK * 2) : 1;
  // B: 64-byte segments (the 32 columns two 16-lane tr groups read per row),
  // PP = rows per 256 B, MAXPH = min(4, segments per row); in 16-byte chunks
  // the XOR value is 4 * phase.
  // PP: rows before a row's bank offset repeats, 256 / gcd(row bytes, 256)
  // (2 for 384-byte rows, whose consecutive rows sit 128 bytes apart in the
  // banks); MAXPH: at most 4, and a power of two dividing the segments per
  // row, so the XOR keeps a chunk inside its row (2 for 6 segments)
  static constexpr int B_PP = 256 / cgcd_(BN * 2, 256);
  static constexpr int B_MAXPH = swizzle_phases(BNC / 4, 4);
  static constexpr int A_STAGE = BM * KCH;  // 16-byte chunks
  static constexpr int B_STAGE = BK * BNC;
  static constexpr int STAGE = A_STAGE + B_STAGE;
  // direct loads per thread per k-tile: whole load rounds of NT chunks; an
  // operand stage of fewer chunks than the rounds cover (8 waves on a
  // 32-deep k-tile of a 64- or 128-wide block) leaves whole waves idle in its
  // last round: those waves issue their load anyway, from kOob (zeros) into a
  // 1 KiB scratch row past the ring that nothing reads, so every wave issues
  // the same loads and one vmcnt depth serves them all
  static constexpr int LA = (A_STAGE + NT - 1) / NT;
  static constexpr int LB = (B_STAGE + NT - 1) / NT;
  static constexpr int LPT = LA + LB;
  static constexpr bool IDLE_ROUNDS = LA * NT != A_STAGE || LB * NT != B_STAGE;
  static constexpr int SCRATCH_CHUNKS = IDLE_ROUNDS ? 64 : 0; // 1 KiB
  static constexpr int LDS_BYTES = (STAGES * STAGE + SCRATCH_CHUNKS) * 16;
  static constexpr int A_ROWS_PER_LOAD = NT / KCH; // rows one load round covers
  static constexpr int B_ROWS_PER_LOAD = NT / BNC;
  // B rows of 24 chunks (192 columns): a load round ends inside a row, so a
  // lane's row and chunk differ per round and each round has its own offset
  static constexpr bool B_RAGGED_ROUNDS = NT % BNC != 0;

  // ---- slot schedule (tiles with >= 4 MFMAs per k step) ------------------
  // A k-tile is NSLOT MFMA slots (KSTEPS x NMFMA). The one barrier per
  // k-tile sits before slot BQ, AFTER slots before the end. The refill of
  // the LDS stage the barrier frees is spread over SPREAD slots from the
  // barrier on: load l of that tile goes load_off(l) slots after the
  // barrier, i.e. in the same k-tile while load_off(l) < AFTER, else in the
  // next k-tile before its barrier. Spreading matters: the L2 -> CU path
  // moves ~56 B/clk per CU and the kernel needs ~32 B/clk on average, so a
  // burst of loads stalls the wave's issue (and its MFMAs) behind the queue.
  static constexpr bool SLOTTED = NMFMA >= 4;
  static constexpr int NSLOT = KSTEPS * NMFMA;
  static constexpr int AFTER = NMFMA / 2;
  static constexpr int BQ = NSLOT - AFTER;
  // default spread: with 3+ stages the freed stage has a whole k-tile before
  // its data is due; with 2 it is due at the next barrier, so the loads go
  // out within one k step to leave the rest of the k-tile as latency slack
  static constexpr int SPREAD =
      SPREAD_REQ > 0 ? SPREAD_REQ : (STAGES >= 3 ? NSLOT : NMFMA);
  static constexpr int load_off(int l) { return SPREAD * l / LPT; }
  static constexpr int count_after() {
    int n = 0;
    for (int l = 0; l < LPT; ++l)
      n += load_off(l) < AFTER ? 1 : 0;
    return n;
  }
  // loads of a refill issued in the k-tile of its barrier
  static constexpr int NA = SLOTTED ? count_after() : LPT;

  // vmcnt allowed at the prologue wait / the per-tile barrier = loads issued
  // after the tile being waited for (vmcnt retires in issue order). The loop
  // waits for tile it+1 while tiles it+2 .. it+STAGES-1 may be in flight
  // (the refill of tile it+STAGES-1 started after the previous barrier and
  // finished before this one). The prologue issues tiles 0 .. STAGES-2 and
  // the first NA loads of tile STAGES-1, then waits for tile 0.
  static constexpr int VM_PROLOGUE = (STAGES - 2) * LPT + NA;
  static constexpr int VM_LOOP = (STAGES - 2) * LPT;
  // f16 C staged through LDS (128- or 256-byte wave-tile rows) when the ring
  // holds every wave's tile; not for 128x128 wave tiles, whose 256
  // accumulator registers leave no room for the staging values
  static constexpr int EPI_ROWB = WTN * 2;         // bytes per staged row
  static constexpr int EPI_CPR = EPI_ROWB / 16;    // 16-byte chunks per row
  static constexpr int EPI_RPP = 256 / EPI_ROWB;   // rows per 256-byte bank period
  static constexpr int EPI_RPI = 64 / EPI_CPR;     // rows per 64-lane read
  // row bit that swaps a staged chunk's 8-byte halves (the one the chunk XOR
  // leaves out of a 16-row quarter wave's 128-byte write window)
  static constexpr int EPI_HALF_BIT = EPI_RPP == 1 ? 3 : 0;
  static constexpr bool STAGED_F16_EPILOGUE =
      SLOTTED && (WTN == 64 || WTN == 128) && WTM * WTN <= 8192 &&
      NW * WTM * EPI_ROWB <= LDS_BYTES;
  // f32 C (C += A*B, plain f32 stores, split-K partials) staged through LDS
  // one 32-row block of the wave tile at a time (F32_ROWB bytes per row):
  // the accumulators go in as 16-byte pieces, come back as whole row
  // segments, and the prior C is read and the result written in full rows.
  // Chunk c of row r sits at c ^ ((r / F32_RPP) % F32_XOR), so the 16 lanes
  // an LDS cycle serves touch 16 different 16-byte bank groups both ways.
  static constexpr int F32_ROWB = WTN * 4;
  static constexpr int F32_CPR = WTN / 4;                  // 16-byte chunks per row
  static constexpr int F32_RPP = F32_ROWB >= 256 ? 1 : 256 / F32_ROWB;
  static constexpr int F32_XOR = F32_CPR < 16 ? F32_CPR : 16;
  static constexpr int F32_RPI = 64 / F32_CPR;             // rows per 64-lane read
  // A 32-row block of every wave that does not fit the ring (4 waves of 32 x
  // 64 on a 24 KiB ring) goes through in two 16-row halves: in each, the
  // lanes holding that half's rows write, and every lane reads back.
  static constexpr bool F32_HALF_BLOCKS =
      NW * 32 * F32_ROWB > LDS_BYTES && NW * 16 * F32_ROWB <= LDS_BYTES;
  static constexpr int F32_BLOCK_ROWS = F32_HALF_BLOCKS ? 16 : 32; // rows per LDS pass
  static constexpr bool STAGED_F32_EPILOGUE =
      (WTN == 32 || WTN == 64 || WTN == 128) && NW * F32_BLOCK_ROWS * F32_ROWB <= LDS_BYTES;

  static_assert(BM % (WGM * 32) == 0 && BN % (WGN * 32) == 0, "wave tile");
  static_assert(KSTEPS == 2 || KSTEPS == 4, "BK must be 32 or 64");
  static_assert(BNC >= 8 && (64 % BNC == 0 || BNC == 24), "B rows of 64..512 halves or 192");
  static_assert(B_RAGGED_ROUNDS || LB == 1 ||
                    (B_ROWS_PER_LOAD % B_PP == 0 && (B_ROWS_PER_LOAD / B_PP) % B_MAXPH == 0),
                "a lane's B swizzle phase is the same in every load round");
  static_assert(A_STAGE % 64 == 0 && B_STAGE % 64 == 0,
                "an operand stage is whole waves' load rounds (idle lanes are whole waves)");
  static_assert(STAGES >= 2 && STAGES <= 4, "2..4 LDS stages");
  static_assert(LDS_BYTES <= 160 * 1024, "gfx950 LDS is 160 KiB per workgroup");
  static_assert(VM_LOOP < 64 && VM_PROLOGUE < 64, "vmcnt range");
  static_assert(!SLOTTED || (SPREAD >= 1 && SPREAD <= NSLOT),
                "a refill must be issued before the next barrier");
};

template <int NMFMA, int NREAD, int NVMEM>
__device__ __forceinline__ void sched_step() {
#pragma unroll
  for (int i = 0; i < NMFMA; ++i) {
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
    if (i < NREAD)
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    if (i < NVMEM)
      __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
  }
}

// ---- 4 waves of 128x128 on a 256x256x64 tile with v_mfma_f32_16x16x32_f16 ------
// The instance the plan selects for the 4-wave 256x256x64 2-stage f16
// configuration (mma = mfma_f32_16x16x32_f16): one wave per SIMD, any M, N
// and K (ragged edges masked at the loads and the C store), tile / grouped /
// persistent order.
// It fills the same LDS ring with the same swizzles as the general loop.
//
// Why 16x16x32: per FLOP it reads and writes a quarter of the accumulator
// registers of 32x32x16 (4 f32 per 16x16x32 against 16 per 32x32x16 at half
// the work), and this part is power-limited: same data movement, same MFMA
// busy cycles, but a ~7% higher sustained clock and ~6% fewer cycles.
//
// The instruction stream is built for a lone wave per SIMD, which has no
// sibling to run its MFMAs while it computes addresses or waits:
//  * every address is fixed before the loop: one vector offset per operand,
//    scalar offsets per load round, per-stage LDS bases; the k step, row
//    group and B half ride in the ds_read immediate offset, and M0 is formed
//    with an immediate add inside the load asm (no SGPR per stage and round);
//  * no per-load address arithmetic for bounds: a lane's A row validity is a
//    compare against a constant per round, its B column validity is fixed,
//    and the ring's lookahead loads past the last k-tile use a descriptor of
//    zero records (zeros);
//  * one loop iteration runs from a k-tile's barrier to the next, so the
//    compiler's waits for fragment reads never land in front of the first
//    MFMAs of a k-tile; the barrier is vmcnt(0) lgkmcnt(0) + s_barrier (this
//    wave's loads have landed and its reads of the stage the barrier frees
//    have returned; that stage is only written by loads issued after it).
// The MFMA is inline asm with the accumulator tied in place ("+a"): the
// builtin's register allocation rotates 16x16 accumulators through copies
// (dst != srcC), 248 extra moves per two k-tiles. Asm carries no hazard
// information, so (a) each accumulator's first MFMA takes srcC = 0 (no
// zeroing write right before it), (b) 24 wait states separate the last MFMA
// from the first accumulator read, and (c) every fragment register is
// rewritten at least 8 MFMA slots after its last MFMA read. The slot
// schedule and these rules are constexpr in Mfma16Schedule (mfma16_schedule.h)
// and static_assert-ed there, so a schedule edit that breaks one does not
// compile. LDS results are waited for by the compiler's lgkmcnt tracking of
// the asm operands.
//
// Per 16x16x32 tile ii, jj (0..7) of the wave's 128x128: lane l holds
// A[16ii + l%16][k0 + 8(l/16) .. +7] (one ds_read_b128) and
// B[k0 + 8(l/16) .. +7][16jj + l%16] (two ds_read_b64_tr_b16); the product is
// formed as C^T += B^T A^T, so lane l ends with C[16ii + l%16][16jj + 4(l/16)
// + r], r = 0..3. Slot schedule per 32-deep k step (64 MFMAs, m = 8ii + jj):
// the reads of the next k step in the order A0, B0 (two halves) .. B7, A1 ..
// A7, op o in slot 8o/3; the barrier before slot 8 of the last k step; after
// it the next k-tile's first reads (op o in slot 8 + 7o/3) and its refill, one
// load every 5 slots (loads 0..11 in slots 8..63, 12..15 in slots 4..19 of
// the next k-tile): a CU then asks the L2 for 64 KiB over ~1200 cycles, about
// what the L2 -> CU path sustains. Bunched into 40 slots, the queued loads
// held up the lone wave's issue (1% slower); every 4 or 3 slots measured
// 0.7% and 1.3% slower than every 5. With the barrier at slot 40 and the
// next k-tile's reads one per slot after it, the k-tile ran 27 cycles (1.2%)
// longer: a lone wave pays for LDS instructions issued back to back; the
// reads spread over the 56 slots after a barrier at slot 8 ran 0.3% faster
// than over the 48 after one at slot 16.
// s_waitcnt depths of the 16x16x32 instance: the prologue issues k-tiles 0
// and 1 whole (16 loads each per lane) and waits for k-tile 0; each
// barrier waits for every load and LDS read of the wave.
constexpr int kMfma16LoadsPerThread = 16;
constexpr int kMfma16VmPrologue = kMfma16LoadsPerThread;
constexpr int kMfma16VmLoop = 0;
constexpr int kMfma16LgkmLoop = 0;

// OUT: kOutF16 (f16 C), kOutF32Partial (a plain f32 C store: never split-K
// here) or kOutF32Accum (f32 C += A*B); the main loop is the same for all.
// Whole k-tiles only: a problem with K % 64 != 0 runs the 16x16x32 loop's
// build of this tile (gemm_mfma16g, the entry's partial-K kernel), which
// masks the partial last k-tile, so this build carries no masking code.
template <int OUT, bool EPI>
__device__ __forceinline__ void mfma16_tile(const GemmParams &p, int m0, int n0, u32x4 *lds) {
  static_assert(OUT == kOutF16 || OUT == kOutF32Partial || OUT == kOutF32Accum,
                "no atomic or split-K output on the 16x16x32 instance");
  // slots, read placement and hazard rules: Mfma16Schedule (compile-time
  // checked)
  using Sched = Mfma16Schedule<>;
  constexpr int BK = 64, BQ = Sched::BQ, LS = 5;
  constexpr uint32_t SLOT = 65536; // ring slot: A [256][64] at 0, B [64][256] at 32 KiB
  constexpr uint32_t B_AT = 32768;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(TBK_LDS void *)lds;
  const int nk = p.K / BK; // k-tiles (K % 64 == 0 here)

  // Direct loads: round l of wave w fills 1 KiB at slot + l * 4 KiB + w * 1 KiB
  // (A rows 32l + 8w .. +7; B k-rows 8l + 2w, +1). B's 16-byte chunk c of
  // row k sits at c ^ 4 (k % 4) ^ 2 ((k / 8) % 2) (the plan's B encoding:
  // the first term over 64-byte segments, the second over 32-byte units; see
  // the fragment reads). The A phase repeats every 16 rows and the B phase
  // every 16 k rows, i.e. every 2 rounds, so a lane fetches one logical
  // chunk in every A round and one per round parity in B; only the scalar
  // offset moves.
  // Ragged edges. A round l covers rows m0 + a_row0 + 32l and is loaded only
  // while that row is below M; B columns at or past N load from kOob. Every
  // such element is refused here, by its offset, rather than left to the
  // buffer range check. Past the edges the ring holds zeros, which only
  // reach C elements that are not stored.
  const int a_row0 = (wave * 64 + lane) >> 3;
  const int a_lc = (lane & 7) ^ ((a_row0 >> 1) & 7);
  const int a_rows_left = p.M - m0 - a_row0;
  const uint32_t a_voff =
      a_rows_left > 0 ? ((uint32_t)a_row0 * (uint32_t)p.lda + a_lc * 8) * 2u : kOob;
  const int b_row0 = (wave * 64 + lane) >> 5; // 0 .. 7: (k / 8) % 2 = round % 2
  const int b_lc = (lane & 31) ^ (4 * (b_row0 & 3));
  const uint32_t b_voff0 =
      n0 + b_lc * 8 < p.N
          ? ((uint32_t)b_row0 * (uint32_t)p.ldb + (uint32_t)(n0 + b_lc * 8)) * 2u
          : kOob;
  const uint32_t b_voff1 =
      n0 + (b_lc ^ 2) * 8 < p.N
          ? ((uint32_t)b_row0 * (uint32_t)p.ldb + (uint32_t)(n0 + (b_lc ^ 2) * 8)) * 2u
          : kOob;
  const uint32_t a_round = 32u * (uint32_t)p.lda * 2u, b_round = 8u * (uint32_t)p.ldb * 2u;
  const uint32_t a_ktile = BK * 2u, b_ktile = BK * 2u * (uint32_t)p.ldb;
  const void *a_tile = rows_at(p.A, m0, p.lda, 2); // A's window starts at row m0
  const uint32_t a_bytes = rows_bytes(m0, p.M, p.lda, 2);
  const uint32_t b_bytes = (uint32_t)p.K * (uint32_t)p.ldb * 2u;
  const uint32_t wlds = lds0 + wave * 1024u;
  // load l of k-tile kt into ring slot ST (l is a constant once unrolled:
  // the LDS offset becomes the literal of the M0 add)
  auto load = [&](const u32x4 &ra, const u32x4 &rb, int kt, auto st_c, int l) {
    constexpr uint32_t base = decltype(st_c)::value * SLOT;
    static_for<16>([&](auto l_c) {
      constexpr int L = decltype(l_c)::value;
      if (L == l) {
        if constexpr (L < 8)
          load_lds16_at<base + L * 4096u>(ra, wlds, L * 32 < a_rows_left ? a_voff : kOob,
                                          (uint32_t)kt * a_ktile + L * a_round);
        else
          load_lds16_at<base + B_AT + (L - 8) * 4096u>(
              rb, wlds, (L & 1) ? b_voff1 : b_voff0, (uint32_t)kt * b_ktile + (L - 8) * b_round);
      }
    });
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;

  // Fragment reads. A tile ii of k step ks from stage st: one ds_read_b128 at
  // a_base[st][ks] + ii * 2 KiB (16 rows of 128 bytes; the row phase
  // (row / 2) % 8 = (l % 16) / 2 is the same for every ii). B tile jj: the 16
  // lanes of group g = l / 16 read k rows 32ks + 8g + l%16/4 (+4 for the
  // second half), columns 16jj + 4(l%4); with the B swizzle chunk ^ 4(k%4) ^
  // 2((k/8)%2) the column group lands at 2(jj ^ 2(l%16/4) ^ (g%2)) 16-byte
  // chunks. A 32-lane LDS cycle serves groups g and g+1, whose rows are 8
  // apart with equal k % 4: the second term puts them in different 32-byte
  // units, so the cycle covers the 64 banks once (without it, 2-way conflict).
  const int g = lane >> 4, ta = (lane >> 2) & 3, tb = lane & 3;
  uint32_t a_base[2][2], b_base[2][8];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      a_base[st][ks] = lds0 + st * SLOT + (wm * 128 + (lane & 15)) * 128 +
                       (((4 * ks + g) ^ ((lane & 15) >> 1)) * 16);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      b_base[st][jj] = lds0 + st * SLOT + B_AT + (8 * g + ta) * 512 +
                       (wn * 16 + 2 * (jj ^ (2 * ta) ^ (g & 1)) + (tb >> 1)) * 16 +
                       8 * (tb & 1);
  }

  f32x4 acc[8][8];
  half8 fa[2][8], fb[2][8];
  // read op o (0..23) of k step ks into buffer buf: A0, B0 (halves 0, 1) ..
  // B7, A1 .. A7
  auto rd = [&](int buf, int st, int ks, int o) {
    if (Sched::op_is_a(o)) {
      const int i = Sched::op_index(o);
      fa[buf][i] = __builtin_bit_cast(
          half8, *(const TBK_LDS u32x4 *)(uintptr_t)(a_base[st][ks] + i * 2048));
    } else {
      const int j = Sched::op_index(o), r = (o - 1) & 1;
      const half4 h = __builtin_bit_cast(
          half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((TBK_LDS short4 *)(uintptr_t)(
                     b_base[st][j] + ks * 16384 + r * 2048)));
      if (r == 0)
        fb[buf][j].lo = h;
      else
        fb[buf][j].hi = h;
    }
  };
  // MFMA m (tile m / 8, m % 8) of buffer buf; `first`: srcC = 0
  auto mfma = [&](int buf, int m, bool first) {
    const int i = m >> 3, j = m & 7;
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
  // k step 0 (stage st): 64 MFMAs, the reads of k step 1, `extra` per slot
  auto kstep0 = [&](int st, auto &&extra, bool first) {
    static_for<64>([&](auto m_c) {
      constexpr int m = decltype(m_c)::value;
      mfma(0, m, first);
      static_for<24>([&](auto o_c) {
        constexpr int o = decltype(o_c)::value;
        if constexpr (Sched::slot_ks0(o) == m)
          rd(1, st, 1, o);
      });
      extra(m);
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  // k step 1, slots LO .. HI-1, `extra` per slot
  auto kstep1x = [&](auto lo_c, auto hi_c, auto &&extra) {
    static_for<64>([&](auto m_c) {
      constexpr int m = decltype(m_c)::value;
      if constexpr (m >= decltype(lo_c)::value && m < decltype(hi_c)::value) {
        mfma(1, m, false);
        extra(m);
        __builtin_amdgcn_sched_barrier(0);
      }
    });
  };
  auto kstep1 = [&](auto lo_c, auto hi_c) { kstep1x(lo_c, hi_c, [](int) {}); };
  using Z = std::integral_constant<int, 0>;
  using Q = std::integral_constant<int, BQ>;
  using E = std::integral_constant<int, 64>;
  auto nothing = [](int) {};

  // f32 C += A*B: the prior C is added into the accumulators during the
  // first 16 loop bodies instead of after the loop, so its 64 MB (at 4096^3)
  // are read while the main loop leaves HBM mostly idle, not after it. Body q
  // (k-tiles q and q+1) adds the prior C of tiles 4q .. 4q+3 (MFMA order
  // m = 8i + j), loaded one body ahead (body 0's in the prologue) in the
  // accumulator layout (16 bytes per lane per tile: lane l holds row 16i + l %
  // 16, columns 16j + 4(l / 16) .. +3). Tile m's add sits 8 MFMA slots after
  // its MFMA in the body's first k step (slot m + 8, or slot m - 56 of the
  // next k step for m >= 56): its accumulators are no MFMA's operand from 8
  // slots before the add (128+ cycles, past rule (b)'s 24 wait states) to 48
  // slots after it. The loads are ordinary buffer loads; each body's barrier
  // (vmcnt(0)) has them landed before the next body adds them. Whole tiles
  // of at least 18 k-tiles only; the others add the prior C in the epilogue.
  constexpr bool C_IN_LOOP = OUT == kOutF32Accum;
  const bool c_in_loop = C_IN_LOOP && nk >= 18 && m0 + 256 <= p.M && n0 + 256 <= p.N;
  f32x4 cbuf[C_IN_LOOP ? 2 : 1][4];
  const __amdgpu_buffer_rsrc_t rcc =
      make_rsrc(rows_at(p.C, m0, p.ldc, 4), rows_bytes(m0, p.M, p.ldc, 4));
  const uint32_t c_voff = ((uint32_t)(wm * 128 + (lane & 15)) * (uint32_t)p.ldc +
                           (uint32_t)(n0 + wn * 128 + 4 * (lane >> 4))) * 4u;
  auto c_load = [&](auto q_c) {
    constexpr int q = decltype(q_c)::value;
    static_for<4>([&](auto t_c) {
      constexpr int t = decltype(t_c)::value, mm = 4 * q + t;
      cbuf[q & 1][t] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     rcc, c_voff, (int)((uint32_t)(16 * (mm >> 3)) * (uint32_t)p.ldc * 4u +
                                        64u * (mm & 7)),
                     0));
    });
  };
  // the add of body q at slot s of its first k step (s < 64) or of the next
  // (s - 64): tile s - 8
  auto c_add = [&](auto q_c, int s) {
    constexpr int q = decltype(q_c)::value;
    static_for<4>([&](auto t_c) {
      constexpr int t = decltype(t_c)::value, mm = 4 * q + t;
      if (s == mm + 8) {
        acc[mm >> 3][mm & 7] += cbuf[q & 1][t];
        // the sum back in its AGPRs in this slot: left to the compiler, the
        // v_accvgpr_write sinks to right before the tile's next asm MFMA,
        // which then reads srcC without the VALU-write wait states
        asm volatile("" : "+a"(acc[mm >> 3][mm & 7]));
      }
    });
  };
  if constexpr (C_IN_LOOP) {
    if (c_in_loop)
      c_load(std::integral_constant<int, 0>{});
  }

  // prologue: k-tiles 0 and 1 in flight, wait for 0, run it up to its barrier
  {
    const u32x4 ra = rsrc_dwords(a_tile, a_bytes), rb = rsrc_dwords(p.B, b_bytes);
    const u32x4 ra1 = rsrc_dwords(a_tile, nk > 1 ? a_bytes : 0u);
    const u32x4 rb1 = rsrc_dwords(p.B, nk > 1 ? b_bytes : 0u);
#pragma unroll
    for (int l = 0; l < 16; ++l)
      load(ra, rb, 0, S0{}, l);
#pragma unroll
    for (int l = 0; l < 16; ++l)
      load(ra1, rb1, 1, S1{}, l);
  }
  wait_vmcnt<kMfma16VmPrologue>();
  barrier();
#pragma unroll
  for (int o = 0; o < 24; ++o)
    rd(0, 0, 0, o);
  kstep0(0, nothing, true);
  kstep1(Z{}, Q{});

  // body(it): k-tile it (stage S) from its barrier on, k-tile it+1 (stage
  // S^1) up to its barrier; stage S is refilled with k-tile it+2.
  auto body_h = [&](int it, auto stage, auto &&start, auto &&k0, auto &&k1) {
    constexpr int S = decltype(stage)::value, Sn = S ^ 1;
    const bool ok = it + 2 < nk;
    const u32x4 ra = rsrc_dwords(a_tile, ok ? a_bytes : 0u);
    const u32x4 rb = rsrc_dwords(p.B, ok ? b_bytes : 0u);
    // k-tile it+1 landed (this wave's part), and this wave's reads of stage
    // S are done (the last A rows of k step 1 are read in k step 0 but only
    // consumed after the barrier, by MFMAs 40..63)
    static_assert(kMfma16VmLoop == 0 && kMfma16LgkmLoop == 0, "barrier wait below");
    wait_vmcnt_lgkm0<kMfma16VmLoop>();
    barrier();
    start();
    static_for<64 - BQ>([&](auto s_c) {
      constexpr int m = BQ + decltype(s_c)::value;
      mfma(1, m, false);
      static_for<Sched::NREAD>([&](auto o_c) {
        constexpr int o = decltype(o_c)::value;
        if constexpr (Sched::slot_ks1(o) == m)
          rd(0, Sn, 0, o);
      });
      if constexpr (((m - BQ) % LS) == 0)
        load(ra, rb, it + 2, stage, (m - BQ) / LS);
      __builtin_amdgcn_sched_barrier(0);
    });
    constexpr int NB = (64 - BQ + LS - 1) / LS; // refill loads issued before k-tile it+1
    constexpr int OFF = NB * LS - (64 - BQ);    // slot of k-tile it+1 with its first load
    static_assert(OFF + (16 - NB - 1) * LS < 64, "refill fits one k-tile");
    auto refill = [&](int m) {
      if (m >= OFF && ((m - OFF) % LS) == 0 && NB + (m - OFF) / LS < 16)
        load(ra, rb, it + 2, stage, NB + (m - OFF) / LS);
      k0(m);
    };
    kstep0(Sn, refill, false);
    kstep1x(Z{}, Q{}, k1);
  };
  auto body = [&](int it, auto stage) {
    auto none = [](int) {};
    body_h(it, stage, []() {}, none, none);
  };
  int it = 0;
  if constexpr (C_IN_LOOP) {
    if (c_in_loop) { // nk >= 18: bodies 0 .. 15, then the loop from k-tile 16
      static_for<16>([&](auto q_c) {
        constexpr int q = decltype(q_c)::value;
        body_h(
            q, std::integral_constant<int, q & 1>{},
            [&]() {
              if constexpr (q + 1 < 16)
                c_load(std::integral_constant<int, q + 1>{});
            },
            [&](int m) { c_add(q_c, m); }, [&](int m) { c_add(q_c, m + 64); });
      });
      it = 16;
    }
  }
  for (; it + 2 <= nk - 1; it += 2) {
    body(it, S0{});
    body(it + 1, S1{});
  }
  if (it < nk - 1)
    body(it, S0{});
  kstep1(Q{}, E{}); // the last k-tile after its barrier point
  // Sched::ACC_READ_WAITS (24) wait states between the last MFMA and the
  // first accumulator read
  static_assert(Sched::ACC_READ_WAITS == 24, "three s_nop 7 in the fence");
  acc_read_fence(acc);
  wait_vmcnt<0>(); // the zero loads past the end have landed too

  // f16 C through LDS: each wave's 128x128 tile goes to its own 32 KiB,
  // 256-byte rows, 16-byte chunk c of row r at c ^ (r % 8) with the chunk's
  // two 8-byte halves swapped when (r / 8) is odd, and comes back as 4 whole
  // rows per ds_read_b128 / buffer store. A ds_write_b64 is served 16 lanes
  // per cycle from a 128-byte window of the banks (measured: 16 lanes writing
  // 8-byte pieces 16 bytes apart conflict 2-way, 16 contiguous pieces do
  // not): the 16 rows a quarter wave writes then land in 16 different 8-byte
  // slots of that window. The fused steps (bias, activation,
  // clamp) run on each tile's f32 values on their way to LDS. The epilogue's
  // lane-derived addresses come from an opaque copy of the lane index, so the
  // compiler cannot hoist them out of a persistent tile loop and keep them
  // live in registers the main loop needs.
  int el = lane_id_fresh();
  const GemmParams pe = params_fresh();
  const EpiArgs ea{pe.bias, pe.epi_bias, pe.epi_act, pe.epi_clamp, pe.clamp_lo, pe.clamp_hi};
  if constexpr (OUT == kOutF16) {
    epi_f32x4 bv[EPI ? 8 : 1];
    if constexpr (EPI) { // every bias load first: one memory latency
      const int ccol = n0 + wn * 128 + 4 * (el >> 4);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        bv[j] = epi_load_bias(ea, ccol + 16 * j, pe.N);
    }
    barrier(); // every wave is past its last fragment read and load
    TBK_LDS char *wl = (TBK_LDS char *)(TBK_LDS void *)lds + wave * 32768;
    // clamp bounds: -inf / +inf for a clamp that is off
    const float lo = (pe.epi_clamp & 1) ? pe.clamp_lo : -__builtin_inff();
    const float hi = (pe.epi_clamp & 2) ? pe.clamp_hi : __builtin_inff();
    // C's window starts at row m0
    const __amdgpu_buffer_rsrc_t rc =
        make_rsrc(rows_at(pe.C, m0, pe.ldc, 2), rows_bytes(m0, pe.M, pe.ldc, 2));
    const int q = el & 15;
    // One 16-row block of the wave tile at a time: its 8 tiles go into LDS,
    // then its 16 rows come back and go out, so the stores of block i run
    // while block i+1's conversions (and fused steps) execute. The region is
    // this wave's alone and a wave's LDS operations complete in order, so no
    // barrier separates a block's writes from its reads.
    auto block = [&](auto i_c, auto act_c, auto clamp_c) {
      constexpr int i = decltype(i_c)::value;
      constexpr int ACT = decltype(act_c)::value;
      constexpr bool CLAMP = decltype(clamp_c)::value;
      epi_variant_fence<ACT, CLAMP>();
      const int r = 16 * i + (el & 15);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
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
        const int chunk = (2 * j + (el >> 5)) ^ (r & 7);
        const int half = ((el >> 4) & 1) ^ ((r >> 3) & 1);
        *(TBK_LDS u32x2 *)(wl + r * 256 + chunk * 16 + half * 8) = v;
        if (j & 1)
          __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int t = 4 * i; t < 4 * i + 4; ++t) {
        const int rr = t * 4 + (el >> 4); // rows 16i .. 16i+15
        u32x4 v = *(const TBK_LDS u32x4 *)(wl + rr * 256 + ((q ^ (rr & 7)) * 16));
        if ((rr >> 3) & 1)
          v = (u32x4){v[2], v[3], v[0], v[1]};
        const int row = m0 + wm * 128 + rr, col = n0 + wn * 128 + 8 * q;
        const uint32_t off =
            row < pe.M && col < pe.N
                ? ((uint32_t)(wm * 128 + rr) * (uint32_t)pe.ldc + (uint32_t)col) * 2u
                : kOob;
        // non-temporal (nt): C is written once and not read again by this
        // kernel; measured 0.7% faster at 4096^3 than the default policy
        __builtin_amdgcn_raw_buffer_store_b128(v, rc, off, 0, kStoreNT);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    epi_for_blocks<8, EPI>(pe, block);
  } else {
    // f32 C through LDS, one 16-row block of the wave tile at a time. Lane l
    // holds row 16i + l%16, columns 16j + 4(l/16) .. +3 of block i (16 bytes
    // per 16x16 tile j); they go to LDS as 512-byte rows, chunk c = 4j + l/16
    // of row r at c ^ r (a quarter wave's 16 rows land in 16 different 16-byte
    // bank groups), and come back as 2 whole rows per ds_read_b128 / buffer
    // store. Blocks rotate over four 8 KiB regions of the wave's 32 KiB: a
    // wave's LDS operations complete in order, so block i+4's writes never
    // overtake block i's reads. C += A*B reads the prior C as the same whole
    // rows, PF blocks ahead of the block being stored, and adds it to the sum
    // before the fused steps (the general loop's order: epilogue(C + acc)).
    constexpr int PF = EPI ? 2 : 4; // 4 blocks (128 VGPRs) spill with the fused steps
    const int q = el & 31, hr = el >> 5; // a lane's 16-byte chunk and row parity
    const int col = n0 + wn * 128 + 4 * q;
    // C's window starts at row m0
    const __amdgpu_buffer_rsrc_t rc =
        make_rsrc(rows_at(pe.C, m0, pe.ldc, 4), rows_bytes(m0, pe.M, pe.ldc, 4));
    auto c_off = [&](int i, int t) -> uint32_t {
      const int rr = wm * 128 + 16 * i + 2 * t + hr; // row of the tile
      return m0 + rr < pe.M && col < pe.N
                 ? ((uint32_t)rr * (uint32_t)pe.ldc + (uint32_t)col) * 4u
                 : kOob;
    };
    f32x4 old[OUT == kOutF32Accum ? PF : 1][8];
    auto load_old = [&](int i) {
      if constexpr (OUT == kOutF32Accum) {
        if (!c_in_loop) {
#pragma unroll
          for (int t = 0; t < 8; ++t)
            old[i % PF][t] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, c_off(i, t), 0, 0));
        }
      }
    };
#pragma unroll
    for (int i = 0; i < PF; ++i)
      load_old(i);
    const epi_f32x4 bias = EPI ? epi_load_bias(ea, col, pe.N) : epi_f32x4{};
    barrier(); // every wave is past its last fragment read and load
    TBK_LDS char *wl = (TBK_LDS char *)(TBK_LDS void *)lds + wave * 32768;
    const float lo = (pe.epi_clamp & 1) ? pe.clamp_lo : -__builtin_inff();
    const float hi = (pe.epi_clamp & 2) ? pe.clamp_hi : __builtin_inff();
    auto block = [&](auto i_c, auto act_c, auto clamp_c) {
      constexpr int i = decltype(i_c)::value;
      constexpr int ACT = decltype(act_c)::value;
      constexpr bool CLAMP = decltype(clamp_c)::value;
      epi_variant_fence<ACT, CLAMP>();
      TBK_LDS char *blk = wl + (i & 3) * 8192;
      const int r = el & 15, g = el >> 4;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        *(TBK_LDS f32x4 *)(blk + r * 512 + (((4 * j + g) ^ r) * 16)) = acc[i][j];
        if (j & 1)
          __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int rr = 2 * t + hr;
        f32x4 v = *(const TBK_LDS f32x4 *)(blk + rr * 512 + ((q ^ rr) * 16));
        if constexpr (OUT == kOutF32Accum) {
          if (!c_in_loop)
            v += old[i % PF][t];
        }
        if constexpr (EPI) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] = epi_apply_t<ACT, CLAMP>(v[e], bias[e], lo, hi);
        }
        // a plain f32 C is written once and not read again by this kernel
        // (non-temporal); C += A*B keeps the default policy
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rc,
                                               c_off(i, t), 0,
                                               OUT == kOutF32Partial ? kStoreNT : 0);
      }
      if (i + PF < 8)
        load_old(i + PF);
      __builtin_amdgcn_sched_barrier(0);
    };
    epi_for_blocks<8, EPI>(pe, block);
  }
}

// EPI: the fused epilogue steps (bias, activation, clamp) are compiled in.
// Plain instances carry none of that code, so their register allocation is
// the main loop's alone.
template <int BM, int BN, int BK, int WGM, int WGN, int OUT, int STAGES,
          int SPREAD_REQ = -1, bool EPI = false>
__global__ __launch_bounds__(WGM *WGN * 64, 1) void gemm_kernel(GemmParams p) {
  using T = GemmTile<BM, BN, BK, WGM, WGN, STAGES, SPREAD_REQ>;
  constexpr int NW = T::NW, KCH = T::KCH, BNC = T::BNC, TM = T::TM, TN = T::TN,
                KSTEPS = T::KSTEPS, NMFMA = T::NMFMA, LA = T::LA, LPT = T::LPT;
  __shared__ u32x4 lds[STAGES * T::STAGE + T::SCRATCH_CHUNKS];
  auto stage_base = [&](int st) -> u32x4 * { return lds + st * T::STAGE; };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave index as a scalar: the LDS bases of the direct loads derive from it
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;

  const u32x4 rb4 = rsrc_dwords(p.B, (uint32_t)p.K * (uint32_t)p.ldb * 2u);

  const bool persistent =
      p.mapping == kMapPersistent || p.mapping == kMapPersistentGrouped;
  int prog = blockIdx.x;
  const int nprog = gridDim.x;
  if (p.xcds > 1 && (nprog % p.xcds) == 0)
    prog = (prog % p.xcds) * (nprog / p.xcds) + prog / p.xcds;

  // ---- direct-load geometry (per thread, fixed for the whole kernel) -----
  // Load round i of wave w writes LDS chunks (i*NW + w)*64 + lane of a stage.
  // A: chunk q -> row q / KCH, physical chunk q % KCH holding logical k chunk
  //    (q % KCH) ^ ((row / A_PP) % KCH); the row advances by A_ROWS_PER_LOAD
  //    per round, so the logical chunk is recomputed per round.
  const int a_row0 = (wave * 64 + lane) / KCH;
  const int a_pc = lane % KCH;
  auto a_lchunk = [&](int i) {
    return a_pc ^ (((a_row0 + i * T::A_ROWS_PER_LOAD) / T::A_PP) % KCH);
  };
  // B: chunk q -> k row q / BNC, physical chunk q % BNC holding logical n
  //    chunk (q % BNC) ^ (4 * ((row / B_PP) % B_MAXPH)), fixed per lane when
  //    a round covers whole rows; else per round (B_RAGGED_ROUNDS)
  const int b_row0 = (wave * 64 + lane) / BNC;
  const int b_pc = (wave * 64 + lane) % BNC;
  const int b_lc = b_pc ^ (4 * ((b_row0 / T::B_PP) % T::B_MAXPH));
  auto b_round_row = [&](int i) { return (i * T::NT + wave * 64 + lane) / BNC; };
  auto b_round_lc = [&](int i) {
    const int q = i * T::NT + wave * 64 + lane;
    return (q % BNC) ^ (4 * (((q / BNC) / T::B_PP) % T::B_MAXPH));
  };

  // ---- fragment-read geometry --------------------------------------------
  const int fr_a = wm * T::WTM + (lane & 31); // A rows of this lane's srcB
  const int khalf = lane >> 5;
  // ds_read_b64_tr_b16 lane roles for the B fragment (srcA of the MFMA):
  // lane l reads 8 bytes at k row 8*(l/32) + (l%16)/4 (+4 for the second
  // read), n column 16*((l/16)%2) + 4*(l%4) of its 32-column tile.
  const int tr_k = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int tr_n = wn * T::WTN + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

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
    // C += A*B on small wave tiles of 4-wave workgroups (512 registers per
    // lane) whose f32 result is not staged through LDS: the prior C is the
    // accumulators' starting value, as in the reference
    // (LowerPipelineToNVGPU.cpp:2246-2263: C loaded into the accumulators
    // before the K loop; the sum is C + a0 b0 + a1 b1 + ... in k order),
    // loaded in their layout before the tile's first A/B loads, so its
    // latency runs beside theirs (the first MFMA waits for k-tile 0, issued
    // after it). Staged tiles read it after the loop as whole rows (fewer,
    // wider requests; loaded first, as rows or in the accumulator layout, it
    // measured no faster for the reference's small cases, which run out of L2).
    constexpr bool PRIOR_C_START = OUT == kOutF32Accum && !T::STAGED_F32_EPILOGUE &&
                                   TM * TN <= 4 && NW <= 4;
    // The staged small tiles load their prior C as the epilogue's whole rows
    // right after the prologue's A/B loads: k-tile 0 arrives first, and the
    // prior C during the first k-tiles' MFMAs instead of after the loop.
    constexpr int NLD32 = 32 / T::F32_RPI; // staged row segments per lane per 32-row block
    constexpr bool C_ROWS_EARLY = OUT == kOutF32Accum && T::STAGED_F32_EPILOGUE &&
                                  TM * TN <= 4 && NW <= 4 &&
                                  T::VM_PROLOGUE + TM * NLD32 < 64;
    f32x4 c_rows[C_ROWS_EARLY ? TM : 1][C_ROWS_EARLY ? NLD32 : 1];
    if constexpr (PRIOR_C_START) {
      const __amdgpu_buffer_rsrc_t rc =
          make_rsrc(rows_at(p.C, m0, p.ldc, 4), rows_bytes(m0, p.M, p.ldc, 4));
      const int row0 = m0 + wm * T::WTM + (lane & 31);
      const int col0 = n0 + wn * T::WTN + 4 * khalf;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int row = row0 + i * 32, col = col0 + j * 32 + 8 * g;
            const uint32_t off =
                (row < p.M && col < p.N)
                    ? ((uint32_t)(row - m0) * (uint32_t)p.ldc + (uint32_t)col) * 4u
                    : kOob;
            const f32x4 c = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, off, 0, 0));
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[i][j][4 * g + r] = c[r];
          }
    } else {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = (f32x16){};
    }

    // The k-dependent part of each global address is wave-uniform and rides
    // in the scalar offset; a row, column or k range outside the problem gets
    // the vector offset kOob, which loads zero. A's window starts at row m0.
    const u32x4 ra4 = rsrc_dwords(rows_at(p.A, m0, p.lda, 2), rows_bytes(m0, p.M, p.lda, 2));
    const uint32_t a_vrow = (uint32_t)a_row0 * (uint32_t)p.lda * 2u;
    const int a_rows_left = p.M - m0 - a_row0; // round i valid iff i*rows < left
    const uint32_t b_voff = (n0 + b_lc * 8) < p.N
                                ? ((uint32_t)b_row0 * (uint32_t)p.ldb +
                                   (uint32_t)(n0 + b_lc * 8)) * 2u
                                : kOob;
    // ragged B rounds: per round the lane's k row and its vector offset
    // (column past N: kOob)
    int b_rrow[T::B_RAGGED_ROUNDS ? T::LB : 1];
    uint32_t b_rvoff[T::B_RAGGED_ROUNDS ? T::LB : 1];
    if constexpr (T::B_RAGGED_ROUNDS) {
#pragma unroll
      for (int i = 0; i < T::LB; ++i) {
        const int row = b_round_row(i), lc = b_round_lc(i);
        b_rrow[i] = row;
        b_rvoff[i] = (n0 + lc * 8) < p.N
                         ? ((uint32_t)row * (uint32_t)p.ldb + (uint32_t)(n0 + lc * 8)) * 2u
                         : kOob;
      }
    }

    // Direct load l (0 .. LPT-1) of k-tile kt into LDS stage `stage`:
    // A load rounds first (l < LA), then B rounds.
    // the scratch row of the idle lanes of a last load round (past the ring),
    // from the array's LDS address (the cast of an offset pointer instead
    // makes the compiler emit an illegal null check against the aperture)
    const uint32_t idle_lds =
        (uint32_t)(uintptr_t)(TBK_LDS void *)lds + STAGES * T::STAGE * 16u;
    auto issue_load = [&](int kt, int stage, int l) {
      const int k0 = kt * BK;
      const bool kt_ok = kt < kt_end;
      // LDS byte address of this wave's first 1 KiB block in the stage
      const uint32_t a_lds =
          (uint32_t)(uintptr_t)(TBK_LDS void *)stage_base(stage) + wave * 1024u;
      if (l < LA) {
        const int i = l;
        const int lc = a_lchunk(i);
        // wave-uniform: the round's chunks of this wave lie inside the stage
        // (always, unless the tile has a partial round)
        const bool live = !T::IDLE_ROUNDS || (i * NW + wave) * 64 < T::A_STAGE;
        const bool ok = live && kt_ok && (k0 + lc * 8) < p.K &&
                        i * T::A_ROWS_PER_LOAD < a_rows_left;
        load_lds16(ra4, live ? a_lds + i * NW * 1024u : idle_lds,
                   ok ? a_vrow + lc * 16u : kOob,
                   k0 * 2 + i * T::A_ROWS_PER_LOAD * p.lda * 2);
      } else {
        const int i = l - LA;
        const uint32_t b_lds = a_lds + T::A_STAGE * 16u;
        const bool live = !T::IDLE_ROUNDS || (i * NW + wave) * 64 < T::B_STAGE;
        if constexpr (T::B_RAGGED_ROUNDS) {
          // the round's rows ride in the vector offset; the k-tile's in the
          // scalar one (unsigned: see below)
          load_lds16(rb4, live ? b_lds + i * NW * 1024u : idle_lds,
                     (live && kt_ok && k0 + b_rrow[i] < p.K) ? b_rvoff[i] : kOob,
                     (uint32_t)k0 * (uint32_t)p.ldb * 2u);
        } else {
          const int krow = k0 + b_row0 + i * T::B_ROWS_PER_LOAD;
          // unsigned: a lookahead k-tile past the end (voffset kOob) may put
          // k0 past K, where the signed product could pass INT_MAX
          load_lds16(rb4, live ? b_lds + i * NW * 1024u : idle_lds,
                     (live && kt_ok && krow < p.K) ? b_voff : kOob,
                     (uint32_t)(k0 + i * T::B_ROWS_PER_LOAD) * (uint32_t)p.ldb * 2u);
        }
      }
    };
    auto issue_tile = [&](int kt, int stage) {
#pragma unroll
      for (int l = 0; l < LPT; ++l)
        issue_load(kt, stage, l);
    };

    half8 fa[2][TM], fb[2][TN];
    // A fragment i of k step ks: one ds_read_b128
    auto read_frag_a = [&](int buf, int stage, int ks, int i) {
      const TBK_LDS u32x4 *As = (const TBK_LDS u32x4 *)stage_base(stage);
      const int c = ks * 2 + khalf;
      const int row = fr_a + i * 32;
      fa[buf][i] = __builtin_bit_cast(
          half8, As[row * KCH + (c ^ ((row / T::A_PP) % KCH))]);
    };
    // B fragment j of k step ks: two ds_read_b64_tr_b16
    auto read_frag_b = [&](int buf, int stage, int ks, int j) {
      const TBK_LDS char *Bs =
          (const TBK_LDS char *)((const TBK_LDS u32x4 *)stage_base(stage) + T::A_STAGE);
      const int n = tr_n + j * 32;
      half4 h[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int k = ks * 16 + tr_k + 4 * r;
        const int pc = (n >> 3) ^ (4 * ((k / T::B_PP) % T::B_MAXPH));
        const TBK_LDS short4 *src = (const TBK_LDS short4 *)(
            Bs + k * (BN * 2) + pc * 16 + (n & 7) * 2);
        h[r] = __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                             (TBK_LDS short4 *)src));
      }
      fb[buf][j] = (half8){h[0][0], h[0][1], h[0][2], h[0][3],
                           h[1][0], h[1][1], h[1][2], h[1][3]};
    };
    // fragment read r (0 .. TM+TN-1) in the order the MFMAs consume them:
    // A0, B0 .. B(TN-1), A1 .. A(TM-1)
    auto read_frag = [&](int buf, int stage, int ks, int r) {
      if (r == 0)
        read_frag_a(buf, stage, ks, 0);
      else if (r <= TN)
        read_frag_b(buf, stage, ks, r - 1);
      else
        read_frag_a(buf, stage, ks, r - TN);
    };
    auto read_frags = [&](int buf, int stage, int ks) {
#pragma unroll
      for (int r = 0; r < TM + TN; ++r)
        read_frag(buf, stage, ks, r);
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

    auto mfma_one = [&](int buf, int q) {
      const int i = q / TN, j = q % TN;
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[buf][j], fa[buf][i],
                                                         acc[i][j], 0, 0, 0);
    };

    // ---- prologue ----------------------------------------------------------
    // Slot schedule: tiles kt0 .. kt0+STAGES-2 whole plus the loads of tile
    // kt0+STAGES-1 that its refill would issue after the barrier; burst
    // schedule: tiles kt0 .. kt0+STAGES-1 whole. One stage per tile.
    if (persistent)
      __syncthreads(); // the previous tile's last fragment reads are done
    if constexpr (T::SLOTTED) {
#pragma unroll
      for (int st = 0; st + 1 < STAGES; ++st)
        issue_tile(kt0 + st, st);
#pragma unroll
      for (int l = 0; l < LPT; ++l)
        if (T::load_off(l) < T::AFTER)
          issue_load(kt0 + STAGES - 1, STAGES - 1, l);
    } else {
#pragma unroll
      for (int st = 0; st < STAGES; ++st)
        issue_tile(kt0 + st, st);
    }
    if constexpr (C_ROWS_EARLY) {
      const __amdgpu_buffer_rsrc_t rc =
          make_rsrc(rows_at(p.C, m0, p.ldc, 4), rows_bytes(m0, p.M, p.ldc, 4));
      const int col = n0 + wn * T::WTN + 4 * (lane % T::F32_CPR);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < NLD32; ++t) {
          const int row = m0 + wm * T::WTM + i * 32 + t * T::F32_RPI + lane / T::F32_CPR;
          const uint32_t off =
              (row < p.M && col < p.N)
                  ? ((uint32_t)(row - m0) * (uint32_t)p.ldc + (uint32_t)col) * 4u
                  : kOob;
          c_rows[i][t] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, off, 0, 0));
        }
      // the prior C loads are the youngest: k-tile 0 has landed once at most
      // VM_PROLOGUE of the A/B loads and all of them are outstanding
      wait_vmcnt<T::VM_PROLOGUE + TM * NLD32>();
    } else {
      wait_vmcnt<T::VM_PROLOGUE>();
    }
    __syncthreads();
    read_frags(0, 0, 0);

    // ---- main loop --------------------------------------------------------
    // Tile `it` is consumed from stage it % STAGES while the next STAGES-1
    // tiles stream into the other stages. Fragments are double-buffered
    // across the 16-deep k steps. The one barrier per k-tile sits in the
    // middle of the last k step: after it, tile it+1 (waited for with vmcnt
    // before the barrier) is visible, and stage it % STAGES is free for tile
    // it+STAGES. All steps are unconditional (out-of-range tiles load zeros).
    int s = 0;
    if constexpr (T::SLOTTED) {
      // Slot schedule: every MFMA slot is pinned in program order with the
      // fragment reads and refill loads assigned to it (see GemmTile).
      // Before the barrier, slot q also carries the loads of the refill that
      // started after the previous barrier (tile it+STAGES-1, stage sp).
      int sp = STAGES - 1;
      for (int it = 0; it < nk; ++it) {
        const int s_next = s + 1 == STAGES ? 0 : s + 1;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
          const int cur = ks & 1;
#pragma unroll
          for (int m = 0; m < NMFMA; ++m) {
            const int q = ks * NMFMA + m;
            if (q == T::BQ) {
              wait_vmcnt<T::VM_LOOP>();
              __syncthreads();
            }
            mfma_one(cur, m);
            constexpr int R = TM + TN;
            if (ks + 1 < KSTEPS) {
#pragma unroll
              for (int r = 0; r < R; ++r)
                if (r * NMFMA / R == m)
                  read_frag(cur ^ 1, s, ks + 1, r);
            } else if (q >= T::BQ) {
#pragma unroll
              for (int r = 0; r < R; ++r)
                if (T::BQ + r * T::AFTER / R == q)
                  read_frag(cur ^ 1, s_next, 0, r);
            }
#pragma unroll
            for (int l = 0; l < LPT; ++l) {
              const int off = T::load_off(l);
              if (off >= T::AFTER && off - T::AFTER == q)
                issue_load(kt0 + it + STAGES - 1, sp, l);
              if (off < T::AFTER && T::BQ + off == q)
                issue_load(kt0 + it + STAGES, s, l);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        sp = s;
        s = s_next;
      }
    } else
    for (int it = 0; it < nk; ++it) {
      const int s_next = s + 1 == STAGES ? 0 : s + 1;
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const int cur = ks & 1;
        if (ks + 1 < KSTEPS) {
          read_frags(cur ^ 1, s, ks + 1);
          mfma_range(cur, 0, NMFMA);
          if (ks == 0)
            sched_step<NMFMA, TM + 2 * TN, 0>();
          else
            sched_step<NMFMA, TM + 2 * TN, 0>();
          __builtin_amdgcn_sched_barrier(0); // k steps do not mix
        } else {
          mfma_range(cur, 0, NMFMA / 2);
          __builtin_amdgcn_sched_barrier(0);
          wait_vmcnt<T::VM_LOOP>();
          __syncthreads();
          read_frags(cur ^ 1, s_next, 0);
          issue_tile(kt0 + it + STAGES, s);
          mfma_range(cur, NMFMA / 2, NMFMA);
          sched_step<NMFMA - NMFMA / 2, TM + 2 * TN, 0>();
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      s = s_next;
    }

    // Drain the (out-of-range, zero) loads still in flight into LDS so none
    // can land after this tile: the next tile or workgroup reuses the space.
    wait_vmcnt<0>();

    // ---- epilogue ---------------------------------------------------------
    // lane holds C[m0 + wm*WTM + i*32 + lane%32][n0 + wn*WTN + j*32 + 8g + 4h + r]
    // in acc[i][j][4g + r], h = lane / 32.
    const int crow_base = m0 + wm * T::WTM + (lane & 31);
    const int ccol_base = n0 + wn * T::WTN + 4 * khalf;

    // Fused epilogue steps (bias, activation, clamp) on the whole f32 result,
    // in place on the accumulators, one 32-column tile j at a time. C += A*B
    // applies them in its store loop, after the prior C is added. EPI
    // instances are never launched for split-K partials (the reduction
    // applies the steps there) nor with atomic output.
    const EpiArgs ea{p.bias, p.epi_bias, p.epi_act, p.epi_clamp, p.clamp_lo, p.clamp_hi};
    if constexpr (EPI && (OUT == kOutF16 || OUT == kOutF32Partial)) {
      // every bias load of the wave tile first: one memory latency, not one
      // per 32-column tile
      epi_f32x4 bv[TN][4];
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          bv[j][g] = epi_load_bias(ea, ccol_base + j * 32 + 8 * g, p.N);
      // the activation dispatched once (no branch per element); the clamps
      // are selects against bounds that are -inf / +inf for a clamp that is off
      const float lo = (p.epi_clamp & 1) ? p.clamp_lo : -__builtin_inff();
      const float hi = (p.epi_clamp & 2) ? p.clamp_hi : __builtin_inff();
      auto steps = [&](auto act_c, auto clamp_c) {
        constexpr int ACT = decltype(act_c)::value;
        constexpr bool CLAMP = decltype(clamp_c)::value;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                acc[i][j][4 * g + r] =
                    epi_apply_t<ACT, CLAMP>(acc[i][j][4 * g + r], bv[j][g][r], lo, hi);
          __builtin_amdgcn_sched_barrier(0); // one 32-column tile at a time
        }
      };
      epi_dispatch_act(p.epi_act, steps);
    }

    if constexpr (OUT == kOutF16 && T::STAGED_F16_EPILOGUE) {
      // f16 C through LDS, so that every global store writes whole rows: a
      // lane's 4 consecutive columns are only 8 bytes, and 8-byte pieces
      // scattered over 32 rows write HBM lines partially. Each wave writes
      // its WTM x WTN f16 tile into a private LDS region of EPI_ROWB bytes
      // per row. Row r's 16-byte chunk c sits at c ^ ((r / EPI_RPP) %
      // EPI_CPR), and the two 8-byte halves of a chunk are swapped when row
      // bit EPI_HALF_BIT is set. A ds_write_b64 is served 16 lanes per cycle
      // from a 128-byte window of the banks: the 16 rows of a quarter wave
      // (one chunk each) then land in 16 different 8-byte slots of the
      // window, and the 16 lanes of a ds_read_b128 quarter (whole rows)
      // cover the 64 banks once. The tile is read back row by row, EPI_CPR
      // lanes x 16 bytes per row, and stored EPI_RPI full rows per
      // instruction.
      __syncthreads(); // every wave drained its loads and finished its reads
      TBK_LDS char *wl =
          (TBK_LDS char *)(TBK_LDS void *)lds + wave * (T::WTM * T::EPI_ROWB);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = i * 32 + (lane & 31);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const _Float16 h0 = (_Float16)acc[i][j][4 * g + 0];
            const _Float16 h1 = (_Float16)acc[i][j][4 * g + 1];
            const _Float16 h2 = (_Float16)acc[i][j][4 * g + 2];
            const _Float16 h3 = (_Float16)acc[i][j][4 * g + 3];
            u32x2 v;
            v[0] = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            v[1] = (uint32_t)__builtin_bit_cast(uint16_t, h2) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16);
            const int chunk = (4 * j + g) ^ ((r / T::EPI_RPP) & (T::EPI_CPR - 1));
            const int half = khalf ^ ((r >> T::EPI_HALF_BIT) & 1);
            *(TBK_LDS u32x2 *)(wl + r * T::EPI_ROWB + chunk * 16 + half * 8) = v;
          }
          __builtin_amdgcn_sched_barrier(0); // one 32x32 tile at a time
        }
      }
      const __amdgpu_buffer_rsrc_t rc =
          make_rsrc(rows_at(p.C, m0, p.ldc, 2), rows_bytes(m0, p.M, p.ldc, 2));
      const int q = lane % T::EPI_CPR;
#pragma unroll
      for (int it2 = 0; it2 < T::WTM / T::EPI_RPI; ++it2) {
        const int r = it2 * T::EPI_RPI + lane / T::EPI_CPR;
        const int chunk = q ^ ((r / T::EPI_RPP) & (T::EPI_CPR - 1));
        u32x4 v = *(const TBK_LDS u32x4 *)(wl + r * T::EPI_ROWB + chunk * 16);
        if ((r >> T::EPI_HALF_BIT) & 1)
          v = (u32x4){v[2], v[3], v[0], v[1]};
        const int row = m0 + wm * T::WTM + r;
        const int col = n0 + wn * T::WTN + 8 * q;
        const uint32_t off =
            (row < p.M && col < p.N)
                ? ((uint32_t)(row - m0) * (uint32_t)p.ldc + (uint32_t)col) * 2u
                : kOob;
        __builtin_amdgcn_raw_buffer_store_b128(v, rc, off, 0, 0);
      }
    } else if constexpr (OUT == kOutF16) {
      const __amdgpu_buffer_rsrc_t rc =
          make_rsrc(rows_at(p.C, m0, p.ldc, 2), rows_bytes(m0, p.M, p.ldc, 2));
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = crow_base + i * 32;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int col = ccol_base + j * 32 + 8 * g;
            const bool ok = row < p.M && col < p.N;
            const uint32_t off =
                ok ? ((uint32_t)(row - m0) * (uint32_t)p.ldc + (uint32_t)col) * 2u : kOob;
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
          // one 32x32 tile at a time: the conversions read the accumulators
          // through VGPRs, and letting them run ahead needs a VGPR each
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else if constexpr ((OUT == kOutF32Partial || OUT == kOutF32Accum ||
                          OUT == kOutF32Atomic) &&
                         T::STAGED_F32_EPILOGUE) {
      // f32 C through LDS, one 32-row block of the wave tile at a time: the
      // prior C (C += A*B) is read and the result written as whole row
      // segments (F32_CPR lanes x 16 bytes per row) instead of 16-byte
      // pieces of 32 rows. Atomic split-K adds each row segment with four
      // buffer_atomic_add_f32, so one instruction's 64 lanes touch a few
      // whole rows' cache lines rather than one line per lane.
      float *base = OUT == kOutF32Partial
                        ? p.ws + (size_t)part * (size_t)p.M * (size_t)p.ws_ld
                        : reinterpret_cast<float *>(p.C);
      const int ld = OUT == kOutF32Partial ? p.ws_ld : p.ldc;
      const __amdgpu_buffer_rsrc_t rc =
          make_rsrc(rows_at(base, m0, ld, 4), rows_bytes(m0, p.M, ld, 4));
      __syncthreads(); // every wave drained its loads and finished its reads
      constexpr int BR = T::F32_BLOCK_ROWS, HB = 32 / BR; // rows per pass, passes
      TBK_LDS char *wl =
          (TBK_LDS char *)(TBK_LDS void *)lds + wave * (BR * T::F32_ROWB);
      constexpr int NLD = 32 / T::F32_RPI; // row segments per lane per block
      constexpr int NLDH = NLD / HB;       // per pass
      static_assert(BR % T::F32_RPI == 0, "a pass reads whole rows");
      const int q = lane % T::F32_CPR;
      const int col = n0 + wn * T::WTN + 4 * q;
      const int rw = lane & 31;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row0 = m0 + wm * T::WTM + i * 32;
        uint32_t off[NLD];
#pragma unroll
        for (int t = 0; t < NLD; ++t) {
          const int row = row0 + t * T::F32_RPI + lane / T::F32_CPR;
          off[t] = (row < p.M && col < p.N)
                       ? ((uint32_t)(row - m0) * (uint32_t)ld + (uint32_t)col) * 4u
                       : kOob;
        }
        f32x4 old[OUT == kOutF32Accum ? NLD : 1];
        if constexpr (C_ROWS_EARLY) {
#pragma unroll
          for (int t = 0; t < NLD; ++t)
            old[t] = c_rows[i][t];
        } else if constexpr (OUT == kOutF32Accum) {
#pragma unroll
          for (int t = 0; t < NLD; ++t)
            old[t] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, off[t], 0, 0));
        }
#pragma unroll
        for (int h = 0; h < HB; ++h) {
          // accumulators in: lane l holds row l % 32, columns 32j + 8g + 4(l / 32);
          // in pass h only the lanes of rows h BR .. h BR + BR - 1 (row rw % BR
          // of the pass region). The lanes read what other lanes wrote, which
          // the compiler's one-thread memory model does not see: a lane that
          // skipped this pass's writes would reuse its previous pass's read of
          // the same address (measured: the reads moved into the masked write
          // block). The memory clobbers make every lane read after the writes
          // (LDS executes one wave's operations in order; no instruction).
          asm volatile("" ::: "memory");
          if (HB == 1 || rw / BR == h) {
            const int rl = rw % BR;
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                const int cs = (8 * j + 2 * g + khalf) ^ ((rl / T::F32_RPP) % T::F32_XOR);
                *(TBK_LDS f32x4 *)(wl + rl * T::F32_ROWB + cs * 16) =
                    (f32x4){acc[i][j][4 * g + 0], acc[i][j][4 * g + 1],
                            acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
              }
          }
          asm volatile("" ::: "memory");
          // whole row segments out: segment t of the block is row t F32_RPI +
          // l / F32_CPR, in pass t / NLDH
#pragma unroll
          for (int t = h * NLDH; t < (h + 1) * NLDH; ++t) {
            const int r = (t - h * NLDH) * T::F32_RPI + lane / T::F32_CPR; // row in the pass
            const int cs = q ^ ((r / T::F32_RPP) % T::F32_XOR);
            f32x4 v = *(const TBK_LDS f32x4 *)(wl + r * T::F32_ROWB + cs * 16);
            if constexpr (OUT == kOutF32Accum) {
              v += old[t];
              if constexpr (EPI) {
                const epi_f32x4 b = epi_load_bias(ea, col, p.N);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  v[e] = epi_apply1(v[e], b[e], ea);
              }
            }
            if constexpr (OUT == kOutF32Atomic) {
              // past the edges off[t] is kOob: the atomics are dropped
#pragma unroll
              for (int e = 0; e < 4; ++e)
                __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(v[e], rc, off[t] + 4u * e, 0, 0);
            } else {
              // f32 results (split-K partials, plain f32 C) are written once
              // and not read again by this kernel: non-temporal, which leaves
              // less dirty data in L2 for the kernel-end release (split-K 512^2
              // x 16384: 15.7 -> 15.1 us per GEMM); C += A*B keeps the default
              __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rc, off[t],
                                                     0, OUT == kOutF32Partial ? kStoreNT : 0);
            }
          }
        }
      }
    } else if constexpr (OUT == kOutF32Partial || OUT == kOutF32Accum) {
      float *base = OUT == kOutF32Partial
                        ? p.ws + (size_t)part * (size_t)p.M * (size_t)p.ws_ld
                        : reinterpret_cast<float *>(p.C);
      const int ld = OUT == kOutF32Partial ? p.ws_ld : p.ldc;
      const __amdgpu_buffer_rsrc_t rc =
          make_rsrc(rows_at(base, m0, ld, 4), rows_bytes(m0, p.M, ld, 4));
      auto c_off = [&](int i, int j, int g) -> uint32_t {
        const int row = crow_base + i * 32, col = ccol_base + j * 32 + 8 * g;
        return (row < p.M && col < p.N)
                   ? ((uint32_t)(row - m0) * (uint32_t)ld + (uint32_t)col) * 4u
                   : kOob;
      };
      // C += A*B reads the prior C first. All loads of a group of tiles (the
      // whole wave tile when it holds at most 4 MFMA tiles, else one row of
      // tiles) are issued before the first add, so the group waits for
      // memory once rather than once per tile.
      constexpr int GI = TM * TN <= 4 ? TM : 1; // tile rows per group
#pragma unroll
      for (int i0 = 0; i0 < TM; i0 += GI) {
        f32x4 old[GI][TN][4];
        if constexpr (OUT == kOutF32Accum && !PRIOR_C_START) {
#pragma unroll
          for (int ii = 0; ii < GI; ++ii)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g)
                old[ii][j][g] = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, c_off(i0 + ii, j, g),
                                                                 0, 0));
        }
#pragma unroll
        for (int ii = 0; ii < GI; ++ii)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const int i = i0 + ii;
              f32x4 v = {acc[i][j][4 * g + 0], acc[i][j][4 * g + 1],
                         acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
              if constexpr (OUT == kOutF32Accum) {
                if constexpr (!PRIOR_C_START)
                  v += old[ii][j][g];
                if constexpr (EPI) {
                  const epi_f32x4 b = epi_load_bias(ea, ccol_base + j * 32 + 8 * g, p.N);
#pragma unroll
                  for (int r = 0; r < 4; ++r)
                    v[r] = epi_apply1(v[r], b[r], ea);
                }
              }
              __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rc,
                                                     c_off(i, j, g), 0, 0);
            }
        __builtin_amdgcn_sched_barrier(0); // one group at a time
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

// ---- producer waves: f32-partial instances with dedicated load waves -------
// The general loop's small-wave-tile instances spend their k-tiles waiting:
// one wave per SIMD issues both the direct loads and the MFMAs, and a load
// the texture path cannot yet accept stalls that wave's next MFMA. Here the
// workgroup has twice the waves: waves NW .. 2NW-1 only issue the direct
// loads (the general loop's load mapping, wave w - NW in the role of wave w)
// and wait for them; waves 0 .. NW-1 only read fragments and run MFMAs. The
// two halves meet at one barrier per k-tile:
//  * before barrier it, a loader waits until its loads of k-tile it+1 have
//    landed (vmcnt((STAGES-2) * LPT)), so after it k-tile it+1 is visible;
//  * before barrier it, a compute wave has read all its fragments of k-tile
//    it (the fence waits for them), so after it the loaders refill k-tile
//    it's stage with k-tile it+STAGES.
// A compute wave reads a whole k-tile's fragments right after each barrier
// (double-buffered across k-tiles), so their latency runs under the previous
// k-tile's MFMAs. Same LDS ring, swizzles, fragment reads, MFMA order and
// staged f32 epilogue as the general instance of the same key: the partials
// are bit-identical. Every wave takes every barrier (prologue, one per
// k-tile, the epilogue's, the persistent loop's), so the counts match.
template <int BM, int BN, int BK, int WGM, int WGN, int STAGES>
__global__ __launch_bounds__(2 * WGM * WGN * 64, 1) void gemm_kernel_pw(GemmParams p) {
  using T = GemmTile<BM, BN, BK, WGM, WGN, STAGES>;
  constexpr int NW = T::NW, KCH = T::KCH, BNC = T::BNC, TM = T::TM, TN = T::TN,
                KSTEPS = T::KSTEPS, NMFMA = T::NMFMA, LA = T::LA, LPT = T::LPT;
  static_assert(!T::IDLE_ROUNDS && !T::B_RAGGED_ROUNDS, "producer waves load whole rows per round");
  static_assert(T::STAGED_F32_EPILOGUE && !T::F32_HALF_BLOCKS,
                "f32 partials staged through LDS in whole 32-row blocks");
  static_assert(KSTEPS == 4, "whole-k-tile fragment buffers sized for BK = 64");
  __shared__ u32x4 lds[STAGES * T::STAGE];
  auto stage_base = [&](int st) -> u32x4 * { return lds + st * T::STAGE; };
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool loader = wave >= NW;
  const u32x4 rb4 = rsrc_dwords(p.B, (uint32_t)p.K * (uint32_t)p.ldb * 2u);
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
    int kt0 = 0, nk = p.tiles_k;
    if (p.mapping == kMapSplitK) {
      // LowerPipelineToNVGPU.cpp:331-356 (contiguous k-tile range per split)
      const int base = p.tiles_k / p.split_k, extra = p.tiles_k % p.split_k;
      kt0 = part * base + (part < extra ? part : extra);
      nk = base + (part < extra ? 1 : 0);
    }
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int kt_end = kt0 + nk;
    if (work != prog)
      __syncthreads(); // the previous tile's staged epilogue has been read back

    if (loader) { // ------------------------------------------------ loads
      const int lw = wave - NW;
      const int a_row0 = (lw * 64 + lane) / KCH;
      const int a_pc = lane % KCH;
      auto a_lchunk = [&](int i) {
        return a_pc ^ (((a_row0 + i * T::A_ROWS_PER_LOAD) / T::A_PP) % KCH);
      };
      const int b_row0 = (lw * 64 + lane) / BNC;
      const int b_pc = lane % BNC;
      const int b_lc = b_pc ^ (4 * ((b_row0 / T::B_PP) % T::B_MAXPH));
      // A's window starts at row m0
      const u32x4 ra4 =
          rsrc_dwords(rows_at(p.A, m0, p.lda, 2), rows_bytes(m0, p.M, p.lda, 2));
      const uint32_t a_vrow = (uint32_t)a_row0 * (uint32_t)p.lda * 2u;
      const int a_rows_left = p.M - m0 - a_row0;
      const uint32_t b_voff = (n0 + b_lc * 8) < p.N
                                  ? ((uint32_t)b_row0 * (uint32_t)p.ldb +
                                     (uint32_t)(n0 + b_lc * 8)) * 2u
                                  : kOob;
      auto issue_load = [&](int kt, int stage, int l) {
        const int k0 = kt * BK;
        const bool kt_ok = kt < kt_end;
        const uint32_t a_lds =
            (uint32_t)(uintptr_t)(TBK_LDS void *)stage_base(stage) + lw * 1024u;
        if (l < LA) {
          const int i = l;
          const int lc = a_lchunk(i);
          const bool ok =
              kt_ok && (k0 + lc * 8) < p.K && i * T::A_ROWS_PER_LOAD < a_rows_left;
          load_lds16(ra4, a_lds + i * NW * 1024u, ok ? a_vrow + lc * 16u : kOob,
                     k0 * 2 + i * T::A_ROWS_PER_LOAD * p.lda * 2);
        } else {
          const int i = l - LA;
          const uint32_t b_lds = a_lds + T::A_STAGE * 16u;
          const int krow = k0 + b_row0 + i * T::B_ROWS_PER_LOAD;
          load_lds16(rb4, b_lds + i * NW * 1024u, (kt_ok && krow < p.K) ? b_voff : kOob,
                     (uint32_t)(k0 + i * T::B_ROWS_PER_LOAD) * (uint32_t)p.ldb * 2u);
        }
      };
      auto issue_tile = [&](int kt, int stage) {
#pragma unroll
        for (int l = 0; l < LPT; ++l)
          issue_load(kt, stage, l);
      };
#pragma unroll
      for (int st = 0; st < STAGES; ++st)
        issue_tile(kt0 + st, st);
      wait_vmcnt<(STAGES - 1) * LPT>();
      __syncthreads(); // k-tile 0 visible
      int s = 0;
      for (int it = 0; it < nk; ++it) {
        wait_vmcnt<(STAGES - 2) * LPT>(); // k-tile it+1 landed
        __syncthreads();                  // the compute waves' barrier of k-tile it
        issue_tile(kt0 + it + STAGES, s); // stage s (k-tile it) is free
        s = s + 1 == STAGES ? 0 : s + 1;
      }
      wait_vmcnt<0>(); // the zero loads past the end have landed too
      __syncthreads(); // the epilogue's barrier
      continue;
    }

    // -------------------------------------------------------------- compute
    const int wm = wave / WGN, wn = wave % WGN;
    const int fr_a = wm * T::WTM + (lane & 31);
    const int khalf = lane >> 5;
    const int tr_k = 8 * (lane >> 5) + ((lane & 15) >> 2);
    const int tr_n = wn * T::WTN + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = (f32x16){};
    // a whole k-tile of fragments per buffer: [buffer][k step][tile]
    half8 fa[2][KSTEPS][TM], fb[2][KSTEPS][TN];
    auto read_tile = [&](int buf, int stage) {
      const TBK_LDS u32x4 *As = (const TBK_LDS u32x4 *)stage_base(stage);
      const TBK_LDS char *Bs = (const TBK_LDS char *)(As + T::A_STAGE);
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int c = ks * 2 + khalf;
          const int row = fr_a + i * 32;
          fa[buf][ks][i] =
              __builtin_bit_cast(half8, As[row * KCH + (c ^ ((row / T::A_PP) % KCH))]);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = tr_n + j * 32;
          half4 h[2];
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const int k = ks * 16 + tr_k + 4 * r;
            const int pc = (n >> 3) ^ (4 * ((k / T::B_PP) % T::B_MAXPH));
            h[r] = __builtin_bit_cast(
                half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((TBK_LDS short4 *)(
                           Bs + k * (BN * 2) + pc * 16 + (n & 7) * 2)));
          }
          fb[buf][ks][j] = (half8){h[0][0], h[0][1], h[0][2], h[0][3],
                                   h[1][0], h[1][1], h[1][2], h[1][3]};
        }
      }
    };
    // C^T tile += B^T-fragment x A-fragment over the k-tile, k steps in order
    auto mfma_tile = [&](int buf) {
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
        for (int q = 0; q < NMFMA; ++q) {
          const int i = q / TN, j = q % TN;
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[buf][ks][j], fa[buf][ks][i],
                                                             acc[i][j], 0, 0, 0);
        }
    };
    __syncthreads(); // k-tile 0 visible
    read_tile(0, 0);
    int s = 0;
    for (int it = 0; it < nk; it += 2) { // two k-tiles: fixed fragment buffers
      const int s1 = s + 1 == STAGES ? 0 : s + 1;
      const int s2 = s1 + 1 == STAGES ? 0 : s1 + 1;
      __syncthreads(); // k-tile it+1 visible; this wave's reads of k-tile it done
      read_tile(1, s1);
      mfma_tile(0);
      __builtin_amdgcn_sched_barrier(0);
      if (it + 1 < nk) {
        __syncthreads();
        read_tile(0, s2);
        mfma_tile(1);
        __builtin_amdgcn_sched_barrier(0);
      }
      s = s2;
    }

    // f32 partials through LDS, as the general loop's staged f32 epilogue
    float *base = p.ws + (size_t)part * (size_t)p.M * (size_t)p.ws_ld;
    const int ld = p.ws_ld;
    const __amdgpu_buffer_rsrc_t rc =
        make_rsrc(rows_at(base, m0, ld, 4), rows_bytes(m0, p.M, ld, 4));
    __syncthreads(); // the loaders drained; every compute wave finished its reads
    TBK_LDS char *wl = (TBK_LDS char *)(TBK_LDS void *)lds + wave * (32 * T::F32_ROWB);
    constexpr int NLD = 32 / T::F32_RPI;
    const int q = lane % T::F32_CPR;
    const int col = n0 + wn * T::WTN + 4 * q;
    const int rw = lane & 31;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row0 = m0 + wm * T::WTM + i * 32;
      uint32_t off[NLD];
#pragma unroll
      for (int t = 0; t < NLD; ++t) {
        const int row = row0 + t * T::F32_RPI + lane / T::F32_CPR;
        off[t] = (row < p.M && col < p.N)
                     ? ((uint32_t)(row - m0) * (uint32_t)ld + (uint32_t)col) * 4u
                     : kOob;
      }
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int cs = (8 * j + 2 * g + khalf) ^ ((rw / T::F32_RPP) % T::F32_XOR);
          *(TBK_LDS f32x4 *)(wl + rw * T::F32_ROWB + cs * 16) =
              (f32x4){acc[i][j][4 * g + 0], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                      acc[i][j][4 * g + 3]};
        }
#pragma unroll
      for (int t = 0; t < NLD; ++t) {
        const int r = t * T::F32_RPI + lane / T::F32_CPR;
        const int cs = q ^ ((r / T::F32_RPP) % T::F32_XOR);
        const f32x4 v = *(const TBK_LDS f32x4 *)(wl + r * T::F32_ROWB + cs * 16);
        // written once, read once by the reduce: non-temporal (see the
        // general loop)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rc, off[t], 0,
                                               kStoreNT);
      }
    }
  }
}

// The programs of the 16x16x32 instance of the 4-wave 256x256x64 2-stage
// configuration (any M, N and K; tile, grouped or persistent order).
template <int OUT, bool EPI>
__device__ __forceinline__ void mfma16_programs(const GemmParams &p, u32x4 *lds) {
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
    mfma16_tile<OUT, EPI>(p, tile_m * 256, tile_n * 256, lds);
  }
}

// f16 C
template <bool EPI>
__global__ __launch_bounds__(256, 1) void gemm_mfma16(GemmParams p) {
  __shared__ u32x4 lds[8192]; // the 2-stage ring of 256x64 + 64x256 halves
  mfma16_programs<kOutF16, EPI>(p, lds);
}

// f32 C: a plain store (OUT = kOutF32Partial) or C += A*B (kOutF32Accum)
template <int OUT, bool EPI>
__global__ __launch_bounds__(256, 1) void gemm_mfma16_f32(GemmParams p) {
  __shared__ u32x4 lds[8192];
  mfma16_programs<OUT, EPI>(p, lds);
}

} // namespace tbk

// One registry entry per instance.
#define TBK_WAITS(BM, BN, BK, WGM, WGN, ST)                                      \
  tbk::GemmTile<BM, BN, BK, WGM, WGN, ST>::VM_PROLOGUE,                          \
      tbk::GemmTile<BM, BN, BK, WGM, WGN, ST>::VM_LOOP, -1

#define TBK_ENTRY(BM, BN, BK, WGM, WGN, OUT, ST)                                 \
  {{BM, BN, BK, WGM, WGN, OUT, ST, 0},                                           \
   reinterpret_cast<const void *>(                                               \
       &tbk::gemm_kernel<BM, BN, BK, WGM, WGN, OUT, ST>),                        \
   "tb_gemm_gfx950_" #BM "x" #BN "x" #BK "_w" #WGM "x" #WGN "_s" #ST "_out" #OUT, \
   TBK_WAITS(BM, BN, BK, WGM, WGN, ST)}

#define TBK_OUTS(BM, BN, BK, WGM, WGN, ST)                                      \
  TBK_ENTRY(BM, BN, BK, WGM, WGN, 0, ST), TBK_ENTRY(BM, BN, BK, WGM, WGN, 1, ST), \
      TBK_ENTRY(BM, BN, BK, WGM, WGN, 2, ST),                                   \
      TBK_ENTRY(BM, BN, BK, WGM, WGN, 3, ST)

// Fused-epilogue instances: f16 C, plain f32 C, and f32 C += A*B (atomic
// split-K cannot carry the steps; split-K partials take them in the reduce).
#define TBK_EPI_ENTRY(BM, BN, BK, WGM, WGN, OUT, ST)                             \
  {{BM, BN, BK, WGM, WGN, OUT, ST, 1},                                           \
   reinterpret_cast<const void *>(                                               \
       &tbk::gemm_kernel<BM, BN, BK, WGM, WGN, OUT, ST, -1, true>),              \
   "tb_gemm_gfx950_" #BM "x" #BN "x" #BK "_w" #WGM "x" #WGN "_s" #ST "_out" #OUT \
   "_epi",                                                                       \
   TBK_WAITS(BM, BN, BK, WGM, WGN, ST)}

#define TBK_EPI_OUTS(BM, BN, BK, WGM, WGN, ST)                                  \
  TBK_EPI_ENTRY(BM, BN, BK, WGM, WGN, 0, ST),                                   \
      TBK_EPI_ENTRY(BM, BN, BK, WGM, WGN, 1, ST),                               \
      TBK_EPI_ENTRY(BM, BN, BK, WGM, WGN, 2, ST)
