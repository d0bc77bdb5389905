// Slot schedule of the 16x16x32 instance (gemm_mfma16 in gemm_gfx950_impl.h)
// and the hazard rules its inline-asm MFMAs rely on, checked at compile time.
//
// The instance issues v_mfma_f32_16x16x32_f16 as inline asm with the
// accumulator tied in place, so the compiler tracks no MFMA hazards for it.
// The rules it must keep instead:
//  (a) each accumulator's first MFMA takes srcC = 0 (no zeroing write lands
//      right before it): every tile of the wave's 8 x 8 grid is the target
//      of exactly one MFMA of a k step, so the first k step's MFMAs cover
//      every accumulator once;
//  (b) the accumulators are read only after ACC_READ_WAITS wait states
//      (three `s_nop 7`) past the last MFMA, at least 3 per MFMA pass;
//  (c) every fragment register is rewritten (by a ds_read of a later k
//      step) at least MIN_REWRITE_SLOTS MFMA slots after its last MFMA
//      read;
//  plus the ordering the barrier depends on: every fragment read of the
//  stage a barrier frees is issued before that barrier (its lgkmcnt(0)
//  then covers it), and every read of the next k-tile comes after it.
//
// Plain constexpr C++ (no HIP): the kernel takes its read slots from here,
// and the CPU tests compile edited schedules to show that an edit breaking
// a rule does not build.
#pragma once

namespace tbk {

template <int BQ_ = 8, int RNUM = 8, int RDEN = 3, int ACC_WAITS = 24, int R1NUM = 7,
          int R1DEN = 3>
struct Mfma16Schedule {
  static constexpr int NSLOT = 64;  // MFMAs per 32-deep k step: 8 x 8 tiles of 16 x 16
  static constexpr int NREAD = 24;  // fragment reads per k step: A0, B0 (2 halves) .. B7, A1 .. A7
  static constexpr int BQ = BQ_;    // the k-tile's barrier sits before slot BQ of k step 1
  static constexpr int PASSES = 8;  // v_mfma_f32_16x16x32_f16
  static constexpr int ACC_READ_WAITS = ACC_WAITS;
  static constexpr int MIN_REWRITE_SLOTS = 8;

  // MFMA m of a k step updates tile (m / 8, m % 8): A fragment m / 8, B m % 8
  static constexpr int mfma_a(int m) { return m >> 3; }
  static constexpr int mfma_b(int m) { return m & 7; }
  // read op o: A (o == 0 or o >= 17) or B, and the fragment index
  static constexpr bool op_is_a(int o) { return o == 0 || o >= 17; }
  static constexpr int op_index(int o) { return o == 0 ? 0 : (o >= 17 ? o - 16 : (o - 1) >> 1); }
  // slot of read op o: in k step 0, the reads of k step 1 (fragment buffer 1);
  // in k step 1 after the barrier, the next k-tile's k step 0 (buffer 0)
  static constexpr int slot_ks0(int o) { return RNUM * o / RDEN; }
  static constexpr int slot_ks1(int o) { return BQ + R1NUM * o / R1DEN; }

  static constexpr int last_read(bool a, int idx) {
    int last = -1;
    for (int m = 0; m < NSLOT; ++m)
      if ((a ? mfma_a(m) : mfma_b(m)) == idx)
        last = m;
    return last;
  }
  // (a): the MFMAs of a k step hit each of the 64 accumulator tiles once
  static constexpr bool covers_every_tile_once() {
    for (int t = 0; t < 64; ++t) {
      int hits = 0;
      for (int m = 0; m < NSLOT; ++m)
        hits += (mfma_a(m) * 8 + mfma_b(m)) == t ? 1 : 0;
      if (hits != 1)
        return false;
    }
    return true;
  }
  // every fragment is read by some op, and each op's slot lies in its k step
  static constexpr bool reads_fit() {
    for (int o = 0; o < NREAD; ++o)
      if (slot_ks0(o) < 0 || slot_ks0(o) >= NSLOT || slot_ks1(o) < BQ ||
          slot_ks1(o) >= NSLOT)
        return false;
    for (int f = 0; f < 8; ++f) {
      int a = 0, b = 0;
      for (int o = 0; o < NREAD; ++o) {
        a += op_is_a(o) && op_index(o) == f ? 1 : 0;
        b += !op_is_a(o) && op_index(o) == f ? 1 : 0;
      }
      if (a != 1 || b != 2) // one ds_read_b128 per A fragment, two halves per B
        return false;
    }
    return true;
  }
  // (c): slots between a fragment's last MFMA read (in the k step that uses
  // its buffer) and the read op that rewrites it (in the other k step)
  static constexpr int min_rewrite_distance() {
    int d = 1 << 30;
    for (int o = 0; o < NREAD; ++o) {
      const int last = last_read(op_is_a(o), op_index(o));
      const int d1 = (NSLOT - last) + slot_ks0(o); // buffer 1: used in k step 1
      const int d0 = (NSLOT - last) + slot_ks1(o); // buffer 0: used in k step 0
      d = d1 < d ? d1 : d;
      d = d0 < d ? d0 : d;
    }
    return d;
  }

  static_assert(covers_every_tile_once(), "(a) first-MFMA srcC = 0 needs one MFMA per tile");
  static_assert(reads_fit(), "fragment reads must fall inside their k step (and after the "
                             "barrier for the next k-tile's reads)");
  static_assert(slot_ks1(NREAD - 1) < NSLOT, "the next k-tile's reads must fit after the barrier");
  static_assert(min_rewrite_distance() >= MIN_REWRITE_SLOTS,
                "(c) a fragment register rewritten too soon after its last MFMA read");
  static_assert(ACC_READ_WAITS >= 3 * PASSES && ACC_READ_WAITS % 8 == 0,
                "(b) accumulator reads need 3 wait states per MFMA pass, issued as s_nop 7");
};

} // namespace tbk
