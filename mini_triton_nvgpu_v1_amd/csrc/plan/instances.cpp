// Host-side table of the compiled gfx950 kernel instances (see instances.h).
#include "instances.h"

#include "../kernels/gemm_tiles.h"

#include <algorithm>
#include <cstdio>
#include <set>
#include <tuple>

namespace tb {

static auto tie(const InstanceKey &k) {
  return std::tie(k.bm, k.bn, k.bk, k.wgm, k.wgn, k.out, k.stages, k.epi, k.mfma);
}
bool InstanceKey::operator<(const InstanceKey &o) const { return tie(*this) < tie(o); }
bool InstanceKey::operator==(const InstanceKey &o) const { return tie(*this) == tie(o); }

namespace {
struct Tile {
  int64_t bm, bn, bk, wgm, wgn, stages;
};
#define TB_TILE(BM, BN, BK, WGM, WGN, ST) Tile{BM, BN, BK, WGM, WGN, ST}
#define TB_SHAPE_TILES(SHAPE) TBK_TILES_##SHAPE(TB_TILE),
const Tile kTiles[] = {TBK_SHAPES(TB_SHAPE_TILES)};
#undef TB_SHAPE_TILES
#undef TB_TILE
} // namespace

const std::vector<InstanceKey> &gfx950Instances() {
  static const std::vector<InstanceKey> all = [] {
    std::vector<InstanceKey> v;
    for (const Tile &t : kTiles) {
      for (int out = kInstOutF16; out <= kInstOutF32Atomic; ++out)
        v.push_back({t.bm, t.bn, t.bk, t.wgm, t.wgn, out, t.stages, 0, TB_MFMA_32X32X16});
      // the fused steps need the whole sum: no atomic-output flavour
      for (int out = kInstOutF16; out <= kInstOutF32Accum; ++out)
        v.push_back({t.bm, t.bn, t.bk, t.wgm, t.wgn, out, t.stages, 1, TB_MFMA_32X32X16});
    }
    // 16x16x32: f16 C, plain f32 C and f32 C += A*B (no split-K)
    for (int out = kInstOutF16; out <= kInstOutF32Accum; ++out)
      for (int epi = 0; epi <= 1; ++epi)
        v.push_back({256, 256, 64, 2, 2, out, 2, epi, TB_MFMA_16X16X32});
    return v;
  }();
  return all;
}

bool hasGfx950Instance(const InstanceKey &k) {
  static const std::set<InstanceKey> keys(gfx950Instances().begin(),
                                          gfx950Instances().end());
  return keys.count(k) != 0;
}

std::string instanceName(const InstanceKey &k) {
  char buf[128];
  snprintf(buf, sizeof buf, "tb_gemm_gfx950_%lldx%lldx%lld_w%lldx%lld_s%lld_out%d%s%s",
           (long long)k.bm, (long long)k.bn, (long long)k.bk, (long long)k.wgm,
           (long long)k.wgn, (long long)k.stages, k.out,
           k.mfma == TB_MFMA_16X16X32 ? "_16x16x32" : "", k.epi ? "_epi" : "");
  return buf;
}

InstanceKey instanceKeyOf(const tb_gemm_config &c) {
  InstanceKey k;
  k.bm = c.block_m;
  k.bn = c.block_n;
  k.bk = c.block_k;
  k.wgm = c.wave_grid_m;
  k.wgn = c.wave_grid_n;
  k.stages = c.stages;
  k.out = instanceOutOf(c.mapping == TB_MAP_SPLIT_K, c.reduction == TB_RED_ATOMIC,
                        c.c_dtype == TB_DTYPE_F16, c.acc_init == TB_ACC_INIT_LOAD_C);
  k.epi = (c.epi_bias || c.epi_activation || c.epi_clamp) && c.mapping != TB_MAP_SPLIT_K;
  k.mfma = c.mfma;
  return k;
}

int instanceOutOf(bool splitK, bool atomicReduction, bool f16C, bool loadC) {
  if (splitK)
    return atomicReduction ? kInstOutF32Atomic : kInstOutF32Partial;
  if (f16C)
    return kInstOutF16;
  return loadC ? kInstOutF32Accum : kInstOutF32Partial;
}

static bool producerTile(const InstanceKey &k) {
#define TB_PRODUCER(BM, BN, BK, WGM, WGN, ST)                                          \
  (k.bm == BM && k.bn == BN && k.bk == BK && k.wgm == WGM && k.wgn == WGN && k.stages == ST) ||
  return TBK_PRODUCER_TILES(TB_PRODUCER) false;
#undef TB_PRODUCER
}

InstanceSchedule instanceSchedule(const InstanceKey &k) {
  InstanceSchedule s;
  if (k.mfma == TB_MFMA_16X16X32) {
    s.issue = "exact_tile_slots";
    s.loadsPerThread = 16; // 256x64 + 64x256 halves, 16-byte loads, 256 lanes
    s.prologueTailLoads = 16;
    s.refillSpreadSlots = 16 * 5; // one load every 5 MFMA slots from the barrier
    s.vmPrologue = 16;
    s.vmLoop = 0;
    s.lgkmLoop = 0;
    return s;
  }
  const int64_t threads = k.wgm * k.wgn * 64;
  const int64_t nmfma = (k.bm / k.wgm / 32) * (k.bn / k.wgn / 32); // per 16-deep k step
  const int64_t lpt = (k.bm * (k.bk / 8) + k.bk * (k.bn / 8)) / threads;
  s.loadsPerThread = lpt;
  if (k.out == kInstOutF32Partial && !k.epi && k.mfma == TB_MFMA_32X32X16 && producerTile(k)) {
    // the loaders issue with the compute waves' thread count: wave w - NW
    // issues wave w's loads
    s.issue = "producer_waves";
    s.loaderWaves = k.wgm * k.wgn;
    s.prologueTailLoads = lpt;
    s.vmPrologue = (k.stages - 1) * lpt;
    s.vmLoop = (k.stages - 2) * lpt;
    s.lgkmLoop = -1;
    return s;
  }
  if (nmfma >= 4) {
    s.issue = "slot_spread";
    const int64_t nslot = (k.bk / 16) * nmfma, after = nmfma / 2;
    s.refillSpreadSlots = k.stages >= 3 ? nslot : nmfma;
    for (int64_t l = 0; l < lpt; ++l) // load l goes refillSpreadSlots * l / lpt slots in
      s.prologueTailLoads += s.refillSpreadSlots * l / lpt < after ? 1 : 0;
  } else {
    s.issue = "burst";
    s.prologueTailLoads = lpt;
  }
  s.vmPrologue = (k.stages - 2) * lpt + s.prologueTailLoads;
  s.vmLoop = (k.stages - 2) * lpt;
  s.lgkmLoop = -1;
  return s;
}

std::vector<std::pair<std::pair<int64_t, int64_t>, int64_t>>
compiledWaveGrids(int64_t bm, int64_t bn, int64_t bk) {
  std::vector<std::pair<std::pair<int64_t, int64_t>, int64_t>> v;
  for (const Tile &t : kTiles)
    if (t.bm == bm && t.bn == bn && t.bk == bk)
      v.push_back({{t.wgm, t.wgn}, t.stages});
  std::sort(v.begin(), v.end(), [](const auto &a, const auto &b) {
    return std::make_tuple(a.first.first * a.first.second, a.first.first, a.second) <
           std::make_tuple(b.first.first * b.first.second, b.first.first, b.second);
  });
  return v;
}

} // namespace tb
