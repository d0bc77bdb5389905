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
// the 16x16x32 loop's tiles (besides the hand-scheduled 256x256x64 one)
#define TB_M16_SHAPE_TILES(SHAPE) TBK_M16_TILES_##SHAPE(TB_TILE),
const Tile kM16Tiles[] = {TBK_M16_SHAPES(TB_M16_SHAPE_TILES)};
#undef TB_M16_SHAPE_TILES
#undef TB_TILE

// the hand-scheduled 16x16x32 instance: 4 waves of 128x128 on 256x256x64, 2 stages
bool handScheduled16(int64_t bm, int64_t bn, int64_t bk, int64_t wgm, int64_t wgn,
                     int64_t stages) {
  return bm == 256 && bn == 256 && bk == 64 && wgm == 2 && wgn == 2 && stages == 2;
}

// Mfma16GTile's issue schedule, restated (gemm_mfma16g.h): loads per thread,
// the refill's spread over the MFMA slots of a loop body
struct M16Geometry {
  int64_t lpt, spread;
};
M16Geometry m16Geometry(const InstanceKey &k) {
  const int64_t nt = k.wgm * k.wgn * 64;
  const int64_t lpt = (k.bm * k.bk * 2 + k.bk * k.bn * 2) / (nt * 16);
  const int64_t nm = (k.bm / k.wgm / 16) * (k.bn / k.wgn / 16), nslot = (k.bk / 32) * nm;
  return {lpt, k.stages == 2 ? nslot * 5 / 8 : nslot - nslot / 8};
}
} // namespace

bool hasMfma16Tile(int64_t bm, int64_t bn, int64_t bk, int64_t wgm, int64_t wgn,
                   int64_t stages) {
  if (handScheduled16(bm, bn, bk, wgm, wgn, stages))
    return true;
  for (const Tile &t : kM16Tiles)
    if (t.bm == bm && t.bn == bn && t.bk == bk && t.wgm == wgm && t.wgn == wgn &&
        t.stages == stages)
      return true;
  return false;
}

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
    // 16x16x32: f16 C, plain f32 C and f32 C += A*B (no split-K), the
    // hand-scheduled 256x256x64 tile and the 16x16x32 loop's tiles
    for (int out = kInstOutF16; out <= kInstOutF32Accum; ++out)
      for (int epi = 0; epi <= 1; ++epi)
        v.push_back({256, 256, 64, 2, 2, out, 2, epi, TB_MFMA_16X16X32});
    for (const Tile &t : kM16Tiles)
      for (int epi = 0; epi <= 1; ++epi)
        for (int out = kInstOutF16; out <= kInstOutF32Accum; ++out)
          v.push_back({t.bm, t.bn, t.bk, t.wgm, t.wgn, out, t.stages, epi, TB_MFMA_16X16X32});
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
  if (k.mfma == TB_MFMA_16X16X32 && !handScheduled16(k.bm, k.bn, k.bk, k.wgm, k.wgn, k.stages)) {
    // the 16x16x32 loop: the prologue issues every stage's k-tile whole;
    // each barrier waits for the next k-tile and for this wave's LDS reads,
    // then the freed stage is refilled, its loads spread over the body
    const M16Geometry g = m16Geometry(k);
    s.issue = "tile16_slots";
    s.loadsPerThread = g.lpt;
    s.prologueTailLoads = g.lpt;
    s.refillSpreadSlots = g.spread;
    s.vmPrologue = (k.stages - 1) * g.lpt;
    s.vmLoop = (k.stages - 2) * g.lpt;
    s.lgkmLoop = 0;
    return s;
  }
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
  // whole load rounds per operand; a last round wider than the operand's
  // stage leaves whole waves idle (they load zeros into a scratch row)
  const int64_t lpt = (k.bm * (k.bk / 8) + threads - 1) / threads +
                      (k.bk * (k.bn / 8) + threads - 1) / threads;
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

namespace {
struct ResourceRow {
  const char *family;
  std::vector<int> args;
  int vgprs, agprs, sgprs, scratch;
};
const ResourceRow kResources[] = {
#include "instance_resources.inc"
};

// The rows of the builds key k binds: the general loop's gemm_kernel (or the
// producer-wave build that replaces its f32-partial entry), or the 16x16x32
// instance with its partial-K build.
bool rowBinds(const ResourceRow &r, const InstanceKey &k, bool partialK) {
  const std::string f = r.family;
  const auto &a = r.args;
  if (k.mfma == TB_MFMA_16X16X32) {
    // the hand-scheduled tile runs whole k-tiles; a partial last k-tile
    // runs the 16x16x32 loop's build of the same tile
    if (handScheduled16(k.bm, k.bn, k.bk, k.wgm, k.wgn, k.stages) && !partialK) {
      if (f == "gemm_mfma16" && k.out == kInstOutF16)
        return a.size() == 1 && a[0] == k.epi;
      if (f == "gemm_mfma16_f32" && k.out != kInstOutF16)
        return a.size() == 2 && a[0] == k.out && a[1] == k.epi;
      return false;
    }
    return f == "gemm_mfma16g" && a.size() == 8 && a[0] == k.bm && a[1] == k.bn &&
           a[2] == k.bk && a[3] == k.wgm && a[4] == k.wgn && a[5] == k.stages &&
           a[6] == k.out && a[7] == k.epi;
  }
  if (k.out == kInstOutF32Partial && !k.epi && producerTile(k))
    return f == "gemm_kernel_pw" && a.size() == 6 && a[0] == k.bm && a[1] == k.bn &&
           a[2] == k.bk && a[3] == k.wgm && a[4] == k.wgn && a[5] == k.stages;
  return f == "gemm_kernel" && a.size() == 9 && a[0] == k.bm && a[1] == k.bn &&
         a[2] == k.bk && a[3] == k.wgm && a[4] == k.wgn && a[5] == k.out &&
         a[6] == k.stages && a[8] == k.epi;
}

std::string familyName(const ResourceRow &r) {
  std::string s = std::string(r.family) + "<";
  for (size_t i = 0; i < r.args.size(); ++i)
    s += (i ? ", " : "") + std::to_string(r.args[i]);
  return s + ">";
}
} // namespace

InstanceResources instanceResources(const InstanceKey &k, bool partialK) {
  InstanceResources res;
  for (const ResourceRow &r : kResources) {
    if (!rowBinds(r, k, partialK))
      continue;
    if (!res.known || r.scratch > res.scratchBytes ||
        (r.scratch == res.scratchBytes && r.vgprs + r.agprs > res.vgprs + res.agprs))
      res.kernel = familyName(r);
    res.known = true;
    res.vgprs = std::max<int64_t>(res.vgprs, r.vgprs);
    res.agprs = std::max<int64_t>(res.agprs, r.agprs);
    res.sgprs = std::max<int64_t>(res.sgprs, r.sgprs);
    res.scratchBytes = std::max<int64_t>(res.scratchBytes, r.scratch);
  }
  return res;
}

std::string spillRefusal(const InstanceKey &k, bool partialK) {
  const InstanceResources r = instanceResources(k, partialK);
  if (!r.known || r.scratchBytes == 0)
    return "";
  return "gfx950 kernel instance " + instanceName(k) +
         (partialK ? " (its build for a partial last k-tile)" : "") + " spills " +
         std::to_string(r.scratchBytes) + " bytes per lane to scratch (" +
         std::to_string(r.vgprs) + " VGPRs, " + std::to_string(r.agprs) +
         " AGPRs per wave, compiler report of " + r.kernel +
         "): the wave tile does not fit the registers of one wave; use more waves or a "
         "smaller block";
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
