// C++ unit tests of the plan derivations (the derive* functions of
// mini_triton_nvgpu_v1_amd/csrc/plan), called directly rather than through
// tb-opt. Each check states a value fixed outside the code under test: the
// reference's own lit expectations, the published Triton program order,
// closed forms, or the compiled instance table. Built and run by
// tests/test_cpp_plans.py; prints one line per failure and exits non-zero.
#include "ir/ir.h"
#include "plan/instances.h"
#include "plan/plans.h"

#include <cstdio>
#include <functional>
#include <set>
#include <string>
#include <tuple>

using namespace tb;

static int failures = 0, checks = 0;
#define CHECK(cond)                                                                \
  do {                                                                             \
    ++checks;                                                                      \
    if (!(cond)) {                                                                 \
      ++failures;                                                                  \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);                  \
    }                                                                              \
  } while (0)
#define CHECK_EQ(a, b)                                                             \
  do {                                                                             \
    ++checks;                                                                      \
    const auto va_ = (a);                                                          \
    const auto vb_ = (b);                                                          \
    if (!(va_ == vb_)) {                                                           \
      ++failures;                                                                  \
      std::printf("FAIL %s:%d: %s == %s (%lld vs %lld)\n", __FILE__, __LINE__, #a, \
                  #b, (long long)va_, (long long)vb_);                             \
    }                                                                              \
  } while (0)

static bool throws(const std::function<void()> &f, const std::string &needle = "") {
  try {
    f();
  } catch (const Error &e) {
    return needle.empty() || std::string(e.what()).find(needle) != std::string::npos;
  }
  return false;
}

// A tb.matmul module as the reference's lit tests write them.
static std::string module(int64_t M, int64_t N, int64_t K, int64_t bm, int64_t bn,
                          int64_t bk, int64_t warps, int64_t stages, bool exact,
                          const std::string &extraModule = "", const std::string &c = "f16") {
  char buf[2048];
  std::snprintf(buf, sizeof buf,
                "module attributes {\"tb.num-warps\" = %lld : i64, \"tb.requested-stages\" = "
                "%lld : i64%s} {\n"
                "  func.func @kernel(%%A: memref<%lldx%lldxf16>, %%B: memref<%lldx%lldxf16>, "
                "%%C: memref<%lldx%lldx%s>) {\n"
                "    tb.matmul %%A, %%B, %%C {block_m = %lld : i64, block_n = %lld : i64, "
                "block_k = %lld : i64, exact_tile = %s}\n"
                "      : memref<%lldx%lldxf16>, memref<%lldx%lldxf16>, memref<%lldx%lldx%s>\n"
                "    func.return\n  }\n}\n",
                (long long)warps, (long long)stages, extraModule.c_str(), (long long)M,
                (long long)K, (long long)K, (long long)N, (long long)M, (long long)N, c.c_str(),
                (long long)bm, (long long)bn, (long long)bk, exact ? "true" : "false",
                (long long)M, (long long)K, (long long)K, (long long)N, (long long)M,
                (long long)N, c.c_str());
  return buf;
}

struct Planned {
  Module m;
  KernelConfig c;
  TargetInfo t;
  ProgramMappingPlan pm;
};
static Planned plan(const std::string &text) {
  Planned p{parseModule(text), {}, deriveTargetInfoForArch("gfx950", ""), {}};
  const Op &op = p.m.funcs.at(0).body.at(0);
  p.c = getKernelConfig(p.m, op);
  p.pm = deriveProgramMappingPlan(p.m, p.c, p.t);
  return p;
}

// build -> print -> parse -> build gives the same text
template <class P, class B, class R>
static bool roundTrips(const P &plan, B build, R parse) {
  const AttrP a = build(plan);
  const std::string text = print(a);
  const AttrP again = build(parse(*a));
  return print(again) == text;
}

static void targetInfo() {
  const TargetInfo t = deriveTargetInfoForArch("gfx950", "");
  CHECK_EQ(t.threadsPerWarp, 64);
  CHECK_EQ(t.numSms, 256);
  CHECK_EQ(t.maxSharedBytesPerCTA, 160 * 1024);
  CHECK_EQ(t.sharedBankCount, 64);
  CHECK_EQ(t.sharedBankBytes, 4);
  CHECK_EQ(t.numXcds, 8);
  CHECK(!t.supportsLdMatrix && !t.supportsMmaSync && t.supportsMfma);
  std::set<std::vector<int64_t>> shapes(t.mfmaInstrShapes.begin(), t.mfmaInstrShapes.end());
  CHECK(shapes.count({16, 16, 32}) == 1 && shapes.count({32, 32, 16}) == 1);
  CHECK(roundTrips(t, buildTargetInfoAttr, parseTargetInfoAttr));
  CHECK(throws([] { deriveTargetInfoForArch("sm_80", ""); }));
}

static void waveGrid() {
  // (block_m, block_n, waves) -> grid: the reference's two-warp lit test
  // (two_warp_shape_closure_contract.mlir:14-15, warp_grid = [2, 1]) and the
  // grids the compiled instance names carry
  const std::tuple<int64_t, int64_t, int64_t, int64_t, int64_t> cases[] = {
      {64, 64, 2, 2, 1},    {256, 256, 4, 2, 2},  {128, 64, 8, 4, 2},
      {128, 64, 4, 4, 1},   {64, 128, 4, 1, 4},   {128, 128, 4, 2, 2},
      {256, 256, 8, 4, 2},  {64, 64, 4, 2, 2},    {256, 128, 8, 4, 2}};
  for (const auto &[bm, bn, w, gm, gn] : cases) {
    KernelConfig c;
    c.blockM = bm;
    c.blockN = bn;
    c.blockK = 64;
    c.numWarps = w;
    const auto g = deriveWaveGrid(c, 32, 32);
    CHECK_EQ(g.first, gm);
    CHECK_EQ(g.second, gn);
    CHECK_EQ(g.first * g.second, w);
  }
}

// Triton's grouped program order (the published tutorial formula the
// reference lowers, LowerPipelineToNVGPU.cpp:286-305)
static void tritonGrouped(int64_t pid, int64_t tm, int64_t tn, int64_t gm, int64_t &m,
                          int64_t &n) {
  const int64_t inGroup = gm * tn, group = pid / inGroup, first = group * gm;
  const int64_t size = std::min(tm - first, gm);
  m = first + (pid % inGroup) % size;
  n = (pid % inGroup) / size;
}

static void programMapping() {
  // grouped: 4096^3 on 256x256 tiles, GROUP_M 8 (16 x 16 tiles)
  {
    Planned p = plan(module(4096, 4096, 4096, 256, 256, 64, 4, 2, true));
    CHECK(p.pm.mappingKind == ProgramMappingKind::GroupedTile);
    CHECK_EQ(p.pm.totalPrograms, 256);
    CHECK_EQ(p.pm.problemTilesK, 64);
    std::set<std::pair<int64_t, int64_t>> seen;
    bool same = true;
    for (int64_t pid = 0; pid < p.pm.totalPrograms; ++pid) {
      int64_t tm, tn, part, m, n;
      programToTile(p.pm, pid, tm, tn, part);
      tritonGrouped(pid, 16, 16, 8, m, n);
      same = same && tm == m && tn == n && part == 0;
      seen.insert({tm, tn});
    }
    CHECK(same);
    CHECK_EQ((int64_t)seen.size(), 256);
    CHECK(roundTrips(p.pm, buildProgramMappingPlanAttr, parseProgramMappingPlanAttr));
  }
  // ragged grouped, a last group shorter than GROUP_M: 9 x 5 tiles
  {
    Planned p = plan(module(9 * 64 - 3, 5 * 64 - 8, 128, 64, 64, 32, 4, 2, false));
    CHECK_EQ(p.pm.problemTilesM, 9);
    CHECK_EQ(p.pm.problemTilesN, 5);
    bool same = true;
    std::set<std::pair<int64_t, int64_t>> seen;
    for (int64_t pid = 0; pid < p.pm.totalPrograms; ++pid) {
      int64_t tm, tn, part, m, n;
      programToTile(p.pm, pid, tm, tn, part);
      tritonGrouped(pid, 9, 5, p.pm.groupM, m, n);
      same = same && tm == m && tn == n;
      seen.insert({tm, tn});
    }
    CHECK(same);
    CHECK_EQ((int64_t)seen.size(), 45);
  }
  // split-K 512^2 x 16384, 8 splits of 128x64 tiles: m = pid / (tilesN S),
  // n = (pid % (tilesN S)) / S, part = pid % S (LowerPipelineToNVGPU.cpp:306-317)
  {
    Planned p = plan(module(512, 512, 16384, 128, 64, 64, 8, 3, true,
                            ", \"tb.split-k\" = 8 : i64, \"tb.reduction-mode\" = "
                            "\"split_k_serial\""));
    CHECK(p.pm.mappingKind == ProgramMappingKind::SplitK);
    CHECK_EQ(p.pm.totalPrograms, 4 * 8 * 8);
    bool same = true;
    for (int64_t pid = 0; pid < p.pm.totalPrograms; ++pid) {
      int64_t tm, tn, part;
      programToTile(p.pm, pid, tm, tn, part);
      same = same && tm == pid / 64 && tn == (pid % 64) / 8 && part == pid % 8;
    }
    CHECK(same);
    const ReductionPlan r = deriveReductionPlan(p.c, p.pm);
    CHECK(r.kind == ReductionPlanKind::SplitKSerial);
    // scratch of one tile's partials per split (ReductionPlan.cpp:158-169)
    CHECK_EQ(r.scratchBytes, 128 * 64 * 4 * 8);
    CHECK_EQ(r.kTilesPerProgram, 32);
    CHECK_EQ(r.remainderKTiles, 0);
    CHECK(roundTrips(r, buildReductionPlanAttr, parseReductionPlanAttr));
  }
  // persistent 8192^3: resident = min(num CTAs, CUs), stride = resident
  // (PersistentWorkPlan.cpp:113-122)
  {
    Planned p = plan(module(8192, 8192, 8192, 256, 256, 64, 4, 2, true,
                            ", \"tb.persistent\" = true, \"tb.num-ctas\" = 300 : i64"));
    const PersistentWorkPlan w = derivePersistentWorkPlan(p.c, p.t, p.pm);
    CHECK(w.enabled);
    CHECK_EQ(w.residentPrograms, 256);
    CHECK_EQ(w.loopStride, 256);
    CHECK_EQ(w.totalWorkItems, 32 * 32);
    CHECK_EQ(w.maxTilesPerProgram, 4);
    CHECK(roundTrips(w, buildPersistentWorkPlanAttr, parsePersistentWorkPlanAttr));
  }
}

static void semanticsAndEncoding() {
  // ragged 96x80 on 64x64 tiles: boundary flags (MatmulSemantics.cpp:234-236)
  {
    Planned p = plan(module(96, 80, 32, 64, 64, 32, 4, 2, false));
    const MatmulSemantics s = deriveMatmulSemantics(p.c, p.m.funcs[0].body[0]);
    CHECK(s.hasBoundaryM && s.hasBoundaryN && !s.hasBoundaryK);
    CHECK(roundTrips(s, buildMatmulSemanticsAttr, parseMatmulSemanticsAttr));
  }
  // exact_tile with a non-divisible shape is refused (KernelConfig.cpp:230-237)
  CHECK(throws([] {
    Planned p = plan(module(96, 80, 32, 64, 64, 32, 4, 2, true));
    verifySupportedKernelConfig(p.c, &p.t);
  }));
  // 4096^3 on the 16x16x32 instance: B's LDS encoding carries the second XOR
  // term (32-byte units, phase (k / 8) % 2) that makes the transposing reads
  // conflict-free; A's is the single 16-byte term over 128-byte rows
  {
    Planned p = plan(module(4096, 4096, 4096, 256, 256, 64, 4, 2, true));
    CHECK(p.c.mmaKind == MmaKind::Mfma16x16x32F16);
    const MatmulSemantics s = deriveMatmulSemantics(p.c, p.m.funcs[0].body[0]);
    const EncodingPlan e = deriveEncodingPlan(p.c, p.t, s, p.pm);
    const SharedSwizzle b = sharedSwizzle(encodingAttr(e, e.bShared, "b shared"));
    CHECK_EQ(b.secondPerPhase, 8);
    CHECK_EQ(b.secondMaxPhase, 2);
    CHECK_EQ(b.secondSwizzlingByteWidth, 32);
    const SharedSwizzle a = sharedSwizzle(encodingAttr(e, e.aShared, "a shared"));
    CHECK(a.secondMaxPhase <= 1);
    CHECK_EQ(a.perPhase * 64 * 2, 256); // rows per 256-byte bank period
    CHECK_EQ(a.maxPhase, 8);            // 16-byte chunks per 128-byte row
    CHECK(mmaWarpsPerCTA(e) == (I64s{2, 2}));
    CHECK(roundTrips(e, buildEncodingPlanAttr, parseEncodingPlanAttr));
    const TransportPlan tr = deriveTransportPlan(p.c, p.t, e);
    CHECK_EQ(tr.operandA.asyncVectorBytes, 16);
    CHECK_EQ(tr.operandB.asyncVectorBytes, 16);
    CHECK(roundTrips(tr, buildTransportPlanAttr, parseTransportPlanAttr));
  }
  // any M, N and K take the 16x16x32 instance on its tile; 8 waves do not
  CHECK(plan(module(1000, 1496, 712, 256, 256, 64, 4, 2, false)).c.mmaKind ==
        MmaKind::Mfma16x16x32F16);
  CHECK(plan(module(4096, 4096, 4096, 256, 256, 64, 8, 2, true)).c.mmaKind ==
        MmaKind::Mfma32x32x16F16);
}

static void instances() {
  // the 16x16x32 instance's waits: 16 loads per lane per k-tile, the prologue
  // waits for k-tile 0 with k-tile 1 in flight, each barrier for everything
  InstanceKey k16{256, 256, 64, 2, 2, 0, 2, 0, 1};
  CHECK(hasGfx950Instance(k16));
  const InstanceSchedule s16 = instanceSchedule(k16);
  CHECK_EQ(s16.loadsPerThread, 16);
  CHECK_EQ(s16.vmPrologue, 16);
  CHECK_EQ(s16.vmLoop, 0);
  CHECK_EQ(s16.lgkmLoop, 0);
  // the split-K tile's f32-partial instance is the producer-wave build: 8
  // load-only waves, 3 loads per lane per k-tile, all 3 k-tiles issued in the
  // prologue, (S - 2) k-tiles in flight at each barrier
  InstanceKey k3{128, 64, 64, 4, 2, kInstOutF32Partial, 3, 0, TB_MFMA_32X32X16};
  CHECK(hasGfx950Instance(k3));
  const InstanceSchedule s3 = instanceSchedule(k3);
  CHECK(s3.issue == "producer_waves");
  CHECK_EQ(s3.loaderWaves, 8);
  CHECK_EQ(s3.loadsPerThread, 3);
  CHECK_EQ(s3.vmPrologue, (3 - 1) * s3.loadsPerThread);
  CHECK_EQ(s3.vmLoop, (3 - 2) * s3.loadsPerThread);
  // the same tile's f16 and C += A*B instances keep the general loop (32x32
  // wave tiles: burst refills), with the same waits and no loader waves
  for (int out : {kInstOutF16, kInstOutF32Accum}) {
    InstanceKey kg = k3;
    kg.out = out;
    const InstanceSchedule sg = instanceSchedule(kg);
    CHECK(sg.issue == "burst");
    CHECK_EQ(sg.loaderWaves, 0);
    CHECK_EQ(sg.vmPrologue, s3.vmPrologue);
    CHECK_EQ(sg.vmLoop, s3.vmLoop);
  }
  // the output mode the plan derives for each (mapping, reduction, C, init)
  CHECK_EQ(instanceOutOf(true, false, true, false), kInstOutF32Partial);
  CHECK_EQ(instanceOutOf(true, true, false, true), kInstOutF32Atomic);
  CHECK_EQ(instanceOutOf(false, false, true, false), kInstOutF16);
  CHECK_EQ(instanceOutOf(false, false, false, false), kInstOutF32Partial);
  CHECK_EQ(instanceOutOf(false, false, false, true), kInstOutF32Accum);
  // every listed instance names its shape and is unique
  std::set<std::string> names;
  for (const InstanceKey &k : gfx950Instances())
    names.insert(instanceName(k));
  CHECK_EQ(names.size(), gfx950Instances().size());
  CHECK(names.count("tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32_epi") == 1);
  CHECK(names.count("tb_gemm_gfx950_128x64x64_w4x2_s3_out1") == 1);
}

int main() {
  const std::pair<const char *, void (*)()> groups[] = {
      {"target info", targetInfo},
      {"wave grid", waveGrid},
      {"program mapping, reduction, persistent work", programMapping},
      {"semantics, encoding, transport", semanticsAndEncoding},
      {"instances", instances}};
  for (const auto &[name, f] : groups) {
    const int before = failures;
    try {
      f();
    } catch (const std::exception &e) {
      ++failures;
      std::printf("FAIL %s: unexpected exception: %s\n", name, e.what());
    }
    std::printf("%-46s %s\n", name, failures == before ? "ok" : "FAILED");
  }
  std::printf("%d checks, %d failures\n", checks, failures);
  return failures ? 1 : 0;
}
