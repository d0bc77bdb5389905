// ProgramMappingPlan, ReductionPlan and PersistentWorkPlan.
#include "serialize.h"

#include <algorithm>

namespace tb {

// ---- ProgramMappingPlan ---------------------------------------------------------
template <class V> void fields(V &v, ProgramMappingPlan &p) {
  v("mapping_kind", p.mappingKind);
  v("problem_tiles_m", p.problemTilesM);
  v("problem_tiles_n", p.problemTilesN);
  v("problem_tiles_k", p.problemTilesK);
  v("tile_m", p.tileM);
  v("tile_n", p.tileN);
  v("tile_k", p.tileK);
  v("group_m", p.groupM);
  v("group_tile_span_m", p.groupTileSpanM);
  v("group_tile_span_n", p.groupTileSpanN);
  v("programs_per_launch_group", p.programsPerLaunchGroup);
  v("launch_group_count", p.launchGroupCount);
  v("total_programs", p.totalPrograms);
  v("split_k", p.splitK);
  v("launch_order", p.launchOrder);
  v("swizzle_kind", p.swizzleKind);
  v("persistent", p.persistent);
  v("reduction_mode", p.reductionMode);
  v("programs_per_tile", p.programsPerTile);
  v("num_ctas", p.numCTAs);
  v("ctas_per_cga", p.ctasPerCGA);
  v("cta_split_num", p.ctaSplitNum);
  v("cta_order", p.ctaOrder);
  v("xcd_remap", p.xcdRemap);
}

// Invariants of the launch formula (reference ProgramMappingPlan.cpp:219-324).
static void validateProgramMappingPlan(const ProgramMappingPlan &p) {
  if (p.problemTilesM <= 0 || p.problemTilesN <= 0 || p.problemTilesK <= 0)
    throw Error("program mapping requires positive tile coverage on M/N/K");
  if (p.groupM <= 0 || p.groupTileSpanM <= 0 || p.groupTileSpanN <= 0 ||
      p.programsPerLaunchGroup <= 0 || p.launchGroupCount <= 0)
    throw Error("program mapping requires positive launch-group geometry");
  if (p.programsPerLaunchGroup != p.groupTileSpanM * p.groupTileSpanN)
    throw Error("programs_per_launch_group must equal group span M x N");
  int64_t tiles = p.problemTilesM * p.problemTilesN;
  switch (p.mappingKind) {
  case ProgramMappingKind::Tile:
  case ProgramMappingKind::PersistentTile:
  case ProgramMappingKind::GroupedTile:
    if (p.totalPrograms != tiles)
      throw Error("total_programs must equal tiles_m x tiles_n");
    break;
  case ProgramMappingKind::SplitK:
    if (p.totalPrograms != tiles * p.splitK || p.programsPerTile != p.splitK)
      throw Error("split-k mapping must launch split_k programs per tile");
    if (p.splitK > p.problemTilesK)
      throw Error("split_k must not exceed the number of k tiles");
    break;
  }
  if (p.mappingKind == ProgramMappingKind::GroupedTile &&
      p.launchGroupCount != ceilDiv(p.problemTilesM, p.groupM))
    throw Error("grouped mapping must cover tiles_m in ceil(tiles_m / group_m) groups");
  if (p.persistent != (p.mappingKind == ProgramMappingKind::PersistentTile))
    throw Error("persistent flag and mapping kind disagree");
  if (p.numCTAs <= 0)
    throw Error("num_ctas must be positive");
  if (p.xcdRemap < 0)
    throw Error("xcd_remap must be non-negative");
}

static int64_t moduleI64Or(const Module &m, const char *name, int64_t dflt) {
  AttrP a = m.attr(name);
  if (!a)
    return dflt;
  if (a->kind != AttrKind::Int)
    throw Error(std::string("module attr `") + name + "` must be an integer");
  return a->i;
}

// Reference: ProgramMappingPlan.cpp:389-444 (kind precedence persistent >
// split-k > grouped > tile). gfx950 differences: a persistent launch keeps
// the grouped-M order when group_m > 1 (the reference forces group_m = 1),
// resident programs are capped at the 256 CUs, and launches with more tiles
// than CUs remap program ids so that consecutive programs share an XCD (each
// of the 8 XCDs has its own L2).
ProgramMappingPlan deriveProgramMappingPlan(const Module &m, const KernelConfig &c,
                                            const TargetInfo &t) {
  ProgramMappingPlan p;
  int64_t numCTAs = moduleI64Or(m, kNumCTAs, 1);
  int64_t splitK = moduleI64Or(m, kSplitK, 1);
  int64_t ppt = moduleI64Or(m, kProgramsPerTile, 0);
  bool persistent = false;
  if (AttrP a = m.attr(kPersistent)) {
    if (a->kind != AttrKind::Bool)
      throw Error(std::string("module attr `") + kPersistent + "` must be a bool");
    persistent = a->b;
  }
  std::string redMode;
  if (AttrP a = m.attr(kReductionMode)) {
    if (a->kind != AttrKind::String)
      throw Error(std::string("module attr `") + kReductionMode + "` must be a string");
    redMode = a->s;
  }
  p.problemTilesM = ceilDiv(c.problemM, c.blockM);
  p.problemTilesN = ceilDiv(c.problemN, c.blockN);
  p.problemTilesK = ceilDiv(c.problemK, c.blockK);
  p.tileM = c.blockM;
  p.tileN = c.blockN;
  p.tileK = c.blockK;
  p.groupM = std::max<int64_t>(1, c.groupM);
  p.splitK = splitK;
  p.persistent = persistent;
  p.numCTAs = numCTAs;
  if (splitK <= 0)
    throw Error(std::string("module attr `") + kSplitK + "` must be positive");
  if (numCTAs <= 0)
    throw Error(std::string("module attr `") + kNumCTAs + "` must be positive");
  if (persistent && splitK != 1)
    throw Error("stage1 does not allow persistent and split-k in the same "
                "program mapping contract yet");
  int64_t tiles = p.problemTilesM * p.problemTilesN;
  bool groupable = p.groupM > 1 && p.problemTilesM > 1 && p.problemTilesN > 1;
  auto rowMajor = [&] {
    p.groupM = 1;
    p.groupTileSpanM = 1;
    p.groupTileSpanN = p.problemTilesN;
    p.launchGroupCount = p.problemTilesM;
    p.launchOrder = ProgramLaunchOrder::RowMajor;
    p.swizzleKind = ProgramSwizzleKind::None;
  };
  auto grouped = [&] {
    p.groupTileSpanM = p.groupM;
    p.groupTileSpanN = p.problemTilesN;
    p.launchGroupCount = ceilDiv(p.problemTilesM, p.groupM);
    p.launchOrder = ProgramLaunchOrder::GroupedM;
    p.swizzleKind = ProgramSwizzleKind::GroupedM;
  };
  if (persistent) {
    p.mappingKind = ProgramMappingKind::PersistentTile;
    groupable ? grouped() : rowMajor();
    p.launchOrder = ProgramLaunchOrder::Persistent;
    p.totalPrograms = tiles;
    p.programsPerTile = 1;
    p.reductionMode = ReductionMode::None;
    p.numCTAs = std::min({p.numCTAs, p.totalPrograms, t.numSms});
  } else if (splitK > 1) {
    p.mappingKind = ProgramMappingKind::SplitK;
    rowMajor();
    p.groupTileSpanN = p.problemTilesN * splitK;
    p.totalPrograms = tiles * splitK;
    p.programsPerTile = splitK;
    if (redMode.empty() || redMode == "split_k_serial")
      p.reductionMode = ReductionMode::SplitKSerial;
    else if (redMode == "split_k_parallel")
      p.reductionMode = ReductionMode::SplitKParallel;
    else
      throw Error(std::string("module attr `") + kReductionMode +
                  "` must be `split_k_serial` or `split_k_parallel`");
  } else if (groupable) {
    p.mappingKind = ProgramMappingKind::GroupedTile;
    grouped();
    p.totalPrograms = tiles;
  } else {
    p.mappingKind = ProgramMappingKind::Tile;
    rowMajor();
    p.totalPrograms = tiles;
  }
  if (ppt > 0 && p.mappingKind != ProgramMappingKind::SplitK && ppt != 1)
    throw Error(std::string("module attr `") + kProgramsPerTile +
                "` other than 1 requires split-k");
  p.programsPerLaunchGroup = p.groupTileSpanM * p.groupTileSpanN;
  p.ctasPerCGA = {p.numCTAs, 1, 1};
  p.ctaSplitNum = {1, 1, 1};
  p.ctaOrder = {0, 1, 2};
  // XCD-aware program order once the output tiles fill the CUs: each XCD
  // (own L2) then works a compact block of tiles instead of every 8th one
  // (4096^3 on 256 tiles: ~0.7% faster). Split-K keeps the plain order, in
  // which each XCD holds one split's K range of A and B.
  p.xcdRemap = tiles >= t.numSms && t.numXcds > 1 &&
                       p.mappingKind != ProgramMappingKind::SplitK
                   ? t.numXcds
                   : 0;
  validateProgramMappingPlan(p);
  return p;
}

AttrP buildProgramMappingPlanAttr(const ProgramMappingPlan &p) { return buildPlanAttr(p); }
ProgramMappingPlan parseProgramMappingPlanAttr(const Attr &a) {
  auto p = parsePlanAttr<ProgramMappingPlan>(a, "`tb.program_mapping_plan`");
  validateProgramMappingPlan(p);
  return p;
}

// Program id -> (tile_m, tile_n, split part). Reference:
// LowerPipelineToNVGPU.cpp:286-317 (the Triton grouped formula and the
// split-k row-major formula); the gfx950 kernels evaluate the same integer
// expressions (persistent programs feed their work index through it).
void programToTile(const ProgramMappingPlan &p, int64_t pid, int64_t &tm,
                   int64_t &tn, int64_t &part) {
  if (p.mappingKind == ProgramMappingKind::SplitK) {
    int64_t ppg = p.problemTilesN * p.splitK;
    tm = pid / ppg;
    tn = (pid % ppg) / p.splitK;
    part = (pid % ppg) % p.splitK;
    return;
  }
  int64_t gm = p.swizzleKind == ProgramSwizzleKind::GroupedM ? p.groupM : 1;
  int64_t ppg = gm * p.problemTilesN;
  int64_t first = (pid / ppg) * gm;
  int64_t gsz = std::min(gm, p.problemTilesM - first);
  tm = first + (pid % ppg) % gsz;
  tn = (pid % ppg) / gsz;
  part = 0;
}

// ---- ReductionPlan ----------------------------------------------------------------
template <class V> void fields(V &v, ReductionPlan &p) {
  v("kind", p.kind);
  v("scratch_space", p.scratchSpace);
  v("split_k", p.splitK);
  v("k_tiles_per_program", p.kTilesPerProgram);
  v("remainder_k_tiles", p.remainderKTiles);
  v("partial_tile_rows", p.partialTileRows);
  v("partial_tile_cols", p.partialTileCols);
  v("producer_programs_per_tile", p.producerProgramsPerTile);
  v("final_reducer_programs", p.finalReducerPrograms);
  v("scratch_rows", p.scratchRows);
  v("scratch_cols", p.scratchCols);
  v("scratch_bytes", p.scratchBytes);
  v("requires_inter_program_reduction", p.requiresInterProgramReduction);
  v("partial_owner", p.partialOwner);
  v("final_executor", p.finalExecutor);
  v("reason", p.reason);
}

// Reference: ReductionPlan.cpp:136-193. gfx950: the serial mode becomes a
// deterministic two-kernel reduction (each split writes an f32 partial tile
// to a global workspace, then one reduce kernel sums the partials in split
// order and casts); the parallel mode accumulates with f32 global atomics and
// therefore needs an f32 C.
ReductionPlan deriveReductionPlan(const KernelConfig &c, const ProgramMappingPlan &pm) {
  ReductionPlan p;
  p.partialTileRows = c.blockM;
  p.partialTileCols = c.blockN;
  p.kTilesPerProgram = pm.problemTilesK;
  p.reason = "single-program workgroup fully owns the K reduction for each tile";
  if (pm.splitK <= 1)
    return p;
  p.splitK = pm.splitK;
  p.kTilesPerProgram = ceilDiv(pm.problemTilesK, p.splitK);
  p.remainderKTiles = pm.problemTilesK % p.splitK;
  p.producerProgramsPerTile = pm.programsPerTile;
  p.finalReducerPrograms = 1;
  p.requiresInterProgramReduction = true;
  p.partialOwner = "per_program_partial_tile";
  p.scratchSpace = ReductionScratchSpace::Global;
  p.scratchRows = c.blockM;
  p.scratchCols = c.blockN;
  p.scratchBytes = c.blockM * c.blockN * 4 * p.splitK;
  switch (pm.reductionMode) {
  case ReductionMode::SplitKSerial:
    p.kind = ReductionPlanKind::SplitKSerial;
    p.finalExecutor = "deterministic_workspace_reduce";
    p.reason = "split-k serial writes one f32 partial tile per split to a global "
               "workspace and a reduce kernel sums them in split order";
    break;
  case ReductionMode::SplitKParallel:
    if (c.cScalar != ScalarKind::F32)
      throw Error("split_k_parallel reduces with f32 global atomics and needs an "
                  "f32 C; use split_k_serial for an f16 C");
    p.kind = ReductionPlanKind::SplitKAtomic;
    p.scratchSpace = ReductionScratchSpace::None;
    p.scratchBytes = 0;
    p.finalExecutor = "global_atomic_accumulate";
    p.reason = "split-k parallel maps multiple programs to one tile and reduces via "
               "global atomic accumulation";
    break;
  case ReductionMode::None:
    throw Error("split-k program mapping requires a reduction mode");
  }
  return p;
}
AttrP buildReductionPlanAttr(const ReductionPlan &p) { return buildPlanAttr(p); }
ReductionPlan parseReductionPlanAttr(const Attr &a) {
  return parsePlanAttr<ReductionPlan>(a, "`tb.reduction_plan`");
}

// ---- PersistentWorkPlan --------------------------------------------------------
template <class V> void fields(V &v, PersistentWorkPlan &p) {
  v("kind", p.kind);
  v("enabled", p.enabled);
  v("resident_programs", p.residentPrograms);
  v("programs_per_wave", p.programsPerWave);
  v("tile_batch_size", p.tileBatchSize);
  v("max_tiles_per_program", p.maxTilesPerProgram);
  v("total_work_items", p.totalWorkItems);
  v("loop_stride", p.loopStride);
  v("requires_outer_serial_loop", p.requiresOuterSerialLoop);
  v("tile_order", p.tileOrder);
  v("owner_scope", p.ownerScope);
  v("completion", p.completion);
  v("reason", p.reason);
}

// Reference: PersistentWorkPlan.cpp:91-133 (resident = min(num_ctas, CUs),
// stride = resident).
PersistentWorkPlan derivePersistentWorkPlan(const KernelConfig &, const TargetInfo &t,
                                            const ProgramMappingPlan &pm) {
  PersistentWorkPlan p;
  p.residentPrograms = std::max<int64_t>(pm.numCTAs, 1);
  p.programsPerWave = p.residentPrograms;
  p.totalWorkItems = std::max<int64_t>(pm.totalPrograms, 1);
  p.loopStride = p.residentPrograms;
  p.reason = "single-tile workgroup launch keeps one program per tile";
  if (!pm.persistent)
    return p;
  p.kind = PersistentWorkKind::TileStrideLoop;
  p.enabled = true;
  p.residentPrograms = std::max<int64_t>(1, std::min(pm.numCTAs, t.numSms));
  p.programsPerWave = p.residentPrograms;
  p.tileBatchSize = std::max<int64_t>(1, pm.programsPerTile);
  p.loopStride = p.residentPrograms;
  p.maxTilesPerProgram = ceilDiv(p.totalWorkItems, p.residentPrograms);
  p.requiresOuterSerialLoop = true;
  p.tileOrder = pm.swizzleKind == ProgramSwizzleKind::GroupedM ? "grouped_m" : "row_major";
  p.ownerScope = "cta_persistent_loop";
  p.completion = "exhaust_program_stride";
  p.reason = "persistent launch keeps resident workgroups fixed and advances each "
             "program through a tile stride loop";
  return p;
}
AttrP buildPersistentWorkPlanAttr(const PersistentWorkPlan &p) { return buildPlanAttr(p); }
PersistentWorkPlan parsePersistentWorkPlanAttr(const Attr &a) {
  return parsePlanAttr<PersistentWorkPlan>(a, "`tb.persistent_work_plan`");
}

} // namespace tb
