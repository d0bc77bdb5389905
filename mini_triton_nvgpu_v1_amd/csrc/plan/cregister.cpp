// The C-register family: AccumulatorPlan, EpiloguePlan, EpilogueReorderPlan,
// SharedWorkspacePlan, WarpDecompositionPlan and ResourceClosurePlan.
#include "serialize.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>

namespace tb {

namespace {
struct WaveGeom {
  int64_t gm, gn, wtM, wtN, tm, tn, iM, iN;
};
WaveGeom waveGeom(const KernelConfig &c, const EncodingPlan &e) {
  I64s w = mmaWarpsPerCTA(e);
  if (w.size() != 2 || w[0] * w[1] != c.numWarps)
    throw Error("MFMA encoding wave grid disagrees with num_warps");
  WaveGeom g;
  g.gm = w[0];
  g.gn = w[1];
  g.wtM = c.blockM / g.gm;
  g.wtN = c.blockN / g.gn;
  g.iM = e.fragmentAcc.instructionShape.at(0);
  g.iN = e.fragmentAcc.instructionShape.at(1);
  g.tm = g.wtM / g.iM;
  g.tn = g.wtN / g.iN;
  return g;
}
} // namespace

// ---- AccumulatorPlan ---------------------------------------------------------------
template <class V> void fields(V &v, AccumulatorPack &p) {
  v("pack_id", p.packId);
  v("row_base", p.rowBase);
  v("col_base", p.colBase);
  v("rows", p.rows);
  v("cols", p.cols);
  v("elem_count", p.elemCount);
  v("vector_width", p.vectorWidth);
  v("warp_owner", p.warpOwner);
  v("mma_group", p.mmaGroup);
  v("epilogue_pack", p.epiloguePack);
}
template <class V> void fields(V &v, AccumulatorPlan &p) {
  v("encoding", p.encoding);
  v("registers_per_warp", p.registersPerWarp);
  v("owner_scope", p.ownerScope);
  v("lane_access", p.laneAccess);
  v("packs", p.packs);
  v("live_across_stages", p.liveAcrossStages);
  v("multi_buffer_depth", p.multiBufferDepth);
}

// Reference: AccumulatorPlan.cpp:193-252 (one pack per MMA tile of the wave
// template). gfx950: one pack per 32x32 MFMA tile; each lane holds 16 f32
// (registers_per_warp counts the per-lane accumulator VGPRs of one wave) as
// 4 runs of 4 consecutive columns 8 apart, on row lane % 32.
AccumulatorPlan deriveAccumulatorPlan(const KernelConfig &c, const TargetInfo &t,
                                      const EncodingPlan &e) {
  WaveGeom g = waveGeom(c, e);
  AccumulatorPlan p;
  p.encoding = e.acc;
  int64_t perTile = g.iM * g.iN / t.threadsPerWarp;
  p.registersPerWarp = g.tm * g.tn * perTile;
  p.laneAccess = {g.iM, 4, 8, {0}};
  for (int64_t i = 0; i < g.tm; ++i)
    for (int64_t j = 0; j < g.tn; ++j) {
      AccumulatorPack k;
      k.packId = i * g.tn + j;
      k.rowBase = i * g.iM;
      k.colBase = j * g.iN;
      k.rows = g.iM;
      k.cols = g.iN;
      k.elemCount = perTile;
      k.vectorWidth = 4;
      k.warpOwner = 0;
      k.mmaGroup = k.packId;
      k.epiloguePack = k.packId;
      p.packs.push_back(k);
    }
  p.liveAcrossStages = true;
  p.multiBufferDepth = 1;
  if (p.registersPerWarp > t.maxRegistersPerThread / 2)
    throw Error("accumulator tile needs " + std::to_string(p.registersPerWarp) +
                " VGPRs per lane, more than half the register file");
  return p;
}
AttrP buildAccumulatorPlanAttr(const AccumulatorPlan &p) { return buildPlanAttr(p); }
AccumulatorPlan parseAccumulatorPlanAttr(const Attr &a) {
  return parsePlanAttr<AccumulatorPlan>(a, "`tb.accumulator_plan`");
}

// ---- EpiloguePlan ----------------------------------------------------------------
template <class V> void fields(V &v, DirectPack &p) {
  v("pack_id", p.packId);
  v("row_base", p.rowBase);
  v("col_base", p.colBase);
  v("rows", p.rows);
  v("cols", p.cols);
  v("vector_width", p.vectorWidth);
  v("warp_owner", p.warpOwner);
  v("fragment_ids", p.fragmentIds);
}
template <class V> void fields(V &v, DirectGlobalVectorPlan &p) {
  v("present", p.present);
  v("owner_scope", p.ownerScope);
  v("lane_access", p.laneAccess);
  v("packs", p.packs);
  v("vector_width", p.vectorWidth);
  v("boundary_aware", p.boundaryAware);
  v("scalar_tail", p.scalarTail);
}
template <class V> void fields(V &v, EpilogueExprOp &p) {
  v("kind", p.kind);
  v("input_scalar", p.inputScalar);
  v("output_scalar", p.outputScalar);
  v("vector_width", p.vectorWidth);
  v("aux", p.aux);
}
template <class V> void fields(V &v, TargetLandingPlan &p) {
  v("kind", p.kind);
  v("global_vector_width", p.globalVectorWidth);
  v("global_access_bytes", p.globalAccessBytes);
  v("producer_fragment_rows", p.producerFragmentRows);
  v("producer_fragment_cols", p.producerFragmentCols);
  v("direct_pack_rows", p.directPackRows);
  v("direct_pack_cols", p.directPackCols);
  v("warp_batching_group", p.warpBatchingGroup);
  v("required_shared_bytes", p.requiredSharedBytes);
  v("expected_register_footprint", p.expectedRegisterFootprint);
  v("shared_tile_rows", p.sharedTileRows);
  v("shared_tile_cols", p.sharedTileCols);
  v("shared_pack_slots", p.sharedPackSlots);
  v("init_shared_store_vector_width", p.initSharedStoreVectorWidth);
  v("init_shared_load_vector_width", p.initSharedLoadVectorWidth);
  v("store_shared_store_vector_width", p.storeSharedStoreVectorWidth);
  v("store_shared_load_vector_width", p.storeSharedLoadVectorWidth);
  v("use_shared_pack_for_init", p.useSharedPackForInit);
  v("use_shared_pack_for_store", p.useSharedPackForStore);
  v("required_sync_kind", p.requiredSyncKind);
  v("reason", p.reason);
}
template <class V> void fields(V &v, EpiloguePlan &p) {
  v("init_mode", p.initMode);
  v("store_mode", p.storeMode);
  v("init", p.init);
  v("store", p.store);
  v("target_landing", p.targetLanding);
  v("exprs", p.exprs);
}

// Reference: EpiloguePlan.cpp:864-1109 (direct global vectors landed from
// register packs). gfx950: every lane owns 4 consecutive columns of one row
// per 32x32 tile and group, so the store is 4-wide straight from registers
// (8 bytes of f16 or 16 bytes of f32 per lane). N is a multiple of 8, hence a
// 4-column vector is either wholly inside or wholly outside the problem and
// the boundary is handled per vector by the buffer store's range check (no
// scalar tail). The C contract follows the output type: an f32 C accumulates
// onto its prior contents (C += A B, the reference's semantics, init by a
// direct vector load), an f16 C receives cast(A B) (init zero, one f32 -> f16
// convert).
// ---- fused epilogue exprs ------------------------------------------------------
static const char *const kActivations[] = {"relu", "gelu_tanh", "silu"};

static bool knownActivation(const std::string &s) {
  for (const char *a : kActivations)
    if (s == a)
      return true;
  return false;
}

// Clamp bounds travel in the Clamp expr's `aux` as `min=<v>,max=<v>` (either
// part optional), each printed with enough digits to read back the f32 value.
static std::string clampAux(const EpilogueRequest &r) {
  char buf[96];
  std::string s;
  if (r.hasMin) {
    snprintf(buf, sizeof buf, "min=%.9g", r.clampMin);
    s += buf;
  }
  if (r.hasMax) {
    snprintf(buf, sizeof buf, "%smax=%.9g", s.empty() ? "" : ",", r.clampMax);
    s += buf;
  }
  return s;
}

static void checkRequest(const EpilogueRequest &r) {
  if (!r.bias.empty() && r.bias != "f16" && r.bias != "f32")
    throw Error("`epilogue_bias` must be \"f16\" or \"f32\", got \"" + r.bias + "\"");
  if (!r.activation.empty() && !knownActivation(r.activation))
    throw Error("`epilogue_activation` must be one of \"relu\", \"gelu_tanh\", "
                "\"silu\", got \"" + r.activation + "\"");
  if ((r.hasMin && !std::isfinite(r.clampMin)) || (r.hasMax && !std::isfinite(r.clampMax)))
    throw Error("epilogue clamp bounds must be finite");
  if (r.hasMin && r.hasMax && r.clampMin > r.clampMax)
    throw Error("`epilogue_clamp_min` must not exceed `epilogue_clamp_max`");
}

EpilogueRequest parseEpilogueRequest(const Op &op) {
  EpilogueRequest r;
  auto str = [&](const char *name, std::string &out) {
    auto it = op.attrs.find(name);
    if (it == op.attrs.end())
      return;
    if (it->second->kind != AttrKind::String)
      throw Error(std::string("`") + name + "` must be a string attribute");
    out = it->second->s;
  };
  auto num = [&](const char *name, bool &has, double &out) {
    auto it = op.attrs.find(name);
    if (it == op.attrs.end())
      return;
    if (it->second->kind == AttrKind::Float)
      out = it->second->f;
    else if (it->second->kind == AttrKind::Int)
      out = (double)it->second->i;
    else
      throw Error(std::string("`") + name + "` must be a float attribute");
    out = (double)(float)out; // the kernels clamp in f32
    has = true;
  };
  str("epilogue_bias", r.bias);
  str("epilogue_activation", r.activation);
  num("epilogue_clamp_min", r.hasMin, r.clampMin);
  num("epilogue_clamp_max", r.hasMax, r.clampMax);
  checkRequest(r);
  return r;
}

EpilogueRequest epilogueRequestOf(const EpiloguePlan &p) {
  EpilogueRequest r;
  // canonical order: LoadBias, Add, Activation, Clamp, Convert
  int stage = 0;
  auto order = [&](int s, const char *what) {
    if (s < stage)
      throw Error(std::string("epilogue expr `") + what +
                  "` is out of order (load_bias, add, activation, clamp, convert)");
    stage = s;
  };
  bool loaded = false, added = false;
  for (const EpilogueExprOp &x : p.exprs) {
    switch (x.kind) {
    case EpilogueExprKind::LoadBias:
      order(0, "load_bias");
      if (loaded || (x.inputScalar != ScalarKind::F16 && x.inputScalar != ScalarKind::F32))
        throw Error("epilogue load_bias must appear once, reading f16 or f32");
      r.bias = x.inputScalar == ScalarKind::F16 ? "f16" : "f32";
      loaded = true;
      break;
    case EpilogueExprKind::Add:
      order(1, "add");
      if (!loaded || added || x.aux != "bias")
        throw Error("epilogue add must follow load_bias and add the bias");
      added = true;
      break;
    case EpilogueExprKind::Activation:
      order(2, "activation");
      if (!r.activation.empty() || !knownActivation(x.aux))
        throw Error("epilogue activation `" + x.aux + "` is not supported on gfx950");
      r.activation = x.aux;
      break;
    case EpilogueExprKind::Clamp: {
      order(3, "clamp");
      if (r.hasMin || r.hasMax)
        throw Error("epilogue clamp must appear once");
      size_t pos = 0;
      while (pos < x.aux.size()) {
        size_t end = x.aux.find(',', pos);
        if (end == std::string::npos)
          end = x.aux.size();
        const std::string part = x.aux.substr(pos, end - pos);
        const bool isMin = part.rfind("min=", 0) == 0, isMax = part.rfind("max=", 0) == 0;
        if (!isMin && !isMax)
          throw Error("epilogue clamp aux `" + x.aux + "` is not `min=<v>,max=<v>`");
        char *stop = nullptr;
        const double v = strtod(part.c_str() + 4, &stop);
        if (stop == part.c_str() + 4 || *stop)
          throw Error("epilogue clamp aux `" + x.aux + "` holds a bad number");
        (isMin ? r.hasMin : r.hasMax) = true;
        (isMin ? r.clampMin : r.clampMax) = v;
        pos = end + 1;
      }
      if (!r.hasMin && !r.hasMax)
        throw Error("epilogue clamp names neither bound");
      break;
    }
    case EpilogueExprKind::Convert:
      order(4, "convert");
      break;
    }
  }
  if (loaded != added)
    throw Error("epilogue load_bias and add come as a pair");
  checkRequest(r);
  return r;
}

EpiloguePlan deriveEpiloguePlan(const KernelConfig &c, const TargetInfo &,
                                const EncodingPlan &e, const AccumulatorPlan &a,
                                const EpilogueRequest &req) {
  checkRequest(req);
  WaveGeom g = waveGeom(c, e);
  bool boundary = c.problemM % c.blockM != 0 || c.problemN % c.blockN != 0;
  DirectGlobalVectorPlan dv;
  dv.present = true;
  dv.ownerScope = "per_warp_template";
  dv.laneAccess = a.laneAccess;
  dv.vectorWidth = 4;
  dv.boundaryAware = boundary;
  dv.scalarTail = false;
  for (const AccumulatorPack &k : a.packs)
    dv.packs.push_back({k.packId, k.rowBase, k.colBase, k.rows, k.cols, 4, 0,
                        {k.mmaGroup}});
  EpiloguePlan p;
  p.storeMode = AccumulatorStoreMode::DirectGlobalVector;
  p.store = dv;
  if (c.cScalar == ScalarKind::F32) {
    p.initMode = AccumulatorInitMode::DirectGlobalVector;
    p.init = dv;
  } else {
    p.initMode = AccumulatorInitMode::Zero;
    p.init.present = false;
    p.init.ownerScope = "none";
  }
  // fused steps on the f32 accumulator, 4 columns per lane at a time
  auto expr = [&](EpilogueExprKind k, ScalarKind in, const std::string &aux) {
    EpilogueExprOp x;
    x.kind = k;
    x.inputScalar = in;
    x.outputScalar = ScalarKind::F32;
    x.vectorWidth = 4;
    x.aux = aux;
    p.exprs.push_back(x);
  };
  if (!req.bias.empty()) {
    expr(EpilogueExprKind::LoadBias,
         req.bias == "f16" ? ScalarKind::F16 : ScalarKind::F32, "bias");
    expr(EpilogueExprKind::Add, ScalarKind::F32, "bias");
  }
  if (!req.activation.empty())
    expr(EpilogueExprKind::Activation, ScalarKind::F32, req.activation);
  if (req.hasMin || req.hasMax)
    expr(EpilogueExprKind::Clamp, ScalarKind::F32, clampAux(req));
  if (c.cScalar != ScalarKind::F32) {
    EpilogueExprOp cvt;
    cvt.kind = EpilogueExprKind::Convert;
    cvt.inputScalar = ScalarKind::F32;
    cvt.outputScalar = ScalarKind::F16;
    cvt.vectorWidth = 4;
    cvt.aux = "round_to_nearest_even";
    p.exprs.push_back(cvt);
  }
  TargetLandingPlan &l = p.targetLanding;
  l.kind = TargetLandingKind::RegisterPackGlobalVector;
  l.globalVectorWidth = 4;
  l.globalAccessBytes = 4 * scalarBytes(c.cScalar);
  l.producerFragmentRows = g.iM;
  l.producerFragmentCols = g.iN;
  l.directPackRows = 1;
  l.directPackCols = 4;
  l.warpBatchingGroup = 1;
  l.expectedRegisterFootprint = a.registersPerWarp;
  l.requiredSyncKind = "none";
  l.reason = "MFMA accumulator lanes own 4 consecutive columns of a row, so C lands "
             "from registers as 4-wide global vectors without an LDS relay";
  return p;
}
AttrP buildEpiloguePlanAttr(const EpiloguePlan &p) { return buildPlanAttr(p); }
EpiloguePlan parseEpiloguePlanAttr(const Attr &a) {
  return parsePlanAttr<EpiloguePlan>(a, "`tb.epilogue_plan`");
}

// ---- EpilogueReorderPlan -------------------------------------------------------
template <class V> void fields(V &v, EpilogueRowVectorMapping &p) {
  v("row_vector_id", p.rowVectorId);
  v("pack_id", p.packId);
  v("warp_owner", p.warpOwner);
  v("row_base", p.rowBase);
  v("col_base", p.colBase);
  v("row_offset", p.rowOffset);
  v("vector_width", p.vectorWidth);
  v("fragment_ids", p.fragmentIds);
}
template <class V> void fields(V &v, EpilogueReorderPlan &p) {
  v("kind", p.kind);
  v("shared_tile_rows", p.sharedTileRows);
  v("shared_tile_cols", p.sharedTileCols);
  v("live_slots", p.liveSlots);
  v("init_shared_store_vector_width", p.initSharedStoreVectorWidth);
  v("init_shared_load_vector_width", p.initSharedLoadVectorWidth);
  v("store_shared_store_vector_width", p.storeSharedStoreVectorWidth);
  v("store_shared_load_vector_width", p.storeSharedLoadVectorWidth);
  v("workspace_barrier_count", p.workspaceBarrierCount);
  v("requires_warp_sync", p.requiresWarpSync);
  v("reorder_needed_for_init", p.reorderNeededForInit);
  v("reorder_needed_for_store", p.reorderNeededForStore);
  v("owner_scope", p.ownerScope);
  v("workspace_sync_kind", p.workspaceSyncKind);
  v("reason", p.reason);
  v("row_vectors", p.rowVectors);
}

// Reference: EpilogueReorderPlan.cpp:214-304 (a workgroup-shared row reorder
// when the tile is ragged and the direct vector width differs from the
// fragment width). On gfx950 the direct vector width equals the accumulator's
// per-lane run (4), so no reorder is needed for any tile shape.
EpilogueReorderPlan deriveEpilogueReorderPlan(const KernelConfig &,
                                              const AccumulatorPlan &a,
                                              const EpiloguePlan &e) {
  EpilogueReorderPlan p;
  int64_t fragmentWidth = a.laneAccess.laneColGroupSize;
  if (e.store.vectorWidth != fragmentWidth)
    throw Error("gfx950 epilogue requires the direct vector width to equal the "
                "accumulator lane run");
  p.kind = EpilogueReorderKind::None;
  p.ownerScope = "none";
  p.workspaceSyncKind = "none";
  p.reason = "direct vector width equals the MFMA accumulator lane run; boundary "
             "vectors are dropped by the buffer range check, no reorder needed";
  return p;
}
AttrP buildEpilogueReorderPlanAttr(const EpilogueReorderPlan &p) { return buildPlanAttr(p); }
EpilogueReorderPlan parseEpilogueReorderPlanAttr(const Attr &a) {
  return parsePlanAttr<EpilogueReorderPlan>(a, "`tb.epilogue_reorder_plan`");
}

// ---- SharedWorkspacePlan -------------------------------------------------------
template <class V> void fields(V &v, SharedWorkspaceSegment &s) {
  v("kind", s.kind);
  v("name", s.name);
  v("byte_offset", s.byteOffset);
  v("byte_size", s.byteSize);
  v("byte_alignment", s.byteAlignment);
  v("logical_rows", s.logicalRows);
  v("logical_cols", s.logicalCols);
  v("stage_count", s.stageCount);
  v("slot_count", s.slotCount);
  v("warp_replicas", s.warpReplicas);
  v("lifetime_begin", s.lifetimeBegin);
  v("lifetime_end", s.lifetimeEnd);
  v("alias_allowed", s.aliasAllowed);
  v("alias_set", s.aliasSet);
  v("producer", s.producer);
  v("consumer", s.consumer);
}
template <class V> void fields(V &v, SharedWorkspacePlan &p) {
  v("contract_model", p.contractModel);
  v("total_bytes", p.totalBytes);
  v("peak_bytes", p.peakBytes);
  v("alias_saved_bytes", p.aliasSavedBytes);
  v("selected_policy", p.selectedPolicy);
  v("reason", p.reason);
  v("segments", p.segments);
}

// Reference: SharedWorkspacePlan.cpp:195-386. gfx950 LDS layout: a ring of
// `stages` slots, slot s at s * (A_stage + B_stage) bytes holding the A tile
// [block_m][block_k] followed by the B tile [block_k][block_n]. No epilogue
// scratch (no reorder) and the split-k partials live in global memory.
SharedWorkspacePlan deriveSharedWorkspacePlan(
    const KernelConfig &c, const TargetInfo &t, const EncodingPlan &,
    const TransportPlan &tr, const EpilogueReorderPlan &ro, const ReductionPlan &rd,
    const PersistentWorkPlan &) {
  if (ro.kind != EpilogueReorderKind::None)
    throw Error("gfx950 workspace has no epilogue reorder scratch");
  if (rd.scratchSpace == ReductionScratchSpace::Shared)
    throw Error("gfx950 split-k keeps partials in global memory");
  SharedWorkspacePlan p;
  p.contractModel = "cta_shared_workspace_v1";
  int64_t aBytes = tr.operandA.transactionBytes, bBytes = tr.operandB.transactionBytes;
  int64_t slot = aBytes + bBytes;
  int64_t S = c.requestedStages;
  for (int64_t s = 0; s < S; ++s) {
    for (int op = 0; op < 2; ++op) {
      SharedWorkspaceSegment g;
      g.kind = op == 0 ? SharedWorkspaceSegmentKind::MainloopAStageBuffer
                       : SharedWorkspaceSegmentKind::MainloopBStageBuffer;
      g.name = std::string(op == 0 ? "a" : "b") + "_stage" + std::to_string(s);
      g.byteOffset = s * slot + (op == 0 ? 0 : aBytes);
      g.byteSize = op == 0 ? aBytes : bBytes;
      g.byteAlignment = 16;
      g.logicalRows = op == 0 ? c.blockM : c.blockK;
      g.logicalCols = op == 0 ? c.blockK : c.blockN;
      g.stageCount = 1;
      g.slotCount = 1;
      g.warpReplicas = 1;
      g.lifetimeBegin = 0;
      g.lifetimeEnd = 1;
      g.aliasAllowed = false;
      g.aliasSet = -1;
      g.producer = "buffer_load_dwordx4_lds";
      g.consumer = op == 0 ? "ds_read_b128" : "ds_read_b64_tr_b16";
      p.segments.push_back(g);
    }
  }
  p.totalBytes = S * slot;
  p.peakBytes = p.totalBytes;
  p.aliasSavedBytes = 0;
  p.selectedPolicy = "single_cta_workspace_stage_ring";
  p.reason = "A/B stage ring only: the epilogue lands from registers and split-k "
             "partials go to a global workspace";
  if (p.totalBytes > t.maxSharedBytesPerCTA)
    throw Error("shared workspace (" + std::to_string(p.totalBytes) +
                " bytes) exceeds the target LDS budget");
  return p;
}
AttrP buildSharedWorkspacePlanAttr(const SharedWorkspacePlan &p) { return buildPlanAttr(p); }
SharedWorkspacePlan parseSharedWorkspacePlanAttr(const Attr &a) {
  return parsePlanAttr<SharedWorkspacePlan>(a, "`tb.shared_workspace_plan`");
}

// ---- WarpDecompositionPlan -----------------------------------------------------
template <class V> void fields(V &v, WarpTileCoverage &w) {
  v("warp_id", w.warpId);
  v("coord_m", w.coordM);
  v("coord_n", w.coordN);
  v("tile_base_m", w.tileBaseM);
  v("tile_base_n", w.tileBaseN);
  v("tile_rows", w.tileRows);
  v("tile_cols", w.tileCols);
  v("mma_group_ids", w.mmaGroupIds);
  v("accumulator_pack_ids", w.accumulatorPackIds);
  v("epilogue_pack_ids", w.epiloguePackIds);
  v("shared_pack_ids", w.sharedPackIds);
  v("reorder_row_vector_ids", w.reorderRowVectorIds);
  v("fragment_to_row_vector_map", w.fragmentToRowVectorMap);
  v("row_vector_store_order", w.rowVectorStoreOrder);
  v("row_vector_load_order", w.rowVectorLoadOrder);
  v("reorder_tile_base", w.reorderTileBase);
  v("reorder_needs_shared", w.reorderNeedsShared);
  v("reduction_partial_ids", w.reductionPartialIds);
  v("persistent_batch_ids", w.persistentBatchIds);
}
template <class V> void fields(V &v, WarpDecompositionPlan &p) {
  v("cta_tile", p.ctaTile);
  v("num_warps", p.numWarps);
  v("warp_grid", p.warpGrid);
  v("warp_tile", p.warpTile);
  v("owner_scope", p.ownerScope);
  v("warp_order", p.warpOrder);
  v("landing_owner", p.landingOwner);
  v("reorder_owner", p.reorderOwner);
  v("reduction_owner", p.reductionOwner);
  v("persistent_owner", p.persistentOwner);
  v("warps", p.warps);
}

// Reference: WarpDecompositionPlan.cpp:268-424. Wave w covers the wave tile
// at grid coordinate (w / grid_n, w % grid_n), row-major like the kernels.
WarpDecompositionPlan deriveWarpDecompositionPlan(
    const KernelConfig &c, const EncodingPlan &e, const AccumulatorPlan &a,
    const EpiloguePlan &, const EpilogueReorderPlan &ro, const ReductionPlan &rd,
    const PersistentWorkPlan &pw) {
  WaveGeom g = waveGeom(c, e);
  WarpDecompositionPlan p;
  p.ctaTile = {c.blockM, c.blockN};
  p.numWarps = c.numWarps;
  p.warpGrid = {g.gm, g.gn};
  p.warpTile = {g.wtM, g.wtN};
  p.landingOwner = "register_pack";
  p.reorderOwner = ro.kind == EpilogueReorderKind::None ? "none" : enumName(ro.kind);
  p.reductionOwner = rd.kind == ReductionPlanKind::None ? "none" : enumName(rd.kind);
  p.persistentOwner = pw.enabled ? pw.ownerScope : "none";
  I64s packIds;
  for (const AccumulatorPack &k : a.packs)
    packIds.push_back(k.packId);
  for (int64_t w = 0; w < c.numWarps; ++w) {
    WarpTileCoverage cv;
    cv.warpId = w;
    cv.coordM = w / g.gn;
    cv.coordN = w % g.gn;
    cv.tileBaseM = cv.coordM * g.wtM;
    cv.tileBaseN = cv.coordN * g.wtN;
    cv.tileRows = g.wtM;
    cv.tileCols = g.wtN;
    cv.mmaGroupIds = packIds;
    cv.accumulatorPackIds = packIds;
    cv.epiloguePackIds = packIds;
    if (rd.kind != ReductionPlanKind::None)
      cv.reductionPartialIds = packIds;
    if (pw.enabled)
      cv.persistentBatchIds = {0};
    p.warps.push_back(cv);
  }
  return p;
}
AttrP buildWarpDecompositionPlanAttr(const WarpDecompositionPlan &p) { return buildPlanAttr(p); }
WarpDecompositionPlan parseWarpDecompositionPlanAttr(const Attr &a) {
  return parsePlanAttr<WarpDecompositionPlan>(a, "`tb.warp_decomposition_plan`");
}

// ---- ResourceClosurePlan -------------------------------------------------------
template <class V> void fields(V &v, ResourceClosurePlan &p) {
  v("estimated_accumulator_regs", p.estimatedAccumulatorRegs);
  v("estimated_epilogue_regs", p.estimatedEpilogueRegs);
  v("estimated_ab_shared", p.estimatedABShared);
  v("estimated_epilogue_shared", p.estimatedEpilogueShared);
  v("estimated_reduction_scratch", p.estimatedReductionScratch);
  v("estimated_persistent_state", p.estimatedPersistentState);
  v("estimated_total_static_shared", p.estimatedTotalStaticShared);
  v("estimated_total_dynamic_shared", p.estimatedTotalDynamicShared);
  v("estimated_total_regs", p.estimatedTotalRegs);
  v("peak_static_shared_bytes", p.peakStaticSharedBytes);
  v("workspace_total_bytes", p.workspaceTotalBytes);
  v("workspace_alias_saved_bytes", p.workspaceAliasSavedBytes);
  v("reorder_shared_bytes", p.reorderSharedBytes);
  v("reduction_shared_bytes", p.reductionSharedBytes);
  v("persistent_shared_bytes", p.persistentSharedBytes);
  v("mainloop_shared_live_begin", p.mainloopSharedLiveBegin);
  v("mainloop_shared_live_end", p.mainloopSharedLiveEnd);
  v("epilogue_reorder_live_begin", p.epilogueReorderLiveBegin);
  v("epilogue_reorder_live_end", p.epilogueReorderLiveEnd);
  v("static_shared_budget", p.staticSharedBudget);
  v("dynamic_shared_budget", p.dynamicSharedBudget);
  v("selected_mainline_kind", p.selectedMainlineKind);
  v("selected_c_landing_kind", p.selectedCLandingKind);
  v("selected_buffering_kind", p.selectedBufferingKind);
  v("selected_shared_workspace_policy", p.selectedSharedWorkspacePolicy);
  v("chosen_landing_tradeoff", p.chosenLandingTradeoff);
  v("chosen_buffering_tradeoff", p.chosenBufferingTradeoff);
  v("reason", p.reason);
  v("global_workspace_bytes", p.globalWorkspaceBytes);
}

// Reference: ResourceClosurePlan.cpp:100-214. Register estimate per lane:
// accumulators + two double-buffered operand fragments (8 f16 = 4 VGPRs per
// 32-row/column fragment) + ~40 for addresses, descriptors and loop state.
ResourceClosurePlan deriveResourceClosurePlan(
    const KernelConfig &c, const TargetInfo &t, const ProgramMappingPlan &pm,
    const ReductionPlan &rd, const PersistentWorkPlan &pw, const AccumulatorPlan &a,
    const EpiloguePlan &, const EpilogueReorderPlan &, const SharedWorkspacePlan &sw,
    const WarpDecompositionPlan &wd) {
  ResourceClosurePlan p;
  int64_t tm = wd.warpTile.at(0) / 32, tn = wd.warpTile.at(1) / 32;
  p.estimatedAccumulatorRegs = a.registersPerWarp;
  p.estimatedEpilogueRegs = 4;
  p.estimatedABShared = sw.totalBytes;
  p.estimatedTotalStaticShared = sw.totalBytes;
  p.estimatedTotalRegs = a.registersPerWarp + 2 * (tm + tn) * 4 + 40;
  p.peakStaticSharedBytes = sw.peakBytes;
  p.workspaceTotalBytes = sw.totalBytes;
  p.workspaceAliasSavedBytes = sw.aliasSavedBytes;
  p.mainloopSharedLiveBegin = 0;
  p.mainloopSharedLiveEnd = 1;
  p.staticSharedBudget = t.maxSharedBytesPerCTA;
  p.dynamicSharedBudget = 0;
  switch (pm.mappingKind) {
  case ProgramMappingKind::PersistentTile:
    p.selectedMainlineKind = "persistent_tile_loop";
    break;
  case ProgramMappingKind::SplitK:
    p.selectedMainlineKind = "split_k";
    break;
  case ProgramMappingKind::GroupedTile:
    p.selectedMainlineKind = "grouped_tile";
    break;
  case ProgramMappingKind::Tile:
    p.selectedMainlineKind = "single_tile";
    break;
  }
  p.selectedCLandingKind = "register_direct_vector";
  p.selectedBufferingKind = "async_ab_plus_register_epilogue";
  p.selectedSharedWorkspacePolicy = sw.selectedPolicy;
  p.chosenLandingTradeoff = "MFMA lane runs of 4 columns store directly; no LDS relay";
  p.chosenBufferingTradeoff = std::to_string(c.requestedStages) +
                              "-slot direct-to-LDS ring ordered by vmcnt + barrier";
  p.globalWorkspaceBytes = rd.kind == ReductionPlanKind::SplitKSerial
                               ? rd.splitK * c.problemM * c.problemN * 4
                               : 0;
  p.reason = pw.enabled ? "persistent workgroups loop over tiles with the same "
                          "per-tile resources"
                        : "one workgroup per program";
  if (p.estimatedTotalStaticShared > p.staticSharedBudget)
    throw Error("static LDS exceeds the gfx950 budget");
  if (p.estimatedTotalRegs > t.maxRegistersPerThread)
    throw Error("estimated " + std::to_string(p.estimatedTotalRegs) +
                " VGPRs per lane exceed the gfx950 register file");
  return p;
}
AttrP buildResourceClosurePlanAttr(const ResourceClosurePlan &p) { return buildPlanAttr(p); }
ResourceClosurePlan parseResourceClosurePlanAttr(const Attr &a) {
  return parsePlanAttr<ResourceClosurePlan>(a, "`tb.resource_closure_plan`");
}

} // namespace tb
