// KernelContract: the public plan attributes of a sealed tb.pipeline_mainline,
// its verifier, and its flattening into the gfx950 launch configuration.
#include "contract.h"
#include "instances.h"
#include "serialize.h"

#include <algorithm>
#include <numeric>
#include <set>
#include <tuple>

namespace tb {

// Reference: KernelContract.cpp:9-65 (every plan parsed back from the op).
KernelContract parseKernelContract(const Module &m, const Op &op) {
  KernelContract k;
  AttrP target = m.attr(kTarget);
  if (!target)
    throw Error("module is missing `tb.target` (run tb-attach-target-info)");
  k.target = parseTargetInfoAttr(*target);
  k.kernel = getKernelConfig(m, op);
  k.semantics = parseMatmulSemanticsAttr(opAttr(op, "tb.semantic_matmul"));
  k.programMapping = parseProgramMappingPlanAttr(opAttr(op, "tb.program_mapping_plan"));
  k.reduction = parseReductionPlanAttr(opAttr(op, "tb.reduction_plan"));
  k.persistentWork = parsePersistentWorkPlanAttr(opAttr(op, "tb.persistent_work_plan"));
  k.encodings = parseEncodingPlanAttr(opAttr(op, "tb.encoding_plan"));
  k.transport = parseTransportPlanAttr(opAttr(op, "tb.transport_plan"));
  k.rewrite = parseMatmulRewritePlanAttr(opAttr(op, "tb.matmul_rewrite"));
  k.buffers = parseBufferModelAttr(opAttr(op, "tb.buffer_model"));
  k.pipelineReady = parsePipelineReadyAttr(opAttr(op, "tb.pipeline_ready"));
  k.async = parseAsyncPlanAttr(opAttr(op, "tb.async_plan"));
  k.accumulator = parseAccumulatorPlanAttr(opAttr(op, "tb.accumulator_plan"));
  k.epilogue = parseEpiloguePlanAttr(opAttr(op, "tb.epilogue_plan"));
  k.epilogueReorder =
      parseEpilogueReorderPlanAttr(opAttr(op, "tb.epilogue_reorder_plan"));
  k.sharedWorkspace =
      parseSharedWorkspacePlanAttr(opAttr(op, "tb.shared_workspace_plan"));
  k.warpDecomposition =
      parseWarpDecompositionPlanAttr(opAttr(op, "tb.warp_decomposition_plan"));
  k.resourceClosure =
      parseResourceClosurePlanAttr(opAttr(op, "tb.resource_closure_plan"));
  return k;
}

static void require(bool ok, const std::string &msg) {
  if (!ok)
    throw Error("pipeline mainline contract: " + msg);
}

// Reference: VerifyPipelineMainlineContract.cpp:183-470. Checks the sealed
// op against its own plans: body clusters vs. buffer-model ops and async
// groups, waits after issues, slot reuse after the last read, program
// mapping / reduction / persistent agreement, LDS and register budgets.
void verifyMainlineContract(const Module &m, const Op &op, const KernelContract &k) {
  const KernelConfig &c = k.kernel;
  verifySupportedKernelConfig(c, &k.target);
  require(op.hasRegion, "tb.pipeline_mainline must own a body");
  // --- body clusters
  std::map<int64_t, std::tuple<int64_t, int64_t, int64_t>> opPos; // id -> (stage, cluster, idx)
  std::set<int64_t> issuedGroups;
  std::map<int64_t, int64_t> groupOfProducer;
  for (const AsyncProducer &p : k.async.producers)
    groupOfProducer[p.opId] = p.groupId;
  int64_t expectOrdinal = 0;
  std::pair<int64_t, int64_t> last{-1, -1};
  for (const Op &cl : op.region) {
    const char *want = cl.name == "tb.async_issue_cluster"     ? "issue"
                       : cl.name == "tb.consumer_wait_cluster" ? "wait"
                       : cl.name == "tb.mma_compute_cluster"   ? "mma"
                                                               : nullptr;
    require(want != nullptr, "unexpected op `" + cl.name + "` in the mainline body");
    Attr d;
    d.kind = AttrKind::Dict;
    d.dict = cl.attrs;
    int64_t ordinal = getI64(d, "ordinal"), stage = getI64(d, "stage"),
            cluster = getI64(d, "cluster"), kg = getI64(d, "k_group");
    require(ordinal == expectOrdinal++, "cluster ordinals must be dense and ordered");
    require(std::make_pair(stage, cluster) > last,
            "clusters must be strictly ordered by (stage, cluster)");
    last = {stage, cluster};
    I64s ids = getDense(d, "op_ids");
    require(!ids.empty(), "empty cluster");
    for (size_t i = 0; i < ids.size(); ++i) {
      int64_t id = ids[i];
      require(id >= 0 && id < (int64_t)k.buffers.ops.size(),
              "cluster names an unknown buffer-model op");
      require(!opPos.count(id), "buffer-model op scheduled twice");
      opPos[id] = {stage, cluster, (int64_t)i};
      const PipelineOp &bo = k.buffers.ops[id];
      require(iterationCoord(bo, "k_group") == kg, "cluster mixes k groups");
      PipelineOpSemanticClass sc = semanticClass(bo.kind);
      bool ok = (std::string(want) == "issue" && sc == PipelineOpSemanticClass::AsyncProducer) ||
                (std::string(want) == "wait" && sc == PipelineOpSemanticClass::SharedConsumer) ||
                (std::string(want) == "mma" && sc == PipelineOpSemanticClass::TensorCoreCompute);
      require(ok, "cluster kind disagrees with the semantic class of op " +
                      std::to_string(id));
      if (sc == PipelineOpSemanticClass::AsyncProducer)
        issuedGroups.insert(groupOfProducer.at(id));
    }
    if (std::string(want) == "wait") {
      require(getBool(d, "needs_barrier"), "gfx950 consumer waits need s_barrier");
      for (int64_t g : getDense(d, "wait_group_ids"))
        require(issuedGroups.count(g), "wait on async group " + std::to_string(g) +
                                           " before it is issued");
    }
  }
  require(opPos.size() == k.buffers.ops.size(),
          "every buffer-model op must appear in exactly one cluster");
  // --- dependencies: each op after the ops defining its inputs
  for (const PipelineOp &bo : k.buffers.ops)
    for (int64_t v : bo.inputs) {
      int64_t def = k.buffers.values.at(v).definingOp;
      auto a = opPos.at(def), b = opPos.at(bo.id);
      require(std::make_tuple(std::get<0>(a), std::get<1>(a)) <
                      std::make_tuple(std::get<0>(b), std::get<1>(b)) ||
                  (std::get<0>(a) == std::get<0>(b) && std::get<1>(a) == std::get<1>(b) &&
                   std::get<2>(a) < std::get<2>(b)),
              "op " + std::to_string(bo.id) + " scheduled before its producer");
    }
  // --- reuse fences: the refill of a slot comes after the slot's last read
  for (const ReuseFence &f : k.async.reuseFences) {
    int64_t acq = k.buffers.values.at(f.acquiringValueId).definingOp;
    auto a = opPos.at(f.afterOpId), b = opPos.at(acq);
    require(std::make_pair(std::get<0>(a), std::get<1>(a)) <
                std::make_pair(std::get<0>(b), std::get<1>(b)),
            "ring slot refilled before its last read");
  }
  // --- pipeline ready
  require(k.pipelineReady.asyncGroups == (int64_t)k.async.groups.size(),
          "pipeline_ready.async_groups disagrees with the async plan");
  require(k.pipelineReady.requestedStages == c.requestedStages,
          "pipeline_ready.requested_stages disagrees with tb.requested-stages");
  // --- mapping / reduction / persistent agreement
  const ProgramMappingPlan &pm = k.programMapping;
  require(pm.tileM == c.blockM && pm.tileN == c.blockN && pm.tileK == c.blockK,
          "program mapping tile disagrees with the semantic tile");
  require((pm.splitK > 1) == (k.reduction.kind != ReductionPlanKind::None),
          "split-k mapping and reduction plan disagree");
  require(pm.persistent == k.persistentWork.enabled,
          "persistent mapping and persistent work plan disagree");
  if (pm.persistent)
    require(k.persistentWork.residentPrograms <= k.target.numSms,
            "persistent residency exceeds the CU count");
  // --- fused epilogue: known steps in canonical order, on a whole sum
  const EpilogueRequest er = epilogueRequestOf(k.epilogue);
  require(er.empty() || k.reduction.kind != ReductionPlanKind::SplitKAtomic,
          "fused epilogue exprs cannot ride on split_k_atomic partial sums");
  const bool hasConvert =
      !k.epilogue.exprs.empty() && k.epilogue.exprs.back().kind == EpilogueExprKind::Convert;
  require(hasConvert == (c.cScalar == ScalarKind::F16),
          "an f16 C needs the f32 -> f16 convert as the last epilogue expr, an f32 C none");
  // --- resources
  require(k.sharedWorkspace.totalBytes ==
              c.requestedStages * (c.blockM + c.blockN) * c.blockK * scalarBytes(c.aScalar),
          "shared workspace must be exactly the A/B stage ring");
  require(k.resourceClosure.estimatedTotalStaticShared <= k.target.maxSharedBytesPerCTA,
          "static LDS exceeds the target budget");
  I64s wg = k.warpDecomposition.warpGrid;
  require(wg.size() == 2 && wg[0] * wg[1] == c.numWarps,
          "wave grid disagrees with tb.num-warps");
  require(mmaWarpsPerCTA(k.encodings) == wg, "MFMA encoding and wave grid disagree");
  AttrP tpw = m.attr(kThreadsPerWarp);
  require(tpw && tpw->kind == AttrKind::Int && tpw->i == k.target.threadsPerWarp,
          "tb.threads-per-warp must match the target wave size");
}

// Swizzle parameters compiled into the gfx950 kernels (A: 16-byte chunks,
// B: 64-byte segments, 256-byte bank period); the lowering refuses a plan
// whose LDS encoding differs.
static void checkKernelSwizzle(const KernelContract &k) {
  const KernelConfig &c = k.kernel;
  SharedSwizzle a = sharedSwizzle(encodingAttr(k.encodings, k.encodings.aShared, "a_shared"));
  SharedSwizzle b = sharedSwizzle(encodingAttr(k.encodings, k.encodings.bShared, "b_shared"));
  int64_t aPP = std::max<int64_t>(1, 256 / (c.blockK * 2)), aMax = c.blockK / 8;
  // B: rows per phase 256 / gcd(row bytes, 256); phases the largest power of
  // two dividing the 64-byte segments per row, at most 4 (GemmTile::B_PP,
  // B_MAXPH)
  const int64_t bSeg = c.blockN / 32;
  int64_t bPP = 256 / std::gcd<int64_t>(c.blockN * 2, 256),
          bMax = std::min<int64_t>(4, bSeg & -bSeg);
  // the 16x16x32 instance's B reads add the second XOR term (32-byte units,
  // phase (k / 8) % 2); the general loop has none
  const bool m16 = c.mmaKind == MmaKind::Mfma16x16x32F16;
  const int64_t b2pp = m16 ? 8 : 0, b2mp = m16 ? 2 : 0, b2w = m16 ? 32 : 0;
  if (a.perPhase != aPP || a.maxPhase != aMax || a.swizzlingByteWidth != 16 ||
      a.secondMaxPhase > 1 || b.perPhase != bPP || b.maxPhase != bMax ||
      b.swizzlingByteWidth != 64 || b.secondPerPhase != b2pp ||
      b.secondMaxPhase != b2mp || b.secondSwizzlingByteWidth != b2w)
    throw Error("LDS encoding of the plan differs from the swizzle compiled into "
                "the gfx950 kernels");
}

// The reference's lowering emits exactly the waits its AsyncPlan derives
// (LowerPipelineToNVGPU.cpp:2279-2294). Here the waits are compiled into
// the kernel instance, so the lowering refuses a plan whose AsyncPlan states
// other waits than the instance it binds: its issue schedule, loads per
// thread, the prologue's vmcnt (k group 0), the per-k-tile barrier's vmcnt
// (every later group) and lgkmcnt.
static void checkKernelWaits(const KernelContract &k, const InstanceKey &key) {
  const InstanceSchedule s = instanceSchedule(key);
  const AsyncPlan &a = k.async;
  auto differ = [&](const std::string &what, int64_t plan, int64_t kernel) {
    throw Error("AsyncPlan " + what + " (" + std::to_string(plan) +
                ") differs from the kernel instance `" + instanceName(key) + "` (" +
                std::to_string(kernel) + ")");
  };
  if (a.issueSchedule != s.issue)
    throw Error("AsyncPlan issue schedule `" + a.issueSchedule +
                "` differs from the kernel instance's `" + s.issue + "`");
  if (a.loadsPerThread != s.loadsPerThread)
    differ("loads per thread", a.loadsPerThread, s.loadsPerThread);
  if (a.prologueTailLoads != s.prologueTailLoads)
    differ("prologue tail loads", a.prologueTailLoads, s.prologueTailLoads);
  if (a.loaderWaves != s.loaderWaves)
    differ("loader waves", a.loaderWaves, s.loaderWaves);
  if (a.waits.empty())
    throw Error("AsyncPlan has no waits");
  for (const WaitInfo &w : a.waits) {
    const int64_t vm = w.groupId == 0 ? s.vmPrologue : s.vmLoop;
    if (w.vmcntAllowance != vm)
      differ("vmcnt of the wait for k group " + std::to_string(w.groupId),
             w.vmcntAllowance, vm);
    if (w.lgkmcntAllowance != s.lgkmLoop)
      differ("lgkmcnt of the wait for k group " + std::to_string(w.groupId),
             w.lgkmcntAllowance, s.lgkmLoop);
  }
}

// Reference: LowerPipelineToNVGPU.cpp:2624-2732 (contract -> gpu.func +
// launch geometry). Here the contract selects a precompiled gfx950 kernel
// instance and fills its launch configuration.
tb_gemm_config lowerContractToConfig(const KernelContract &k) {
  const KernelConfig &c = k.kernel;
  checkKernelSwizzle(k);
  tb_gemm_config g{};
  g.m = c.problemM;
  g.n = c.problemN;
  g.k = c.problemK;
  g.lda = c.problemK;
  g.ldb = c.problemN;
  g.ldc = c.problemN;
  g.c_dtype = c.cScalar == ScalarKind::F16 ? TB_DTYPE_F16 : TB_DTYPE_F32;
  g.acc_init = k.epilogue.initMode == AccumulatorInitMode::Zero ? TB_ACC_INIT_ZERO
                                                                : TB_ACC_INIT_LOAD_C;
  g.block_m = c.blockM;
  g.block_n = c.blockN;
  g.block_k = c.blockK;
  g.num_waves = c.numWarps;
  g.wave_grid_m = k.warpDecomposition.warpGrid.at(0);
  g.wave_grid_n = k.warpDecomposition.warpGrid.at(1);
  g.stages = c.requestedStages;
  const ProgramMappingPlan &pm = k.programMapping;
  switch (pm.mappingKind) {
  case ProgramMappingKind::Tile:
    g.mapping = TB_MAP_TILE;
    break;
  case ProgramMappingKind::GroupedTile:
    g.mapping = TB_MAP_GROUPED_TILE;
    break;
  case ProgramMappingKind::SplitK:
    g.mapping = TB_MAP_SPLIT_K;
    break;
  case ProgramMappingKind::PersistentTile:
    g.mapping = pm.swizzleKind == ProgramSwizzleKind::GroupedM ? TB_MAP_PERSISTENT_GROUPED
                                                                : TB_MAP_PERSISTENT_TILE;
    break;
  }
  g.group_m = pm.groupM;
  g.split_k = pm.splitK;
  switch (k.reduction.kind) {
  case ReductionPlanKind::None:
    g.reduction = TB_RED_NONE;
    break;
  case ReductionPlanKind::SplitKSerial:
    g.reduction = TB_RED_WORKSPACE;
    break;
  case ReductionPlanKind::SplitKAtomic:
    g.reduction = TB_RED_ATOMIC;
    break;
  }
  g.num_programs = pm.persistent ? k.persistentWork.residentPrograms : pm.totalPrograms;
  g.xcd_remap = pm.xcdRemap;
  const EpilogueRequest r = epilogueRequestOf(k.epilogue);
  g.epi_bias = r.bias.empty() ? TB_EPI_BIAS_NONE
                              : (r.bias == "f16" ? TB_EPI_BIAS_F16 : TB_EPI_BIAS_F32);
  g.epi_activation = r.activation.empty()       ? TB_ACT_NONE
                     : r.activation == "relu"   ? TB_ACT_RELU
                     : r.activation == "silu"   ? TB_ACT_SILU
                                                : TB_ACT_GELU_TANH;
  g.epi_clamp = (r.hasMin ? TB_CLAMP_MIN : 0) | (r.hasMax ? TB_CLAMP_MAX : 0);
  g.clamp_min = r.hasMin ? (float)r.clampMin : 0.0f;
  g.clamp_max = r.hasMax ? (float)r.clampMax : 0.0f;
  g.mfma = c.mmaKind == MmaKind::Mfma16x16x32F16 ? TB_MFMA_16X16X32 : TB_MFMA_32X32X16;
  if (g.mfma == TB_MFMA_16X16X32 && g.mapping == TB_MAP_SPLIT_K)
    throw Error("mma = `mfma_f32_16x16x32_f16` has no split-k instance");
  // the lowering names only kernels that exist
  const InstanceKey key = instanceKeyOf(g);
  if (!hasGfx950Instance(key))
    throw Error("no gfx950 kernel instance `" + instanceName(key) +
                "` for this contract (see tb-opt --list-instances)");
  // register truth: the compiler's report of the instance (build-time table)
  if (const std::string why = spillRefusal(key, g.k % g.block_k != 0); !why.empty())
    throw Error(why);
  checkKernelWaits(k, key);
  return g;
}

} // namespace tb
