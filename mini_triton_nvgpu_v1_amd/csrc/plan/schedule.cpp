// The schedule chain: MatmulRewritePlan, BufferModel, LoopPlan, LatencyPlan,
// PipelinePlan, AsyncPlan, PipelineExpansion and PipelineReady.
//
// gfx950 model of the main loop. A k group is one fill of one LDS slot
// (block_k deep); it holds block_k / 16 MFMA k steps. Group g is loaded into
// ring slot g % S (S = requested stages) and consumed S groups later, and
// the load of group g + S reuses the slot of group g right after group g's
// last fragment read:
//   time slot t:  consume group t - S (wait, fragment reads, MFMAs), then
//                 issue the loads of group t into the slot just freed.
// Slots 0 .. S-1 are the prologue (loads only). Within a slot the clusters
// run consumer_wait (0), mma_compute (1), async_issue (2): refill after
// consume, which is what lets the kernels use one barrier per k group.
//
// The reference unrolls every k group of the problem into the model
// (BufferModel.cpp:1075-1193), O(k groups x fragments) host work and IR
// size. Here the model covers a steady-state window of min(k groups, S + 1)
// groups, which shows every slot's load, reuse and wait once; LoopPlan's
// iteration_count records the real trip count the kernels run.
#include "instances.h"
#include "serialize.h"

#include <algorithm>
#include <set>

namespace tb {

// ---- MatmulRewritePlan ----------------------------------------------------------
template <class V> void fields(V &v, OperandFragmentPath &p) {
  v("role", p.role);
  v("instruction_shape", p.instructionShape);
  v("fragment_shape", p.fragmentShape);
  v("fragments_per_k_group", p.fragmentsPerKGroup);
  v("consumer_tile_span_m", p.consumerTileSpanM);
  v("consumer_tile_span_n", p.consumerTileSpanN);
  v("uses_ldmatrix", p.usesLdMatrix);
}
template <class V> void fields(V &v, MatmulRewritePlan &p) {
  v("contract_model", p.contractModel);
  v("mainloop_kind", p.mainloopKind);
  v("instruction_m", p.instructionM);
  v("instruction_n", p.instructionN);
  v("instruction_k", p.instructionK);
  v("k_groups", p.kGroups);
  v("acc_tiles_m", p.accTilesM);
  v("acc_tiles_n", p.accTilesN);
  v("b_group_count", p.bGroupCount);
  v("accumulator_fragments", p.accumulatorFragments);
  v("direct_accumulator_init", p.directAccumulatorInit);
  v("direct_accumulator_store", p.directAccumulatorStore);
  v("a_path", p.aPath);
  v("b_path", p.bPath);
  v("k_group_depth", p.kGroupDepth);
  v("k_steps_per_group", p.kStepsPerGroup);
}

// Reference: MatmulRewritePlan.cpp:167-220. k_groups counts the k groups
// one program runs (split-k programs each run a contiguous share).
MatmulRewritePlan deriveMatmulRewritePlan(const KernelConfig &c, const EncodingPlan &e,
                                          const AccumulatorPlan &,
                                          const EpiloguePlan &ep) {
  MatmulRewritePlan p;
  p.contractModel = "triton_layout_driven_matmul_rewrite_v2";
  p.mainloopKind = "mfma_direct_to_lds_async";
  p.instructionM = e.fragmentA.instructionShape.at(0);
  p.instructionK = e.fragmentA.instructionShape.at(1);
  p.instructionN = e.fragmentB.instructionShape.at(1);
  p.kGroupDepth = c.blockK;
  p.kStepsPerGroup = c.blockK / p.instructionK;
  p.kGroups = ceilDiv(c.problemK, c.blockK);
  p.accTilesM = e.fragmentAcc.repeatShape.at(0);
  p.accTilesN = e.fragmentAcc.repeatShape.at(1);
  p.bGroupCount = 1; // one B fragment bundle (all n tiles of the wave) per k step
  p.accumulatorFragments = p.accTilesM * p.accTilesN;
  p.directAccumulatorInit = ep.initMode == AccumulatorInitMode::DirectGlobalVector;
  p.directAccumulatorStore = ep.storeMode == AccumulatorStoreMode::DirectGlobalVector;
  p.aPath = {"a", e.fragmentA.instructionShape, e.fragmentA.logicalShape,
             p.accTilesM * p.kStepsPerGroup, p.accTilesM, 1, true};
  p.bPath = {"b", e.fragmentB.instructionShape, e.fragmentB.logicalShape,
             p.accTilesN * p.kStepsPerGroup, 1, p.accTilesN, true};
  if (p.kStepsPerGroup * p.instructionK != c.blockK)
    throw Error("block_k must be a whole number of MFMA k steps");
  return p;
}
AttrP buildMatmulRewritePlanAttr(const MatmulRewritePlan &p) { return buildPlanAttr(p); }
MatmulRewritePlan parseMatmulRewritePlanAttr(const Attr &a) {
  return parsePlanAttr<MatmulRewritePlan>(a, "`tb.matmul_rewrite`");
}

// ---- BufferModel ----------------------------------------------------------------
template <class V> void fields(V &v, BufferBacking &b) {
  v("id", b.id);
  v("role", b.role);
  v("desc_type", b.descType);
  v("depth", b.depth);
  v("alias_group", b.aliasGroup);
  v("stage_indexed", b.stageIndexed);
  v("debug_name", b.debugName);
}
template <class V> void fields(V &v, BufferView &b) {
  v("id", b.id);
  v("backing", b.backing);
  v("kind", b.kind);
  v("stage", b.stage);
  v("buffer_index", b.bufferIndex);
  v("encoding", b.encoding);
  v("offsets", b.offsets);
  v("shape", b.shape);
  v("debug_name", b.debugName);
}
template <class V> void fields(V &v, ValueState &s) {
  v("id", s.id);
  v("kind", s.kind);
  v("defining_op", s.definingOp);
  v("users", s.users);
  v("owner_view", s.ownerView);
  v("loop_distance", s.loopDistance);
  v("bundle", s.bundle);
  v("first_use_ordinal", s.firstUseOrdinal);
  v("last_use_ordinal", s.lastUseOrdinal);
  v("debug_name", s.debugName);
}
template <class V> void fields(V &v, IterationCoord &c) {
  v("axis", c.axis);
  v("value", c.value);
}
template <class V> void fields(V &v, PipelineOp &o) {
  v("id", o.id);
  v("kind", o.kind);
  v("inputs", o.inputs);
  v("outputs", o.outputs);
  v("iteration_coords", o.iterationCoords);
}
template <class V> void fields(V &v, BufferModel &m) {
  v("backings", m.backings);
  v("views", m.views);
  v("values", m.values);
  v("ops", m.ops);
}

const char *bufferOpKindName(BufferOpKind k) { return enumName(k); }
PipelineOpSemanticClass semanticClass(BufferOpKind k) {
  switch (k) {
  case BufferOpKind::LoadA:
  case BufferOpKind::LoadB:
    return PipelineOpSemanticClass::AsyncProducer;
  case BufferOpKind::LocalLoadA:
  case BufferOpKind::LocalLoadB:
    return PipelineOpSemanticClass::SharedConsumer;
  case BufferOpKind::Mma:
    return PipelineOpSemanticClass::TensorCoreCompute;
  case BufferOpKind::AccumulatorInit:
    return PipelineOpSemanticClass::EpilogueInit;
  case BufferOpKind::AccumulatorStore:
    return PipelineOpSemanticClass::EpilogueStore;
  }
  return PipelineOpSemanticClass::TensorCoreCompute;
}
int64_t iterationCoord(const PipelineOp &op, const std::string &axis) {
  for (const IterationCoord &c : op.iterationCoords)
    if (c.axis == axis)
      return c.value;
  return -1;
}

static AttrP memdesc(I64s shape, const std::string &elem, AttrP enc,
                     const std::string &space, bool mut, I64s alloc) {
  auto d = std::make_shared<Attr>();
  d->kind = AttrKind::Type;
  d->typeDialect = "memdesc";
  d->params = {{"shape", IntList(shape)},  {"elementType", TypeText(elem)},
               {"encoding", enc},           {"memorySpace", Str(space)},
               {"mutableMemory", Bool(mut)}, {"allocShape", IntList(alloc)}};
  return d;
}

BufferModel deriveBufferModel(const KernelConfig &c, const EncodingPlan &e,
                              const AccumulatorPlan &, const EpiloguePlan &,
                              const MatmulRewritePlan &rw) {
  const int64_t S = c.requestedStages, KS = rw.kStepsPerGroup;
  const int64_t window = std::min(rw.kGroups, S + 1);
  const std::string cElem = scalarName(c.cScalar);
  BufferModel m;
  auto backing = [&](BufferRole role, AttrP desc, int64_t depth, bool staged,
                     const char *name) {
    m.backings.push_back({(int64_t)m.backings.size(), role, desc, depth, -1, staged, name});
    return (int64_t)m.backings.size() - 1;
  };
  auto view = [&](int64_t b, ViewKind k, int64_t stage, int64_t idx, int enc,
                  I64s off, I64s shape, std::string name) {
    m.views.push_back({(int64_t)m.views.size(), b, k, stage, idx, enc, off, shape, name});
    return (int64_t)m.views.size() - 1;
  };
  const AttrP &aSh = e.encodings.at(e.aShared).encodingAttr;
  const AttrP &bSh = e.encodings.at(e.bShared).encodingAttr;
  int64_t wtM = e.fragmentAcc.logicalShape.at(0), wtN = e.fragmentAcc.logicalShape.at(1);
  int64_t aG = backing(BufferRole::OperandA,
                       memdesc({c.problemM, c.problemK}, "f16",
                               e.encodings.at(e.aGlobal).encodingAttr, "global",
                               false, {c.problemM, c.problemK}),
                       1, false, "a_global");
  int64_t bG = backing(BufferRole::OperandB,
                       memdesc({c.problemK, c.problemN}, "f16",
                               e.encodings.at(e.bGlobal).encodingAttr, "global",
                               false, {c.problemK, c.problemN}),
                       1, false, "b_global");
  int64_t aS = backing(BufferRole::OperandA,
                       memdesc({S, c.blockM, c.blockK}, "f16", aSh, "shared", true,
                               {S, c.blockM, c.blockK}),
                       S, true, "a_shared_ring");
  int64_t bS = backing(BufferRole::OperandB,
                       memdesc({S, c.blockK, c.blockN}, "f16", bSh, "shared", true,
                               {S, c.blockK, c.blockN}),
                       S, true, "b_shared_ring");
  int64_t aR = backing(BufferRole::OperandA,
                       memdesc({2, wtM, rw.instructionK}, "f16",
                               e.encodings.at(e.aDot).encodingAttr, "registers",
                               true, {2, wtM, rw.instructionK}),
                       2, true, "a_fragments");
  int64_t bR = backing(BufferRole::OperandB,
                       memdesc({2, rw.instructionK, wtN}, "f16",
                               e.encodings.at(e.bDot).encodingAttr, "registers",
                               true, {2, rw.instructionK, wtN}),
                       2, true, "b_fragments");
  int64_t accB = backing(BufferRole::Accumulator,
                         memdesc({wtM, wtN}, "f32", e.encodings.at(e.acc).encodingAttr,
                                 "registers", true, {wtM, wtN}),
                         1, false, "accumulator");
  backing(BufferRole::Output,
          memdesc({c.problemM, c.problemN}, cElem, e.encodings.at(e.cStore).encodingAttr,
                  "global", true, {c.problemM, c.problemN}),
          1, false, "c_global");
  int64_t aGV = view(aG, ViewKind::FullBuffer, -1, -1, e.aGlobal, {0, 0},
                     {c.problemM, c.problemK}, "a_global");
  int64_t bGV = view(bG, ViewKind::FullBuffer, -1, -1, e.bGlobal, {0, 0},
                     {c.problemK, c.problemN}, "b_global");
  (void)aGV;
  (void)bGV;
  I64s aStage(S), bStage(S);
  for (int64_t s = 0; s < S; ++s) {
    aStage[s] = view(aS, ViewKind::StageSlice, s, s, e.aShared, {s, 0, 0},
                     {c.blockM, c.blockK}, "a_stage" + std::to_string(s));
    bStage[s] = view(bS, ViewKind::StageSlice, s, s, e.bShared, {s, 0, 0},
                     {c.blockK, c.blockN}, "b_stage" + std::to_string(s));
  }
  I64s aFrag(2), bFrag(2);
  for (int64_t i = 0; i < 2; ++i) {
    aFrag[i] = view(aR, ViewKind::Fragment, -1, i, e.aDot, {i, 0, 0},
                    {wtM, rw.instructionK}, "a_frag" + std::to_string(i));
    bFrag[i] = view(bR, ViewKind::Fragment, -1, i, e.bDot, {i, 0, 0},
                    {rw.instructionK, wtN}, "b_frag" + std::to_string(i));
  }
  int64_t accV = view(accB, ViewKind::FullBuffer, -1, -1, e.acc, {0, 0}, {wtM, wtN},
                      "accumulator");

  auto value = [&](BufferValueKind k, int64_t def, int64_t owner, int64_t bundle,
                   const std::string &name) {
    ValueState s;
    s.id = (int64_t)m.values.size();
    s.kind = k;
    s.definingOp = def;
    s.ownerView = owner;
    s.bundle = bundle;
    s.debugName = name;
    m.values.push_back(s);
    return s.id;
  };
  auto use = [&](int64_t v, int64_t op) {
    ValueState &s = m.values[v];
    s.users.push_back(op);
    if (s.firstUseOrdinal < 0)
      s.firstUseOrdinal = op;
    s.lastUseOrdinal = op;
    m.ops[op].inputs.push_back(v);
  };
  auto op = [&](BufferOpKind k, int64_t kg, int64_t ks, int64_t bundle) {
    PipelineOp o;
    o.id = (int64_t)m.ops.size();
    o.kind = k;
    o.iterationCoords = {{"bundle", bundle}, {"k_group", kg}, {"k_step", ks},
                         {"m_tile", -1}, {"n_tile", -1}, {"acc_index", -1}};
    m.ops.push_back(o);
    return o.id;
  };
  int64_t prevAcc = -1;
  for (int64_t g = 0; g < window; ++g) {
    int64_t la = op(BufferOpKind::LoadA, g, -1, g);
    int64_t aVal = value(BufferValueKind::SharedTile, la, aStage[g % S], g, "a_shared");
    m.ops[la].outputs.push_back(aVal);
    int64_t lb = op(BufferOpKind::LoadB, g, -1, g);
    int64_t bVal = value(BufferValueKind::SharedTile, lb, bStage[g % S], g, "b_shared");
    m.ops[lb].outputs.push_back(bVal);
    for (int64_t ks = 0; ks < KS; ++ks) {
      int64_t step = g * KS + ks, buf = step % 2;
      int64_t lla = op(BufferOpKind::LocalLoadA, g, ks, step);
      use(aVal, lla);
      int64_t fa = value(BufferValueKind::DotOperandFragment, lla, aFrag[buf], step, "a_frag");
      m.ops[lla].outputs.push_back(fa);
      int64_t llb = op(BufferOpKind::LocalLoadB, g, ks, step);
      use(bVal, llb);
      int64_t fb = value(BufferValueKind::DotOperandFragment, llb, bFrag[buf], step, "b_frag");
      m.ops[llb].outputs.push_back(fb);
      int64_t mm = op(BufferOpKind::Mma, g, ks, step);
      use(fa, mm);
      use(fb, mm);
      if (prevAcc >= 0)
        use(prevAcc, mm);
      prevAcc = value(BufferValueKind::AccumulatorFragment, mm, accV, step, "acc");
      m.ops[mm].outputs.push_back(prevAcc);
    }
  }
  // loop-carry distance of each value (k groups between def and later users)
  for (ValueState &s : m.values) {
    int64_t defG = iterationCoord(m.ops[s.definingOp], "k_group");
    int64_t dist = 0;
    for (int64_t u : s.users) {
      int64_t d = iterationCoord(m.ops[u], "k_group") - defG;
      if (d > 0) {
        if (dist && dist != d)
          throw Error("buffer model accepts one loop-carry distance per value");
        dist = d;
      }
    }
    s.loopDistance = dist;
  }
  return m;
}
AttrP buildBufferModelAttr(const BufferModel &m) { return buildPlanAttr(m); }
BufferModel parseBufferModelAttr(const Attr &a) {
  return parsePlanAttr<BufferModel>(a, "`tb.buffer_model`");
}

// ---- LoopPlan ------------------------------------------------------------------
template <class V> void fields(V &v, LoopIterationPlan &p) {
  v("k_group", p.kGroup);
  v("async_producer_ops", p.asyncProducerOps);
  v("consumer_ops", p.consumerOps);
  v("compute_ops", p.computeOps);
}
template <class V> void fields(V &v, LoopCarriedValue &p) {
  v("value_id", p.valueId);
  v("defining_op", p.definingOp);
  v("owner_view", p.ownerView);
  v("loop_distance", p.loopDistance);
  v("users", p.users);
  v("reason", p.reason);
}
template <class V> void fields(V &v, LoopPlan &p) {
  v("loop_axis", p.loopAxis);
  v("iteration_count", p.iterationCount);
  v("single_main_loop", p.singleMainLoop);
  v("iterations", p.iterations);
  v("carried_values", p.carriedValues);
  v("template_iterations", p.templateIterations);
}

// Reference: LoopPlan.cpp:253-364 (one k loop, ops bucketed per k group).
LoopPlan deriveLoopPlan(const BufferModel &m, const MatmulRewritePlan &rw) {
  LoopPlan p;
  p.loopAxis = "k_group";
  p.iterationCount = rw.kGroups;
  p.singleMainLoop = true;
  int64_t groups = 0;
  for (const PipelineOp &o : m.ops)
    groups = std::max(groups, iterationCoord(o, "k_group") + 1);
  p.templateIterations = groups;
  p.iterations.resize(groups);
  for (int64_t g = 0; g < groups; ++g)
    p.iterations[g].kGroup = g;
  for (const PipelineOp &o : m.ops) {
    LoopIterationPlan &it = p.iterations.at(iterationCoord(o, "k_group"));
    switch (semanticClass(o.kind)) {
    case PipelineOpSemanticClass::AsyncProducer:
      it.asyncProducerOps.push_back(o.id);
      break;
    case PipelineOpSemanticClass::SharedConsumer:
      it.consumerOps.push_back(o.id);
      break;
    default:
      it.computeOps.push_back(o.id);
    }
  }
  for (const ValueState &s : m.values)
    if (s.loopDistance > 0)
      p.carriedValues.push_back({s.id, s.definingOp, s.ownerView, s.loopDistance,
                                 s.users, "accumulator carried into the next k group"});
  return p;
}
AttrP buildLoopPlanAttr(const LoopPlan &p) { return buildPlanAttr(p); }
LoopPlan parseLoopPlanAttr(const Attr &a) { return parsePlanAttr<LoopPlan>(a, "`tb.loop_plan`"); }

// ---- LatencyPlan ------------------------------------------------------------------
template <class V> void fields(V &v, OpLatencyInfo &p) {
  v("op_id", p.opId);
  v("target_latency", p.targetLatency);
  v("self_latency", p.selfLatency);
  v("buffer_distance", p.bufferDistance);
  v("pipelineable", p.pipelineable);
  v("acc_multi_buffer", p.accMultiBuffer);
  v("reason", p.reason);
}
template <class V> void fields(V &v, LatencyPlan &p) { v("ops", p.ops); }

// Reference: LatencyPlan.cpp:215-383 (loads get buffer_distance = depth - 1
// because its cp.async refill is issued before the slot's consumers). The
// gfx950 ring refills a slot only after its last fragment read, so a load
// leads its consumers by the full ring depth S.
LatencyPlan deriveLatencyPlan(const KernelConfig &c, const TargetInfo &t,
                              const BufferModel &m, const LoopPlan &) {
  LatencyPlan p;
  for (const PipelineOp &o : m.ops) {
    OpLatencyInfo i;
    i.opId = o.id;
    switch (semanticClass(o.kind)) {
    case PipelineOpSemanticClass::AsyncProducer:
      i.targetLatency = t.globalToSharedStageLatency;
      i.selfLatency = 1;
      i.bufferDistance = c.requestedStages;
      i.pipelineable = true;
      i.reason = "direct-to-LDS load leads its consumers by the ring depth";
      break;
    case PipelineOpSemanticClass::SharedConsumer:
      i.targetLatency = t.sharedToRegisterStageLatency;
      i.selfLatency = 1;
      i.bufferDistance = 0;
      i.pipelineable = true;
      i.reason = "fragment read one k step ahead into the other register buffer";
      break;
    default:
      i.targetLatency = t.mmaStageLatency;
      i.selfLatency = 1;
      i.bufferDistance = 0;
      i.pipelineable = false;
      i.reason = "MFMA accumulates in place";
    }
    p.ops.push_back(i);
  }
  return p;
}
AttrP buildLatencyPlanAttr(const LatencyPlan &p) { return buildPlanAttr(p); }
LatencyPlan parseLatencyPlanAttr(const Attr &a) {
  return parsePlanAttr<LatencyPlan>(a, "`tb.latency_plan`");
}

// ---- PipelinePlan -------------------------------------------------------------
template <class V> void fields(V &v, PipelinePlacement &p) {
  v("op_id", p.opId);
  v("stage", p.stage);
  v("cluster", p.cluster);
  v("order", p.order);
  v("reason", p.reason);
}
template <class V> void fields(V &v, StageBufferUse &p) {
  v("view_id", p.viewId);
  v("backing", p.backing);
  v("stage", p.stage);
  v("buffer_index", p.bufferIndex);
  v("producer_op", p.producerOp);
  v("first_consumer_op", p.firstConsumerOp);
  v("last_consumer_op", p.lastConsumerOp);
}
template <class V> void fields(V &v, PipelinePlan &p) {
  v("scheduled_max_stage", p.scheduledMaxStage);
  v("placements", p.placements);
  v("stage_owned_buffers", p.stageOwnedBuffers);
}

static constexpr int64_t kClusterConsumer = 0, kClusterMma = 1, kClusterIssue = 2;

// Reference: PipelinePlan.cpp:319-546 (stage = max(input ready, k-group
// anchor)). A load of group g is anchored at time slot g; its consumers run
// in slot g + buffer_distance.
PipelinePlan derivePipelinePlan(const BufferModel &m, const LoopPlan &,
                                const LatencyPlan &lat) {
  PipelinePlan p;
  std::map<int64_t, int64_t> stageOf;
  int64_t loadDistance = 0;
  for (const OpLatencyInfo &i : lat.ops)
    if (semanticClass(m.ops.at(i.opId).kind) == PipelineOpSemanticClass::AsyncProducer)
      loadDistance = std::max(loadDistance, i.bufferDistance);
  std::map<std::pair<int64_t, int64_t>, int64_t> order;
  for (const PipelineOp &o : m.ops) {
    int64_t g = iterationCoord(o, "k_group");
    PipelinePlacement pl;
    pl.opId = o.id;
    switch (semanticClass(o.kind)) {
    case PipelineOpSemanticClass::AsyncProducer:
      pl.stage = g;
      pl.cluster = kClusterIssue;
      pl.reason = "k-group anchor; refill after the slot's previous consumers";
      break;
    case PipelineOpSemanticClass::SharedConsumer:
      pl.stage = g + loadDistance;
      pl.cluster = kClusterConsumer;
      pl.reason = "ring slot lands buffer_distance groups after its load";
      break;
    default:
      pl.stage = g + loadDistance;
      pl.cluster = kClusterMma;
      pl.reason = "MFMA consumes the fragments of its k step";
    }
    pl.order = order[{pl.stage, pl.cluster}]++;
    stageOf[o.id] = pl.stage;
    p.scheduledMaxStage = std::max(p.scheduledMaxStage, pl.stage);
    p.placements.push_back(pl);
  }
  // stage-owned ring slots: producer and the first/last consumer of each
  for (const ValueState &v : m.values) {
    const BufferView &view = m.views.at(v.ownerView);
    if (view.kind != ViewKind::StageSlice)
      continue;
    StageBufferUse u;
    u.viewId = view.id;
    u.backing = view.backing;
    u.stage = stageOf[v.definingOp];
    u.bufferIndex = view.bufferIndex;
    u.producerOp = v.definingOp;
    u.firstConsumerOp = v.users.empty() ? -1 : v.users.front();
    u.lastConsumerOp = v.users.empty() ? -1 : v.users.back();
    p.stageOwnedBuffers.push_back(u);
  }
  return p;
}
AttrP buildPipelinePlanAttr(const PipelinePlan &p) { return buildPlanAttr(p); }
PipelinePlan parsePipelinePlanAttr(const Attr &a) {
  return parsePlanAttr<PipelinePlan>(a, "`tb.pipeline_plan`");
}

// ---- AsyncPlan --------------------------------------------------------------------
template <class V> void fields(V &v, AsyncProducer &p) {
  v("op_id", p.opId);
  v("kind", p.kind);
  v("value_id", p.valueId);
  v("src_view", p.srcView);
  v("dst_view", p.dstView);
  v("src_offsets", p.srcOffsets);
  v("group_id", p.groupId);
  v("vec_bytes", p.vecBytes);
  v("transaction_bytes", p.transactionBytes);
  v("zero_fill", p.zeroFill);
  v("predicated", p.predicated);
  v("bypass_l1", p.bypassL1);
  v("barrier_kind", p.barrierKind);
  v("cache_policy", p.cachePolicy);
  v("legal", p.legal);
  v("reason", p.reason);
}
template <class V> void fields(V &v, AsyncGroup &g) {
  v("id", g.id);
  v("producers", g.producers);
}
template <class V> void fields(V &v, WaitInfo &w) {
  v("group_id", w.groupId);
  v("before_op_id", w.beforeOpId);
  v("required_stage", w.requiredStage);
  v("required_cluster", w.requiredCluster);
  v("required_order", w.requiredOrder);
  v("needs_barrier", w.needsBarrier);
  v("reason", w.reason);
  v("vmcnt_allowance", w.vmcntAllowance);
  v("lgkmcnt_allowance", w.lgkmcntAllowance);
}
template <class V> void fields(V &v, ReuseFence &f) {
  v("view_id", f.viewId);
  v("backing", f.backing);
  v("retiring_value_id", f.retiringValueId);
  v("acquiring_value_id", f.acquiringValueId);
  v("after_op_id", f.afterOpId);
  v("required_after_stage", f.requiredAfterStage);
  v("required_after_cluster", f.requiredAfterCluster);
  v("required_after_order", f.requiredAfterOrder);
  v("reason", f.reason);
}
template <class V> void fields(V &v, AsyncPlan &p) {
  v("producers", p.producers);
  v("groups", p.groups);
  v("waits", p.waits);
  v("reuse_fences", p.reuseFences);
  v("issue_schedule", p.issueSchedule);
  v("loads_per_thread", p.loadsPerThread);
  v("prologue_tail_loads", p.prologueTailLoads);
  v("refill_spread_slots", p.refillSpreadSlots);
  v("loader_waves", p.loaderWaves);
}

// Loads one thread issues per k group: each 16-byte vector of the A and B
// tiles is one buffer_load_dwordx4 ... lds, spread over the workgroup in
// rounds of one vector per lane. An operand's vectors are whole waves' rounds;
// when they do not fill the last round, the waves past them still issue that
// load (zeros into a scratch row of LDS), so every lane issues the same count.
static int64_t loadsPerThread(const KernelConfig &c, const TransportPlan &tr) {
  int64_t threads = c.numWarps * 64;
  int64_t va = tr.operandA.transactionBytes / tr.operandA.asyncVectorBytes;
  int64_t vb = tr.operandB.transactionBytes / tr.operandB.asyncVectorBytes;
  if (va % 64 || vb % 64)
    throw Error("A/B tiles must split into whole wavefront rounds of 16-byte loads");
  return (va + threads - 1) / threads + (vb + threads - 1) / threads;
}

// Reference: AsyncPlan.cpp:543-843 (one producer group per stage-owned
// buffer, a wait at the first-use frontier, reuse fences before a slot is
// refilled). gfx950: the producers are direct-to-LDS buffer loads, counted
// per lane by vmcnt in issue order. The waits' depths are those of the
// kernel instance the plan binds, which follow from how it issues its loads
// (InstanceSchedule): at the per-k-tile barrier the loads of the S - 2 later
// groups stay outstanding (vmcnt((S-2) x loads per thread)); at the
// prologue's wait also the part of group S-1 the prologue issues. Each wait
// is followed by s_barrier so every wave's share has landed; the 16x16x32
// instance also waits lgkmcnt(0) there (its LDS reads of the stage the
// barrier frees have returned).
AsyncPlan deriveAsyncPlan(const KernelConfig &c, const BufferModel &m,
                          const TransportPlan &tr, const LatencyPlan &,
                          const PipelinePlan &pp, int out, bool epi) {
  AsyncPlan p;
  const int64_t S = c.requestedStages, lpt = loadsPerThread(c, tr);
  InstanceKey key;
  const auto grid = deriveWaveGrid(c, 32, 32);
  key.bm = c.blockM;
  key.bn = c.blockN;
  key.bk = c.blockK;
  key.wgm = grid.first;
  key.wgn = grid.second;
  key.stages = S;
  key.out = out;
  key.epi = epi ? 1 : 0;
  key.mfma = c.mmaKind == MmaKind::Mfma16x16x32F16 ? TB_MFMA_16X16X32 : TB_MFMA_32X32X16;
  const InstanceSchedule sched = instanceSchedule(key);
  if (sched.loadsPerThread != lpt)
    throw Error("transport plan loads per thread (" + std::to_string(lpt) +
                ") disagree with the kernel's issue schedule (" +
                std::to_string(sched.loadsPerThread) + ")");
  if (sched.vmPrologue > 63)
    throw Error("outstanding loads per lane exceed the vmcnt counter (63)");
  p.issueSchedule = sched.issue;
  p.loadsPerThread = lpt;
  p.prologueTailLoads = sched.prologueTailLoads;
  p.refillSpreadSlots = sched.refillSpreadSlots;
  p.loaderWaves = sched.loaderWaves;
  std::map<int64_t, const PipelinePlacement *> place;
  for (const PipelinePlacement &pl : pp.placements)
    place[pl.opId] = &pl;
  bool boundary = c.problemM % c.blockM || c.problemN % c.blockN || c.problemK % c.blockK;
  std::map<int64_t, AsyncGroup> groups;
  std::map<int64_t, int64_t> sharedValueOfGroupA;
  for (const PipelineOp &o : m.ops) {
    if (semanticClass(o.kind) != PipelineOpSemanticClass::AsyncProducer)
      continue;
    bool isA = o.kind == BufferOpKind::LoadA;
    int64_t g = iterationCoord(o, "k_group");
    AsyncProducer a;
    a.opId = o.id;
    a.kind = AsyncProducerKind::BufferLoadLds;
    a.valueId = o.outputs.at(0);
    a.srcView = isA ? 0 : 1;
    a.dstView = m.values.at(a.valueId).ownerView;
    a.srcOffsets = isA ? I64s{0, g * c.blockK} : I64s{g * c.blockK, 0};
    a.groupId = g;
    a.vecBytes = (isA ? tr.operandA : tr.operandB).asyncVectorBytes;
    a.transactionBytes = (isA ? tr.operandA : tr.operandB).transactionBytes;
    a.zeroFill = boundary;
    a.predicated = boundary;
    a.bypassL1 = false;
    a.barrierKind = AsyncBarrierKind::VmcntBarrier;
    a.cachePolicy = AsyncCachePolicy::Default;
    a.legal = true;
    a.reason = "buffer_load_dwordx4 lds into ring slot " +
               std::to_string(g % S) + "; out-of-range lanes land zeros";
    groups[g].id = g;
    groups[g].producers.push_back(o.id);
    p.producers.push_back(a);
  }
  for (auto &kv : groups)
    p.groups.push_back(kv.second);
  // waits: before the first fragment read of each group
  for (const AsyncGroup &g : p.groups) {
    const PipelineOp *first = nullptr;
    for (const PipelineOp &o : m.ops)
      if (semanticClass(o.kind) == PipelineOpSemanticClass::SharedConsumer &&
          iterationCoord(o, "k_group") == g.id) {
        first = &o;
        break;
      }
    if (!first)
      continue;
    const PipelinePlacement *pl = place.at(first->id);
    WaitInfo w;
    w.groupId = g.id;
    w.beforeOpId = first->id;
    w.requiredStage = pl->stage;
    w.requiredCluster = pl->cluster;
    w.requiredOrder = pl->order;
    w.needsBarrier = true;
    w.vmcntAllowance = g.id == 0 ? (S - 2) * lpt + sched.prologueTailLoads : (S - 2) * lpt;
    w.lgkmcntAllowance = sched.lgkmLoop;
    w.reason = g.id == 0 ? "prologue: k groups 0 .. S-2 and the first " +
                               std::to_string(sched.prologueTailLoads) +
                               " loads of group S-1 issued, wait for group 0"
                         : "waited before the previous slot's refill, sharing its barrier";
    p.waits.push_back(w);
  }
  // reuse fences: the load of group g + S overwrites group g's slot
  for (const AsyncProducer &later : p.producers) {
    int64_t g = later.groupId - S;
    if (g < 0)
      continue;
    for (const AsyncProducer &earlier : p.producers) {
      if (earlier.groupId != g || earlier.dstView == -1)
        continue;
      const BufferView &ev = m.views.at(earlier.dstView);
      const BufferView &lv = m.views.at(later.dstView);
      if (ev.backing != lv.backing)
        continue;
      const ValueState &retiring = m.values.at(earlier.valueId);
      int64_t lastUse = retiring.users.empty() ? earlier.opId : retiring.users.back();
      const PipelinePlacement *pl = place.at(lastUse);
      ReuseFence f;
      f.viewId = ev.id;
      f.backing = ev.backing;
      f.retiringValueId = earlier.valueId;
      f.acquiringValueId = later.valueId;
      f.afterOpId = lastUse;
      f.requiredAfterStage = pl->stage;
      f.requiredAfterCluster = pl->cluster;
      f.requiredAfterOrder = pl->order;
      f.reason = "slot refilled only after the barrier that follows its last read";
      p.reuseFences.push_back(f);
    }
  }
  return p;
}
AttrP buildAsyncPlanAttr(const AsyncPlan &p) { return buildPlanAttr(p); }
AsyncPlan parseAsyncPlanAttr(const Attr &a) {
  return parsePlanAttr<AsyncPlan>(a, "`tb.async_plan`");
}

// ---- PipelineExpansion ------------------------------------------------------------
template <class V> void fields(V &v, ExpandedCluster &c) {
  v("ordinal", c.ordinal);
  v("stage", c.stage);
  v("cluster", c.cluster);
  v("k_group", c.kGroup);
  v("kind", c.kind);
  v("op_ids", c.opIds);
  v("wait_group_ids", c.waitGroupIds);
  v("needs_barrier", c.needsBarrier);
  v("reason", c.reason);
}
template <class V> void fields(V &v, PipelineExpansion &p) { v("clusters", p.clusters); }

// Reference: PipelineExpansion.cpp:304-448 (one cluster per (stage, cluster)
// holding ops of one kind, in schedule order).
PipelineExpansion derivePipelineExpansion(const BufferModel &m, const PipelinePlan &pp,
                                          const AsyncPlan &ap) {
  std::map<std::pair<int64_t, int64_t>, ExpandedCluster> byKey;
  std::map<int64_t, const PipelinePlacement *> place;
  for (const PipelinePlacement &pl : pp.placements)
    place[pl.opId] = &pl;
  std::vector<const PipelinePlacement *> sorted;
  for (const PipelinePlacement &pl : pp.placements)
    sorted.push_back(&pl);
  std::stable_sort(sorted.begin(), sorted.end(), [](auto *a, auto *b) {
    return std::tie(a->stage, a->cluster, a->order) <
           std::tie(b->stage, b->cluster, b->order);
  });
  for (const PipelinePlacement *pl : sorted) {
    const PipelineOp &o = m.ops.at(pl->opId);
    ExpandedCluster &c = byKey[{pl->stage, pl->cluster}];
    ExpandedClusterKind kind =
        pl->cluster == kClusterIssue      ? ExpandedClusterKind::AsyncIssue
        : pl->cluster == kClusterConsumer ? ExpandedClusterKind::ConsumerWait
                                          : ExpandedClusterKind::MmaCompute;
    if (c.opIds.empty()) {
      c.stage = pl->stage;
      c.cluster = pl->cluster;
      c.kGroup = iterationCoord(o, "k_group");
      c.kind = kind;
    } else if (c.kGroup != iterationCoord(o, "k_group")) {
      throw Error("a pipeline cluster must hold one k group");
    }
    c.opIds.push_back(o.id);
  }
  PipelineExpansion p;
  int64_t ordinal = 0;
  for (auto &kv : byKey) {
    ExpandedCluster c = kv.second;
    c.ordinal = ordinal++;
    if (c.kind == ExpandedClusterKind::ConsumerWait) {
      for (const WaitInfo &w : ap.waits)
        if (std::find(c.opIds.begin(), c.opIds.end(), w.beforeOpId) != c.opIds.end()) {
          c.waitGroupIds.push_back(w.groupId);
          c.needsBarrier = c.needsBarrier || w.needsBarrier;
        }
      c.reason = "s_waitcnt vmcnt + s_barrier, then fragment reads of k group " +
                 std::to_string(c.kGroup);
    } else if (c.kind == ExpandedClusterKind::AsyncIssue) {
      c.reason = "direct-to-LDS loads of k group " + std::to_string(c.kGroup);
    } else {
      c.reason = "MFMAs of k group " + std::to_string(c.kGroup);
    }
    p.clusters.push_back(c);
  }
  return p;
}
AttrP buildPipelineExpansionAttr(const PipelineExpansion &p) { return buildPlanAttr(p); }
PipelineExpansion parsePipelineExpansionAttr(const Attr &a) {
  return parsePlanAttr<PipelineExpansion>(a, "`tb.pipeline_expansion`");
}

// ---- PipelineReady ------------------------------------------------------------------
template <class V> void fields(V &v, PipelineReady &p) {
  v("scheduled_max_stage", p.scheduledMaxStage);
  v("async_groups", p.asyncGroups);
  v("requested_stages", p.requestedStages);
}
AttrP buildPipelineReadyAttr(const PipelineReady &p) { return buildPlanAttr(p); }
PipelineReady parsePipelineReadyAttr(const Attr &a) {
  return parsePlanAttr<PipelineReady>(a, "`tb.pipeline_ready`");
}

} // namespace tb
