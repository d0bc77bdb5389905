// Pass implementations of tb-opt. Each pass reads the plans it needs back
// from the IR (the text is the checkpoint, so every pass can run on its own
// from tb-opt), derives its plan and writes it as an attribute, exactly as
// the reference passes do (lib/Transforms/*.cpp).
#include "passes.h"
#include "../plan/instances.h"
#include "../ir/verify.h"

#include "../plan/contract.h"
#include "../plan/plans.h"

#include <cstdio>
#include <functional>
#include <set>

namespace tb {

namespace {

// ---- helpers -----------------------------------------------------------------
void forEachOp(Module &m, const char *name, const std::function<void(Op &)> &fn) {
  for (Func &f : m.funcs)
    for (Op &op : f.body)
      if (op.name == name)
        fn(op);
}

TargetInfo moduleTarget(const Module &m) {
  AttrP t = m.attr(kTarget);
  if (!t)
    throw Error("module is missing `tb.target`; run tb-attach-target-info first");
  return parseTargetInfoAttr(*t);
}

const Attr &need(const Op &op, const char *attr, const char *producer) {
  auto it = op.attrs.find(attr);
  if (it == op.attrs.end())
    throw Error(std::string("tb.matmul is missing `") + attr + "`; run " + producer +
                " first");
  return *it->second;
}

KernelConfig checkedConfig(const Module &m, const Op &op, const TargetInfo *t) {
  KernelConfig c = getKernelConfig(m, op);
  verifySupportedKernelConfig(c, t);
  if (t) // with the gfx950 target: the bound instance holds its registers
    verifyInstanceRegisters(m, op, c);
  return c;
}

// ---- passes ------------------------------------------------------------------------
// Reference: VerifyScope.cpp:19-30 (+ the IR subset this build accepts).
void verifyScope(Module &m, const PassOptions &) {
  static const std::set<std::string> allowed = {
      "tb.matmul", "tb.convert_layout", "tb.pipeline_mainline", "tb.gfx950_launch",
      "func.return"};
  for (Func &f : m.funcs)
    for (Op &op : f.body)
      if (!allowed.count(op.name))
        throw Error("operation `" + op.name + "` is outside the stage1 scope");
  forEachOp(m, "tb.matmul", [&](Op &op) {
    checkedConfig(m, op, nullptr);
    parseEpilogueRequest(op);
  });
}

// Reference: AttachTargetInfo.cpp:35-82.
void attachTargetInfo(Module &m, const PassOptions &o) {
  auto arch = o.find("gpu-arch");
  if (arch == o.end() || arch->second.empty())
    throw Error("tb-attach-target-info requires explicit `gpu-arch`; stage1 target "
                "ownership must not fall back to a hidden default chip");
  auto feat = o.find("ptx-features");
  std::string features = feat == o.end() ? "" : feat->second;
  forEachOp(m, "tb.matmul", [&](Op &op) {
    if (!m.attr(kNumWarps) || !m.attr(kRequestedStages))
      throw Error("tb-attach-target-info requires module attrs `tb.num-warps` and "
                  "`tb.requested-stages`");
    TargetInfo t = deriveTargetInfoForArch(arch->second, features);
    m.attrs[kTarget] = buildTargetInfoAttr(t);
    m.attrs[kThreadsPerWarp] = I64(t.threadsPerWarp);
    op.attrs.erase("tb.target_info");
  });
}

// Reference: SemanticizeMatmul.cpp:22-45.
void semanticize(Module &m, const PassOptions &) {
  forEachOp(m, "tb.matmul", [&](Op &op) {
    KernelConfig c = checkedConfig(m, op, nullptr);
    op.attrs["tb.semantic_matmul"] = buildMatmulSemanticsAttr(deriveMatmulSemantics(c, op));
  });
}

// Reference: BuildProgramMappingPlan.cpp:30-70.
void buildProgramMapping(Module &m, const PassOptions &) {
  forEachOp(m, "tb.matmul", [&](Op &op) {
    TargetInfo t = moduleTarget(m);
    KernelConfig c = checkedConfig(m, op, &t);
    need(op, "tb.semantic_matmul", "tb-semanticize-matmul");
    ProgramMappingPlan pm = deriveProgramMappingPlan(m, c, t);
    ReductionPlan rd = deriveReductionPlan(c, pm);
    PersistentWorkPlan pw = derivePersistentWorkPlan(c, t, pm);
    op.attrs["tb.program_mapping_plan"] = buildProgramMappingPlanAttr(pm);
    op.attrs["tb.reduction_plan"] = buildReductionPlanAttr(rd);
    op.attrs["tb.persistent_work_plan"] = buildPersistentWorkPlanAttr(pw);
    // the launch's CTA count as module context (BuildProgramMappingPlan.cpp:67-72)
    m.attrs[kNumCTAs] = I64(pm.numCTAs);
  });
}

// Reference: BuildLayoutPlan.cpp:26-55.
void buildLayout(Module &m, const PassOptions &) {
  forEachOp(m, "tb.matmul", [&](Op &op) {
    TargetInfo t = moduleTarget(m);
    KernelConfig c = checkedConfig(m, op, &t);
    MatmulSemantics s = parseMatmulSemanticsAttr(
        need(op, "tb.semantic_matmul", "tb-semanticize-matmul"));
    ProgramMappingPlan pm = parseProgramMappingPlanAttr(
        need(op, "tb.program_mapping_plan", "tb-build-program-mapping-plan"));
    op.attrs.erase("tb.layout_plan");
    op.attrs["tb.encoding_plan"] = buildEncodingPlanAttr(deriveEncodingPlan(c, t, s, pm));
  });
}

// Reference: BuildTransportPlan.cpp:24-52.
void buildTransport(Module &m, const PassOptions &) {
  forEachOp(m, "tb.matmul", [&](Op &op) {
    TargetInfo t = moduleTarget(m);
    KernelConfig c = checkedConfig(m, op, &t);
    EncodingPlan e =
        parseEncodingPlanAttr(need(op, "tb.encoding_plan", "tb-build-layout-plan"));
    op.attrs["tb.transport_plan"] = buildTransportPlanAttr(deriveTransportPlan(c, t, e));
  });
}

// Reference: BuildCRegisterPlan.cpp:30-135.
void buildCRegister(Module &m, const PassOptions &) {
  forEachOp(m, "tb.matmul", [&](Op &op) {
    TargetInfo t = moduleTarget(m);
    KernelConfig c = checkedConfig(m, op, &t);
    EncodingPlan e =
        parseEncodingPlanAttr(need(op, "tb.encoding_plan", "tb-build-layout-plan"));
    TransportPlan tr =
        parseTransportPlanAttr(need(op, "tb.transport_plan", "tb-build-transport-plan"));
    ProgramMappingPlan pm = parseProgramMappingPlanAttr(
        need(op, "tb.program_mapping_plan", "tb-build-program-mapping-plan"));
    ReductionPlan rd = parseReductionPlanAttr(
        need(op, "tb.reduction_plan", "tb-build-program-mapping-plan"));
    PersistentWorkPlan pw = parsePersistentWorkPlanAttr(
        need(op, "tb.persistent_work_plan", "tb-build-program-mapping-plan"));
    AccumulatorPlan a = deriveAccumulatorPlan(c, t, e);
    const EpilogueRequest req = parseEpilogueRequest(op);
    if (!req.empty() && rd.kind == ReductionPlanKind::SplitKAtomic)
      throw Error("fused epilogue exprs apply to the whole sum; split_k_atomic "
                  "accumulates partial sums straight into C and cannot carry them");
    EpiloguePlan ep = deriveEpiloguePlan(c, t, e, a, req);
    EpilogueReorderPlan ro = deriveEpilogueReorderPlan(c, a, ep);
    SharedWorkspacePlan sw = deriveSharedWorkspacePlan(c, t, e, tr, ro, rd, pw);
    WarpDecompositionPlan wd = deriveWarpDecompositionPlan(c, e, a, ep, ro, rd, pw);
    ResourceClosurePlan rc =
        deriveResourceClosurePlan(c, t, pm, rd, pw, a, ep, ro, sw, wd);
    op.attrs.erase("tb.c_register_plan");
    op.attrs["tb.accumulator_plan"] = buildAccumulatorPlanAttr(a);
    op.attrs["tb.epilogue_plan"] = buildEpiloguePlanAttr(ep);
    op.attrs["tb.epilogue_reorder_plan"] = buildEpilogueReorderPlanAttr(ro);
    op.attrs["tb.shared_workspace_plan"] = buildSharedWorkspacePlanAttr(sw);
    op.attrs["tb.warp_decomposition_plan"] = buildWarpDecompositionPlanAttr(wd);
    op.attrs["tb.resource_closure_plan"] = buildResourceClosurePlanAttr(rc);
  });
}

// Reference: RewriteMatmulMainloop.cpp:24-55.
void rewriteMainloop(Module &m, const PassOptions &) {
  forEachOp(m, "tb.matmul", [&](Op &op) {
    TargetInfo t = moduleTarget(m);
    KernelConfig c = checkedConfig(m, op, &t);
    EncodingPlan e =
        parseEncodingPlanAttr(need(op, "tb.encoding_plan", "tb-build-layout-plan"));
    AccumulatorPlan a = parseAccumulatorPlanAttr(
        need(op, "tb.accumulator_plan", "tb-build-c-register-plan"));
    EpiloguePlan ep =
        parseEpiloguePlanAttr(need(op, "tb.epilogue_plan", "tb-build-c-register-plan"));
    op.attrs["tb.matmul_rewrite"] =
        buildMatmulRewritePlanAttr(deriveMatmulRewritePlan(c, e, a, ep));
  });
}

// Reference: CleanupLayoutConversions.cpp:20-55. Folds identity conversions
// and conversion round trips, then drops unused conversions.
void cleanupLayoutConversions(Module &m, const PassOptions &) {
  for (Func &f : m.funcs) {
    bool changed = true;
    while (changed) {
      changed = false;
      std::map<std::string, const Op *> defOf;
      for (const Op &op : f.body)
        for (const std::string &r : op.results)
          defOf[r] = &op;
      for (size_t i = 0; i < f.body.size(); ++i) {
        Op &op = f.body[i];
        if (op.name != "tb.convert_layout" || op.operands.size() != 1 ||
            op.results.size() != 1 || op.operandTypes.size() != 1 ||
            op.resultTypes.size() != 1)
          continue;
        std::string replacement;
        if (equal(op.operandTypes[0], op.resultTypes[0])) {
          replacement = op.operands[0];
        } else if (auto d = defOf.find(op.operands[0]);
                   d != defOf.end() && d->second->name == "tb.convert_layout" &&
                   d->second->operandTypes.size() == 1 &&
                   equal(d->second->operandTypes[0], op.resultTypes[0])) {
          replacement = d->second->operands[0];
        }
        if (replacement.empty())
          continue;
        std::string result = op.results[0];
        f.body.erase(f.body.begin() + i);
        for (Op &user : f.body)
          for (std::string &o : user.operands)
            if (o == result)
              o = replacement;
        changed = true;
        break;
      }
    }
    std::set<std::string> used;
    for (const Op &op : f.body)
      used.insert(op.operands.begin(), op.operands.end());
    std::vector<Op> kept;
    for (Op &op : f.body)
      if (!(op.name == "tb.convert_layout" && op.results.size() == 1 &&
            !used.count(op.results[0])))
        kept.push_back(op);
    f.body = kept;
  }
}

// Reference: BuildMainloopGraph.cpp:24-60.
void buildMainloopGraph(Module &m, const PassOptions &) {
  forEachOp(m, "tb.matmul", [&](Op &op) {
    TargetInfo t = moduleTarget(m);
    KernelConfig c = checkedConfig(m, op, &t);
    EncodingPlan e =
        parseEncodingPlanAttr(need(op, "tb.encoding_plan", "tb-build-layout-plan"));
    AccumulatorPlan a = parseAccumulatorPlanAttr(
        need(op, "tb.accumulator_plan", "tb-build-c-register-plan"));
    EpiloguePlan ep =
        parseEpiloguePlanAttr(need(op, "tb.epilogue_plan", "tb-build-c-register-plan"));
    MatmulRewritePlan rw = parseMatmulRewritePlanAttr(
        need(op, "tb.matmul_rewrite", "tb-rewrite-matmul-mainloop"));
    op.attrs.erase("tb.mainloop_graph");
    op.attrs["tb.buffer_model"] = buildBufferModelAttr(deriveBufferModel(c, e, a, ep, rw));
  });
}

// Reference: RegularizeKLoop.cpp:22-50.
void regularizeKLoop(Module &m, const PassOptions &) {
  forEachOp(m, "tb.matmul", [&](Op &op) {
    BufferModel bm =
        parseBufferModelAttr(need(op, "tb.buffer_model", "tb-build-mainloop-graph"));
    MatmulRewritePlan rw = parseMatmulRewritePlanAttr(
        need(op, "tb.matmul_rewrite", "tb-rewrite-matmul-mainloop"));
    op.attrs["tb.loop_plan"] = buildLoopPlanAttr(deriveLoopPlan(bm, rw));
  });
}

// Reference: AssignLatencies.cpp:22-60.
void assignLatencies(Module &m, const PassOptions &) {
  forEachOp(m, "tb.matmul", [&](Op &op) {
    TargetInfo t = moduleTarget(m);
    KernelConfig c = checkedConfig(m, op, &t);
    BufferModel bm =
        parseBufferModelAttr(need(op, "tb.buffer_model", "tb-build-mainloop-graph"));
    LoopPlan lp = parseLoopPlanAttr(need(op, "tb.loop_plan", "tb-regularize-k-loop"));
    op.attrs["tb.latency_plan"] = buildLatencyPlanAttr(deriveLatencyPlan(c, t, bm, lp));
  });
}

// Reference: ScheduleLoops.cpp:22-56.
void scheduleLoops(Module &m, const PassOptions &) {
  forEachOp(m, "tb.matmul", [&](Op &op) {
    BufferModel bm =
        parseBufferModelAttr(need(op, "tb.buffer_model", "tb-build-mainloop-graph"));
    LoopPlan lp = parseLoopPlanAttr(need(op, "tb.loop_plan", "tb-regularize-k-loop"));
    LatencyPlan lat =
        parseLatencyPlanAttr(need(op, "tb.latency_plan", "tb-assign-latencies"));
    op.attrs.erase("tb.schedule_plan");
    op.attrs["tb.pipeline_plan"] = buildPipelinePlanAttr(derivePipelinePlan(bm, lp, lat));
  });
}

// Reference: DeriveWaits.cpp:22-56.
void deriveWaits(Module &m, const PassOptions &) {
  forEachOp(m, "tb.matmul", [&](Op &op) {
    TargetInfo t = moduleTarget(m);
    KernelConfig c = checkedConfig(m, op, &t);
    BufferModel bm =
        parseBufferModelAttr(need(op, "tb.buffer_model", "tb-build-mainloop-graph"));
    TransportPlan tr =
        parseTransportPlanAttr(need(op, "tb.transport_plan", "tb-build-transport-plan"));
    LatencyPlan lat =
        parseLatencyPlanAttr(need(op, "tb.latency_plan", "tb-assign-latencies"));
    PipelinePlan pp =
        parsePipelinePlanAttr(need(op, "tb.pipeline_plan", "tb-schedule-loops"));
    // the instance flavour the lowering will bind (instanceKeyOf)
    const ProgramMappingPlan pm = parseProgramMappingPlanAttr(
        need(op, "tb.program_mapping_plan", "tb-build-program-mapping-plan"));
    const ReductionPlan rd =
        parseReductionPlanAttr(need(op, "tb.reduction_plan", "tb-build-program-mapping-plan"));
    const EpiloguePlan ep =
        parseEpiloguePlanAttr(need(op, "tb.epilogue_plan", "tb-build-c-register-plan"));
    const bool splitK = pm.mappingKind == ProgramMappingKind::SplitK;
    const int out = instanceOutOf(splitK, rd.kind == ReductionPlanKind::SplitKAtomic,
                                  c.cScalar == ScalarKind::F16,
                                  ep.initMode != AccumulatorInitMode::Zero);
    const bool epi = !splitK && !epilogueRequestOf(ep).empty();
    op.attrs.erase("tb.wait_plan");
    op.attrs["tb.async_plan"] =
        buildAsyncPlanAttr(deriveAsyncPlan(c, bm, tr, lat, pp, out, epi));
  });
}

// Reference: ExpandPipeline.cpp:22-57.
void expandPipeline(Module &m, const PassOptions &) {
  forEachOp(m, "tb.matmul", [&](Op &op) {
    BufferModel bm =
        parseBufferModelAttr(need(op, "tb.buffer_model", "tb-build-mainloop-graph"));
    PipelinePlan pp =
        parsePipelinePlanAttr(need(op, "tb.pipeline_plan", "tb-schedule-loops"));
    AsyncPlan ap = parseAsyncPlanAttr(need(op, "tb.async_plan", "tb-derive-waits"));
    op.attrs["tb.pipeline_expansion"] =
        buildPipelineExpansionAttr(derivePipelineExpansion(bm, pp, ap));
  });
}

// Reference: CleanupPipeline.cpp:172-348. Seals tb.matmul into
// tb.pipeline_mainline: the private scheduling attrs are dropped, the public
// plans stay, and the expansion becomes the body's cluster ops.
void cleanupPipeline(Module &m, const PassOptions &) {
  static const std::set<std::string> dropped = {
      "block_m", "block_n", "block_k", "num_warps", "num_stages", "group_m",
      "exact_tile", "mma", "tb.target_info", "tb.layout_plan", "tb.c_register_plan",
      "tb.mainloop_graph", "tb.schedule_plan", "tb.wait_plan", "tb.loop_plan",
      "tb.latency_plan", "tb.pipeline_plan", "tb.pipeline_expansion",
      "tb.pipeline_ready", "epilogue_bias", "epilogue_activation",
      "epilogue_clamp_min", "epilogue_clamp_max"};
  forEachOp(m, "tb.matmul", [&](Op &op) {
    TargetInfo t = moduleTarget(m);
    KernelConfig c = checkedConfig(m, op, &t);
    PipelinePlan pp =
        parsePipelinePlanAttr(need(op, "tb.pipeline_plan", "tb-schedule-loops"));
    AsyncPlan ap = parseAsyncPlanAttr(need(op, "tb.async_plan", "tb-derive-waits"));
    PipelineExpansion ex = parsePipelineExpansionAttr(
        need(op, "tb.pipeline_expansion", "tb-expand-pipeline"));
    for (const char *a : {"tb.buffer_model", "tb.latency_plan", "tb.loop_plan",
                          "tb.epilogue_plan", "tb.epilogue_reorder_plan",
                          "tb.shared_workspace_plan", "tb.resource_closure_plan"})
      need(op, a, "the stage1 plan passes");
    PipelineReady ready{pp.scheduledMaxStage, (int64_t)ap.groups.size(),
                        c.requestedStages};
    Op sealed;
    sealed.name = "tb.pipeline_mainline";
    sealed.operands = op.operands;
    sealed.operandTypes = op.operandTypes;
    for (auto &kv : op.attrs)
      if (!dropped.count(kv.first))
        sealed.attrs[kv.first] = kv.second;
    sealed.attrs["tb.pipeline_ready"] = buildPipelineReadyAttr(ready);
    sealed.hasRegion = true;
    std::vector<const ExpandedCluster *> ordered;
    for (const ExpandedCluster &cl : ex.clusters)
      ordered.push_back(&cl);
    std::stable_sort(ordered.begin(), ordered.end(),
                     [](auto *a, auto *b) { return a->ordinal < b->ordinal; });
    for (const ExpandedCluster *cl : ordered) {
      Op body;
      body.attrs["ordinal"] = I64(cl->ordinal);
      body.attrs["stage"] = I64(cl->stage);
      body.attrs["cluster"] = I64(cl->cluster);
      body.attrs["k_group"] = I64(cl->kGroup);
      body.attrs["op_ids"] = Dense(cl->opIds);
      body.attrs["reason"] = Str(cl->reason);
      switch (cl->kind) {
      case ExpandedClusterKind::AsyncIssue:
        body.name = "tb.async_issue_cluster";
        break;
      case ExpandedClusterKind::ConsumerWait:
        body.name = "tb.consumer_wait_cluster";
        body.attrs["wait_group_ids"] = Dense(cl->waitGroupIds);
        body.attrs["needs_barrier"] = Bool(cl->needsBarrier);
        break;
      case ExpandedClusterKind::MmaCompute:
        body.name = "tb.mma_compute_cluster";
        break;
      }
      sealed.region.push_back(body);
    }
    op = sealed;
  });
}

// Reference: VerifyPipelineMainlineContract.cpp:183-470.
void verifyMainline(Module &m, const PassOptions &) {
  int count = 0;
  forEachOp(m, "tb.pipeline_mainline", [&](Op &op) {
    ++count;
    verifyMainlineContract(m, op, parseKernelContract(m, op));
  });
  forEachOp(m, "tb.matmul", [&](Op &) {
    throw Error("tb.matmul survived to the mainline verifier; run tb-cleanup-pipeline");
  });
  (void)count;
}

// Replaces tb-lower-pipeline-to-nvgpu (LowerPipelineToNVGPU.cpp:2624-2732):
// the sealed contract becomes a tb.gfx950_launch op naming the gfx950
// kernel instance and its launch configuration (grid, block, LDS bytes,
// global workspace bytes, and every tb_gemm_config field).
void lowerToGfx950(Module &m, const PassOptions &) {
  forEachOp(m, "tb.pipeline_mainline", [&](Op &op) {
    KernelContract k = parseKernelContract(m, op);
    verifyMainlineContract(m, op, k);
    tb_gemm_config g = lowerContractToConfig(k);
    Op launch;
    launch.name = "tb.gfx950_launch";
    launch.operands = op.operands;
    launch.operandTypes = op.operandTypes;
    std::map<std::string, AttrP> cfg = {
        {"m", I64(g.m)}, {"n", I64(g.n)}, {"k", I64(g.k)},
        {"lda", I64(g.lda)}, {"ldb", I64(g.ldb)}, {"ldc", I64(g.ldc)},
        {"c_dtype", I64(g.c_dtype)}, {"acc_init", I64(g.acc_init)},
        {"block_m", I64(g.block_m)}, {"block_n", I64(g.block_n)},
        {"block_k", I64(g.block_k)}, {"num_waves", I64(g.num_waves)},
        {"wave_grid_m", I64(g.wave_grid_m)}, {"wave_grid_n", I64(g.wave_grid_n)},
        {"stages", I64(g.stages)}, {"mapping", I64(g.mapping)},
        {"group_m", I64(g.group_m)}, {"split_k", I64(g.split_k)},
        {"reduction", I64(g.reduction)}, {"num_programs", I64(g.num_programs)},
        {"xcd_remap", I64(g.xcd_remap)}};
    if (g.mfma != TB_MFMA_32X32X16)
      cfg["mfma"] = I64(g.mfma);
    if (g.epi_bias || g.epi_activation || g.epi_clamp) {
      cfg["epi_bias"] = I64(g.epi_bias);
      cfg["epi_activation"] = I64(g.epi_activation);
      cfg["epi_clamp"] = I64(g.epi_clamp);
      cfg["clamp_min"] = F32(g.clamp_min);
      cfg["clamp_max"] = F32(g.clamp_max);
    }
    launch.attrs["config"] = Dict(cfg);
    launch.attrs["kernel"] = Str(kernelInstanceName(g));
    // the s_waitcnt depths of the AsyncPlan, which the lowering checked
    // against the instance: vmcnt at the prologue, vmcnt and lgkmcnt at the
    // per-k-tile barrier (the runtime checks them against the compiled kernel)
    const InstanceSchedule sched = instanceSchedule(instanceKeyOf(g));
    launch.attrs["waits"] = Dense({sched.vmPrologue, sched.vmLoop, sched.lgkmLoop});
    launch.attrs["grid"] = Dense({g.num_programs, 1, 1});
    // the wave grid's waves plus the instance's load-only waves, if any
    launch.attrs["block"] =
        Dense({(g.num_waves + sched.loaderWaves) * k.target.threadsPerWarp, 1, 1});
    launch.attrs["lds_bytes"] = I64(k.sharedWorkspace.totalBytes);
    launch.attrs["workspace_bytes"] = I64(k.resourceClosure.globalWorkspaceBytes);
    op = launch;
  });
}

// Reference: lib/Transforms/LowerEpilogueVectorIO.cpp covers the epilogue C
// IO as IR ops; on gfx950 the epilogue is part of the kernel instance, so
// there is no separate IR to lower and the pass only checks its scope.
void lowerEpilogueVectorIO(Module &m, const PassOptions &) {
  for (Func &f : m.funcs)
    for (Op &op : f.body)
      if (op.name == "tb.epilogue_global_vector_load" ||
          op.name == "tb.epilogue_global_vector_store")
        throw Error("standalone epilogue vector IO ops are not part of the gfx950 "
                    "flow; the epilogue is fused into the kernel instance");
}

struct PassEntry {
  const char *name, *summary;
  void (*fn)(Module &, const PassOptions &);
};

const std::vector<PassEntry> &passTable() {
  static const std::vector<PassEntry> t = {
      {"tb-verify-scope", "check every tb.matmul against the supported envelope",
       verifyScope},
      {"tb-attach-target-info", "attach the gfx950 capability table (gpu-arch=gfx950)",
       attachTargetInfo},
      {"tb-semanticize-matmul", "derive tb.semantic_matmul", semanticize},
      {"tb-build-program-mapping-plan",
       "derive program mapping, reduction and persistent work plans",
       buildProgramMapping},
      {"tb-build-layout-plan", "derive the MFMA/LDS encoding plan", buildLayout},
      {"tb-build-encoding-plan", "alias of tb-build-layout-plan", buildLayout},
      {"tb-build-transport-plan", "derive the direct-to-LDS transport plan",
       buildTransport},
      {"tb-build-c-register-plan",
       "derive accumulator, epilogue, reorder, workspace, wave and resource plans",
       buildCRegister},
      {"tb-rewrite-matmul-mainloop", "derive tb.matmul_rewrite", rewriteMainloop},
      {"tb-cleanup-layout-conversions", "fold redundant tb.convert_layout ops",
       cleanupLayoutConversions},
      {"tb-build-mainloop-graph", "derive tb.buffer_model", buildMainloopGraph},
      {"tb-regularize-k-loop", "derive tb.loop_plan", regularizeKLoop},
      {"tb-assign-latencies", "derive tb.latency_plan", assignLatencies},
      {"tb-schedule-loops", "derive tb.pipeline_plan", scheduleLoops},
      {"tb-derive-waits", "derive tb.async_plan", deriveWaits},
      {"tb-expand-pipeline", "derive tb.pipeline_expansion", expandPipeline},
      {"tb-cleanup-pipeline", "seal tb.matmul into tb.pipeline_mainline",
       cleanupPipeline},
      {"tb-verify-pipeline-mainline-contract", "verify the sealed mainline contract",
       verifyMainline},
      {"tb-lower-pipeline-to-gfx950",
       "lower the sealed mainline to a tb.gfx950_launch of a gfx950 kernel instance",
       lowerToGfx950},
      {"tb-lower-epilogue-vector-io", "epilogue IO check (fused on gfx950)",
       lowerEpilogueVectorIO},
  };
  return t;
}

std::string trim(const std::string &s) {
  size_t b = s.find_first_not_of(" \t\n'\"");
  size_t e = s.find_last_not_of(" \t\n'\"");
  return b == std::string::npos ? "" : s.substr(b, e - b + 1);
}

} // namespace

PassOptions parsePassOptions(const std::string &text) {
  PassOptions o;
  size_t i = 0;
  while (i < text.size()) {
    while (i < text.size() && (text[i] == ' ' || text[i] == ','))
      ++i;
    size_t b = i;
    while (i < text.size() && text[i] != ' ' && text[i] != ',')
      ++i;
    std::string kv = text.substr(b, i - b);
    if (kv.empty())
      continue;
    size_t eq = kv.find('=');
    if (eq == std::string::npos)
      o[kv] = "true";
    else
      o[kv.substr(0, eq)] = kv.substr(eq + 1);
  }
  return o;
}

std::vector<PassSpec> parsePassPipeline(const std::string &raw) {
  std::string text = trim(raw);
  const std::string outer = "builtin.module(";
  if (text.rfind(outer, 0) == 0) {
    if (text.back() != ')')
      throw Error("pass pipeline `" + raw + "` is missing its closing `)`");
    text = text.substr(outer.size(), text.size() - outer.size() - 1);
  }
  std::vector<PassSpec> out;
  size_t i = 0;
  while (i < text.size()) {
    while (i < text.size() && (text[i] == ',' || text[i] == ' '))
      ++i;
    if (i >= text.size())
      break;
    size_t b = i;
    while (i < text.size() && text[i] != ',' && text[i] != '{')
      ++i;
    PassSpec p;
    p.name = trim(text.substr(b, i - b));
    if (i < text.size() && text[i] == '{') {
      size_t close = text.find('}', i);
      if (close == std::string::npos)
        throw Error("unterminated options of pass `" + p.name + "`");
      p.options = parsePassOptions(text.substr(i + 1, close - i - 1));
      i = close + 1;
    }
    out.push_back(p);
  }
  // expand the registered pipelines
  std::vector<PassSpec> expanded;
  for (const PassSpec &p : out) {
    if (p.name == "tb-stage1-full-to-gfx950-pipeline" ||
        p.name == "tb-stage1-mainline-pipeline") {
      auto pick = [&](std::initializer_list<const char *> keys, const char *dflt) {
        for (const char *k : keys)
          if (p.options.count(k))
            return p.options.at(k);
        return std::string(dflt);
      };
      std::string chip = pick({"cubin-chip", "gpu-arch", "chip"}, "gfx950");
      std::string feat = pick({"cubin-features", "ptx-features", "features"}, "");
      for (PassSpec &q : stage1Pipeline(chip, feat,
                                        p.name == "tb-stage1-full-to-gfx950-pipeline"))
        expanded.push_back(q);
    } else {
      expanded.push_back(p);
    }
  }
  return expanded;
}

void runPass(Module &m, const PassSpec &p) {
  for (const PassEntry &e : passTable())
    if (p.name == e.name) {
      try {
        e.fn(m, p.options);
        verifyModule(m); // after every pass, as MLIR's pass manager does
      } catch (const Error &err) {
        throw Error(p.name + ": " + err.what());
      }
      return;
    }
  throw Error("unknown pass `" + p.name + "`");
}

void runPipeline(Module &m, const std::vector<PassSpec> &passes) {
  for (const PassSpec &p : passes)
    runPass(m, p);
}

std::vector<PassInfo> registeredPasses() {
  std::vector<PassInfo> v;
  for (const PassEntry &e : passTable())
    v.push_back({e.name, e.summary});
  v.push_back({"tb-stage1-full-to-gfx950-pipeline",
               "the whole stage1 plan pipeline plus the gfx950 lowering "
               "(options cubin-chip, cubin-features)"});
  v.push_back({"tb-stage1-mainline-pipeline",
               "the stage1 plan pipeline up to the sealed, verified mainline"});
  return v;
}

std::vector<PassSpec> stage1Pipeline(const std::string &gpuArch,
                                     const std::string &features, bool lower) {
  std::vector<PassSpec> p = {
      {"tb-verify-scope", {}},
      {"tb-attach-target-info", {{"gpu-arch", gpuArch}, {"ptx-features", features}}},
      {"tb-semanticize-matmul", {}},
      {"tb-build-program-mapping-plan", {}},
      {"tb-build-layout-plan", {}},
      {"tb-build-transport-plan", {}},
      {"tb-build-c-register-plan", {}},
      {"tb-rewrite-matmul-mainloop", {}},
      {"tb-cleanup-layout-conversions", {}},
      {"tb-build-mainloop-graph", {}},
      {"tb-regularize-k-loop", {}},
      {"tb-assign-latencies", {}},
      {"tb-schedule-loops", {}},
      {"tb-derive-waits", {}},
      {"tb-expand-pipeline", {}},
      {"tb-cleanup-pipeline", {}},
      {"tb-verify-pipeline-mainline-contract", {}}};
  if (lower)
    p.push_back({"tb-lower-pipeline-to-gfx950", {}});
  return p;
}

tb_gemm_config launchConfigOf(const Op &launch) {
  if (launch.name != "tb.gfx950_launch")
    throw Error("expected a tb.gfx950_launch op");
  const Attr &c = opAttr(launch, "config");
  tb_gemm_config g{};
  g.m = getI64(c, "m");
  g.n = getI64(c, "n");
  g.k = getI64(c, "k");
  g.lda = getI64(c, "lda");
  g.ldb = getI64(c, "ldb");
  g.ldc = getI64(c, "ldc");
  g.c_dtype = (int32_t)getI64(c, "c_dtype");
  g.acc_init = (int32_t)getI64(c, "acc_init");
  g.block_m = getI64(c, "block_m");
  g.block_n = getI64(c, "block_n");
  g.block_k = getI64(c, "block_k");
  g.num_waves = getI64(c, "num_waves");
  g.wave_grid_m = getI64(c, "wave_grid_m");
  g.wave_grid_n = getI64(c, "wave_grid_n");
  g.stages = getI64(c, "stages");
  g.mapping = (int32_t)getI64(c, "mapping");
  g.group_m = getI64(c, "group_m");
  g.split_k = getI64(c, "split_k");
  g.reduction = (int32_t)getI64(c, "reduction");
  g.num_programs = getI64(c, "num_programs");
  g.xcd_remap = (int32_t)getI64(c, "xcd_remap");
  // the MFMA kind is printed only for 16x16x32, the fused epilogue fields
  // only when some step is requested
  if (has(c, "mfma"))
    g.mfma = (int32_t)getI64(c, "mfma");
  if (has(c, "epi_bias")) {
    g.epi_bias = (int32_t)getI64(c, "epi_bias");
    g.epi_activation = (int32_t)getI64(c, "epi_activation");
    g.epi_clamp = (int32_t)getI64(c, "epi_clamp");
    g.clamp_min = (float)getF64(c, "clamp_min");
    g.clamp_max = (float)getF64(c, "clamp_max");
  }
  return g;
}

// The instance the runtime binds (instances.h), so tb-opt can name the
// kernel without a GPU.
std::string kernelInstanceName(const tb_gemm_config &c) {
  return instanceName(instanceKeyOf(c));
}

} // namespace tb
