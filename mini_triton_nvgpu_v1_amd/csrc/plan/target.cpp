// TargetInfo (gfx950 capability table), KernelConfig legality and
// MatmulSemantics.
#include "instances.h"
#include "serialize.h"

#include <cstdlib>

namespace tb {

// ---- shared helpers -----------------------------------------------------------
const Attr &opAttr(const Op &op, const std::string &name) {
  auto it = op.attrs.find(name);
  if (it == op.attrs.end())
    throw Error("missing `" + name + "` attribute on " + op.name);
  return *it->second;
}

std::map<std::string, AttrP> dictOf(const Attr &a) {
  if (a.kind != AttrKind::Dict)
    throw Error("expected a dictionary attribute");
  return a.dict;
}

// ---- TargetInfo ------------------------------------------------------------------
template <class V> void fields(V &v, TargetInfo &t) {
  v("gpu_arch", t.gpuArch);
  v("target_triple", t.targetTriple);
  v("ptx_features", t.ptxFeatures);
  v("threads_per_warp", t.threadsPerWarp);
  v("shared_bank_bytes", t.sharedBankBytes);
  v("num_sms", t.numSms);
  v("max_warps_per_cta", t.maxWarpsPerCTA);
  v("max_registers_per_thread", t.maxRegistersPerThread);
  v("max_registers_per_cta", t.maxRegistersPerCTA);
  v("max_shared_bytes_per_cta", t.maxSharedBytesPerCTA);
  v("supports_async_copy", t.supportsAsyncCopy);
  v("supports_ldmatrix", t.supportsLdMatrix);
  v("supports_mma_sync", t.supportsMmaSync);
  v("supports_mbarrier", t.supportsMBarrier);
  v("supports_tma", t.supportsTMA);
  v("supports_wgmma", t.supportsWGMMA);
  v("async_copy_min_bytes", t.asyncCopyMinBytes);
  v("async_copy_max_bytes", t.asyncCopyMaxBytes);
  v("async_copy_preferred_bytes", t.asyncCopyPreferredBytes);
  v("global_to_shared_stage_latency", t.globalToSharedStageLatency);
  v("shared_to_register_stage_latency", t.sharedToRegisterStageLatency);
  v("mma_stage_latency", t.mmaStageLatency);
  v("preferred_async_transport", t.preferredAsyncTransport);
  v("mma_instr_shape", t.mmaInstrShape);
  v("shared_bank_count", t.sharedBankCount);
  v("num_xcds", t.numXcds);
  v("supports_mfma", t.supportsMfma);
  v("supports_direct_to_lds", t.supportsDirectToLds);
  v("supports_lds_transpose_read", t.supportsLdsTransposeRead);
  v("mfma_instr_shapes", t.mfmaInstrShapes);
}

static void validateTargetInfo(const TargetInfo &t) {
  if (t.threadsPerWarp != 64)
    throw Error("gfx950 target requires 64-lane wavefronts");
  if (t.numSms <= 0 || t.maxWarpsPerCTA <= 0 || t.maxSharedBytesPerCTA <= 0)
    throw Error("target info requires positive CU, wave and LDS limits");
  if (t.mmaInstrShape.size() != 3)
    throw Error("target info requires a rank-3 mma instruction shape");
  if (t.sharedBankBytes <= 0 || t.sharedBankCount <= 0)
    throw Error("target info requires positive LDS bank geometry");
}

// Reference table: TargetInfo.cpp:118-215 (per-SM-arch entries). This build
// targets MI355X only; the capability numbers are the CDNA4 ones the kernels
// are written against (64-lane waves, 256 CUs in 8 XCDs, 160 KiB LDS per
// workgroup served by 64 banks of 4 bytes, 512 VGPR+AGPR per lane).
TargetInfo deriveTargetInfoForArch(const std::string &gpuArch,
                                   const std::string &features) {
  std::string chip = gpuArch.substr(0, gpuArch.find(':'));
  if (chip != "gfx950")
    throw Error("tb-attach-target-info supports gpu-arch `gfx950` (MI355X), "
                "got `" + gpuArch + "`");
  TargetInfo t;
  t.gpuArch = "gfx950";
  t.targetTriple = "amdgcn-amd-amdhsa";
  t.ptxFeatures = features;
  t.threadsPerWarp = 64;
  t.sharedBankBytes = 4;
  t.sharedBankCount = 64;
  t.numSms = 256;
  t.numXcds = 8;
  t.maxWarpsPerCTA = 16;
  t.maxRegistersPerThread = 512;
  t.maxRegistersPerCTA = 131072;
  t.maxSharedBytesPerCTA = 163840;
  t.supportsAsyncCopy = true;
  t.supportsLdMatrix = false;
  t.supportsMmaSync = false;
  t.supportsMBarrier = false;
  t.supportsTMA = false;
  t.supportsWGMMA = false;
  t.supportsMfma = true;
  t.supportsDirectToLds = true;
  t.supportsLdsTransposeRead = true;
  t.asyncCopyMinBytes = 4;
  t.asyncCopyMaxBytes = 16;
  t.asyncCopyPreferredBytes = 16;
  t.globalToSharedStageLatency = 2;
  t.sharedToRegisterStageLatency = 1;
  t.mmaStageLatency = 1;
  t.preferredAsyncTransport = "buffer_load_dwordx4_lds";
  t.mmaInstrShape = {32, 32, 16};
  t.mfmaInstrShapes = {{32, 32, 16}, {16, 16, 32}, {32, 32, 8}, {16, 16, 16}};
  validateTargetInfo(t);
  return t;
}

AttrP buildTargetInfoAttr(const TargetInfo &t) { return buildPlanAttr(t); }
TargetInfo parseTargetInfoAttr(const Attr &a) {
  TargetInfo t = parsePlanAttr<TargetInfo>(a, "`tb.target`");
  validateTargetInfo(t);
  return t;
}

// ---- KernelConfig ---------------------------------------------------------------
const char *scalarName(ScalarKind k) { return enumName(k); }
const char *mmaKindName(MmaKind k) { return enumName(k); }
int64_t scalarBytes(ScalarKind k) { return k == ScalarKind::F16 ? 2 : 4; }

static int64_t moduleI64(const Module &m, const char *name, bool required,
                         int64_t dflt) {
  AttrP a = m.attr(name);
  if (!a) {
    if (required)
      throw Error(std::string("missing required module attr `") + name + "`");
    return dflt;
  }
  if (a->kind != AttrKind::Int)
    throw Error(std::string("module attr `") + name + "` must be an integer");
  return a->i;
}

static ScalarKind scalarOf(const std::string &t, const char *role) {
  if (t == "f16")
    return ScalarKind::F16;
  if (t == "f32")
    return ScalarKind::F32;
  throw Error(std::string("operand `") + role + "` must have f16 or f32 elements, got `" +
              t + "`");
}

static int64_t opI64(const Op &op, const char *name, bool required, int64_t dflt) {
  auto it = op.attrs.find(name);
  if (it == op.attrs.end()) {
    if (required)
      throw Error(std::string("tb.matmul requires `") + name + "`");
    return dflt;
  }
  if (it->second->kind != AttrKind::Int)
    throw Error(std::string("`") + name + "` must be an integer attribute");
  return it->second->i;
}

// gfx950: v_mfma_f32_16x16x32_f16 instances exist for the 4-wave
// 256x256x64 2-stage tile (hand-scheduled) and for the tiles of the
// 16x16x32 loop (kernels/gemm_tiles.h, TBK_M16_TILES_*), on the wave grid
// the plan derives, with an f16 C, a plain f32 C or f32 C += A*B, plain or
// fused, any M, N and K (they mask ragged edges). Per FLOP it moves a
// quarter of the accumulator register traffic of 32x32x16, which this
// power-limited part turns into a higher sustained clock, and its wave
// tiles of 128x128 (and 256x64, 96x128) hold their accumulators without
// spilling. (Split-K has no 16x16x32 instance: the caller checks.)
bool mfma16x16x32Supported(const KernelConfig &c) {
  std::pair<int64_t, int64_t> g;
  try {
    g = deriveWaveGrid(c, 32, 32);
  } catch (const Error &) {
    return false;
  }
  return hasMfma16Tile(c.blockM, c.blockN, c.blockK, g.first, g.second, c.requestedStages);
}

// Reference: KernelConfig.cpp:86-132 (tb.matmul) and the post-cleanup
// derivation from module attrs + semantic/mapping plans.
KernelConfig getKernelConfig(const Module &m, const Op &op) {
  if (op.operandTypes.size() != 3)
    throw Error(op.name + " must have three memref operands");
  MemRefInfo a = parseMemRef(op.operandTypes[0]);
  MemRefInfo b = parseMemRef(op.operandTypes[1]);
  MemRefInfo c = parseMemRef(op.operandTypes[2]);
  if (a.shape.size() != 2 || b.shape.size() != 2 || c.shape.size() != 2)
    throw Error("tb.matmul currently requires rank-2 memrefs");
  KernelConfig k;
  k.problemM = a.shape[0];
  k.problemK = a.shape[1];
  k.problemN = b.shape[1];
  k.aScalar = scalarOf(a.elementType, "a");
  k.bScalar = scalarOf(b.elementType, "b");
  k.cScalar = scalarOf(c.elementType, "c");
  if (b.shape[0] != k.problemK || c.shape[0] != k.problemM || c.shape[1] != k.problemN)
    throw Error("tb.matmul operand shapes disagree: A is MxK, B is KxN, C is MxN");
  k.numWarps = moduleI64(m, kNumWarps, true, 0);
  k.requestedStages = moduleI64(m, kRequestedStages, true, 0);
  if (op.name == "tb.matmul") {
    k.blockM = opI64(op, "block_m", true, 0);
    k.blockN = opI64(op, "block_n", true, 0);
    k.blockK = opI64(op, "block_k", true, 0);
    k.groupM = opI64(op, "group_m", false, 8);
    auto et = op.attrs.find("exact_tile");
    if (et == op.attrs.end() || et->second->kind != AttrKind::Bool)
      throw Error("tb.matmul requires bool `exact_tile`");
    k.exactTile = et->second->b;
    // `mma` names the instruction; without it the plan takes 16x16x32
    // wherever that instance exists (no split-K: its partials are f32 planes
    // of the general loop), else 32x32x16
    const bool splitK = moduleI64(m, kSplitK, false, 1) > 1;
    auto mma = op.attrs.find("mma");
    if (mma != op.attrs.end()) {
      if (mma->second->kind != AttrKind::String)
        throw Error("`mma` must be a string attribute");
      k.mmaKind = enumFromName<MmaKind>(mma->second->s, "mma");
      if (k.mmaKind == MmaKind::Mfma16x16x32F16 && splitK)
        throw Error("mma = `mfma_f32_16x16x32_f16` has no split-k instance");
    } else {
      k.mmaKind = mfma16x16x32Supported(k) && !splitK ? MmaKind::Mfma16x16x32F16
                                                       : MmaKind::Mfma32x32x16F16;
    }
  } else {
    MatmulSemantics s = parseMatmulSemanticsAttr(opAttr(op, "tb.semantic_matmul"));
    ProgramMappingPlan pm =
        parseProgramMappingPlanAttr(opAttr(op, "tb.program_mapping_plan"));
    k.blockM = s.tileM;
    k.blockN = s.tileN;
    k.blockK = s.tileK;
    k.exactTile = s.exactTile;
    k.groupM = pm.groupM;
    EncodingPlan e = parseEncodingPlanAttr(opAttr(op, "tb.encoding_plan"));
    const Attr &parent = param(encodingAttr(e, e.acc, "acc"), "parent");
    I64s instr = paramInts(parent, "instrShape");
    k.mmaKind = instr == I64s{16, 16, 32} ? MmaKind::Mfma16x16x32F16
                                          : MmaKind::Mfma32x32x16F16;
  }
  return k;
}

// The gfx950 kernels are compiled instances (kernels/gemm_tiles.h): a
// 32x32x16 configuration is legal only where the wave grid the encoding plan
// will derive has an instance for this block shape and stage count. (The
// reference emits a kernel for any legal contract, LowerPipelineToNVGPU.cpp:
// 678-1554; here the legality stops what the lowering could not bind.) A
// configuration with no legal wave grid at all is left to the encoding
// plan's own diagnostic.
static void verifyCompiledInstance(const KernelConfig &c) {
  if (c.mmaKind != MmaKind::Mfma32x32x16F16)
    return; // 16x16x32: mfma16x16x32Supported above
  std::pair<int64_t, int64_t> g;
  try {
    g = deriveWaveGrid(c, 32, 32);
  } catch (const Error &) {
    return;
  }
  for (const auto &[grid, stages] : compiledWaveGrids(c.blockM, c.blockN, c.blockK))
    if (grid == g && stages == c.requestedStages)
      return;
  std::string have;
  for (const auto &[grid, stages] : compiledWaveGrids(c.blockM, c.blockN, c.blockK))
    have += (have.empty() ? "" : ", ") + std::to_string(grid.first) + "x" +
            std::to_string(grid.second) + " s" + std::to_string(stages);
  throw Error("no gfx950 kernel instance for block " + std::to_string(c.blockM) + "x" +
              std::to_string(c.blockN) + "x" + std::to_string(c.blockK) + " on " +
              std::to_string(c.numWarps) + " waves (wave grid " +
              std::to_string(g.first) + "x" + std::to_string(g.second) + ") with " +
              std::to_string(c.requestedStages) + " LDS stages; compiled wave grids " +
              "and stages for this block: " + (have.empty() ? "none" : have));
}

void verifyInstanceRegisters(const Module &m, const Op &op, const KernelConfig &c) {
  if (op.name != "tb.matmul")
    return; // past the rewrite the lowering checks the exact instance
  std::pair<int64_t, int64_t> g;
  try {
    g = deriveWaveGrid(c, 32, 32);
  } catch (const Error &) {
    return; // the encoding plan reports the missing wave grid
  }
  const bool splitK = moduleI64(m, kSplitK, false, 1) > 1;
  bool atomic = false;
  if (AttrP a = m.attr(kReductionMode))
    atomic = a->kind == AttrKind::String && a->s == "split_k_parallel";
  const bool f16C = c.cScalar == ScalarKind::F16;
  bool fused = false;
  for (const char *name : {"epilogue_bias", "epilogue_activation", "epilogue_clamp_min",
                           "epilogue_clamp_max"})
    fused = fused || op.attrs.count(name) != 0;
  InstanceKey key;
  key.bm = c.blockM;
  key.bn = c.blockN;
  key.bk = c.blockK;
  key.wgm = g.first;
  key.wgn = g.second;
  key.stages = c.requestedStages;
  key.out = instanceOutOf(splitK, splitK && atomic, f16C, !f16C);
  key.epi = fused && !splitK ? 1 : 0;
  key.mfma = c.mmaKind == MmaKind::Mfma16x16x32F16 ? TB_MFMA_16X16X32 : TB_MFMA_32X32X16;
  if (!hasGfx950Instance(key))
    return; // the lowering names the missing instance
  if (const std::string why = spillRefusal(key, c.problemK % c.blockK != 0); !why.empty())
    throw Error(why);
}

// Reference: KernelConfig.cpp:202-246. gfx950 legality: f16 x f16 into an
// f16 or f32 C through v_mfma_f32_32x32x16_f16, so the block shape must be
// a multiple of the MFMA tile (32 x 32, k 16) and block_k one or two
// 16-byte LDS chunks per k step pair (32 or 64).
void verifySupportedKernelConfig(const KernelConfig &c, const TargetInfo *t) {
  if (c.aScalar != ScalarKind::F16 || c.bScalar != ScalarKind::F16)
    throw Error("gfx950 stage1 supports fp16 x fp16 -> fp16/fp32 matmul kernels");
  if (c.mmaKind != MmaKind::Mfma32x32x16F16 && c.mmaKind != MmaKind::Mfma16x16x32F16)
    throw Error("gfx950 stage1 supports mma = `mfma_f32_32x32x16_f16` or "
                "`mfma_f32_16x16x32_f16`");
  if (c.mmaKind == MmaKind::Mfma16x16x32F16 && !mfma16x16x32Supported(c))
    throw Error("mma = `mfma_f32_16x16x32_f16` has no gfx950 kernel instance for "
                "this block, wave count and stage count (see tb-opt --list-instances)");
  if (c.problemM <= 0 || c.problemN <= 0 || c.problemK <= 0)
    throw Error("problem M/N/K must be positive");
  if (c.blockM <= 0 || c.blockN <= 0 || c.blockK <= 0)
    throw Error("block M/N/K must be positive");
  if (c.blockM % 32 != 0 || c.blockN % 32 != 0 ||
      (c.blockK != 32 && c.blockK != 64))
    throw Error("gfx950 requires block_m % 32 == 0, block_n % 32 == 0 and "
                "block_k in {32, 64} for mfma_f32_32x32x16_f16 legality");
  if (c.requestedStages < 2 || c.requestedStages > 4)
    throw Error("stage1 currently supports num_stages in [2, 4]");
  if (c.numWarps <= 0)
    throw Error("num_warps must be positive");
  if (t && c.numWarps > t->maxWarpsPerCTA)
    throw Error("num_warps exceeds target max warps per CTA");
  if (c.groupM <= 0)
    throw Error("group_m must be positive");
  if (c.problemN % 8 != 0 || c.problemK % 8 != 0)
    throw Error("gfx950 buffer transport requires N and K to be multiples of 8 "
                "(16-byte rows chunks of f16)");
  if (c.exactTile && ((c.problemM % c.blockM) != 0 ||
                      (c.problemN % c.blockN) != 0 ||
                      (c.problemK % c.blockK) != 0))
    throw Error("exact_tile=true requires problem M/N/K to be divisible by "
                "block M/N/K");
  int64_t lds = c.requestedStages * (c.blockM + c.blockN) * c.blockK *
                scalarBytes(c.aScalar);
  if (t && lds > t->maxSharedBytesPerCTA)
    throw Error("A/B stage buffers (" + std::to_string(lds) +
                " bytes) exceed the target LDS budget");
  if (t) // with the gfx950 target attached: its compiled kernels
    verifyCompiledInstance(c);
}

// ---- MatmulSemantics -------------------------------------------------------------
template <class V> void fields(V &v, MatmulSemantics &s) {
  v("contract_model", s.contractModel);
  v("a_desc_type", s.aDescType);
  v("b_desc_type", s.bDescType);
  v("c_desc_type", s.cDescType);
  I64s ps{s.problemM, s.problemN, s.problemK}, ts{s.tileM, s.tileN, s.tileK};
  v("problem_shape", ps);
  v("tile_shape", ts);
  if (ps.size() != 3 || ts.size() != 3)
    throw Error("problem_shape and tile_shape must have three entries");
  s.problemM = ps[0], s.problemN = ps[1], s.problemK = ps[2];
  s.tileM = ts[0], s.tileN = ts[1], s.tileK = ts[2];
  v("exact_tile", s.exactTile);
  v("boundary_m", s.hasBoundaryM);
  v("boundary_n", s.hasBoundaryN);
  v("boundary_k", s.hasBoundaryK);
}

static AttrP semanticDesc(const MemRefInfo &info, int64_t rows, int64_t cols) {
  // identity row-major layout: strides [cols, 1], minor dimension 1
  AttrP layout = Dialect("semantic_layout",
                         {{"order", IntList({1, 0})},
                          {"strides", IntList({cols, 1})},
                          {"zeroOffset", Bool(true)},
                          {"hasStaticStrides", Bool(true)},
                          {"unitStrideOnMinor", Bool(true)},
                          {"contiguous", Bool(true)}});
  auto d = std::make_shared<Attr>();
  d->kind = AttrKind::Type;
  d->typeDialect = "memdesc";
  d->params = {{"shape", IntList({rows, cols})},
               {"elementType", TypeText(info.elementType)},
               {"encoding", layout},
               {"memorySpace", Str("global")},
               {"mutableMemory", Bool(true)},
               {"allocShape", IntList({rows, cols})}};
  return d;
}

// Reference: MatmulSemantics.cpp:64-127 (layout truth) and :202-256. The
// IR subset accepts identity-layout memrefs only, i.e. row-major contiguous
// operands with unit minor stride, which is what the gfx950 kernels load.
MatmulSemantics deriveMatmulSemantics(const KernelConfig &c, const Op &op) {
  const char *roles[3] = {"a", "b", "c"};
  MemRefInfo info[3];
  for (int i = 0; i < 3; ++i) {
    info[i] = parseMemRef(op.operandTypes[i]);
    if (!info[i].identityLayout)
      throw Error(std::string("semantic operand `") + roles[i] +
                  "` must use the identity (row-major, zero offset) layout");
  }
  MatmulSemantics s;
  s.contractModel = "triton_matmul_semantics_v3";
  s.problemM = c.problemM;
  s.problemN = c.problemN;
  s.problemK = c.problemK;
  s.tileM = c.blockM;
  s.tileN = c.blockN;
  s.tileK = c.blockK;
  s.exactTile = c.exactTile;
  s.hasBoundaryM = c.problemM % c.blockM != 0;
  s.hasBoundaryN = c.problemN % c.blockN != 0;
  s.hasBoundaryK = c.problemK % c.blockK != 0;
  s.aDescType = semanticDesc(info[0], c.problemM, c.problemK);
  s.bDescType = semanticDesc(info[1], c.problemK, c.problemN);
  s.cDescType = semanticDesc(info[2], c.problemM, c.problemN);
  return s;
}
AttrP buildMatmulSemanticsAttr(const MatmulSemantics &s) { return buildPlanAttr(s); }
MatmulSemantics parseMatmulSemanticsAttr(const Attr &a) {
  return parsePlanAttr<MatmulSemantics>(a, "`tb.semantic_matmul`");
}

} // namespace tb
