// Triton-aligned plan structures of the tb.matmul compiler, gfx950 edition.
//
// Struct and field names mirror the reference's plan headers
// (include/tb/Analysis/*.h) because they are the API surface; each plan is
// derived by a pass and serialized as a dictionary attribute on the op
// (snake_case keys as in the reference's build*Attr functions). What changes
// for MI355X is the content of the five target-facing plans: TargetInfo
// describes gfx950; ProgramMappingPlan adds grouped persistent order and an
// XCD count; EncodingPlan carries MFMA operand layouts and 64-bank LDS
// swizzles; TransportPlan/AsyncPlan describe direct-to-LDS buffer loads
// ordered by s_waitcnt vmcnt + s_barrier; AccumulatorPlan/EpiloguePlan carry
// the MFMA 32x32 accumulator layout, the f32->f16 convert and the split-K
// workspace reduction.
#pragma once

#include "../ir/ir.h"

#include <cstdint>
#include <string>
#include <vector>

namespace tb {

using I64s = std::vector<int64_t>;

// Module context attribute names (reference TargetInfo.h:15-21,
// ProgramMappingPlan.h:14-17).
inline const char *kTarget = "tb.target";
inline const char *kNumWarps = "tb.num-warps";
inline const char *kThreadsPerWarp = "tb.threads-per-warp";
inline const char *kNumCTAs = "tb.num-ctas";
inline const char *kRequestedStages = "tb.requested-stages";
inline const char *kSplitK = "tb.split-k";
inline const char *kPersistent = "tb.persistent";
inline const char *kProgramsPerTile = "tb.programs-per-tile";
inline const char *kReductionMode = "tb.reduction-mode";

// ---- TargetInfo (reference include/tb/Analysis/TargetInfo.h:23-49) --------
struct TargetInfo {
  std::string gpuArch, targetTriple, ptxFeatures;
  int64_t threadsPerWarp = 64;
  int64_t sharedBankBytes = 4;
  int64_t numSms = 0; // compute units
  int64_t maxWarpsPerCTA = 0;
  int64_t maxRegistersPerThread = 0;
  int64_t maxRegistersPerCTA = 0;
  int64_t maxSharedBytesPerCTA = 0;
  bool supportsAsyncCopy = true;
  bool supportsLdMatrix = false;
  bool supportsMmaSync = false;
  bool supportsMBarrier = false;
  bool supportsTMA = false;
  bool supportsWGMMA = false;
  int64_t asyncCopyMinBytes = 4;
  int64_t asyncCopyMaxBytes = 16;
  int64_t asyncCopyPreferredBytes = 16;
  int64_t globalToSharedStageLatency = 2;
  int64_t sharedToRegisterStageLatency = 1;
  int64_t mmaStageLatency = 1;
  std::string preferredAsyncTransport;
  I64s mmaInstrShape;
  // gfx950 additions
  int64_t sharedBankCount = 64;   // LDS banks (x sharedBankBytes per cycle)
  int64_t numXcds = 8;            // accelerator complex dies (own L2 each)
  bool supportsMfma = true;
  bool supportsDirectToLds = true;     // buffer_load_dwordx4 ... lds
  bool supportsLdsTransposeRead = true; // ds_read_b64_tr_b16
  std::vector<I64s> mfmaInstrShapes; // f16 MFMA shapes [M, N, K]
};
TargetInfo deriveTargetInfoForArch(const std::string &gpuArch,
                                   const std::string &features);
AttrP buildTargetInfoAttr(const TargetInfo &t);
TargetInfo parseTargetInfoAttr(const Attr &a);

// ---- KernelConfig (reference KernelConfig.h:13-37) ------------------------
enum class ScalarKind { F16, F32 };
enum class MmaKind { M16N8K16, Mfma32x32x16F16, Mfma16x16x32F16 };
struct KernelConfig {
  int64_t problemM = 0, problemN = 0, problemK = 0;
  int64_t blockM = 0, blockN = 0, blockK = 0;
  int64_t numWarps = 0, requestedStages = 0, groupM = 8;
  bool exactTile = false;
  MmaKind mmaKind = MmaKind::Mfma32x32x16F16;
  ScalarKind aScalar = ScalarKind::F16, bScalar = ScalarKind::F16,
             cScalar = ScalarKind::F32;
};
const char *scalarName(ScalarKind k);
bool mfma16x16x32Supported(const KernelConfig &c);
const char *mmaKindName(MmaKind k);
int64_t scalarBytes(ScalarKind k);
KernelConfig getKernelConfig(const Module &m, const Op &matmul);
void verifySupportedKernelConfig(const KernelConfig &c, const TargetInfo *t);
// Register truth at KernelConfig legality: the instance a tb.matmul binds
// (its output mode and fused steps follow from the module's split-k and
// reduction attrs, C's type and the op's epilogue attrs) must not spill
// to scratch in the compiler's report of its build.
void verifyInstanceRegisters(const Module &m, const Op &op, const KernelConfig &c);
// The wave grid the EncodingPlan derives (reference EncodingPlan.cpp:283-320):
// minimal |wave_tile_m - wave_tile_n| over grids of whole instrM x instrN
// tiles, ties to more waves along the longer block side.
std::pair<int64_t, int64_t> deriveWaveGrid(const KernelConfig &c, int64_t instrM,
                                           int64_t instrN);

// ---- MatmulSemantics (reference MatmulSemantics.h:15-31) ------------------
struct MatmulSemantics {
  std::string contractModel;
  AttrP aDescType, bDescType, cDescType;
  int64_t problemM = 0, problemN = 0, problemK = 0;
  int64_t tileM = 0, tileN = 0, tileK = 0;
  bool exactTile = false, hasBoundaryM = false, hasBoundaryN = false,
       hasBoundaryK = false;
};
MatmulSemantics deriveMatmulSemantics(const KernelConfig &c, const Op &matmul);
AttrP buildMatmulSemanticsAttr(const MatmulSemantics &s);
MatmulSemantics parseMatmulSemanticsAttr(const Attr &a);

// ---- ProgramMappingPlan (reference ProgramMappingPlan.h:19-71) ------------
enum class ProgramMappingKind { Tile, GroupedTile, SplitK, PersistentTile };
enum class ProgramLaunchOrder { RowMajor, GroupedM, Persistent };
enum class ProgramSwizzleKind { None, GroupedM };
enum class ReductionMode { None, SplitKSerial, SplitKParallel };
struct ProgramMappingPlan {
  ProgramMappingKind mappingKind = ProgramMappingKind::Tile;
  int64_t problemTilesM = 0, problemTilesN = 0, problemTilesK = 0;
  int64_t tileM = 0, tileN = 0, tileK = 0;
  int64_t groupM = 1, groupTileSpanM = 1, groupTileSpanN = 1;
  int64_t programsPerLaunchGroup = 1, launchGroupCount = 1, totalPrograms = 1;
  int64_t splitK = 1;
  ProgramLaunchOrder launchOrder = ProgramLaunchOrder::RowMajor;
  ProgramSwizzleKind swizzleKind = ProgramSwizzleKind::None;
  bool persistent = false;
  ReductionMode reductionMode = ReductionMode::None;
  int64_t programsPerTile = 1, numCTAs = 1;
  I64s ctasPerCGA{1, 1, 1}, ctaSplitNum{1, 1, 1}, ctaOrder{0, 1, 2};
  int64_t xcdRemap = 0; // gfx950: program ids remapped across this many XCDs
};
ProgramMappingPlan deriveProgramMappingPlan(const Module &m,
                                            const KernelConfig &c,
                                            const TargetInfo &t);
AttrP buildProgramMappingPlanAttr(const ProgramMappingPlan &p);
ProgramMappingPlan parseProgramMappingPlanAttr(const Attr &a);
// pid -> (tile_m, tile_n, split part) exactly as the kernel computes it
void programToTile(const ProgramMappingPlan &p, int64_t pid, int64_t &tm,
                   int64_t &tn, int64_t &part);

// ---- ReductionPlan (reference ReductionPlan.h:15-46) ----------------------
enum class ReductionPlanKind { None, SplitKSerial, SplitKAtomic };
enum class ReductionScratchSpace { None, Global, Shared };
struct ReductionPlan {
  ReductionPlanKind kind = ReductionPlanKind::None;
  ReductionScratchSpace scratchSpace = ReductionScratchSpace::None;
  int64_t splitK = 1, kTilesPerProgram = 0, remainderKTiles = 0;
  int64_t partialTileRows = 0, partialTileCols = 0;
  int64_t producerProgramsPerTile = 1, finalReducerPrograms = 1;
  int64_t scratchRows = 0, scratchCols = 0, scratchBytes = 0;
  bool requiresInterProgramReduction = false;
  std::string partialOwner = "none", finalExecutor = "none", reason;
};
ReductionPlan deriveReductionPlan(const KernelConfig &c,
                                  const ProgramMappingPlan &pm);
AttrP buildReductionPlanAttr(const ReductionPlan &p);
ReductionPlan parseReductionPlanAttr(const Attr &a);

// ---- PersistentWorkPlan (reference PersistentWorkPlan.h:15-37) ------------
enum class PersistentWorkKind { None, TileStrideLoop };
struct PersistentWorkPlan {
  PersistentWorkKind kind = PersistentWorkKind::None;
  bool enabled = false;
  int64_t residentPrograms = 1, programsPerWave = 1, tileBatchSize = 1;
  int64_t maxTilesPerProgram = 1, totalWorkItems = 1, loopStride = 1;
  bool requiresOuterSerialLoop = false;
  std::string tileOrder = "row_major", ownerScope = "none",
              completion = "single_tile", reason;
};
PersistentWorkPlan derivePersistentWorkPlan(const KernelConfig &c,
                                            const TargetInfo &t,
                                            const ProgramMappingPlan &pm);
AttrP buildPersistentWorkPlanAttr(const PersistentWorkPlan &p);
PersistentWorkPlan parsePersistentWorkPlanAttr(const Attr &a);

// ---- EncodingPlan (reference EncodingPlan.h:19-62) ------------------------
struct FragmentEncodingSpec {
  std::string role;
  I64s instructionShape, repeatShape, logicalShape, registerShape, registerOrder;
  int64_t laneRowModulus = 0, laneColDivisor = 0, laneColStride = 0;
  int64_t valuesPerLane = 0;
  // LDS reads per fragment and whether they transpose (gfx950: A = one
  // ds_read_b128, B = two ds_read_b64_tr_b16)
  int64_t ldmatrixTileCount = 0;
  bool ldmatrixTranspose = false;
};
struct EncodingEntry {
  std::string name;
  AttrP encodingAttr;
};
struct SharedEncodingSpec {
  I64s logicalShape, allocShape;
};
struct EncodingPlan {
  std::string contractModel;
  SharedEncodingSpec aSharedSpec, bSharedSpec;
  FragmentEncodingSpec fragmentA, fragmentB, fragmentAcc;
  std::vector<EncodingEntry> encodings;
  int aGlobal = -1, bGlobal = -1, aShared = -1, bShared = -1, aDot = -1,
      bDot = -1, acc = -1, cStore = -1;
};
EncodingPlan deriveEncodingPlan(const KernelConfig &c, const TargetInfo &t,
                                const MatmulSemantics &s,
                                const ProgramMappingPlan &pm);
AttrP buildEncodingPlanAttr(const EncodingPlan &p);
EncodingPlan parseEncodingPlanAttr(const Attr &a);
const Attr &encodingAttr(const EncodingPlan &p, int id, const char *role);
I64s mmaWarpsPerCTA(const EncodingPlan &p);
I64s accumulatorTileShape(const EncodingPlan &p);
// swizzle parameters of a #tb.shared encoding
struct SharedSwizzle {
  I64s order;
  int64_t perPhase = 1, maxPhase = 1, swizzlingByteWidth = 0;
  bool transposed = false;
  // gfx950: a second XOR term, on units of secondSwizzlingByteWidth inside a
  // first-term unit, phase (row / secondPerPhase) % secondMaxPhase
  // (secondMaxPhase <= 1: none)
  int64_t secondPerPhase = 0, secondMaxPhase = 0, secondSwizzlingByteWidth = 0;
};
SharedSwizzle sharedSwizzle(const Attr &shared);

// ---- TransportPlan (reference TransportPlan.h:15-34) ----------------------
struct TransportSpec {
  std::string role;
  int64_t dstEncoding = -1;
  std::string kind;
  int64_t vectorBytes = 0, asyncVectorBytes = 0, transactionBytes = 0;
  bool asyncEligible = false, bypassL1 = false;
  std::string cachePolicy;
};
struct TransportPlan {
  std::string contractModel;
  TransportSpec operandA, operandB;
};
TransportPlan deriveTransportPlan(const KernelConfig &c, const TargetInfo &t,
                                  const EncodingPlan &e);
AttrP buildTransportPlanAttr(const TransportPlan &p);
TransportPlan parseTransportPlanAttr(const Attr &a);

// ---- AccumulatorPlan (reference AccumulatorPlan.h:15-44) ------------------
struct LaneAccessPattern {
  int64_t laneRowGroupSize = 0, laneColGroupSize = 0, laneColStride = 0;
  I64s rowOffsets;
};
struct AccumulatorPack {
  int64_t packId = 0, rowBase = 0, colBase = 0, rows = 0, cols = 0;
  int64_t elemCount = 0, vectorWidth = 0, warpOwner = 0, mmaGroup = -1,
          epiloguePack = -1;
};
struct AccumulatorPlan {
  int encoding = -1;
  int64_t registersPerWarp = 0;
  std::string ownerScope = "per_warp_template";
  LaneAccessPattern laneAccess;
  std::vector<AccumulatorPack> packs;
  bool liveAcrossStages = false;
  int64_t multiBufferDepth = 1;
};
AccumulatorPlan deriveAccumulatorPlan(const KernelConfig &c, const TargetInfo &t,
                                      const EncodingPlan &e);
AttrP buildAccumulatorPlanAttr(const AccumulatorPlan &p);
AccumulatorPlan parseAccumulatorPlanAttr(const Attr &a);

// ---- EpiloguePlan (reference EpiloguePlan.h:16-114) -----------------------
enum class AccumulatorInitMode { Zero, DirectGlobalVector, SharedRelay };
enum class AccumulatorStoreMode { DirectGlobalVector, SharedRelay };
enum class TargetLandingKind { None, RegisterPackGlobalVector,
                               SharedPackThenGlobalVector,
                               SharedRelayThenGlobalVector };
enum class EpilogueExprKind { LoadBias, Add, Convert, Activation, Clamp };
struct DirectPack {
  int64_t packId = 0, rowBase = 0, colBase = 0, rows = 0, cols = 0;
  int64_t vectorWidth = 0, warpOwner = 0;
  I64s fragmentIds;
};
struct DirectGlobalVectorPlan {
  bool present = false;
  std::string ownerScope = "per_warp_template";
  LaneAccessPattern laneAccess;
  std::vector<DirectPack> packs;
  int64_t vectorWidth = 0;
  bool boundaryAware = false, scalarTail = false;
};
struct EpilogueExprOp {
  EpilogueExprKind kind = EpilogueExprKind::Add;
  ScalarKind inputScalar = ScalarKind::F32, outputScalar = ScalarKind::F32;
  int64_t vectorWidth = 0;
  std::string aux;
};
struct TargetLandingPlan {
  TargetLandingKind kind = TargetLandingKind::None;
  int64_t globalVectorWidth = 0, globalAccessBytes = 0;
  int64_t producerFragmentRows = 0, producerFragmentCols = 0;
  int64_t directPackRows = 0, directPackCols = 0, warpBatchingGroup = 0;
  int64_t requiredSharedBytes = 0, expectedRegisterFootprint = 0;
  int64_t sharedTileRows = 0, sharedTileCols = 0, sharedPackSlots = 0;
  int64_t initSharedStoreVectorWidth = 0, initSharedLoadVectorWidth = 0;
  int64_t storeSharedStoreVectorWidth = 0, storeSharedLoadVectorWidth = 0;
  bool useSharedPackForInit = false, useSharedPackForStore = false;
  std::string requiredSyncKind = "none", reason;
};
struct EpiloguePlan {
  AccumulatorInitMode initMode = AccumulatorInitMode::Zero;
  AccumulatorStoreMode storeMode = AccumulatorStoreMode::DirectGlobalVector;
  DirectGlobalVectorPlan init, store; // init.present == false for Zero
  TargetLandingPlan targetLanding;
  std::vector<EpilogueExprOp> exprs;
};
// Fused epilogue steps requested on tb.matmul through the optional attrs
// `epilogue_bias` ("f16" | "f32": a length-N vector added to every row),
// `epilogue_activation` ("relu" | "gelu_tanh" | "silu"), `epilogue_clamp_min`
// and `epilogue_clamp_max` (f32). The reference declares the expr kinds
// (include/tb/Analysis/EpiloguePlan.h:61-75, serialized at
// lib/Analysis/EpiloguePlan.cpp:423-459) but never derives them and gives
// tb.matmul no way to ask for them; these attrs are that surface. The steps
// always apply in the order bias, activation, clamp, then the C conversion.
struct EpilogueRequest {
  std::string bias;       // "", "f16" or "f32"
  std::string activation; // "", "relu", "gelu_tanh" or "silu"
  bool hasMin = false, hasMax = false;
  double clampMin = 0.0, clampMax = 0.0;
  bool empty() const { return bias.empty() && activation.empty() && !hasMin && !hasMax; }
};
// From the tb.matmul attrs (validated; an op without them gives an empty request).
EpilogueRequest parseEpilogueRequest(const Op &matmul);
// Back from a derived plan's exprs (validated: canonical order, known kinds).
EpilogueRequest epilogueRequestOf(const EpiloguePlan &p);

EpiloguePlan deriveEpiloguePlan(const KernelConfig &c, const TargetInfo &t,
                                const EncodingPlan &e, const AccumulatorPlan &a,
                                const EpilogueRequest &req = {});
AttrP buildEpiloguePlanAttr(const EpiloguePlan &p);
EpiloguePlan parseEpiloguePlanAttr(const Attr &a);

// ---- EpilogueReorderPlan (reference EpilogueReorderPlan.h:17-53) ----------
enum class EpilogueReorderKind { None, CTASharedRowReorder, CTASharedRelay };
struct EpilogueRowVectorMapping {
  int64_t rowVectorId = -1, packId = -1, warpOwner = -1, rowBase = 0,
          colBase = 0, rowOffset = 0, vectorWidth = 0;
  I64s fragmentIds;
};
struct EpilogueReorderPlan {
  EpilogueReorderKind kind = EpilogueReorderKind::None;
  int64_t sharedTileRows = 0, sharedTileCols = 0, liveSlots = 0;
  int64_t initSharedStoreVectorWidth = 0, initSharedLoadVectorWidth = 0;
  int64_t storeSharedStoreVectorWidth = 0, storeSharedLoadVectorWidth = 0;
  int64_t workspaceBarrierCount = 0;
  bool requiresWarpSync = false, reorderNeededForInit = false,
       reorderNeededForStore = false;
  std::string ownerScope = "none", workspaceSyncKind = "none", reason;
  std::vector<EpilogueRowVectorMapping> rowVectors;
};
EpilogueReorderPlan deriveEpilogueReorderPlan(const KernelConfig &c,
                                              const AccumulatorPlan &a,
                                              const EpiloguePlan &e);
AttrP buildEpilogueReorderPlanAttr(const EpilogueReorderPlan &p);
EpilogueReorderPlan parseEpilogueReorderPlanAttr(const Attr &a);

// ---- SharedWorkspacePlan (reference SharedWorkspacePlan.h:22-62) ----------
enum class SharedWorkspaceSegmentKind { MainloopAStageBuffer, MainloopBStageBuffer,
                                        EpilogueReorderScratch,
                                        SplitKReductionScratch,
                                        PersistentStateScratch };
struct SharedWorkspaceSegment {
  SharedWorkspaceSegmentKind kind = SharedWorkspaceSegmentKind::MainloopAStageBuffer;
  std::string name;
  int64_t byteOffset = 0, byteSize = 0, byteAlignment = 1;
  int64_t logicalRows = 0, logicalCols = 0, stageCount = 1, slotCount = 1,
          warpReplicas = 1, lifetimeBegin = 0, lifetimeEnd = 0;
  bool aliasAllowed = false;
  int64_t aliasSet = -1;
  std::string producer, consumer;
};
struct SharedWorkspacePlan {
  std::string contractModel;
  int64_t totalBytes = 0, peakBytes = 0, aliasSavedBytes = 0;
  std::string selectedPolicy, reason;
  std::vector<SharedWorkspaceSegment> segments;
};
SharedWorkspacePlan deriveSharedWorkspacePlan(
    const KernelConfig &c, const TargetInfo &t, const EncodingPlan &e,
    const TransportPlan &tr, const EpilogueReorderPlan &ro,
    const ReductionPlan &rd, const PersistentWorkPlan &pw);
AttrP buildSharedWorkspacePlanAttr(const SharedWorkspacePlan &p);
SharedWorkspacePlan parseSharedWorkspacePlanAttr(const Attr &a);

// ---- WarpDecompositionPlan (reference WarpDecompositionPlan.h:18-57) ------
struct WarpTileCoverage {
  int64_t warpId = -1, coordM = -1, coordN = -1, tileBaseM = 0, tileBaseN = 0,
          tileRows = 0, tileCols = 0;
  I64s mmaGroupIds, accumulatorPackIds, epiloguePackIds, sharedPackIds,
      reorderRowVectorIds, fragmentToRowVectorMap, rowVectorStoreOrder,
      rowVectorLoadOrder, reorderTileBase;
  bool reorderNeedsShared = false;
  I64s reductionPartialIds, persistentBatchIds;
};
struct WarpDecompositionPlan {
  I64s ctaTile;
  int64_t numWarps = 0;
  I64s warpGrid, warpTile;
  std::string ownerScope = "per_warp_template", warpOrder = "row_major",
              landingOwner = "register_pack", reorderOwner = "none",
              reductionOwner = "none", persistentOwner = "none";
  std::vector<WarpTileCoverage> warps;
};
WarpDecompositionPlan deriveWarpDecompositionPlan(
    const KernelConfig &c, const EncodingPlan &e, const AccumulatorPlan &a,
    const EpiloguePlan &ep, const EpilogueReorderPlan &ro,
    const ReductionPlan &rd, const PersistentWorkPlan &pw);
AttrP buildWarpDecompositionPlanAttr(const WarpDecompositionPlan &p);
WarpDecompositionPlan parseWarpDecompositionPlanAttr(const Attr &a);

// ---- ResourceClosurePlan (reference ResourceClosurePlan.h:21-51) ----------
struct ResourceClosurePlan {
  int64_t estimatedAccumulatorRegs = 0, estimatedEpilogueRegs = 0,
          estimatedABShared = 0, estimatedEpilogueShared = 0,
          estimatedReductionScratch = 0, estimatedPersistentState = 0,
          estimatedTotalStaticShared = 0, estimatedTotalDynamicShared = 0,
          estimatedTotalRegs = 0, peakStaticSharedBytes = 0,
          workspaceTotalBytes = 0, workspaceAliasSavedBytes = 0,
          reorderSharedBytes = 0, reductionSharedBytes = 0,
          persistentSharedBytes = 0, mainloopSharedLiveBegin = 0,
          mainloopSharedLiveEnd = 0, epilogueReorderLiveBegin = 0,
          epilogueReorderLiveEnd = 0, staticSharedBudget = 0,
          dynamicSharedBudget = 0;
  std::string selectedMainlineKind, selectedCLandingKind, selectedBufferingKind,
      selectedSharedWorkspacePolicy, chosenLandingTradeoff,
      chosenBufferingTradeoff, reason;
  int64_t globalWorkspaceBytes = 0; // gfx950: split-K f32 partials in HBM
};
ResourceClosurePlan deriveResourceClosurePlan(
    const KernelConfig &c, const TargetInfo &t, const ProgramMappingPlan &pm,
    const ReductionPlan &rd, const PersistentWorkPlan &pw,
    const AccumulatorPlan &a, const EpiloguePlan &ep,
    const EpilogueReorderPlan &ro, const SharedWorkspacePlan &sw,
    const WarpDecompositionPlan &wd);
AttrP buildResourceClosurePlanAttr(const ResourceClosurePlan &p);
ResourceClosurePlan parseResourceClosurePlanAttr(const Attr &a);

// ---- MatmulRewritePlan (reference MatmulRewritePlan.h:17-44) --------------
struct OperandFragmentPath {
  std::string role;
  I64s instructionShape, fragmentShape;
  int64_t fragmentsPerKGroup = 0, consumerTileSpanM = 1, consumerTileSpanN = 1;
  bool usesLdMatrix = false; // gfx950: fragment comes from LDS reads
};
struct MatmulRewritePlan {
  std::string contractModel, mainloopKind;
  int64_t instructionM = 0, instructionN = 0, instructionK = 0, kGroups = 0;
  int64_t accTilesM = 0, accTilesN = 0, bGroupCount = 0, accumulatorFragments = 0;
  bool directAccumulatorInit = false, directAccumulatorStore = false;
  OperandFragmentPath aPath, bPath;
  // gfx950: a k group is one LDS stage fill (block_k deep) holding
  // kStepsPerGroup MFMA k steps
  int64_t kGroupDepth = 0, kStepsPerGroup = 1;
};
MatmulRewritePlan deriveMatmulRewritePlan(const KernelConfig &c,
                                          const EncodingPlan &e,
                                          const AccumulatorPlan &a,
                                          const EpiloguePlan &ep);
AttrP buildMatmulRewritePlanAttr(const MatmulRewritePlan &p);
MatmulRewritePlan parseMatmulRewritePlanAttr(const Attr &a);

// ---- BufferModel (reference BufferModel.h:19-119) -------------------------
enum class MemorySpace { Global, Shared, Registers };
enum class BufferRole { OperandA, OperandB, Output, Accumulator, EpilogueRelay,
                        Descriptor, Generic };
enum class ViewKind { FullBuffer, StageSlice, TileSlice, Fragment, Pack };
enum class BufferValueKind { GlobalTile, SharedTile, DotOperandFragment,
                             AccumulatorFragment, EpilogueFragment };
enum class BufferOpKind { LoadA, LoadB, LocalLoadA, LocalLoadB, Mma,
                          AccumulatorInit, AccumulatorStore };
enum class PipelineOpSemanticClass { AsyncProducer, SharedConsumer,
                                     TensorCoreCompute, EpilogueInit,
                                     EpilogueStore };
struct BufferBacking {
  int64_t id = -1;
  BufferRole role = BufferRole::Generic;
  AttrP descType;
  int64_t depth = 1, aliasGroup = -1;
  bool stageIndexed = false;
  std::string debugName;
};
struct BufferView {
  int64_t id = -1, backing = -1;
  ViewKind kind = ViewKind::FullBuffer;
  int64_t stage = -1, bufferIndex = -1;
  int encoding = -1;
  I64s offsets, shape;
  std::string debugName;
};
struct ValueState {
  int64_t id = -1;
  BufferValueKind kind = BufferValueKind::SharedTile;
  int64_t definingOp = -1;
  I64s users;
  int64_t ownerView = -1, loopDistance = 0, bundle = -1, firstUseOrdinal = -1,
          lastUseOrdinal = -1;
  std::string debugName;
};
struct IterationCoord {
  std::string axis;
  int64_t value = -1;
};
struct PipelineOp {
  int64_t id = -1;
  BufferOpKind kind = BufferOpKind::Mma;
  I64s inputs, outputs;
  std::vector<IterationCoord> iterationCoords;
};
struct BufferModel {
  std::vector<BufferBacking> backings;
  std::vector<BufferView> views;
  std::vector<ValueState> values;
  std::vector<PipelineOp> ops;
};
const char *bufferOpKindName(BufferOpKind k);
PipelineOpSemanticClass semanticClass(BufferOpKind k);
int64_t iterationCoord(const PipelineOp &op, const std::string &axis);
BufferModel deriveBufferModel(const KernelConfig &c, const EncodingPlan &e,
                              const AccumulatorPlan &a, const EpiloguePlan &ep,
                              const MatmulRewritePlan &rw);
AttrP buildBufferModelAttr(const BufferModel &m);
BufferModel parseBufferModelAttr(const Attr &a);

// ---- LoopPlan (reference LoopPlan.h:15-34) --------------------------------
struct LoopIterationPlan {
  int64_t kGroup = -1;
  I64s asyncProducerOps, consumerOps, computeOps;
};
struct LoopCarriedValue {
  int64_t valueId = -1, definingOp = -1, ownerView = -1, loopDistance = 0;
  I64s users;
  std::string reason;
};
struct LoopPlan {
  std::string loopAxis;
  int64_t iterationCount = 0;
  bool singleMainLoop = false;
  std::vector<LoopIterationPlan> iterations;
  std::vector<LoopCarriedValue> carriedValues;
  // gfx950: the plan models a steady-state window of `iterations.size()`
  // k groups; the kernel runs the loop `iterationCount` times
  int64_t templateIterations = 0;
};
LoopPlan deriveLoopPlan(const BufferModel &m, const MatmulRewritePlan &rw);
AttrP buildLoopPlanAttr(const LoopPlan &p);
LoopPlan parseLoopPlanAttr(const Attr &a);

// ---- LatencyPlan (reference LatencyPlan.h:16-29) --------------------------
struct OpLatencyInfo {
  int64_t opId = -1, targetLatency = 0, selfLatency = 0, bufferDistance = 0;
  bool pipelineable = false, accMultiBuffer = false;
  std::string reason;
};
struct LatencyPlan {
  std::vector<OpLatencyInfo> ops;
};
LatencyPlan deriveLatencyPlan(const KernelConfig &c, const TargetInfo &t,
                              const BufferModel &m, const LoopPlan &l);
AttrP buildLatencyPlanAttr(const LatencyPlan &p);
LatencyPlan parseLatencyPlanAttr(const Attr &a);

// ---- PipelinePlan (reference PipelinePlan.h:16-37) ------------------------
struct PipelinePlacement {
  int64_t opId = -1, stage = 0, cluster = 0, order = 0;
  std::string reason;
};
struct StageBufferUse {
  int64_t viewId = -1, backing = -1, stage = -1, bufferIndex = -1,
          producerOp = -1, firstConsumerOp = -1, lastConsumerOp = -1;
};
struct PipelinePlan {
  int64_t scheduledMaxStage = 0;
  std::vector<PipelinePlacement> placements;
  std::vector<StageBufferUse> stageOwnedBuffers;
};
PipelinePlan derivePipelinePlan(const BufferModel &m, const LoopPlan &l,
                                const LatencyPlan &lat);
AttrP buildPipelinePlanAttr(const PipelinePlan &p);
PipelinePlan parsePipelinePlanAttr(const Attr &a);

// ---- AsyncPlan (reference AsyncPlan.h:17-91) ------------------------------
enum class AsyncProducerKind { CpAsync, TMA, BulkCopy, SyncCopyFallback,
                               BufferLoadLds };
enum class AsyncBarrierKind { AsyncGroup, CTA, MBarrier, None, VmcntBarrier };
enum class AsyncCachePolicy { Default, BypassL1, CacheAll };
struct AsyncProducer {
  int64_t opId = -1;
  AsyncProducerKind kind = AsyncProducerKind::BufferLoadLds;
  int64_t valueId = -1, srcView = -1, dstView = -1;
  I64s srcOffsets;
  int64_t groupId = -1, vecBytes = 0, transactionBytes = 0;
  bool zeroFill = false, predicated = false, bypassL1 = false;
  AsyncBarrierKind barrierKind = AsyncBarrierKind::VmcntBarrier;
  AsyncCachePolicy cachePolicy = AsyncCachePolicy::Default;
  bool legal = false;
  std::string reason;
};
struct AsyncGroup {
  int64_t id = -1;
  I64s producers;
};
struct WaitInfo {
  int64_t groupId = -1, beforeOpId = -1, requiredStage = -1,
          requiredCluster = -1, requiredOrder = -1;
  bool needsBarrier = true;
  std::string reason;
  int64_t vmcntAllowance = 0;  // gfx950: s_waitcnt vmcnt(N) outstanding loads
  int64_t lgkmcntAllowance = -1; // gfx950: s_waitcnt lgkmcnt(N) with the barrier
                                 // (-1: none; the compiler orders LDS reads)
};
struct ReuseFence {
  int64_t viewId = -1, backing = -1, retiringValueId = -1, acquiringValueId = -1,
          afterOpId = -1, requiredAfterStage = -1, requiredAfterCluster = -1,
          requiredAfterOrder = -1;
  std::string reason;
};
struct AsyncPlan {
  std::vector<AsyncProducer> producers;
  std::vector<AsyncGroup> groups;
  std::vector<WaitInfo> waits;
  std::vector<ReuseFence> reuseFences;
  // gfx950: how the bound kernel instance issues its loads, from which the
  // waits' depths follow (instances.h, InstanceSchedule)
  std::string issueSchedule;
  int64_t loadsPerThread = 0, prologueTailLoads = 0, refillSpreadSlots = 0;
  int64_t loaderWaves = 0; // load-only waves beside the wave grid ("producer_waves")
};
// `out` (InstanceOut) and `epi` name the instance flavour the lowering binds
// (instanceOutOf), which with the tile decides the issue schedule.
AsyncPlan deriveAsyncPlan(const KernelConfig &c, const BufferModel &m,
                          const TransportPlan &tr, const LatencyPlan &lat,
                          const PipelinePlan &pp, int out, bool epi);
AttrP buildAsyncPlanAttr(const AsyncPlan &p);
AsyncPlan parseAsyncPlanAttr(const Attr &a);

// ---- PipelineExpansion (reference PipelineExpansion.h:16-41) --------------
enum class ExpandedClusterKind { AsyncIssue, ConsumerWait, MmaCompute };
struct ExpandedCluster {
  int64_t ordinal = -1, stage = -1, cluster = -1, kGroup = -1;
  ExpandedClusterKind kind = ExpandedClusterKind::AsyncIssue;
  I64s opIds, waitGroupIds;
  bool needsBarrier = false;
  std::string reason;
};
struct PipelineExpansion {
  std::vector<ExpandedCluster> clusters;
};
PipelineExpansion derivePipelineExpansion(const BufferModel &m,
                                          const PipelinePlan &pp,
                                          const AsyncPlan &ap);
AttrP buildPipelineExpansionAttr(const PipelineExpansion &p);
PipelineExpansion parsePipelineExpansionAttr(const Attr &a);

// ---- PipelineReady (reference PipelineReady.h:11-15) ----------------------
struct PipelineReady {
  int64_t scheduledMaxStage = 0, asyncGroups = 0, requestedStages = 0;
};
AttrP buildPipelineReadyAttr(const PipelineReady &p);
PipelineReady parsePipelineReadyAttr(const Attr &a);

// ---- KernelContract (reference KernelContract.h:31-52) --------------------
struct KernelContract {
  KernelConfig kernel;
  MatmulSemantics semantics;
  TargetInfo target;
  ProgramMappingPlan programMapping;
  ReductionPlan reduction;
  PersistentWorkPlan persistentWork;
  EncodingPlan encodings;
  TransportPlan transport;
  MatmulRewritePlan rewrite;
  BufferModel buffers;
  PipelineReady pipelineReady;
  AsyncPlan async;
  AccumulatorPlan accumulator;
  EpiloguePlan epilogue;
  EpilogueReorderPlan epilogueReorder;
  SharedWorkspacePlan sharedWorkspace;
  WarpDecompositionPlan warpDecomposition;
  ResourceClosurePlan resourceClosure;
};
// Reads the public plan attributes of a tb.pipeline_mainline op.
KernelContract parseKernelContract(const Module &m, const Op &mainline);

// ---- helpers shared by the plan files --------------------------------------
inline int64_t ceilDiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
const Attr &opAttr(const Op &op, const std::string &name);
std::map<std::string, AttrP> dictOf(const Attr &a);

} // namespace tb
