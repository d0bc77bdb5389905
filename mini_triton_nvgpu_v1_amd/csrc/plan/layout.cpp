// EncodingPlan (wave grid, MFMA fragments, LDS swizzles) and TransportPlan.
#include "serialize.h"

#include <algorithm>
#include <numeric>
#include <cstdlib>
#include <limits>

namespace tb {

template <class V> void fields(V &v, SharedEncodingSpec &s) {
  v("logical_shape", s.logicalShape);
  v("alloc_shape", s.allocShape);
}
template <class V> void fields(V &v, FragmentEncodingSpec &s) {
  v("role", s.role);
  v("instruction_shape", s.instructionShape);
  v("repeat_shape", s.repeatShape);
  v("logical_shape", s.logicalShape);
  v("register_shape", s.registerShape);
  v("register_order", s.registerOrder);
  v("lane_row_modulus", s.laneRowModulus);
  v("lane_col_divisor", s.laneColDivisor);
  v("lane_col_stride", s.laneColStride);
  v("values_per_lane", s.valuesPerLane);
  v("ldmatrix_tile_count", s.ldmatrixTileCount);
  v("ldmatrix_transpose", s.ldmatrixTranspose);
}
template <class V> void fields(V &v, EncodingEntry &e) {
  v("name", e.name);
  v("encoding", e.encodingAttr);
}
template <class V> void fields(V &v, EncodingPlan &p) {
  v("contract_model", p.contractModel);
  v("a_shared_spec", p.aSharedSpec);
  v("b_shared_spec", p.bSharedSpec);
  v("fragment_a", p.fragmentA);
  v("fragment_b", p.fragmentB);
  v("fragment_acc", p.fragmentAcc);
  v("encodings", p.encodings);
  v("a_global", p.aGlobal);
  v("b_global", p.bGlobal);
  v("a_shared", p.aShared);
  v("b_shared", p.bShared);
  v("a_dot", p.aDot);
  v("b_dot", p.bDot);
  v("acc", p.acc);
  v("c_store", p.cStore);
}

// Reference: EncodingPlan.cpp:283-320. Minimise |wave_tile_m - wave_tile_n|
// over wave grids whose wave tiles are whole MFMA tiles; ties go to more
// waves along the longer block side (M for a square block, which the
// reference's two_warp_shape_closure_contract test pins).
std::pair<int64_t, int64_t> deriveWaveGrid(const KernelConfig &c, int64_t instrM,
                                           int64_t instrN) {
  int64_t bestM = -1, bestN = -1, bestScore = std::numeric_limits<int64_t>::max();
  for (int64_t gm = 1; gm <= c.numWarps; ++gm) {
    if (c.numWarps % gm)
      continue;
    int64_t gn = c.numWarps / gm;
    if (c.blockM % gm || c.blockN % gn)
      continue;
    int64_t tm = c.blockM / gm, tn = c.blockN / gn;
    if (tm % instrM || tn % instrN)
      continue;
    int64_t score = std::llabs(tm - tn);
    bool tieWins = score == bestScore &&
                   ((c.blockM >= c.blockN && gm > bestM) ||
                    (c.blockM < c.blockN && gn > bestN));
    if (score < bestScore || tieWins) {
      bestScore = score;
      bestM = gm;
      bestN = gn;
    }
  }
  if (bestM <= 0)
    throw Error("failed to derive a legal wave grid from module num-warps, block "
                "shape and MFMA instruction shape");
  return {bestM, bestN};
}

// gfx950 LDS swizzle heuristic. The reference (EncodingPlan.cpp:340-379)
// sizes the phase period by the 128-byte bank period of its target; gfx950
// LDS serves 64 banks x 4 bytes = 256 bytes per cycle, i.e. 16 lanes of a
// 16-byte ds_read_b128 or 32 lanes of an 8-byte ds_read_b64_tr_b16. The XOR
// unit is the bytes one lane group reads contiguously from a row:
//  * A ([block_m][block_k], read row-wise with ds_read_b128): 16 bytes,
//    phases = 16-byte chunks per row, rows per phase = rows per 256 bytes;
//  * B ([block_k][block_n], read with transposing ds_read_b64_tr_b16, two
//    16-lane groups covering 32 columns = 64 bytes of a row): 64 bytes,
//    phases = min(256 / 64, 64-byte segments per row).
// Rows per phase: rows before a row's bank offset repeats, period / gcd(row
// bytes, period) (period / row bytes for power-of-two rows under the period,
// 1 from the period up, 2 for 384-byte rows). Phases: at most period / unit
// and a power of two dividing the units per row, so a unit XOR-ed with the
// phase stays inside its row (the reference keeps it inside with a modulo,
// LowerPipelineToNVGPU.cpp:1589-1621; a power of two needs none).
static SharedSwizzle deriveSwizzle(const TargetInfo &t, int64_t rowBytes,
                                   int64_t unitBytes) {
  SharedSwizzle s;
  s.order = {1, 0};
  int64_t period = t.sharedBankCount * t.sharedBankBytes;
  if (rowBytes < unitBytes || rowBytes % unitBytes)
    return s;
  s.swizzlingByteWidth = unitBytes;
  s.perPhase = period / std::gcd(rowBytes, period);
  const int64_t units = rowBytes / unitBytes;
  s.maxPhase = std::max<int64_t>(1, std::min(units & -units, period / unitBytes));
  return s;
}

SharedSwizzle sharedSwizzle(const Attr &shared) {
  if (shared.kind != AttrKind::Dialect || shared.s != "shared")
    throw Error("expected a #tb.shared encoding");
  SharedSwizzle s;
  s.order = paramInts(shared, "order");
  s.perPhase = paramI64(shared, "perPhase");
  s.maxPhase = paramI64(shared, "maxPhase");
  s.transposed = paramBool(shared, "transposed");
  s.swizzlingByteWidth = paramI64(shared, "swizzlingByteWidth");
  for (const auto &kv : shared.params)
    if (kv.first == "secondPerPhase") {
      s.secondPerPhase = paramI64(shared, "secondPerPhase");
      s.secondMaxPhase = paramI64(shared, "secondMaxPhase");
      s.secondSwizzlingByteWidth = paramI64(shared, "secondSwizzlingByteWidth");
    }
  return s;
}

const Attr &encodingAttr(const EncodingPlan &p, int id, const char *role) {
  if (id < 0 || id >= (int)p.encodings.size() || !p.encodings[id].encodingAttr)
    throw Error(std::string("encoding plan has no `") + role + "` encoding");
  return *p.encodings[id].encodingAttr;
}

I64s mmaWarpsPerCTA(const EncodingPlan &p) {
  return paramInts(param(encodingAttr(p, p.acc, "acc"), "parent"), "warpsPerCTA");
}
I64s accumulatorTileShape(const EncodingPlan &p) { return p.fragmentAcc.logicalShape; }

// Reference: EncodingPlan.cpp:400-575 (layout freeze). gfx950 content:
//  * one LDS stage holds a whole block_k slab: A [block_m][block_k] and
//    B [block_k][block_n], both row-major with the swizzles above;
//  * v_mfma_f32_32x32x16_f16 operand layouts: lane l holds
//    A[l % 32][8 (l / 32) .. +7] (one ds_read_b128) and
//    B[8 (l / 32) .. +7][l % 32] (two ds_read_b64_tr_b16);
//  * the accumulator is computed transposed (B fragment as the MFMA's first
//    source) so that lane l holds C[l % 32][8 g + 4 (l / 32) + r], g, r in
//    0..3: 16 f32 values as 4 groups of 4 consecutive columns, which the
//    epilogue stores as 4 vectors of 4 elements per 32x32 tile.
EncodingPlan deriveEncodingPlan(const KernelConfig &c, const TargetInfo &t,
                                const MatmulSemantics &s,
                                const ProgramMappingPlan &pm) {
  for (const AttrP &d : {s.aDescType, s.bDescType, s.cDescType}) {
    if (!d || d->typeDialect != "memdesc")
      throw Error("semanticization must provide !tb.memdesc operands");
    const Attr &layout = param(*d, "encoding");
    if (!paramBool(layout, "zeroOffset") || !paramBool(layout, "hasStaticStrides") ||
        !paramBool(layout, "unitStrideOnMinor"))
      throw Error("layout freeze requires zero-offset, statically strided operands "
                  "with unit stride on the minor dimension");
  }
  // the wave grid is chosen on 32x32 MFMA tiles whatever the instruction,
  // so both instructions see the same wave tiles
  auto [gm, gn] = deriveWaveGrid(c, t.mmaInstrShape[0], t.mmaInstrShape[1]);
  const I64s instr = c.mmaKind == MmaKind::Mfma16x16x32F16 ? I64s{16, 16, 32}
                                                           : t.mmaInstrShape;
  const int64_t iM = instr[0], iN = instr[1], iK = instr[2];
  const int64_t wtM = c.blockM / gm, wtN = c.blockN / gn;
  const int64_t elem = scalarBytes(c.aScalar);
  const int64_t lanes = t.threadsPerWarp;

  EncodingPlan p;
  p.contractModel = "strict_v2_layout_owner";
  p.aSharedSpec = {{c.blockM, c.blockK}, {c.blockM, c.blockK}};
  p.bSharedSpec = {{c.blockK, c.blockN}, {c.blockK, c.blockN}};
  const int64_t kPerLane = iK * iM / lanes; // 8 f16 per lane per operand
  p.fragmentA = {"a", {iM, iK}, {wtM / iM, c.blockK / iK}, {wtM, c.blockK},
                 {1, kPerLane}, {1, 0}, iM, iM, kPerLane, kPerLane,
                 /*ds reads*/ 1, /*transpose*/ false};
  p.fragmentB = {"b", {iK, iN}, {c.blockK / iK, wtN / iN}, {c.blockK, wtN},
                 {kPerLane, 1}, {0, 1}, iN, iN, kPerLane, kPerLane, 2, true};
  p.fragmentAcc = {"acc", {iM, iN}, {wtM / iM, wtN / iN}, {wtM, wtN},
                   {4, 4}, {0, 1}, iM, iM, 4, iM * iN / lanes, 0, false};

  AttrP cga = Dialect("cga", {{"ctasPerCGA", IntList(pm.ctasPerCGA)},
                              {"ctaSplitNum", IntList(pm.ctaSplitNum)},
                              {"ctaOrder", IntList(pm.ctaOrder)}});
  AttrP mfma = Dialect("amd_mfma", {{"versionMajor", IntU(4)},
                                    {"versionMinor", IntU(0)},
                                    {"warpsPerCTA", IntList({gm, gn})},
                                    {"instrShape", IntList(instr)},
                                    {"isTransposed", Bool(true)},
                                    {"cga", cga}});
  auto add = [&](const std::string &name, AttrP a) {
    p.encodings.push_back({name, a});
    return (int)p.encodings.size() - 1;
  };
  // global-side layouts: one 16-byte vector (8 f16) per lane, consecutive
  // lanes along the contiguous dimension
  auto blocked = [&](int64_t cols, I64s warps) {
    int64_t chunks = std::max<int64_t>(1, std::min(lanes, cols / 8));
    return Dialect("blocked", {{"sizePerThread", IntList({1, 8})},
                               {"threadsPerWarp", IntList({lanes / chunks, chunks})},
                               {"warpsPerCTA", IntList(warps)},
                               {"order", IntList({1, 0})},
                               {"cga", cga}});
  };
  auto shared = [&](const SharedSwizzle &sw) {
    Fields f = {{"order", IntList(sw.order)},
                {"perPhase", IntU(sw.perPhase)},
                {"maxPhase", IntU(sw.maxPhase)},
                {"transposed", Bool(sw.transposed)},
                {"swizzlingByteWidth", IntU(sw.swizzlingByteWidth)},
                {"cga", cga}};
    if (sw.secondMaxPhase > 1) {
      f.push_back({"secondPerPhase", IntU(sw.secondPerPhase)});
      f.push_back({"secondMaxPhase", IntU(sw.secondMaxPhase)});
      f.push_back({"secondSwizzlingByteWidth", IntU(sw.secondSwizzlingByteWidth)});
    }
    return Dialect("shared", f);
  };
  auto dot = [&](int64_t idx) {
    return Dialect("dot_operand", {{"operandIndex", IntU(idx)},
                                   {"parent", mfma},
                                   {"kWidth", IntU(kPerLane)}});
  };
  int64_t nw = gm * gn;
  p.aGlobal = add("a_global", blocked(c.blockK, {nw, 1}));
  p.bGlobal = add("b_global", blocked(c.blockN, {nw, 1}));
  p.aShared = add("a_shared", shared(deriveSwizzle(t, c.blockK * elem, 16)));
  // B's transposing reads: each 32-lane LDS cycle of a ds_read_b64_tr_b16
  // serves two 16-lane groups, each reading 4 k rows of iN columns. With the
  // 32x32 layout the two groups read the same rows, 16 columns apart: one
  // 64-byte segment per row, which the first term spreads over the banks.
  // With the 16x16 layout they read the same iN = 16 columns of rows iK/4 = 8
  // apart, so rows with equal k % 4 collide; a second XOR term on iN-column
  // (32-byte) units with phase (k / 8) % 2 separates the groups.
  SharedSwizzle bSwizzle = deriveSwizzle(t, c.blockN * elem, 64);
  if (iM == 16 && bSwizzle.maxPhase > 1 && iN * elem * 2 <= bSwizzle.swizzlingByteWidth) {
    bSwizzle.secondPerPhase = iK / 4;
    bSwizzle.secondMaxPhase = 2;
    bSwizzle.secondSwizzlingByteWidth = iN * elem;
  }
  p.bShared = add("b_shared", shared(bSwizzle));
  p.aDot = add("a_dot", dot(0));
  p.bDot = add("b_dot", dot(1));
  p.acc = add("acc", Dialect("accumulator",
                             {{"parent", mfma},
                              {"logicalShape", IntList(p.fragmentAcc.logicalShape)},
                              {"instructionShape", IntList(p.fragmentAcc.instructionShape)},
                              {"repeatShape", IntList(p.fragmentAcc.repeatShape)},
                              {"repeatOrder", IntList(p.fragmentAcc.registerOrder)}}));
  // C stores: lane l owns row l % 32 and 4 consecutive columns at 4 (l / 32)
  p.cStore = add("c_store", Dialect("blocked", {{"sizePerThread", IntList({1, 4})},
                                                {"threadsPerWarp", IntList({iM, lanes / iM})},
                                                {"warpsPerCTA", IntList({gm, gn})},
                                                {"order", IntList({0, 1})},
                                                {"cga", cga}}));
  return p;
}
AttrP buildEncodingPlanAttr(const EncodingPlan &p) { return buildPlanAttr(p); }
EncodingPlan parseEncodingPlanAttr(const Attr &a) {
  return parsePlanAttr<EncodingPlan>(a, "`tb.encoding_plan`");
}

// ---- TransportPlan -------------------------------------------------------------
template <class V> void fields(V &v, TransportSpec &s) {
  v("role", s.role);
  v("dst_encoding", s.dstEncoding);
  v("kind", s.kind);
  v("vector_bytes", s.vectorBytes);
  v("async_vector_bytes", s.asyncVectorBytes);
  v("transaction_bytes", s.transactionBytes);
  v("async_eligible", s.asyncEligible);
  v("bypass_l1", s.bypassL1);
  v("cache_policy", s.cachePolicy);
}
template <class V> void fields(V &v, TransportPlan &p) {
  v("contract_model", p.contractModel);
  v("operand_a", p.operandA);
  v("operand_b", p.operandB);
}

// Reference: TransportPlan.cpp:139-305 (async vector = the largest candidate
// <= min(16, contiguous bytes, swizzle unit) dividing the contiguous bytes).
// gfx950 transport: buffer_load_dwordx4 with the LDS-direct modifier, one
// 16-byte vector per lane straight into the swizzled LDS stage; lanes whose
// row or column lies outside the problem get an out-of-range buffer offset
// and land zeros (the zero-fill of the reference's predicated cp.async).
static TransportSpec transportFor(const char *role, int dst, const TargetInfo &t,
                                  int64_t rowBytes, const SharedSwizzle &sw,
                                  int64_t stageBytes) {
  TransportSpec s;
  s.role = role;
  s.dstEncoding = dst;
  int64_t cap = std::min<int64_t>(t.asyncCopyMaxBytes, rowBytes);
  if (sw.swizzlingByteWidth > 0)
    cap = std::min(cap, sw.swizzlingByteWidth);
  int64_t vec = 0;
  for (int64_t cand : {16, 8, 4})
    if (cand <= cap && rowBytes % cand == 0 && cand >= t.asyncCopyMinBytes) {
      vec = cand;
      break;
    }
  if (vec != 16 || !t.supportsDirectToLds)
    throw Error(std::string("operand ") + role +
                " cannot use 16-byte direct-to-LDS buffer loads");
  s.kind = "buffer_load_dwordx4_lds";
  s.vectorBytes = vec;
  s.asyncVectorBytes = vec;
  s.transactionBytes = stageBytes;
  s.asyncEligible = true;
  s.bypassL1 = false;
  s.cachePolicy = "default";
  return s;
}

TransportPlan deriveTransportPlan(const KernelConfig &c, const TargetInfo &t,
                                  const EncodingPlan &e) {
  TransportPlan p;
  p.contractModel = "gfx950_direct_to_lds_v1";
  int64_t elem = scalarBytes(c.aScalar);
  p.operandA = transportFor("a", e.aShared, t, c.blockK * elem,
                            sharedSwizzle(encodingAttr(e, e.aShared, "a_shared")),
                            c.blockM * c.blockK * elem);
  p.operandB = transportFor("b", e.bShared, t, c.blockN * elem,
                            sharedSwizzle(encodingAttr(e, e.bShared, "b_shared")),
                            c.blockK * c.blockN * elem);
  return p;
}
AttrP buildTransportPlanAttr(const TransportPlan &p) { return buildPlanAttr(p); }
TransportPlan parseTransportPlanAttr(const Attr &a) {
  return parsePlanAttr<TransportPlan>(a, "`tb.transport_plan`");
}

} // namespace tb
