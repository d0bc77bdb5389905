// Verifiers of the tb IR subset (see verify.h).
#include "verify.h"

#include <algorithm>
#include <set>

namespace tb {

namespace {

[[noreturn]] void attrError(const std::string &mnemonic, const std::string &msg) {
  throw Error("invalid `#tb." + mnemonic + "`: " + msg);
}

[[noreturn]] void opError(const std::string &op, const std::string &msg) {
  throw Error("'" + op + "' op " + msg);
}

// ---- parameter schemas ---------------------------------------------------------
// Kinds: i integer, l integer list, b bool, s string, c #tb.cga, m an MMA
// parent (#tb.amd_mfma or #tb.nvgpu_mma), e any #tb encoding, t a type.
struct ParamSpec {
  const char *name;
  char kind;
};
struct Schema {
  std::vector<ParamSpec> required;
  // optional trailing groups: all of a group's parameters or none
  std::vector<std::vector<ParamSpec>> optional;
};

const std::map<std::string, Schema> &schemas() {
  static const std::map<std::string, Schema> s = {
      {"semantic_layout",
       {{{"order", 'l'}, {"strides", 'l'}, {"zeroOffset", 'b'}, {"hasStaticStrides", 'b'},
         {"unitStrideOnMinor", 'b'}, {"contiguous", 'b'}},
        {}}},
      {"cga", {{{"ctasPerCGA", 'l'}, {"ctaSplitNum", 'l'}, {"ctaOrder", 'l'}}, {}}},
      {"blocked",
       {{{"sizePerThread", 'l'}, {"threadsPerWarp", 'l'}, {"warpsPerCTA", 'l'},
         {"order", 'l'}, {"cga", 'c'}},
        {}}},
      // gfx950 adds an optional second XOR term (secondPerPhase, ...)
      {"shared",
       {{{"order", 'l'}, {"perPhase", 'i'}, {"maxPhase", 'i'}, {"transposed", 'b'},
         {"swizzlingByteWidth", 'i'}, {"cga", 'c'}},
        {{{"paddingIntervals", 'l'}, {"paddings", 'l'}},
         {{"secondPerPhase", 'i'}, {"secondMaxPhase", 'i'},
          {"secondSwizzlingByteWidth", 'i'}}}}},
      {"nvgpu_mma",
       {{{"mmaFamily", 's'}, {"versionMajor", 'i'}, {"versionMinor", 'i'},
         {"warpsPerCTA", 'l'}, {"instrShape", 'l'}, {"cga", 'c'}},
        {}}},
      {"amd_mfma",
       {{{"versionMajor", 'i'}, {"versionMinor", 'i'}, {"warpsPerCTA", 'l'},
         {"instrShape", 'l'}, {"isTransposed", 'b'}, {"cga", 'c'}},
        {}}},
      {"dot_operand", {{{"operandIndex", 'i'}, {"parent", 'm'}, {"kWidth", 'i'}}, {}}},
      {"accumulator",
       {{{"parent", 'm'}, {"logicalShape", 'l'}, {"instructionShape", 'l'},
         {"repeatShape", 'l'}, {"repeatOrder", 'l'}},
        {}}},
  };
  return s;
}

bool isIntList(const Attr &a) {
  if (a.kind != AttrKind::Array)
    return false;
  for (const AttrP &e : a.elems)
    if (!e || e->kind != AttrKind::Int)
      return false;
  return true;
}

void checkKind(const std::string &owner, const ParamSpec &p, const Attr &v) {
  bool ok = false;
  switch (p.kind) {
  case 'i': ok = v.kind == AttrKind::Int; break;
  case 'l': ok = isIntList(v); break;
  case 'b': ok = v.kind == AttrKind::Bool; break;
  case 's': ok = v.kind == AttrKind::String; break;
  case 'c': ok = v.kind == AttrKind::Dialect && v.s == "cga"; break;
  case 'm':
    ok = v.kind == AttrKind::Dialect && (v.s == "amd_mfma" || v.s == "nvgpu_mma");
    break;
  case 'e': ok = v.kind == AttrKind::Dialect; break;
  case 't': ok = v.kind == AttrKind::Type; break;
  }
  if (!ok) {
    static const std::map<char, const char *> what = {
        {'i', "an integer"}, {'l', "an integer list"}, {'b', "a bool"},
        {'s', "a string"}, {'c', "a #tb.cga encoding"},
        {'m', "an MMA parent encoding (#tb.amd_mfma or #tb.nvgpu_mma)"},
        {'e', "a #tb encoding"}, {'t', "a type"}};
    attrError(owner, std::string("`") + p.name + "` must be " + what.at(p.kind));
  }
}

// The parameters of `a` must be the schema's required ones, in order, then
// whole optional groups.
void checkParams(const std::string &owner, const Fields &params, const Schema &s) {
  size_t i = 0;
  auto take = [&](const ParamSpec &p) {
    if (i >= params.size() || params[i].first != p.name)
      attrError(owner, std::string("expected parameter `") + p.name + "`" +
                           (i < params.size() ? ", found `" + params[i].first + "`"
                                              : ", found the end"));
    checkKind(owner, p, *params[i].second);
    ++i;
  };
  for (const ParamSpec &p : s.required)
    take(p);
  for (const auto &group : s.optional) {
    if (i < params.size() && params[i].first == group.front().name)
      for (const ParamSpec &p : group)
        take(p);
  }
  if (i != params.size())
    attrError(owner, "unexpected parameter `" + params[i].first + "`");
}

const Attr &paramOf(const Attr &a, const char *name) {
  for (const auto &kv : a.params)
    if (kv.first == name)
      return *kv.second;
  attrError(a.s, std::string("missing `") + name + "`");
}

bool hasParam(const Attr &a, const char *name) {
  for (const auto &kv : a.params)
    if (kv.first == name)
      return true;
  return false;
}

std::vector<int64_t> ints(const Attr &a) {
  std::vector<int64_t> v;
  for (const AttrP &e : a.elems)
    v.push_back(e->i);
  return v;
}

// Reference: TBAttrs.cpp:23-43.
void positiveArray(const std::string &owner, const char *name,
                   const std::vector<int64_t> &v) {
  if (std::any_of(v.begin(), v.end(), [](int64_t x) { return x <= 0; }))
    attrError(owner, std::string(name) + " entries must be positive");
}
void permutation(const std::string &owner, const char *name,
                 const std::vector<int64_t> &v) {
  std::vector<bool> seen(v.size(), false);
  for (int64_t x : v) {
    if (x < 0 || x >= (int64_t)v.size())
      attrError(owner, std::string(name) + " must be a permutation of [0, rank)");
    if (seen[x])
      attrError(owner, std::string(name) + " must not contain duplicates");
    seen[x] = true;
  }
}

void verifyDialect(const Attr &a) {
  auto it = schemas().find(a.s);
  if (it == schemas().end())
    throw Error("unknown tb attribute `#tb." + a.s + "`");
  checkParams(a.s, a.params, it->second);
  for (const auto &kv : a.params)
    verifyAttr(*kv.second);
  const std::string &m = a.s;
  if (m == "semantic_layout") { // TBAttrs.cpp:47-73
    auto order = ints(paramOf(a, "order")), strides = ints(paramOf(a, "strides"));
    const bool stat = paramOf(a, "hasStaticStrides").b;
    const bool unit = paramOf(a, "unitStrideOnMinor").b;
    const bool contig = paramOf(a, "contiguous").b;
    if (order.empty())
      attrError(m, "semantic layout must have non-empty order");
    if (order.size() != strides.size())
      attrError(m, "semantic layout stride rank must match order rank");
    permutation(m, "order", order);
    if (stat) {
      if (std::any_of(strides.begin(), strides.end(), [](int64_t x) { return x <= 0; }))
        attrError(m, "semantic layout static strides must be positive");
    } else if (std::any_of(strides.begin(), strides.end(),
                           [](int64_t x) { return x == 0; })) {
      attrError(m, "semantic layout strides must use positive values or -1 for "
                   "dynamic metadata");
    }
    if ((unit || contig) && !stat)
      attrError(m, "semantic layout contiguity flags require static stride metadata");
    if (contig && !unit)
      attrError(m, "semantic layout contiguous=true requires unitStrideOnMinor=true");
  } else if (m == "cga") { // TBAttrs.cpp:75-90
    auto per = ints(paramOf(a, "ctasPerCGA")), split = ints(paramOf(a, "ctaSplitNum")),
         order = ints(paramOf(a, "ctaOrder"));
    if (per.size() != 3 || split.size() != 3 || order.size() != 3)
      attrError(m, "cga encoding must carry rank-3 ctas_per_cga/cta_split_num/cta_order");
    positiveArray(m, "ctas_per_cga", per);
    positiveArray(m, "cta_split_num", split);
    permutation(m, "cta_order", order);
  } else if (m == "blocked") { // TBAttrs.cpp:92-118
    auto spt = ints(paramOf(a, "sizePerThread")), tpw = ints(paramOf(a, "threadsPerWarp")),
         wpc = ints(paramOf(a, "warpsPerCTA")), order = ints(paramOf(a, "order"));
    if (spt.empty())
      attrError(m, "blocked encoding must have non-empty size_per_thread");
    if (spt.size() != tpw.size())
      attrError(m, "size_per_thread/threads_per_warp rank mismatch: " +
                       std::to_string(spt.size()) + " vs " + std::to_string(tpw.size()));
    if (spt.size() != wpc.size())
      attrError(m, "size_per_thread/warps_per_cta rank mismatch: " +
                       std::to_string(spt.size()) + " vs " + std::to_string(wpc.size()));
    if (spt.size() != order.size())
      attrError(m, "order rank must match blocked encoding rank");
    positiveArray(m, "size_per_thread", spt);
    positiveArray(m, "threads_per_warp", tpw);
    positiveArray(m, "warps_per_cta", wpc);
    permutation(m, "order", order);
  } else if (m == "shared") { // TBAttrs.cpp:120-148
    auto order = ints(paramOf(a, "order"));
    const int64_t pp = paramOf(a, "perPhase").i, mp = paramOf(a, "maxPhase").i;
    const int64_t sw = paramOf(a, "swizzlingByteWidth").i;
    if (order.empty())
      attrError(m, "shared encoding must have non-empty order");
    std::vector<int64_t> pi, pd;
    if (hasParam(a, "paddingIntervals")) {
      pi = ints(paramOf(a, "paddingIntervals"));
      pd = ints(paramOf(a, "paddings"));
    }
    if (pi.size() != pd.size())
      attrError(m, "padding_intervals and paddings must have same rank");
    if (!pi.empty() && pi.size() != order.size())
      attrError(m, "padding rank must match shared encoding rank");
    if (pp < 0 || mp < 0)
      attrError(m, "per_phase and max_phase must be non-negative");
    if (sw < 0)
      attrError(m, "swizzling_byte_width must be non-negative");
    permutation(m, "order", order);
    if (std::any_of(pi.begin(), pi.end(), [](int64_t x) { return x < 0; }) ||
        std::any_of(pd.begin(), pd.end(), [](int64_t x) { return x < 0; }))
      attrError(m, "shared padding metadata must be non-negative");
    if (hasParam(a, "secondPerPhase")) { // gfx950: a second XOR term
      const int64_t pp2 = paramOf(a, "secondPerPhase").i;
      const int64_t mp2 = paramOf(a, "secondMaxPhase").i;
      const int64_t sw2 = paramOf(a, "secondSwizzlingByteWidth").i;
      if (pp2 <= 0 || mp2 <= 0 || sw2 <= 0)
        attrError(m, "the second XOR term's per_phase, max_phase and swizzling byte "
                     "width must be positive");
      if (sw2 % 16 || sw <= 0 || sw % sw2 || (sw2 * mp2) > sw)
        attrError(m, "the second XOR term must permute whole 16-byte chunks inside "
                     "one swizzling unit of the first (second byte width a multiple "
                     "of 16 dividing the first, times its max_phase at most the first)");
    }
  } else if (m == "nvgpu_mma" || m == "amd_mfma") { // TBAttrs.cpp:150-169
    if (m == "nvgpu_mma" && paramOf(a, "mmaFamily").s.empty())
      attrError(m, "mma_family must be non-empty");
    if (paramOf(a, "versionMajor").i < 0 || paramOf(a, "versionMinor").i < 0)
      attrError(m, "mma version must be non-negative");
    auto wpc = ints(paramOf(a, "warpsPerCTA")), instr = ints(paramOf(a, "instrShape"));
    if (wpc.size() != 2)
      attrError(m, "warps_per_cta must have rank 2");
    if (instr.size() != 3)
      attrError(m, "instr_shape must have rank 3");
    positiveArray(m, "warps_per_cta", wpc);
    positiveArray(m, "instr_shape", instr);
  } else if (m == "dot_operand") { // TBAttrs.cpp:171-181
    const int64_t idx = paramOf(a, "operandIndex").i;
    if (idx != 0 && idx != 1)
      attrError(m, "operand_index must be 0 or 1");
    if (paramOf(a, "kWidth").i <= 0)
      attrError(m, "k_width must be positive");
  }
}

// Reference: TBTypes.cpp:16-46.
void verifyMemDesc(const Attr &t) {
  static const Schema s = {{{"shape", 'l'}, {"elementType", 't'}, {"encoding", 'e'},
                            {"memorySpace", 's'}, {"mutableMemory", 'b'},
                            {"allocShape", 'l'}},
                           {}};
  const std::string owner = "memdesc";
  size_t i = 0;
  for (const ParamSpec &p : s.required) {
    if (i >= t.params.size() || t.params[i].first != p.name)
      throw Error(std::string("invalid `!tb.memdesc`: expected parameter `") + p.name + "`");
    const Attr &v = *t.params[i].second;
    if (p.kind == 'l' && !isIntList(v))
      throw Error(std::string("invalid `!tb.memdesc`: `") + p.name +
                  "` must be an integer list");
    if (p.kind == 's' && v.kind != AttrKind::String)
      throw Error("invalid `!tb.memdesc`: `memorySpace` must be a string");
    if (p.kind == 'b' && v.kind != AttrKind::Bool)
      throw Error("invalid `!tb.memdesc`: `mutableMemory` must be a bool");
    if (p.kind == 'e' && v.kind != AttrKind::Dialect)
      throw Error("invalid `!tb.memdesc`: `encoding` must be a #tb encoding");
    ++i;
  }
  if (i != t.params.size())
    throw Error("invalid `!tb.memdesc`: unexpected parameter `" + t.params[i].first + "`");
  auto get = [&](const char *n) -> const Attr & {
    for (const auto &kv : t.params)
      if (kv.first == n)
        return *kv.second;
    throw Error("invalid `!tb.memdesc`");
  };
  auto fail = [](const std::string &msg) { throw Error("invalid `!tb.memdesc`: " + msg); };
  auto shape = ints(get("shape")), alloc = ints(get("allocShape"));
  const std::string space = get("memorySpace").s;
  const Attr &enc = get("encoding");
  verifyAttr(enc);
  if (shape.empty())
    fail("shape must be non-empty");
  if (shape.size() != alloc.size())
    fail("alloc_shape rank must match shape rank");
  if (std::any_of(shape.begin(), shape.end(), [](int64_t d) { return d <= 0; }))
    fail("shape dimensions must be positive");
  if (std::any_of(alloc.begin(), alloc.end(), [](int64_t d) { return d <= 0; }))
    fail("alloc_shape dimensions must be positive");
  if (get("elementType").s.empty())
    fail("element_type must be present");
  if (space != "global" && space != "shared" && space != "registers")
    fail("memory_space must be one of global/shared/registers");
  if (enc.s == "semantic_layout" && space != "global")
    fail("semantic layout requires global memory_space");
  if (enc.s == "shared" && space != "shared")
    fail("shared encoding requires shared memory_space");
  if ((enc.s == "dot_operand" || enc.s == "accumulator") && space != "registers")
    fail("register fragment encodings require registers memory_space");
}

// Reference: TBOps.cpp:16-60 (three rank-2 memref operands, A:[M,K],
// B:[K,N], C:[M,N]). gfx950 also takes an f16 C (f32 accumulation, f16
// store).
void verifyKernelOperands(const Op &op) {
  if (op.operandTypes.size() != 3)
    opError(op.name, "expected three memref operands `a`, `b`, `c`");
  static const char *names[3] = {"a", "b", "c"};
  MemRefInfo info[3];
  for (int i = 0; i < 3; ++i) {
    const Attr &t = *op.operandTypes[i];
    if (t.kind != AttrKind::Type || !t.typeDialect.empty() || t.s.rfind("memref<", 0) != 0)
      opError(op.name, std::string("expected `") + names[i] + "` to be a memref");
    info[i] = parseMemRef(op.operandTypes[i]);
    if (info[i].shape.size() != 2)
      opError(op.name, std::string("expected `") + names[i] + "` to be a rank-2 memref");
  }
  if (info[0].elementType != "f16" || info[1].elementType != "f16" ||
      (info[2].elementType != "f32" && info[2].elementType != "f16"))
    opError(op.name, "expected fp16 x fp16 -> fp32 (or fp16) operand element types");
  if (info[0].shape[1] != info[1].shape[0] || info[0].shape[0] != info[2].shape[0] ||
      info[1].shape[1] != info[2].shape[1])
    opError(op.name, "expected A:[M,K], B:[K,N], C:[M,N] operand shapes");
}

int64_t intAttr(const Op &op, const char *name, bool required, int64_t dflt) {
  auto it = op.attrs.find(name);
  if (it == op.attrs.end()) {
    if (required)
      opError(op.name, std::string("requires attribute `") + name + "`");
    return dflt;
  }
  if (it->second->kind != AttrKind::Int)
    opError(op.name, std::string("attribute `") + name + "` must be an integer");
  return it->second->i;
}

// Reference: TBOps.cpp:174-182.
void verifyMatmul(const Op &op) {
  verifyKernelOperands(op);
  if (intAttr(op, "block_m", true, 0) <= 0 || intAttr(op, "block_n", true, 0) <= 0 ||
      intAttr(op, "block_k", true, 0) <= 0)
    opError(op.name, "block sizes must be positive");
  if (intAttr(op, "group_m", false, 8) <= 0)
    opError(op.name, "group_m must be positive");
  auto et = op.attrs.find("exact_tile");
  if (et == op.attrs.end() || et->second->kind != AttrKind::Bool)
    opError(op.name, "requires bool attribute `exact_tile`");
}

// Reference: TBOps.cpp:128-158.
void verifyConvertLayout(const Op &op) {
  if (op.operandTypes.size() != 1 || op.resultTypes.size() != 1)
    opError(op.name, "expects one source and one result");
  const Attr &s = *op.operandTypes[0], &d = *op.resultTypes[0];
  if (s.typeDialect != "memdesc" || d.typeDialect != "memdesc")
    opError(op.name, "requires !tb.memdesc source/result types for explicit layout "
                     "ownership transfer");
  auto p = [](const Attr &t, const char *n) -> AttrP {
    for (const auto &kv : t.params)
      if (kv.first == n)
        return kv.second;
    return nullptr;
  };
  if (!equal(p(s, "shape"), p(d, "shape")))
    opError(op.name, "source/result logical shapes must match for layout conversion");
  if (!equal(p(s, "elementType"), p(d, "elementType")))
    opError(op.name, "source/result element types must match for layout conversion");
  if (!equal(p(s, "memorySpace"), p(d, "memorySpace")))
    opError(op.name, "source/result memory spaces must match for layout conversion");
  if (!equal(p(s, "mutableMemory"), p(d, "mutableMemory")))
    opError(op.name, "source/result mutability must match for layout conversion");
  if (!p(s, "encoding") || !p(d, "encoding"))
    opError(op.name, "layout conversion requires concrete source/result encodings");
  if (equal(p(s, "encoding"), p(d, "encoding")) &&
      equal(p(s, "allocShape"), p(d, "allocShape")))
    opError(op.name, "layout conversion must change encoding or alloc_shape");
}

int64_t clusterInt(const Op &cl, const char *name) {
  auto it = cl.attrs.find(name);
  if (it == cl.attrs.end() || it->second->kind != AttrKind::Int)
    opError(cl.name, std::string("requires integer attribute `") + name + "`");
  return it->second->i;
}

// Reference: TBOps.cpp:62-71 and :276-304.
void verifyCluster(const Op &cl) {
  const int64_t ordinal = clusterInt(cl, "ordinal"), stage = clusterInt(cl, "stage"),
                cluster = clusterInt(cl, "cluster"), kg = clusterInt(cl, "k_group");
  if (ordinal < 0 || stage < 0 || cluster < 0 || kg < 0)
    opError(cl.name, "cluster metadata must be non-negative");
  auto ids = cl.attrs.find("op_ids");
  if (ids == cl.attrs.end() || ids->second->kind != AttrKind::DenseI64 ||
      ids->second->ints.empty())
    opError(cl.name, "cluster must carry non-empty op_ids");
  if (cl.name == "tb.consumer_wait_cluster") {
    auto w = cl.attrs.find("wait_group_ids");
    if (w == cl.attrs.end() || w->second->kind != AttrKind::DenseI64 ||
        w->second->ints.empty())
      opError(cl.name, "consumer_wait_cluster must carry non-empty wait_group_ids");
    auto b = cl.attrs.find("needs_barrier");
    if (b == cl.attrs.end() || b->second->kind != AttrKind::Bool || !b->second->b)
      opError(cl.name, "consumer_wait_cluster must own the CTA barrier");
  }
}

// Reference: TBOps.cpp:184-272.
void verifyMainline(const Module &m, const Op &op) {
  verifyKernelOperands(op);
  for (const char *a :
       {"tb.semantic_matmul", "tb.program_mapping_plan", "tb.reduction_plan",
        "tb.persistent_work_plan", "tb.encoding_plan", "tb.transport_plan",
        "tb.accumulator_plan", "tb.matmul_rewrite", "tb.epilogue_plan", "tb.buffer_model",
        "tb.async_plan", "tb.pipeline_ready"})
    if (!op.attrs.count(a))
      opError(op.name, std::string("requires `") + a + "` to be present");
  for (const char *a : {"tb.target", "tb.num-warps", "tb.threads-per-warp", "tb.num-ctas",
                        "tb.requested-stages"})
    if (!m.attr(a))
      opError(op.name, std::string("requires module attr `") + a + "`");
  for (const char *a : {"tb.target_info", "tb.layout_plan", "tb.c_register_plan",
                        "tb.mainloop_graph", "tb.schedule_plan", "tb.wait_plan",
                        "tb.loop_plan", "tb.latency_plan", "tb.pipeline_plan",
                        "tb.pipeline_expansion"})
    if (op.attrs.count(a))
      opError(op.name, std::string("must not retain transient attr `") + a +
                           "` after post-pipeline cleanup");
  if (!op.hasRegion || op.region.empty())
    opError(op.name, "pipeline_mainline must carry a non-empty body");
  int64_t expect = 0, prevStage = -1, prevCluster = -1, maxKg = -1;
  std::set<int64_t> kgs;
  for (const Op &cl : op.region) {
    if (cl.name != "tb.async_issue_cluster" && cl.name != "tb.consumer_wait_cluster" &&
        cl.name != "tb.mma_compute_cluster")
      opError(op.name, "pipeline_mainline body may only contain explicit pipeline "
                       "cluster ops");
    verifyCluster(cl);
    const int64_t ordinal = clusterInt(cl, "ordinal"), stage = clusterInt(cl, "stage"),
                  cluster = clusterInt(cl, "cluster"), kg = clusterInt(cl, "k_group");
    if (ordinal != expect++)
      opError(op.name, "pipeline_mainline cluster ordinals must be contiguous from zero");
    if (stage < prevStage || (stage == prevStage && cluster < prevCluster))
      opError(op.name, "pipeline_mainline clusters must stay ordered by stage/cluster");
    prevStage = stage;
    prevCluster = cluster;
    kgs.insert(kg);
    maxKg = std::max(maxKg, kg);
  }
  for (int64_t g = 0; g <= maxKg; ++g)
    if (!kgs.count(g))
      opError(op.name, "pipeline_mainline must carry contiguous explicit k_group "
                       "coverage after cleanup");
}

// The lowered launch op (this backend's counterpart of the reference's
// gpu.binary payload).
void verifyLaunch(const Op &op) {
  verifyKernelOperands(op);
  auto cfg = op.attrs.find("config");
  if (cfg == op.attrs.end() || cfg->second->kind != AttrKind::Dict)
    opError(op.name, "requires a `config` dictionary");
  for (const char *k : {"m", "n", "k", "lda", "ldb", "ldc", "c_dtype", "acc_init",
                        "block_m", "block_n", "block_k", "num_waves", "wave_grid_m",
                        "wave_grid_n", "stages", "mapping", "group_m", "split_k",
                        "reduction", "num_programs", "xcd_remap"}) {
    auto it = cfg->second->dict.find(k);
    if (it == cfg->second->dict.end() || it->second->kind != AttrKind::Int)
      opError(op.name, std::string("`config` requires integer `") + k + "`");
  }
  auto kn = op.attrs.find("kernel");
  if (kn == op.attrs.end() || kn->second->kind != AttrKind::String ||
      kn->second->s.empty())
    opError(op.name, "requires a non-empty `kernel` name");
  for (const char *k : {"grid", "block"}) {
    auto it = op.attrs.find(k);
    if (it == op.attrs.end() || it->second->kind != AttrKind::DenseI64 ||
        it->second->ints.size() != 3 ||
        std::any_of(it->second->ints.begin(), it->second->ints.end(),
                    [](int64_t x) { return x <= 0; }))
      opError(op.name, std::string("`") + k + "` must be three positive extents");
  }
  auto w = op.attrs.find("waits");
  if (w != op.attrs.end() &&
      (w->second->kind != AttrKind::DenseI64 || w->second->ints.size() != 3))
    opError(op.name, "`waits` must be array<i64: vmcnt prologue, vmcnt loop, lgkmcnt loop>");
}

void verifyAttrMap(const std::map<std::string, AttrP> &attrs) {
  for (const auto &kv : attrs)
    if (kv.second)
      verifyAttr(*kv.second);
}

void verifyOp(const Module &m, const Op &op) {
  verifyAttrMap(op.attrs);
  for (const AttrP &t : op.operandTypes)
    verifyAttr(*t);
  for (const AttrP &t : op.resultTypes)
    verifyAttr(*t);
  if (op.name == "tb.matmul")
    verifyMatmul(op);
  else if (op.name == "tb.convert_layout")
    verifyConvertLayout(op);
  else if (op.name == "tb.pipeline_mainline")
    verifyMainline(m, op);
  else if (op.name == "tb.gfx950_launch")
    verifyLaunch(op);
  for (const Op &nested : op.region)
    verifyAttrMap(nested.attrs);
}

} // namespace

void verifyAttr(const Attr &a) {
  switch (a.kind) {
  case AttrKind::Dialect:
    verifyDialect(a);
    break;
  case AttrKind::Type:
    if (a.typeDialect == "memdesc")
      verifyMemDesc(a);
    break;
  case AttrKind::Array:
    for (const AttrP &e : a.elems)
      if (e)
        verifyAttr(*e);
    break;
  case AttrKind::Dict:
    verifyAttrMap(a.dict);
    break;
  default:
    break;
  }
}

void verifyModule(const Module &m) {
  verifyAttrMap(m.attrs);
  verifyAttrMap(m.aliases);
  for (const Func &f : m.funcs) {
    for (const auto &arg : f.args)
      verifyAttr(*arg.second);
    for (const AttrP &t : f.resultTypes)
      verifyAttr(*t);
    for (const Op &op : f.body)
      verifyOp(m, op);
  }
}

} // namespace tb
