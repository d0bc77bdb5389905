// Field-list serialization of the plan structs.
//
// Each plan declares its fields once, `template <class V> void fields(V &v,
// Plan &p) { v("key", p.member); ... }`; the same list drives the dictionary
// attribute builder (Writer) and the parser (Reader), so the IR text is a
// lossless checkpoint of every plan (the reference keeps the same property
// with hand-written build*/parse* pairs, e.g. ProgramMappingPlan.cpp:460-581).
// Keys are snake_case and dictionaries print sorted, as MLIR's
// DictionaryAttr does.
#pragma once

#include "plans.h"

#include <type_traits>

namespace tb {

template <class E> struct EnumTable;
#define TB_ENUM_NAMES(E, ...)                                                  \
  template <> struct EnumTable<E> {                                            \
    static constexpr const char *names[] = {__VA_ARGS__};                      \
    static constexpr size_t size = sizeof(names) / sizeof(names[0]);           \
  };

TB_ENUM_NAMES(ScalarKind, "f16", "f32")
TB_ENUM_NAMES(MmaKind, "m16n8k16", "mfma_f32_32x32x16_f16",
              "mfma_f32_16x16x32_f16")
TB_ENUM_NAMES(ProgramMappingKind, "tile", "grouped_tile", "split_k",
              "persistent_tile")
TB_ENUM_NAMES(ProgramLaunchOrder, "row_major", "grouped_m", "persistent")
TB_ENUM_NAMES(ProgramSwizzleKind, "none", "grouped_m")
TB_ENUM_NAMES(ReductionMode, "none", "split_k_serial", "split_k_parallel")
TB_ENUM_NAMES(ReductionPlanKind, "none", "split_k_serial", "split_k_atomic")
TB_ENUM_NAMES(ReductionScratchSpace, "none", "global", "shared")
TB_ENUM_NAMES(PersistentWorkKind, "none", "tile_stride_loop")
TB_ENUM_NAMES(AccumulatorInitMode, "zero", "direct_global_vector", "shared_relay")
TB_ENUM_NAMES(AccumulatorStoreMode, "direct_global_vector", "shared_relay")
TB_ENUM_NAMES(TargetLandingKind, "none", "register_pack_global_vector",
              "shared_pack_then_global_vector", "shared_relay_then_global_vector")
TB_ENUM_NAMES(EpilogueExprKind, "load_bias", "add", "convert", "activation",
              "clamp")
TB_ENUM_NAMES(EpilogueReorderKind, "none", "cta_shared_row_reorder",
              "cta_shared_relay")
TB_ENUM_NAMES(SharedWorkspaceSegmentKind, "mainloop_a_stage_buffer",
              "mainloop_b_stage_buffer", "epilogue_reorder_scratch",
              "split_k_reduction_scratch", "persistent_state_scratch")
TB_ENUM_NAMES(MemorySpace, "global", "shared", "registers")
TB_ENUM_NAMES(BufferRole, "operand_a", "operand_b", "output", "accumulator",
              "epilogue_relay", "descriptor", "generic")
TB_ENUM_NAMES(ViewKind, "full_buffer", "stage_slice", "tile_slice", "fragment",
              "pack")
TB_ENUM_NAMES(BufferValueKind, "global_tile", "shared_tile",
              "dot_operand_fragment", "accumulator_fragment",
              "epilogue_fragment")
TB_ENUM_NAMES(BufferOpKind, "load_a", "load_b", "local_load_a", "local_load_b",
              "mma", "accumulator_init", "accumulator_store")
TB_ENUM_NAMES(AsyncProducerKind, "cp_async", "tma", "bulk_copy",
              "sync_copy_fallback", "buffer_load_lds")
TB_ENUM_NAMES(AsyncBarrierKind, "async_group", "cta", "mbarrier", "none",
              "vmcnt_barrier")
TB_ENUM_NAMES(AsyncCachePolicy, "default", "bypass_l1", "cache_all")
TB_ENUM_NAMES(ExpandedClusterKind, "async_issue", "consumer_wait", "mma_compute")
#undef TB_ENUM_NAMES

template <class E> const char *enumName(E e) {
  size_t i = static_cast<size_t>(e);
  if (i >= EnumTable<E>::size)
    throw Error("enum value out of range");
  return EnumTable<E>::names[i];
}
template <class E> E enumFromName(const std::string &s, const char *key) {
  for (size_t i = 0; i < EnumTable<E>::size; ++i)
    if (s == EnumTable<E>::names[i])
      return static_cast<E>(i);
  throw Error(std::string("unknown value `") + s + "` for field `" + key + "`");
}

// ---- encode ----------------------------------------------------------------
inline AttrP enc(int64_t x) { return I64(x); }
inline AttrP enc(int x) { return I64(x); }
inline AttrP enc(bool x) { return Bool(x); }
inline AttrP enc(const std::string &x) { return Str(x); }
inline AttrP enc(const I64s &x) { return Dense(x); }
inline AttrP enc(const AttrP &x) { return x ? x : Unit(); }
template <class E, std::enable_if_t<std::is_enum_v<E>, int> = 0>
AttrP enc(E e) { return Str(enumName(e)); }
template <class T> AttrP enc(const std::vector<T> &v);
template <class S, std::enable_if_t<std::is_class_v<S>, int> = 0>
AttrP enc(const S &s);

struct Writer {
  std::map<std::string, AttrP> d;
  template <class T> void operator()(const char *key, const T &x) {
    d[key] = enc(x);
  }
};
template <class T> AttrP enc(const std::vector<T> &v) {
  std::vector<AttrP> e;
  for (const T &x : v)
    e.push_back(enc(x));
  return Arr(e);
}
template <class S, std::enable_if_t<std::is_class_v<S>, int>>
AttrP enc(const S &s) {
  Writer w;
  fields(w, const_cast<S &>(s));
  return Dict(w.d);
}

// ---- decode ----------------------------------------------------------------
inline void dec(const AttrP &a, int64_t &x, const char *k) {
  if (a->kind != AttrKind::Int)
    throw Error(std::string("missing integer field `") + k + "`");
  x = a->i;
}
inline void dec(const AttrP &a, int &x, const char *k) {
  int64_t v;
  dec(a, v, k);
  x = static_cast<int>(v);
}
inline void dec(const AttrP &a, bool &x, const char *k) {
  if (a->kind != AttrKind::Bool)
    throw Error(std::string("missing bool field `") + k + "`");
  x = a->b;
}
inline void dec(const AttrP &a, std::string &x, const char *k) {
  if (a->kind != AttrKind::String)
    throw Error(std::string("missing string field `") + k + "`");
  x = a->s;
}
inline void dec(const AttrP &a, I64s &x, const char *k) {
  if (a->kind != AttrKind::DenseI64)
    throw Error(std::string("missing dense i64 array field `") + k + "`");
  x = a->ints;
}
inline void dec(const AttrP &a, AttrP &x, const char *) { x = a; }
template <class E, std::enable_if_t<std::is_enum_v<E>, int> = 0>
void dec(const AttrP &a, E &e, const char *k) {
  std::string s;
  dec(a, s, k);
  e = enumFromName<E>(s, k);
}
template <class T> void dec(const AttrP &a, std::vector<T> &v, const char *k);
template <class S, std::enable_if_t<std::is_class_v<S>, int> = 0>
void dec(const AttrP &a, S &s, const char *k);

struct Reader {
  const Attr &d;
  template <class T> void operator()(const char *key, T &x) {
    if (d.kind != AttrKind::Dict)
      throw Error(std::string("expected a dictionary holding `") + key + "`");
    auto it = d.dict.find(key);
    if (it == d.dict.end())
      throw Error(std::string("missing field `") + key + "`");
    dec(it->second, x, key);
  }
};
template <class T> void dec(const AttrP &a, std::vector<T> &v, const char *k) {
  if (a->kind != AttrKind::Array)
    throw Error(std::string("missing array field `") + k + "`");
  v.clear();
  for (const AttrP &e : a->elems) {
    T x{};
    dec(e, x, k);
    v.push_back(x);
  }
}
template <class S, std::enable_if_t<std::is_class_v<S>, int>>
void dec(const AttrP &a, S &s, const char *k) {
  if (a->kind != AttrKind::Dict)
    throw Error(std::string("missing dictionary field `") + k + "`");
  Reader r{*a};
  fields(r, s);
}

template <class S> AttrP buildPlanAttr(const S &s) { return enc(s); }
template <class S> S parsePlanAttr(const Attr &a, const char *what) {
  S s{};
  if (a.kind != AttrKind::Dict)
    throw Error(std::string(what) + " must be a dictionary attribute");
  try {
    Reader r{a};
    fields(r, s);
  } catch (const Error &e) {
    throw Error(std::string("malformed ") + what + ": " + e.what());
  }
  return s;
}

// ---- field lists -------------------------------------------------------------
template <class V> void fields(V &v, LaneAccessPattern &p) {
  v("lane_row_group_size", p.laneRowGroupSize);
  v("lane_col_group_size", p.laneColGroupSize);
  v("lane_col_stride", p.laneColStride);
  v("row_offsets", p.rowOffsets);
}

} // namespace tb
