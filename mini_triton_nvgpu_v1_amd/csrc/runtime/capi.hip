// C ABI of the gfx950 backend (include/tb_gfx950.h): descriptor creation,
// kernel-instance selection and stream-ordered launch.
//
// Replaces the reference's lowering entry (TBLowerPipelineToNVGPU,
// lib/Transforms/LowerPipelineToNVGPU.cpp:2624-2732: parseKernelContract ->
// validateLoweringContract -> gpu.func) and its external launcher
// (cuLaunchKernel with grid = programs, block = num_warps*32,
// tools/bench_stage1_fair.py:665-699). Here block = num_waves*64 and the
// kernel is a precompiled gfx950 instance chosen by tile shape.
#include "tb_gfx950.h"

#include "../kernels/gemm_gfx950.h"
#include "../plan/instances.h"
#include "desc.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <mutex>
#include <string>

namespace {

thread_local std::string g_last_error;

int fail(const std::string &msg) {
  g_last_error = msg;
  return -1;
}

int check_hip(hipError_t e, const char *what) {
  if (e == hipSuccess)
    return 0;
  return fail(std::string(what) + ": " + hipGetErrorString(e));
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

} // namespace

namespace tbrt {

void set_error(const std::string &msg) { g_last_error = msg; }

void desc_waits(const tb_gemm_desc *d, int64_t out[3]) {
  out[0] = d->entry->vm_prologue;
  out[1] = d->entry->vm_loop;
  out[2] = d->entry->lgkm_loop;
}

// Validate a flattened config and bind it to a compiled instance.
int create_desc(const tb_gemm_config &c, tb_gemm_desc **out) {
  if (!out)
    return fail("tb_desc_create: out is NULL");
  *out = nullptr;
  if (c.m <= 0 || c.n <= 0 || c.k <= 0)
    return fail("problem M/N/K must be positive");
  if (c.lda < c.k || c.ldb < c.n || c.ldc < c.n)
    return fail("leading dimensions must cover the row lengths (lda >= K, "
                "ldb >= N, ldc >= N)");
  if (c.k % 8 || c.n % 8 || c.lda % 8 || c.ldb % 8 || c.ldc % 8)
    return fail("gfx950 16-byte row transport requires K, N and every "
                "leading dimension to be multiples of 8 elements");
  if (c.c_dtype != TB_DTYPE_F16 && c.c_dtype != TB_DTYPE_F32)
    return fail("c_dtype must be TB_DTYPE_F16 or TB_DTYPE_F32");
  if (c.acc_init != TB_ACC_INIT_ZERO && c.acc_init != TB_ACC_INIT_LOAD_C)
    return fail("acc_init must be TB_ACC_INIT_ZERO or TB_ACC_INIT_LOAD_C");
  if (c.acc_init == TB_ACC_INIT_LOAD_C && c.c_dtype != TB_DTYPE_F32)
    return fail("accumulating into C (C += A*B) requires f32 C");
  if (c.block_m <= 0 || c.block_n <= 0 || c.block_k <= 0)
    return fail("block M/N/K must be positive");
  if (c.wave_grid_m * c.wave_grid_n != c.num_waves)
    return fail("wave grid must multiply to num_waves");
  if (c.split_k < 1)
    return fail("split_k must be >= 1");
  if (c.epi_bias < TB_EPI_BIAS_NONE || c.epi_bias > TB_EPI_BIAS_F32)
    return fail("epi_bias must be TB_EPI_BIAS_NONE, _F16 or _F32");
  if (c.epi_activation < TB_ACT_NONE || c.epi_activation > TB_ACT_SILU)
    return fail("epi_activation must be TB_ACT_NONE, _RELU, _GELU_TANH or _SILU");
  if (c.epi_clamp & ~(TB_CLAMP_MIN | TB_CLAMP_MAX))
    return fail("epi_clamp holds unknown bits");
  if (((c.epi_clamp & TB_CLAMP_MIN) && !std::isfinite(c.clamp_min)) ||
      ((c.epi_clamp & TB_CLAMP_MAX) && !std::isfinite(c.clamp_max)))
    return fail("clamp bounds must be finite");
  if ((c.epi_clamp & TB_CLAMP_MIN) && (c.epi_clamp & TB_CLAMP_MAX) &&
      c.clamp_min > c.clamp_max)
    return fail("clamp_min must not exceed clamp_max");
  const bool fused = c.epi_bias || c.epi_activation || c.epi_clamp;
  if (fused && c.reduction == TB_RED_ATOMIC)
    return fail("fused epilogue steps need the whole sum; atomic split-K "
                "accumulates partial sums into C");
  if (c.group_m < 1)
    return fail("group_m must be >= 1");
  if (c.mfma != TB_MFMA_32X32X16 && c.mfma != TB_MFMA_16X16X32)
    return fail("mfma must be TB_MFMA_32X32X16 or TB_MFMA_16X16X32");
  if (c.mfma == TB_MFMA_16X16X32 && c.mapping == TB_MAP_SPLIT_K)
    return fail("the 16x16x32 instance has no split-K");
  const int64_t tiles_m = ceil_div(c.m, c.block_m);
  const int64_t tiles_n = ceil_div(c.n, c.block_n);
  const int64_t tiles_k = ceil_div(c.k, c.block_k);
  int64_t total_work = tiles_m * tiles_n;
  int out_mode = tbk::kOutF16;
  switch (c.mapping) {
  case TB_MAP_TILE:
  case TB_MAP_GROUPED_TILE:
  case TB_MAP_PERSISTENT_TILE:
  case TB_MAP_PERSISTENT_GROUPED:
    if (c.split_k != 1 || c.reduction != TB_RED_NONE)
      return fail("tile/grouped/persistent mappings carry no split-K reduction");
    if (c.c_dtype == TB_DTYPE_F16)
      out_mode = tbk::kOutF16;
    else
      out_mode = c.acc_init == TB_ACC_INIT_LOAD_C ? tbk::kOutF32Accum
                                                  : tbk::kOutF32Partial;
    if (c.c_dtype == TB_DTYPE_F32 && c.acc_init == TB_ACC_INIT_ZERO &&
        c.ldc > std::numeric_limits<int>::max())
      return fail("ldc too large");
    break;
  case TB_MAP_SPLIT_K:
    if (c.split_k < 2)
      return fail("split_k mapping requires split_k >= 2");
    total_work = tiles_m * tiles_n * c.split_k;
    if (c.reduction == TB_RED_WORKSPACE) {
      out_mode = tbk::kOutF32Partial;
    } else if (c.reduction == TB_RED_ATOMIC) {
      if (c.c_dtype != TB_DTYPE_F32 || c.acc_init != TB_ACC_INIT_LOAD_C)
        return fail("atomic split-K accumulates into f32 C (C += A*B)");
      out_mode = tbk::kOutF32Atomic;
    } else {
      return fail("split_k mapping requires a reduction");
    }
    break;
  default:
    return fail("unknown mapping kind");
  }
  const bool persistent = c.mapping == TB_MAP_PERSISTENT_TILE ||
                          c.mapping == TB_MAP_PERSISTENT_GROUPED;
  int64_t programs = persistent ? c.num_programs : total_work;
  if (persistent && (programs <= 0 || programs > total_work))
    programs = std::min<int64_t>(total_work, programs <= 0 ? 256 : programs);
  if (!persistent && c.num_programs > 0 && c.num_programs != total_work)
    return fail("num_programs disagrees with the mapping's launch formula");

  // 32-bit buffer offsets: A, C and the split-K partial planes are addressed
  // through windows that start at each tile's first row, so a tile's rows
  // (block_m of them) must span less than 1 GiB (well inside the offsets'
  // 2^31 range); B is addressed whole and must span less than 2 GiB. The
  // operands' total sizes are otherwise free.
  const int64_t lim = (int64_t)1 << 31, tile_lim = (int64_t)1 << 30;
  if (c.block_m * c.lda * 2 >= tile_lim || c.block_m * c.ldc * 4 >= tile_lim ||
      c.block_m * c.n * 4 >= tile_lim)
    return fail("a tile's rows of A or C span 1 GiB or more (leading dimensions too "
                "large for the 32-bit buffer offsets of this backend)");
  if (c.k * c.ldb * 2 >= lim)
    return fail("B larger than 2 GiB is not supported by the 32-bit buffer "
                "addressing of this backend");
  if (c.m >= lim || c.n >= lim || c.k >= lim)
    return fail("M, N and K must be below 2^31");
  if (total_work > std::numeric_limits<int>::max())
    return fail("too many programs");

  // split-K partials take the fused steps in the reduction instead
  const int epi = fused && c.mapping != TB_MAP_SPLIT_K ? 1 : 0;
  tbk::KernelKey key{(int)c.block_m, (int)c.block_n, (int)c.block_k,
                     (int)c.wave_grid_m, (int)c.wave_grid_n, out_mode,
                     (int)c.stages, epi, (int)c.mfma};
  const tbk::KernelEntry *e = tbk::find_kernel(key);
  // an instance that spills to scratch is refused, as the plan refuses it
  // (the build-time table of the compiler's register report)
  if (e) {
    tb::InstanceKey ik;
    ik.bm = c.block_m;
    ik.bn = c.block_n;
    ik.bk = c.block_k;
    ik.wgm = c.wave_grid_m;
    ik.wgn = c.wave_grid_n;
    ik.out = out_mode;
    ik.stages = c.stages;
    ik.epi = epi;
    ik.mfma = c.mfma;
    if (const std::string why = tb::spillRefusal(ik, c.k % c.block_k != 0); !why.empty())
      return fail(why);
  }
  if (!e) {
    char buf[256];
    snprintf(buf, sizeof buf,
             "no gfx950 kernel instance for tile %lldx%lldx%lld, wave grid "
             "%lldx%lld, %lld LDS stages, output mode %d%s%s",
             (long long)c.block_m, (long long)c.block_n, (long long)c.block_k,
             (long long)c.wave_grid_m, (long long)c.wave_grid_n,
             (long long)c.stages, out_mode, epi ? " with fused epilogue steps" : "",
             c.mfma == TB_MFMA_16X16X32 ? " on mfma_f32_16x16x32_f16" : "");
    return fail(buf);
  }
  tb_gemm_desc *d = new tb_gemm_desc();
  d->cfg = c;
  d->cfg.num_programs = programs;
  d->entry = e;
  d->out_mode = out_mode;
  d->tiles_m = tiles_m;
  d->tiles_n = tiles_n;
  d->tiles_k = tiles_k;
  d->total_work = total_work;
  d->lds_bytes = c.stages * (c.block_m + c.block_n) * c.block_k * 2;
  d->workspace_bytes = c.reduction == TB_RED_WORKSPACE
                           ? (size_t)(c.split_k * c.m * c.n * 4)
                           : 0;
  *out = d;
  return 0;
}

} // namespace tbrt

// ---- the scratch of tb_gemm_launch_noalloc --------------------------------
// The split-K workspace of the entry point that allocates nothing: a static
// device array of TB_NOALLOC_SCRATCH_BYTES, one copy per GPU, held until the
// process ends. Host code never passes `scratch` itself to a kernel (in host
// code the name is a host-side stand-in, not a device address): the device
// address comes from hipGetSymbolAddress, once per device with that device
// current, and is kept per device. Calls on one GPU share its array; each
// call writes every partial its reduction reads, so nothing needs clearing,
// and calls that overlap on one GPU race.
static __device__ __align__(256) float scratch[TB_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The scratch of the device the kernels run on: the stream's device (the
// current device for the null stream). Its address is looked up once, with
// that device made current for the lookup and the caller's current device
// restored afterwards.
int scratch_address(hipStream_t stream, void **out) {
  int dev = 0;
  if (stream) {
    hipDevice_t sd = 0;
    if (int rc = check_hip(hipStreamGetDevice(stream, &sd), "hipStreamGetDevice"))
      return rc;
    dev = (int)sd;
  } else if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) {
    return rc;
  }
  if (dev < 0 || dev >= kMaxDevices)
    return fail("tb_gemm_launch_noalloc: device index " + std::to_string(dev) +
                " beyond the library's table of " + std::to_string(kMaxDevices));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = 0;
    if (int rc = check_hip(hipGetDevice(&cur), "hipGetDevice"))
      return rc;
    if (cur != dev)
      if (int rc = check_hip(hipSetDevice(dev), "hipSetDevice"))
        return rc;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev)
      if (int rc = check_hip(hipSetDevice(cur), "hipSetDevice (restore)"))
        return rc;
    if (int rc = check_hip(e, "hipGetSymbolAddress(scratch)"))
      return rc;
    if (!ptr)
      return fail("tb_gemm_launch_noalloc: hipGetSymbolAddress returned no address");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

static int launch_impl(const tb_gemm_desc *d, const void *a, const void *b, void *c,
                       const void *bias, void *workspace, void *stream, const char *who) {
  if (!d)
    return fail(std::string(who) + ": desc is NULL");
  if (!a || !b || !c)
    return fail("tb_gemm_launch: A, B and C must be device pointers");
  // every kernel moves 16-byte vectors from these bases
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
       reinterpret_cast<uintptr_t>(c)) % 16)
    return fail("tb_gemm_launch: A, B and C must be 16-byte aligned");
  if (d->cfg.epi_bias != TB_EPI_BIAS_NONE) {
    // the epilogue reads 4 bias values per vector load
    const uintptr_t align = d->cfg.epi_bias == TB_EPI_BIAS_F16 ? 8 : 16;
    if (!bias)
      return fail("tb_gemm_launch_ex: this descriptor adds a bias; bias is NULL");
    if (reinterpret_cast<uintptr_t>(bias) % align)
      return fail("tb_gemm_launch_ex: the bias must be " + std::to_string(align) +
                  "-byte aligned");
  } else if (bias) {
    return fail("tb_gemm_launch_ex: this descriptor has no bias step; pass NULL");
  }
  if (d->workspace_bytes && !workspace)
    return fail("tb_gemm_launch: this descriptor needs a workspace of " +
                std::to_string(d->workspace_bytes) + " bytes");
  if (d->workspace_bytes && reinterpret_cast<uintptr_t>(workspace) % 16)
    return fail("tb_gemm_launch: the workspace must be 16-byte aligned");
  const tb_gemm_config &cf = d->cfg;
  tbk::GemmParams p{};
  p.A = a;
  p.B = b;
  p.C = c;
  p.ws = reinterpret_cast<float *>(workspace);
  p.M = (int)cf.m;
  p.N = (int)cf.n;
  p.K = (int)cf.k;
  p.lda = (int)cf.lda;
  p.ldb = (int)cf.ldb;
  p.ldc = (int)cf.ldc;
  p.tiles_m = (int)d->tiles_m;
  p.tiles_n = (int)d->tiles_n;
  p.tiles_k = (int)d->tiles_k;
  p.group_m = (int)cf.group_m;
  p.split_k = (int)cf.split_k;
  p.mapping = cf.mapping;
  p.total_work = (int)d->total_work;
  p.xcds = cf.xcd_remap;
  p.ws_ld = (int)cf.n;
  p.bias = bias;
  p.epi_bias = cf.epi_bias;
  p.epi_act = cf.epi_activation;
  p.epi_clamp = cf.epi_clamp;
  p.clamp_lo = cf.clamp_min;
  p.clamp_hi = cf.clamp_max;
  if (d->out_mode == tbk::kOutF32Partial && cf.mapping != TB_MAP_SPLIT_K) {
    p.ws = reinterpret_cast<float *>(c); // plain f32 store into C
    p.ws_ld = (int)cf.ldc;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  void *args[] = {&p};
  const dim3 grid((unsigned)cf.num_programs),
      block((unsigned)(d->entry->threads ? d->entry->threads : cf.num_waves * 64));
  const void *fn = d->entry->fn_partial_k && cf.k % cf.block_k ? d->entry->fn_partial_k
                                                               : d->entry->fn;
  if (int rc = check_hip(hipLaunchKernel(fn, grid, block, args, 0, s),
                         "hipLaunchKernel(gemm)"))
    return rc;
  if (cf.mapping == TB_MAP_SPLIT_K && cf.reduction == TB_RED_WORKSPACE) {
    if (int rc = check_hip(
            tbk::launch_reduce_ex(p.ws, c, p.M, p.N, p.ldc, p.split_k,
                                  cf.c_dtype == TB_DTYPE_F16 ? 1 : 0,
                                  cf.acc_init == TB_ACC_INIT_LOAD_C ? 1 : 0,
                                  tbk::EpiArgs{bias, cf.epi_bias, cf.epi_activation,
                                               cf.epi_clamp, cf.clamp_min,
                                               cf.clamp_max},
                                  s),
            "hipLaunchKernel(split-k reduce)"))
      return rc;
  }
  return 0;
}

} // namespace

extern "C" {

const char *tb_last_error(void) { return g_last_error.c_str(); }

int tb_abi_version(void) { return TB_GFX950_ABI_VERSION; }

int tb_desc_create(const tb_gemm_config *cfg, tb_gemm_desc **out) {
  if (!cfg)
    return fail("tb_desc_create: cfg is NULL");
  return tbrt::create_desc(*cfg, out);
}

int tb_desc_get_config(const tb_gemm_desc *desc, tb_gemm_config *out) {
  if (!desc || !out)
    return fail("tb_desc_get_config: NULL argument");
  *out = desc->cfg;
  return 0;
}

const char *tb_desc_kernel_name(const tb_gemm_desc *desc) {
  return desc && desc->entry ? desc->entry->name : "";
}

int64_t tb_desc_lds_bytes(const tb_gemm_desc *desc) {
  return desc ? desc->lds_bytes : 0;
}

size_t tb_workspace_bytes(const tb_gemm_desc *desc) {
  return desc ? desc->workspace_bytes : 0;
}

void tb_desc_free(tb_gemm_desc *desc) { delete desc; }

int tb_gemm_launch(const tb_gemm_desc *d, const void *a, const void *b,
                   void *c, void *workspace, void *stream) {
  if (d && d->cfg.epi_bias != TB_EPI_BIAS_NONE)
    return fail("tb_gemm_launch: this descriptor adds a bias; pass it through "
                "tb_gemm_launch_ex");
  return tb_gemm_launch_ex(d, a, b, c, nullptr, workspace, stream);
}

int tb_gemm_launch_ex(const tb_gemm_desc *d, const void *a, const void *b,
                      void *c, const void *bias, void *workspace, void *stream) {
  return launch_impl(d, a, b, c, bias, workspace, stream, "tb_gemm_launch");
}

int tb_gemm_launch_noalloc(const tb_gemm_desc *d, const void *a, const void *b,
                           void *c, const void *bias, void *stream) {
  if (!d)
    return fail("tb_gemm_launch_noalloc: desc is NULL");
  void *ws = nullptr;
  if (d->workspace_bytes) {
    if (d->workspace_bytes > (size_t)TB_NOALLOC_SCRATCH_BYTES)
      return fail("tb_gemm_launch_noalloc: this descriptor needs " +
                  std::to_string(d->workspace_bytes) +
                  " bytes of split-K workspace, more than the library's static scratch of " +
                  std::to_string((size_t)TB_NOALLOC_SCRATCH_BYTES) +
                  " bytes; use tb_gemm_launch_ex with a caller-provided workspace");
    if (int rc = scratch_address(reinterpret_cast<hipStream_t>(stream), &ws))
      return rc;
  }
  return launch_impl(d, a, b, c, bias, ws, stream, "tb_gemm_launch_noalloc");
}

int tb_fill_seeded_f16(void *dst, int64_t rows, int64_t cols, int64_t ld,
                       uint64_t seed, int32_t dist, double scale, void *stream) {
  if (!dst || rows < 0 || cols < 0 || ld < cols)
    return fail("tb_fill_seeded_f16: bad arguments");
  if (dist != 0 && dist != 1)
    return fail("tb_fill_seeded_f16: dist must be 0 (uniform) or 1 (normal)");
  return check_hip(tbk::launch_fill(dst, rows, cols, ld, seed, dist, scale,
                                    reinterpret_cast<hipStream_t>(stream)),
                   "hipLaunchKernel(fill)");
}

int tb_clock_probe(uint64_t *out, int32_t workgroups, int32_t window_ticks, void *stream) {
  if (!out || workgroups < 1 || workgroups > 1024)
    return fail("tb_clock_probe: out must be a device pointer and workgroups in 1..1024");
  if (window_ticks < 1 || window_ticks > 100000)
    return fail("tb_clock_probe: window_ticks must be in 1..100000 (1 ms)");
  if (reinterpret_cast<uintptr_t>(out) % 8)
    return fail("tb_clock_probe: out must be 8-byte aligned");
  return check_hip(tbk::launch_clock_probe(reinterpret_cast<unsigned long long *>(out),
                                           workgroups, (unsigned)window_ticks,
                                           reinterpret_cast<hipStream_t>(stream)),
                   "hipLaunchKernel(clock probe)");
}

int tb_clock_stamp(uint64_t *out, int32_t workgroups, void *stream) {
  if (!out || workgroups < 1 || workgroups > 1024)
    return fail("tb_clock_stamp: out must be a device pointer and workgroups in 1..1024");
  if (reinterpret_cast<uintptr_t>(out) % 8)
    return fail("tb_clock_stamp: out must be 8-byte aligned");
  return check_hip(tbk::launch_clock_stamp(reinterpret_cast<unsigned long long *>(out),
                                           workgroups, reinterpret_cast<hipStream_t>(stream)),
                   "hipLaunchKernel(clock stamp)");
}

int tb_kernel_count(void) { return tbk::kernel_count(); }

const char *tb_kernel_name(int i) {
  const tbk::KernelEntry *e = tbk::kernel_at(i);
  return e ? e->name : "";
}

int tb_kernel_waits(int i, int32_t *vm_prologue, int32_t *vm_loop, int32_t *lgkm_loop) {
  const tbk::KernelEntry *e = tbk::kernel_at(i);
  if (!e || !vm_prologue || !vm_loop || !lgkm_loop)
    return fail("tb_kernel_waits: no instance " + std::to_string(i) + " or NULL output");
  *vm_prologue = e->vm_prologue;
  *vm_loop = e->vm_loop;
  *lgkm_loop = e->lgkm_loop;
  return 0;
}

int tb_kernel_resources(int i, int32_t partial_k, int32_t *vgprs, int32_t *agprs,
                        int32_t *scratch_bytes) {
  const tbk::KernelEntry *e = tbk::kernel_at(i);
  if (!e || !vgprs || !agprs || !scratch_bytes)
    return fail("tb_kernel_resources: no instance " + std::to_string(i) + " or NULL output");
  tb::InstanceKey ik;
  ik.bm = e->key.bm;
  ik.bn = e->key.bn;
  ik.bk = e->key.bk;
  ik.wgm = e->key.wgm;
  ik.wgn = e->key.wgn;
  ik.out = e->key.out;
  ik.stages = e->key.stages;
  ik.epi = e->key.epi;
  ik.mfma = e->key.mfma;
  const tb::InstanceResources r = tb::instanceResources(ik, partial_k != 0);
  if (!r.known)
    return fail(std::string("tb_kernel_resources: no compiler report for ") + e->name);
  *vgprs = (int32_t)r.vgprs;
  *agprs = (int32_t)r.agprs;
  *scratch_bytes = (int32_t)r.scratchBytes;
  return 0;
}

} // extern "C"
