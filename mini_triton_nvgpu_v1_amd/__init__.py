"""MI355X (gfx950) backend for the tb.matmul GEMM compiler path.

Python host layer over the C ABI in ``include/tb_gfx950.h`` (library
``lib/libtb_gfx950.so``, built in-tree by ``make -C mini_triton_nvgpu_v1_amd``).
The reference's user surface is the ``tb-opt`` driver plus an external
launcher (``tools/bench_stage1_fair.py:531-564``, ``:665-699``); here
:func:`plan_from_mlir` runs the same plan pipeline in-process and
:meth:`GemmDesc.launch` enqueues the gfx950 kernel on a HIP stream.

There is no CPU fallback: every entry point raises if the HIP library is
missing.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

__all__ = [
    "GemmConfig", "GemmDesc", "TbError", "lib", "build", "plan_from_mlir",
    "plan_from_file", "fill_seeded_f16", "kernel_names", "LIB_PATH", "TB_OPT",
    "DTYPE_F16", "DTYPE_F32", "ACC_INIT_ZERO", "ACC_INIT_LOAD_C", "MAP_TILE",
    "MAP_GROUPED_TILE", "MAP_SPLIT_K", "MAP_PERSISTENT_TILE",
    "MAP_PERSISTENT_GROUPED", "RED_NONE", "RED_WORKSPACE", "RED_ATOMIC",
    "EPI_BIAS_NONE", "EPI_BIAS_F16", "EPI_BIAS_F32", "ACT_NONE", "ACT_RELU",
    "ACT_GELU_TANH", "ACT_SILU", "CLAMP_MIN", "CLAMP_MAX", "MFMA_32X32X16",
    "MFMA_16X16X32", "NOALLOC_SCRATCH_BYTES",
]

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libtb_gfx950.so")
TB_OPT = os.path.join(PKG_DIR, "bin", "tb-opt")

DTYPE_F16, DTYPE_F32 = 0, 1
ACC_INIT_ZERO, ACC_INIT_LOAD_C = 0, 1
(MAP_TILE, MAP_GROUPED_TILE, MAP_SPLIT_K, MAP_PERSISTENT_TILE,
 MAP_PERSISTENT_GROUPED) = range(5)
RED_NONE, RED_WORKSPACE, RED_ATOMIC = 0, 1, 2
# fused epilogue steps (bias, activation, clamp), applied in that order
EPI_BIAS_NONE, EPI_BIAS_F16, EPI_BIAS_F32 = 0, 1, 2
ACT_NONE, ACT_RELU, ACT_GELU_TANH, ACT_SILU = 0, 1, 2, 3
CLAMP_MIN, CLAMP_MAX = 1, 2
# MFMA instruction of the instance (the EncodingPlan's instrShape)
MFMA_32X32X16, MFMA_16X16X32 = 0, 1
# static split-K scratch of tb_gemm_launch_noalloc per GPU
NOALLOC_SCRATCH_BYTES = 32 * 1024 * 1024


class TbError(RuntimeError):
    """An error reported by libtb_gfx950 (tb_last_error())."""


class GemmConfig(ctypes.Structure):
    """Mirror of ``tb_gemm_config`` (include/tb_gfx950.h)."""
    _fields_ = [
        ("m", ctypes.c_int64), ("n", ctypes.c_int64), ("k", ctypes.c_int64),
        ("lda", ctypes.c_int64), ("ldb", ctypes.c_int64), ("ldc", ctypes.c_int64),
        ("c_dtype", ctypes.c_int32), ("acc_init", ctypes.c_int32),
        ("block_m", ctypes.c_int64), ("block_n", ctypes.c_int64),
        ("block_k", ctypes.c_int64), ("num_waves", ctypes.c_int64),
        ("wave_grid_m", ctypes.c_int64), ("wave_grid_n", ctypes.c_int64),
        ("stages", ctypes.c_int64), ("mapping", ctypes.c_int32),
        ("group_m", ctypes.c_int64), ("split_k", ctypes.c_int64),
        ("reduction", ctypes.c_int32), ("num_programs", ctypes.c_int64),
        ("xcd_remap", ctypes.c_int32),
        ("epi_bias", ctypes.c_int32), ("epi_activation", ctypes.c_int32),
        ("epi_clamp", ctypes.c_int32), ("clamp_min", ctypes.c_float),
        ("clamp_max", ctypes.c_float), ("mfma", ctypes.c_int32),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}

    def __eq__(self, other) -> bool:
        return isinstance(other, GemmConfig) and self.as_dict() == other.as_dict()

    def __repr__(self) -> str:
        return f"GemmConfig({self.as_dict()})"


_lib = None


def build() -> None:
    """Compile the backend in-tree (make always runs; it rebuilds what changed)."""
    jobs = str(min(16, os.cpu_count() or 4))
    subprocess.run(["make", "-s", "-j" + jobs, "-C", PKG_DIR], check=True)


def lib() -> ctypes.CDLL:
    """Load libtb_gfx950.so; raises TbError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise TbError(
            f"{LIB_PATH} is missing: build the gfx950 backend first "
            "(make -C mini_triton_nvgpu_v1_amd, or __graft_entry__.build())")
    # PyTorch-ROCm ships its own HIP runtime (torch/lib/libamdhip64.so, with
    # its own HSA runtime). Loaded first, torch's copy is the one this
    # library binds (same soname); loaded after this library had pulled in
    # /opt/rocm's, torch would load its copy as well, and two runtimes in one
    # process do not share the GPU (hipLaunchKernel: "no ROCm-capable
    # device"). So torch, when installed, is imported before the library.
    import importlib.util
    if importlib.util.find_spec("torch") is not None:
        import torch  # noqa: F401
    L = ctypes.CDLL(LIB_PATH)
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    pdesc = ctypes.POINTER(vp)
    L.tb_last_error.restype = ctypes.c_char_p
    L.tb_last_error.argtypes = []
    L.tb_abi_version.restype = ctypes.c_int
    L.tb_desc_create.argtypes = [ctypes.POINTER(GemmConfig), pdesc]
    L.tb_desc_create.restype = ctypes.c_int
    L.tb_plan_from_mlir.argtypes = [ctypes.c_char_p, ctypes.c_size_t,
                                    ctypes.c_char_p, pdesc]
    L.tb_plan_from_mlir.restype = ctypes.c_int
    L.tb_plan_from_file.argtypes = [ctypes.c_char_p, pdesc]
    L.tb_plan_from_file.restype = ctypes.c_int
    L.tb_desc_get_config.argtypes = [vp, ctypes.POINTER(GemmConfig)]
    L.tb_desc_get_config.restype = ctypes.c_int
    L.tb_desc_kernel_name.argtypes = [vp]
    L.tb_desc_kernel_name.restype = ctypes.c_char_p
    L.tb_desc_lds_bytes.argtypes = [vp]
    L.tb_desc_lds_bytes.restype = i64
    L.tb_workspace_bytes.argtypes = [vp]
    L.tb_workspace_bytes.restype = ctypes.c_size_t
    L.tb_gemm_launch.argtypes = [vp, vp, vp, vp, vp, vp]
    L.tb_gemm_launch.restype = ctypes.c_int
    L.tb_gemm_launch_ex.argtypes = [vp, vp, vp, vp, vp, vp, vp]
    L.tb_gemm_launch_ex.restype = ctypes.c_int
    L.tb_gemm_launch_noalloc.argtypes = [vp, vp, vp, vp, vp, vp]
    L.tb_gemm_launch_noalloc.restype = ctypes.c_int
    L.tb_desc_free.argtypes = [vp]
    L.tb_desc_free.restype = None
    L.tb_fill_seeded_f16.argtypes = [vp, i64, i64, i64, ctypes.c_uint64, i32,
                                     ctypes.c_double, vp]
    L.tb_fill_seeded_f16.restype = ctypes.c_int
    L.tb_clock_probe.argtypes = [vp, i32, i32, vp]
    L.tb_clock_probe.restype = ctypes.c_int
    L.tb_clock_stamp.argtypes = [vp, i32, vp]
    L.tb_clock_stamp.restype = ctypes.c_int
    L.tb_kernel_count.restype = ctypes.c_int
    L.tb_kernel_resources.argtypes = [i32, i32] + [ctypes.POINTER(ctypes.c_int32)] * 3
    L.tb_kernel_resources.restype = ctypes.c_int
    L.tb_kernel_name.argtypes = [ctypes.c_int]
    L.tb_kernel_name.restype = ctypes.c_char_p
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != 0:
        raise TbError(lib().tb_last_error().decode())


def _ptr(x) -> int | None:
    """Device address of a torch tensor, an int address, or None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _stream_handle(stream) -> int | None:
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream  # torch.cuda.Stream -> hipStream_t


def _is_tensor(x) -> bool:
    return hasattr(x, "data_ptr") and hasattr(x, "untyped_storage")


def _check_operand(x, role: str, dtypes: tuple, rows: int, cols: int, ld: int,
                   elem: int) -> None:
    """Check a torch tensor against what the kernels will touch through its
    address: the element type, the row-major (rows x cols, leading dimension
    ld) footprint inside the tensor's storage and the layout of a 2-D
    tensor. Raw integer addresses are the caller's responsibility, as in the
    C ABI."""
    if x is None or not _is_tensor(x):
        return
    names = " or ".join(str(d).replace("torch.", "") for d in dtypes)
    if x.dtype not in dtypes:
        raise TbError(f"{role}: expected a {names} tensor, got {x.dtype}")
    need = ((rows - 1) * ld + cols) * elem if rows > 0 and cols > 0 else 0
    st = x.untyped_storage()
    avail = st.data_ptr() + st.nbytes() - x.data_ptr()
    if need > avail:
        raise TbError(f"{role}: the descriptor touches {need} bytes from the tensor's "
                      f"address, its storage holds {avail}")
    if x.dim() == 2 and rows > 1 and cols > 1:
        if x.shape[0] < rows or x.shape[1] < cols or x.stride(1) != 1 or x.stride(0) != ld:
            raise TbError(f"{role}: a 2-D tensor must be at least {rows} x {cols}, "
                          f"row-major with leading dimension {ld} (got shape "
                          f"{tuple(x.shape)}, strides {tuple(x.stride())})")


class GemmDesc:
    """Owning handle of a ``tb_gemm_desc``."""

    def __init__(self, handle: int):
        self._h = ctypes.c_void_p(handle)

    @classmethod
    def from_config(cls, cfg: GemmConfig | None = None, **fields) -> "GemmDesc":
        if cfg is None:
            cfg = GemmConfig(**fields)
        h = ctypes.c_void_p()
        _check(lib().tb_desc_create(ctypes.byref(cfg), ctypes.byref(h)))
        return cls(h.value)

    @property
    def handle(self) -> int:
        return self._h.value

    @property
    def config(self) -> GemmConfig:
        cfg = GemmConfig()
        _check(lib().tb_desc_get_config(self._h, ctypes.byref(cfg)))
        return cfg

    @property
    def kernel_name(self) -> str:
        return lib().tb_desc_kernel_name(self._h).decode()

    @property
    def lds_bytes(self) -> int:
        return lib().tb_desc_lds_bytes(self._h)

    @property
    def workspace_bytes(self) -> int:
        return lib().tb_workspace_bytes(self._h)

    def check_operands(self, a, b, c, workspace=None, bias=None) -> None:
        """Check torch tensors against this descriptor before their addresses
        go to the C ABI: A (M x K, lda) and B (K x N, ldb) f16, C (M x N, ldc)
        of the config's C type, the bias (N values of the bias type) and the
        workspace (workspace_bytes). The kernels bound their accesses by the
        descriptor's sizes, not the tensor's, so a short or mistyped tensor
        would be written past its end. Raises TbError; raw integer addresses
        pass unchecked."""
        if not any(_is_tensor(x) for x in (a, b, c, workspace, bias)):
            return
        import torch
        cf = self.config
        f16, f32 = (torch.float16,), (torch.float32,)
        _check_operand(a, "A", f16, cf.m, cf.k, cf.lda, 2)
        _check_operand(b, "B", f16, cf.k, cf.n, cf.ldb, 2)
        cdt, ce = (f16, 2) if cf.c_dtype == DTYPE_F16 else (f32, 4)
        _check_operand(c, "C", cdt, cf.m, cf.n, cf.ldc, ce)
        if cf.epi_bias != EPI_BIAS_NONE:
            bdt, be = (f16, 2) if cf.epi_bias == EPI_BIAS_F16 else (f32, 4)
            _check_operand(bias, "bias", bdt, 1, cf.n, cf.n, be)
        if self.workspace_bytes and _is_tensor(workspace):
            _check_operand(workspace, "workspace", (workspace.dtype,), 1,
                           self.workspace_bytes, self.workspace_bytes, 1)
        for role, x in (("A", a), ("B", b), ("C", c), ("workspace", workspace),
                        ("bias", bias)):
            if _is_tensor(x) and not x.is_cuda:
                raise TbError(f"{role}: the tensor must be on a GPU (got {x.device})")
        devs = {x.device for x in (a, b, c, workspace, bias) if _is_tensor(x)}
        if len(devs) > 1:
            raise TbError(f"operands are on different devices: {sorted(map(str, devs))}")

    @staticmethod
    def _default_stream(stream, *xs):
        """An explicit stream wins; else torch's current stream of the
        tensors' device (work queued there by torch then orders with the
        GEMM); else the null stream."""
        if stream is not None:
            return _stream_handle(stream)
        for x in xs:
            if _is_tensor(x) and x.is_cuda:
                import torch
                return torch.cuda.current_stream(x.device).cuda_stream
        return None

    def launch(self, a, b, c, workspace=None, stream=None, bias=None) -> None:
        """Enqueue C = A*B (or C += A*B), then the config's fused epilogue
        steps, for device tensors/addresses. ``bias`` (N values) is required
        exactly when the config adds one. Tensors are checked against the
        descriptor (check_operands); ``stream`` defaults to torch's current
        stream of the tensors' device."""
        self.check_operands(a, b, c, workspace, bias)
        st = self._default_stream(stream, a, b, c)
        if bias is None:
            _check(lib().tb_gemm_launch(self._h, _ptr(a), _ptr(b), _ptr(c),
                                        _ptr(workspace), st))
        else:
            _check(lib().tb_gemm_launch_ex(self._h, _ptr(a), _ptr(b), _ptr(c),
                                           _ptr(bias), _ptr(workspace), st))

    def launch_noalloc(self, a, b, c, stream=None, bias=None) -> None:
        """Like launch, with no workspace argument: a split-K descriptor's
        partials go to the library's static per-GPU scratch
        (NOALLOC_SCRATCH_BYTES), and nothing is allocated. Calls that overlap
        on one GPU share that scratch and race."""
        self.check_operands(a, b, c, None, bias)
        st = self._default_stream(stream, a, b, c)
        _check(lib().tb_gemm_launch_noalloc(self._h, _ptr(a), _ptr(b), _ptr(c),
                                            _ptr(bias), st))

    def bind(self, a, b, c, workspace=None, stream=None, bias=None):
        """A zero-argument launcher for repeated launches on the same buffers
        and stream: the operands are checked, and device addresses and the
        stream handle resolved, once, so each call is one C call (the shape of
        the reference's driver loop, tools/bench_stage1_fair.py:680-699). The
        buffers must outlive it."""
        self.check_operands(a, b, c, workspace, bias)
        L = lib()
        args = (self._h, _ptr(a), _ptr(b), _ptr(c))
        ws, st = _ptr(workspace), self._default_stream(stream, a, b, c)
        if bias is None:
            fn, args = L.tb_gemm_launch, args + (ws, st)
        else:
            fn, args = L.tb_gemm_launch_ex, args + (_ptr(bias), ws, st)
        keep = (self, a, b, c, workspace, bias)  # hold the buffers and descriptor

        def launch() -> None:
            if fn(*args):
                _check(-1)
        launch.keep = keep
        return launch

    def close(self) -> None:
        if self._h and self._h.value:
            lib().tb_desc_free(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def plan_from_mlir(text: str, gpu_arch: str = "gfx950") -> GemmDesc:
    """Run the tb plan pipeline on a module holding one tb.matmul."""
    data = text.encode()
    h = ctypes.c_void_p()
    _check(lib().tb_plan_from_mlir(data, len(data), gpu_arch.encode(),
                                   ctypes.byref(h)))
    return GemmDesc(h.value)


def plan_from_file(path: str) -> GemmDesc:
    """Load the descriptor side-file written by tb-lower-pipeline-to-gfx950."""
    h = ctypes.c_void_p()
    _check(lib().tb_plan_from_file(path.encode(), ctypes.byref(h)))
    return GemmDesc(h.value)


def fill_seeded_f16(dst, rows: int, cols: int, seed: int, dist: int = 0,
                    scale: float = 1.0, ld: int | None = None,
                    stream=None) -> None:
    """Device-side seeded f16 fill (SplitMix64; dist 0 uniform, 1 normal)."""
    _check(lib().tb_fill_seeded_f16(_ptr(dst), rows, cols,
                                    cols if ld is None else ld, seed, dist,
                                    scale, _stream_handle(stream)))


def clock_probe(out, workgroups: int = 8, window_ticks: int = 2000, stream=None) -> None:
    """Probe the shader clock from `workgroups` one-wave workgroups over
    `window_ticks` ticks of the 100 MHz counter, into the 64-bit device tensor
    `out` (XCC id, cycles, ticks per workgroup), on `stream`."""
    _check(lib().tb_clock_probe(_ptr(out), workgroups, window_ticks, _stream_handle(stream)))


def probe_clock_mhz(readings) -> float | None:
    """The mean shader clock of a clock_probe reading (a host list of
    (XCC id, cycles, ticks) triples): total cycles / total ticks * 100 MHz."""
    cyc = sum(int(readings[3 * i + 1]) for i in range(len(readings) // 3))
    ticks = sum(int(readings[3 * i + 2]) for i in range(len(readings) // 3))
    return cyc / ticks * 100.0 if ticks > 0 else None


def clock_stamp(out, workgroups: int = 1024, stream=None) -> None:
    """Stamp (where, shader-clock count, 100 MHz count) from `workgroups`
    one-wave workgroups into the 64-bit device tensor `out`, on `stream`;
    `where` is XCC id << 8 | the SE, SH and CU fields of HW_ID."""
    _check(lib().tb_clock_stamp(_ptr(out), workgroups, _stream_handle(stream)))


def stamps_clock_mhz(before, after) -> dict:
    """Per-CU mean shader clock between two clock_stamp readings (host lists
    of (where, cycles, ticks) triples): for each CU present in both, (cycles
    after - cycles before) / (ticks after - ticks before) * 100 MHz. A CU's
    counter is its own, so only stamps of the same CU are paired (the first
    reading of each CU in each stamp); pairs whose counters did not advance
    are left out."""
    def by_cu(r):
        d = {}
        for i in range(len(r) // 3):
            d.setdefault(int(r[3 * i]), (int(r[3 * i + 1]), int(r[3 * i + 2])))
        return d
    b, a = by_cu(before), by_cu(after)
    out = {}
    for x in sorted(set(b) & set(a)):
        dc, dt = a[x][0] - b[x][0], a[x][1] - b[x][1]
        if dc > 0 and dt > 0:
            out[x] = dc / dt * 100.0
    return out


def kernel_names() -> list[str]:
    L = lib()
    return [L.tb_kernel_name(i).decode() for i in range(L.tb_kernel_count())]


def kernel_resources(partial_k: bool = False) -> dict[str, tuple[int, int, int]]:
    """name -> (VGPRs, AGPRs, scratch bytes per lane) of every compiled
    instance (partial_k: its build for a partial last k-tile), from the
    compiler's report. The plan and tb_desc_create refuse an instance whose
    scratch is not zero."""
    L = lib()
    out = {}
    for i in range(L.tb_kernel_count()):
        v = [ctypes.c_int32() for _ in range(3)]
        _check(L.tb_kernel_resources(i, int(partial_k), *[ctypes.byref(x) for x in v]))
        out[L.tb_kernel_name(i).decode()] = tuple(x.value for x in v)
    return out
