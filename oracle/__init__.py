"""CPU oracle for the tb.matmul GEMM path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker or the
reported CPU baseline. The product library (``libtb_gfx950.so``) never loads
it and has no CPU fallback.

Thin ctypes/numpy wrapper over ``oracle/liboracle.so`` (built from
``oracle/oracle.c`` by ``oracle/Makefile``). Each C function cites the
reference file:line it restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

UNIFORM = 0
NORMAL = 1

# mapping codes of tbo_program_to_tile
MAP_TILE, MAP_GROUPED, MAP_SPLIT_K, MAP_PERSISTENT, MAP_PERSISTENT_GROUPED = range(5)


def build() -> None:
    """Compile liboracle.so with make (always runs make; make skips if fresh)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        u64, i64, dbl, vp = ctypes.c_uint64, ctypes.c_int64, ctypes.c_double, ctypes.c_void_p
        pi64 = ctypes.POINTER(i64)
        L.tbo_splitmix64_at.argtypes = [u64, u64]
        L.tbo_splitmix64_at.restype = u64
        L.tbo_uniform_at.argtypes = [u64, u64]
        L.tbo_uniform_at.restype = dbl
        L.tbo_normal_at.argtypes = [u64, u64]
        L.tbo_normal_at.restype = dbl
        L.tbo_f64_to_f16.argtypes = [dbl]
        L.tbo_f64_to_f16.restype = ctypes.c_uint16
        L.tbo_f16_to_f64.argtypes = [ctypes.c_uint16]
        L.tbo_f16_to_f64.restype = dbl
        L.tbo_fill_f16.argtypes = [vp, i64, i64, i64, u64, ctypes.c_int, dbl]
        L.tbo_fill_f16.restype = None
        L.tbo_gemm_f64.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, i64, i64,
                                   i64, i64, i64, ctypes.c_int]
        L.tbo_gemm_f64.restype = None
        L.tbo_check_tolerance.argtypes = [vp, ctypes.c_int, i64, vp, i64, i64,
                                          i64, i64, dbl, ctypes.POINTER(dbl),
                                          pi64, pi64]
        L.tbo_check_tolerance.restype = i64
        L.tbo_gemm_f32.argtypes = [vp, vp, vp, i64, i64, i64, ctypes.c_int]
        L.tbo_gemm_f32.restype = None
        L.tbo_epilogue_f64.argtypes = [vp, i64, i64, i64, vp, ctypes.c_int,
                                       ctypes.c_int, dbl, dbl]
        L.tbo_epilogue_f64.restype = None
        L.tbo_max_threads.argtypes = []
        L.tbo_max_threads.restype = ctypes.c_int
        L.tbo_program_to_tile.argtypes = [ctypes.c_int, i64, i64, i64, i64, i64,
                                          pi64, pi64, pi64]
        L.tbo_program_to_tile.restype = None
        L.tbo_split_k_range.argtypes = [i64, i64, i64, pi64, pi64]
        L.tbo_split_k_range.restype = None
        L.tbo_swizzle_minor.argtypes = [i64, i64, i64, i64, i64, i64]
        L.tbo_swizzle_minor.restype = i64
        L.tbo_swizzle_minor2.argtypes = [i64] * 9
        L.tbo_swizzle_minor2.restype = i64
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def splitmix64_at(seed: int, i: int) -> int:
    return lib().tbo_splitmix64_at(seed, i)


def f64_to_f16_bits(x: float) -> int:
    return lib().tbo_f64_to_f16(x)


def f16_bits_to_f64(h: int) -> float:
    return lib().tbo_f16_to_f64(h)


def fill_f16(rows: int, cols: int, seed: int, dist: int = UNIFORM,
             scale: float = 1.0) -> np.ndarray:
    """Seeded f16 matrix (row-major) returned as a numpy float16 array."""
    out = np.empty((rows, cols), dtype=np.uint16)
    lib().tbo_fill_f16(_ptr(out), rows, cols, cols, seed, dist, scale)
    return out.view(np.float16)


def config_inputs(M: int, N: int, K: int, seed: int, dist: int):
    """A uses stream `seed`, B uses `seed ^ 0xB`; normal inputs scaled 1/sqrt(K)."""
    scale = 1.0 / np.sqrt(K) if dist == NORMAL else 1.0
    A = fill_f16(M, K, seed, dist, scale)
    B = fill_f16(K, N, seed ^ 0xB, dist, scale)
    return A, B


def gemm_f64(A: np.ndarray, B: np.ndarray, init: np.ndarray | None = None,
             row_begin: int = 0, row_end: int | None = None,
             threads: int = 0) -> np.ndarray:
    """f64 reference of init + A@B for rows [row_begin, row_end)."""
    A = np.ascontiguousarray(A, dtype=np.float16)
    B = np.ascontiguousarray(B, dtype=np.float16)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    if row_end is None:
        row_end = M
    ref = np.empty((row_end - row_begin, N), dtype=np.float64)
    init_ptr = None
    ldi = 0
    if init is not None:
        init = np.ascontiguousarray(init, dtype=np.float32)
        assert init.shape == (M, N)
        init_ptr = _ptr(init)
        ldi = N
    lib().tbo_gemm_f64(_ptr(A), _ptr(B), init_ptr, _ptr(ref), M, N, K, K, N,
                       ldi, N, row_begin, row_end, threads)
    return ref


def epilogue_f64(ref: np.ndarray, bias: np.ndarray | None = None, act: int = 0,
                 clamp_bits: int = 0, lo: float = 0.0, hi: float = 0.0) -> np.ndarray:
    """Fused epilogue steps applied in place to an f64 result (bias, then
    activation 0 none / 1 relu / 2 gelu_tanh / 3 silu, then clamp)."""
    assert ref.dtype == np.float64 and ref.flags.c_contiguous
    rows, N = ref.shape
    bias_ptr = None
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.float64)
        assert bias.shape == (N,)
        bias_ptr = _ptr(bias)
    lib().tbo_epilogue_f64(_ptr(ref), rows, N, N, bias_ptr, act, clamp_bits,
                           float(lo), float(hi))
    return ref


def check_tolerance(got: np.ndarray, ref: np.ndarray, row_begin: int = 0,
                    rtol: float = 1e-2):
    """Count elements violating |got-ref| <= rtol*(|ref|+1) (NaN counts as bad).

    `got` is the whole M x N result; `ref` holds rows [row_begin,
    row_begin + ref.shape[0]) of the reference (as returned by gemm_f64).
    Returns (violations, max_abs_err, (worst_row, worst_col))."""
    got = np.ascontiguousarray(got)
    is_f32 = got.dtype == np.float32
    assert is_f32 or got.dtype == np.float16
    N = got.shape[1]
    row_end = row_begin + ref.shape[0]
    if got.shape[0] < row_end or ref.shape[1] != N:
        raise ValueError(f"check_tolerance: result has {got.shape} but the "
                         f"reference covers rows [{row_begin}, {row_end}) x {ref.shape[1]}")
    err = ctypes.c_double()
    wr, wc = ctypes.c_int64(), ctypes.c_int64()
    bad = lib().tbo_check_tolerance(_ptr(got), int(is_f32), N, _ptr(ref), N, N,
                                    row_begin, row_end, rtol, ctypes.byref(err),
                                    ctypes.byref(wr), ctypes.byref(wc))
    return bad, err.value, (wr.value, wc.value)


def gemm_f32(A: np.ndarray, B: np.ndarray, threads: int = 0) -> np.ndarray:
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    M, K = A.shape
    _, N = B.shape
    C = np.empty((M, N), dtype=np.float32)
    lib().tbo_gemm_f32(_ptr(A), _ptr(B), _ptr(C), M, N, K, threads)
    return C


def max_threads() -> int:
    return lib().tbo_max_threads()


def program_to_tile(mapping: int, pid: int, tiles_m: int, tiles_n: int,
                    group_m: int = 1, split_k: int = 1):
    m, n, p = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    lib().tbo_program_to_tile(mapping, pid, tiles_m, tiles_n, group_m, split_k,
                              ctypes.byref(m), ctypes.byref(n), ctypes.byref(p))
    return m.value, n.value, p.value


def split_k_range(tiles_k: int, split_k: int, part: int):
    s, c = ctypes.c_int64(), ctypes.c_int64()
    lib().tbo_split_k_range(tiles_k, split_k, part, ctypes.byref(s), ctypes.byref(c))
    return s.value, c.value


def swizzle_minor(major: int, minor: int, per_phase: int, max_phase: int,
                  span_elems: int, minor_extent: int) -> int:
    return lib().tbo_swizzle_minor(major, minor, per_phase, max_phase,
                                   span_elems, minor_extent)


def swizzle_minor2(major: int, minor: int, per_phase: int, max_phase: int,
                   span_elems: int, per_phase2: int, max_phase2: int,
                   span2_elems: int, minor_extent: int) -> int:
    """swizzle_minor, then the gfx950 second XOR term on span2 units."""
    return lib().tbo_swizzle_minor2(major, minor, per_phase, max_phase, span_elems,
                                    per_phase2, max_phase2, span2_elems, minor_extent)
