"""The five benchmark/parity workloads of the tb.matmul gfx950 path.

Each workload is a ``tb.matmul`` module (the reference's own input format,
``examples/*.mlir``) plus the seeded-input recipe. Shapes follow
``examples/smoke_64x64x32.mlir``, ``examples/smoke_96x80x32.mlir``,
``examples/smoke_128x128x32.mlir``, and scaled-up versions of
``examples/smoke_splitk_64x64x64.mlir`` and
``examples/smoke_persistent_192x128x32.mlir``. Unlike the reference
(f32 C, C += A*B) these write f16 C = A*B with f32 accumulation.
"""
from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass, field

from . import (ACC_INIT_LOAD_C, ACC_INIT_ZERO, ACT_GELU_TANH, ACT_NONE, ACT_RELU, ACT_SILU,
               CLAMP_MAX, CLAMP_MIN, DTYPE_F16, DTYPE_F32, EPI_BIAS_F16, EPI_BIAS_F32,
               EPI_BIAS_NONE, MAP_GROUPED_TILE, MAP_PERSISTENT_GROUPED,
               MAP_SPLIT_K, MAP_TILE, MFMA_16X16X32, MFMA_32X32X16, RED_NONE,
               RED_WORKSPACE, GemmConfig)

ACTIVATIONS = {"": ACT_NONE, "relu": ACT_RELU, "gelu_tanh": ACT_GELU_TANH,
               "silu": ACT_SILU}
BIAS_KINDS = {"": EPI_BIAS_NONE, "f16": EPI_BIAS_F16, "f32": EPI_BIAS_F32}

UNIFORM, NORMAL = 0, 1


def wave_grid(block_m: int, block_n: int, num_waves: int, instr: int = 32):
    """The plan's wave-grid choice: minimise |wave_tile_m - wave_tile_n| over
    grids whose wave tiles are whole MFMA tiles, ties to more waves along the
    longer block side (reference EncodingPlan.cpp:283-320)."""
    best, best_score = None, None
    for gm in range(1, num_waves + 1):
        if num_waves % gm:
            continue
        gn = num_waves // gm
        if block_m % gm or block_n % gn:
            continue
        tm, tn = block_m // gm, block_n // gn
        if tm % instr or tn % instr:
            continue
        score = abs(tm - tn)
        tie = best is not None and score == best_score and (
            (block_m >= block_n and gm > best[0]) or (block_m < block_n and gn > best[1]))
        if best is None or score < best_score or tie:
            best, best_score = (gm, gn), score
    if best is None:
        raise ValueError("no legal wave grid")
    return best


_M16_TILES = None


def mfma16_tiles() -> set:
    """(BM, BN, BK, wave grid M, wave grid N, stages) of every 16x16x32
    instance: the hand-scheduled tile and the TBK_M16_TILES_* lists of
    csrc/kernels/gemm_tiles.h, read from the header the kernels and the
    plan's instance table are built from."""
    global _M16_TILES
    if _M16_TILES is None:
        import os
        import re
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc", "kernels",
                            "gemm_tiles.h")
        text = open(path).read()
        tiles = {(256, 256, 64, 2, 2, 2)}
        for m in re.finditer(r"#define TBK_M16_TILES_\w+\(X\)((?:.*\\\n)*.*)", text):
            for t in re.findall(r"X\(([^)]*)\)", m.group(1)):
                tiles.add(tuple(int(v) for v in t.split(",")))
        _M16_TILES = tiles
    return _M16_TILES


@dataclass(frozen=True)
class Workload:
    name: str
    M: int
    N: int
    K: int
    seed: int
    dist: int
    block: tuple  # (block_m, block_n, block_k)
    num_waves: int
    stages: int = 2
    group_m: int = 8
    exact_tile: bool = True
    split_k: int = 1
    persistent: bool = False
    num_ctas: int = 1
    module_attrs: dict = field(default_factory=dict)
    # fused epilogue steps (tb.matmul `epilogue_*` attrs)
    bias: str = ""          # "", "f16" or "f32"
    activation: str = ""    # "", "relu", "gelu_tanh" or "silu"
    clamp_min: float | None = None
    clamp_max: float | None = None
    # f32 C with C += A*B (the reference's own tb.matmul semantics) instead of
    # f16 C = A*B
    c_f32: bool = False

    @property
    def flop(self) -> int:
        return 2 * self.M * self.N * self.K

    @property
    def algo_bytes(self) -> int:
        """Algorithmic HBM bytes: A and B moved once, and the f16 C written
        once (an f32 C += A*B: read and written once)."""
        c_bytes = 8 * self.M * self.N if self.c_f32 else 2 * self.M * self.N
        return 2 * (self.M * self.K + self.K * self.N) + c_bytes

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.K) if self.dist == NORMAL else 1.0

    @property
    def seed_b(self) -> int:
        return self.seed ^ 0xB

    def mlir(self, c_type: str | None = None) -> str:
        """The tb.matmul module fed to the plan pipeline (an f32 C makes it
        C += A*B)."""
        c_type = c_type or ("f32" if self.c_f32 else "f16")
        attrs = {"tb.num-warps": f"{self.num_waves} : i64",
                 "tb.requested-stages": f"{self.stages} : i64"}
        if self.split_k > 1:
            attrs["tb.split-k"] = f"{self.split_k} : i64"
            attrs["tb.reduction-mode"] = '"split_k_serial"'
        if self.persistent:
            attrs["tb.persistent"] = "true"
            attrs["tb.num-ctas"] = f"{self.num_ctas} : i64"
        attrs.update(self.module_attrs)
        mattr = ", ".join(f'"{k}" = {v}' for k, v in attrs.items())
        bm, bn, bk = self.block
        M, N, K = self.M, self.N, self.K
        a, b, c = (f"memref<{M}x{K}xf16>", f"memref<{K}x{N}xf16>",
                   f"memref<{M}x{N}x{c_type}>")
        gm = f",\n                          group_m = {self.group_m} : i64"
        if self.bias:
            gm += f',\n                          epilogue_bias = "{self.bias}"'
        if self.activation:
            gm += f',\n                          epilogue_activation = "{self.activation}"'
        if self.clamp_min is not None:
            gm += f",\n                          epilogue_clamp_min = {float(self.clamp_min)!r} : f32"
        if self.clamp_max is not None:
            gm += f",\n                          epilogue_clamp_max = {float(self.clamp_max)!r} : f32"
        return (
            f"module attributes {{{mattr}}} {{\n"
            f"  func.func @kernel(%A: {a}, %B: {b},\n"
            f"                    %C: {c}) {{\n"
            f"    tb.matmul %A, %B, %C {{block_m = {bm} : i64, block_n = {bn} : i64,\n"
            f"                          block_k = {bk} : i64, exact_tile = "
            f"{'true' if self.exact_tile else 'false'}{gm}}}\n"
            f"      : {a}, {b}, {c}\n"
            f"    func.return\n"
            f"  }}\n"
            f"}}\n")

    def direct_config(self) -> GemmConfig:
        """Flattened descriptor equal to what the plan pipeline derives
        (tb_plan_from_mlir on ``self.mlir()``); the tests check the two agree
        field by field."""
        bm, bn, bk = self.block
        wg = wave_grid(bm, bn, self.num_waves)
        tiles_m, tiles_n = -(-self.M // bm), -(-self.N // bn)
        if self.persistent:
            mapping = MAP_PERSISTENT_GROUPED
            programs = min(self.num_ctas, tiles_m * tiles_n)
        elif self.split_k > 1:
            mapping = MAP_SPLIT_K
            programs = tiles_m * tiles_n * self.split_k
        elif self.group_m > 1 and tiles_m > 1 and tiles_n > 1:
            mapping = MAP_GROUPED_TILE
            programs = tiles_m * tiles_n
        else:
            mapping = MAP_TILE
            programs = tiles_m * tiles_n
        return GemmConfig(
            m=self.M, n=self.N, k=self.K, lda=self.K, ldb=self.N, ldc=self.N,
            c_dtype=DTYPE_F32 if self.c_f32 else DTYPE_F16,
            acc_init=ACC_INIT_LOAD_C if self.c_f32 else ACC_INIT_ZERO, block_m=bm, block_n=bn,
            block_k=bk, num_waves=self.num_waves, wave_grid_m=wg[0],
            wave_grid_n=wg[1], stages=self.stages, mapping=mapping,
            group_m=self.group_m if mapping not in (MAP_TILE, MAP_SPLIT_K) else 1,
            split_k=self.split_k,
            reduction=RED_WORKSPACE if self.split_k > 1 else RED_NONE,
            num_programs=programs,
            # XCD-aware program order once the tiles fill the 256 CUs
            # (not for split-K: there each XCD holds one split's K range)
            xcd_remap=8 if tiles_m * tiles_n >= 256 and mapping != MAP_SPLIT_K else 0,
            epi_bias=BIAS_KINDS[self.bias],
            epi_activation=ACTIVATIONS[self.activation],
            epi_clamp=(CLAMP_MIN if self.clamp_min is not None else 0)
            | (CLAMP_MAX if self.clamp_max is not None else 0),
            clamp_min=self.clamp_min or 0.0, clamp_max=self.clamp_max or 0.0,
            mfma=MFMA_16X16X32 if self.mfma16_supported() else MFMA_32X32X16)

    def mfma16_supported(self) -> bool:
        """The plan's choice of v_mfma_f32_16x16x32_f16 (without an `mma`
        attribute): every tile with a 16x16x32 instance on the plan's wave
        grid (the hand-scheduled 4-wave 256x256x64 2-stage tile and the
        16x16x32 loop's lists), f16 or f32 C, any M, N and K, no split-K."""
        if self.split_k != 1:
            return False
        wg = wave_grid(*self.block[:2], self.num_waves)
        return (*self.block, *wg, self.stages) in mfma16_tiles()


SMOKE = Workload("smoke_64x64x32", 64, 64, 32, 0x5EED0001, UNIFORM,
                 (64, 64, 32), num_waves=4)
RAGGED = Workload("ragged_96x80x32", 96, 80, 32, 0x5EED0002, UNIFORM,
                  (64, 64, 32), num_waves=4, exact_tile=False)
RAGGED_128 = Workload("tile_128x128x32", 128, 128, 32, 0x5EED0003, UNIFORM,
                      (128, 128, 32), num_waves=4)
# 4 waves of 128x128 (one per SIMD) on the 256x256 tile: a third fewer LDS
# fragment bytes per MFMA than 8 waves of 64x128, and the
# 16x16x32 instance, a quarter of the accumulator register traffic per FLOP:
# less energy per launch, a higher sustained clock on this power-limited part
# (~14% faster than 8 waves of 32x32x16)
ROOFLINE = Workload("gemm_4096", 4096, 4096, 4096, 0x5EED0004, NORMAL,
                    (256, 256, 64), num_waves=4, stages=2, group_m=8)
# 128x64 tiles with 3 LDS stages: 32 tiles x 8 splits = 256 workgroups, one
# per CU (128x128 tiles would leave half the CUs idle); 8 waves of 32x32 (two
# per SIMD, one issuing while the other waits on its loads) measured 4% faster
# per call than 4 waves of 32x64
SPLIT_K = Workload("splitk_512x512x16384", 512, 512, 16384, 0x5EED0005,
                   UNIFORM, (128, 64, 64), num_waves=8, stages=3, split_k=8)
PERSISTENT = Workload("persistent_8192", 8192, 8192, 8192, 0x5EED0006, NORMAL,
                      (256, 256, 64), num_waves=4, group_m=8, persistent=True,
                      num_ctas=256)

ALL = [SMOKE, RAGGED, RAGGED_128, ROOFLINE, SPLIT_K, PERSISTENT]
# The roofline GEMM with fused epilogue steps (a bias row and the tanh GELU
# on the f32 result before the f16 store): what the fusion costs.
FUSED = [dataclasses.replace(ROOFLINE, name="gemm_4096_bias_gelu", bias="f16",
                             activation="gelu_tanh")]
# The roofline GEMM in the reference's own semantics: f32 C += A*B (the
# prior C read, the sum written back as f32).
F32_ACCUMULATE = [dataclasses.replace(ROOFLINE, name="gemm_4096_f32_accumulate",
                                      c_f32=True)]
# Profiling rows (not bench lines): the 16x16x32 loop's 4-wave 128x128 tile at
# 2048^3 (1024 tiles, four per CU), against the hand-scheduled 256x256 tile's
# MFMA-busy fraction at 4096^3.
PROFILE_ROWS = [Workload("gemm_2048_tile128", 2048, 2048, 2048, 0x5EED0007, NORMAL,
                         (128, 128, 64), num_waves=4, stages=3, group_m=8)]
BY_NAME = {w.name: w for w in ALL + FUSED + F32_ACCUMULATE + PROFILE_ROWS}
