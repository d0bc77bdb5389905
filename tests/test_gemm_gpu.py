"""GPU parity of the gfx950 GEMM kernels against the fp64 oracle.

Inputs come from the oracle's seeded generator on the CPU and are uploaded;
the kernel runs through the C ABI (libtb_gfx950.so); the result is checked
per element with |got - ref| <= 1e-2 * (|ref| + 1) (f16 A/B, f32
accumulation: the path's stated tolerance). Outputs are pre-filled
with NaN so an element the kernel fails to write fails the check.
"""
import dataclasses
import time

import numpy as np
import pytest
import torch

import mini_triton_nvgpu_v1_amd as tb
import oracle
from mini_triton_nvgpu_v1_amd import configs

pytestmark = pytest.mark.gpu
RTOL = 1e-2


def _dev(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def run_desc(desc: tb.GemmDesc, A16, B16, device, c_init=None, c_dtype=torch.float16,
             M=None, N=None):
    M = A16.shape[0] if M is None else M
    N = B16.shape[1] if N is None else N
    dA, dB = _dev(A16, device), _dev(B16, device)
    if c_init is None:
        dC = torch.full((M, N), float("nan"), dtype=c_dtype, device=device)
    else:
        dC = _dev(c_init, device)
    ws = None
    if desc.workspace_bytes:
        ws = torch.empty(desc.workspace_bytes, dtype=torch.uint8, device=device)
    desc.launch(dA, dB, dC, ws)
    torch.cuda.synchronize()
    return dC.cpu().numpy()


def check(got, A16, B16, init=None, rows=None):
    """Full check, or a list of (row_begin, row_end) blocks."""
    blocks = rows or [(0, A16.shape[0])]
    for r0, r1 in blocks:
        ref = oracle.gemm_f64(A16, B16, init=init, row_begin=r0, row_end=r1)
        bad, err, worst = oracle.check_tolerance(got, ref, row_begin=r0, rtol=RTOL)
        print(f"rows [{r0},{r1}): violations={bad} max|err|={err:.3e} at {worst}", flush=True)
        assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"


@pytest.mark.parametrize("w", [configs.SMOKE, configs.RAGGED, configs.RAGGED_128,
                               configs.SPLIT_K, configs.ROOFLINE],
                         ids=lambda w: w.name)
def test_workload_parity(w, device):
    """The product path: tb.matmul module text -> plan pipeline -> kernel."""
    print(f"workload {w.name} {w.M}x{w.N}x{w.K}", flush=True)
    A, B = oracle.config_inputs(w.M, w.N, w.K, w.seed, w.dist)
    desc = tb.plan_from_mlir(w.mlir())
    got = run_desc(desc, A, B, device)
    check(got, A, B)


@pytest.fixture(scope="module")
def persistent_8192_ref():
    """The 8192^3 workload's seeded inputs and the whole fp64 product (all
    8192 rows; the OpenMP oracle takes tens of seconds on the box's cores)."""
    w = configs.PERSISTENT
    A, B = oracle.config_inputs(w.M, w.N, w.K, w.seed, w.dist)
    t0 = time.perf_counter()
    ref = oracle.gemm_f64(A, B)
    print(f"fp64 oracle 8192^3: {time.perf_counter() - t0:.1f} s", flush=True)
    return A, B, ref


def _check_full(got, ref):
    bad, err, worst = oracle.check_tolerance(got, ref, rtol=RTOL)
    print(f"all {ref.shape[0]} rows: violations={bad} max|err|={err:.3e} at {worst}",
          flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"


def test_persistent_8192_parity(device, persistent_8192_ref):
    """8192^3 through the plan (256x256 tiles, 256 resident programs striding
    over 1024 tiles in grouped order): every element against fp64."""
    w = configs.PERSISTENT
    print(f"workload {w.name}", flush=True)
    A, B, ref = persistent_8192_ref
    desc = tb.plan_from_mlir(w.mlir())
    assert desc.config.num_programs == 256
    _check_full(run_desc(desc, A, B, device), ref)


def test_persistent_8192_192x128_tiles(device, persistent_8192_ref):
    """The persistent configuration on 192x128 tiles (the reference's
    smoke_persistent_192x128x32 shape family, scaled): 43 x 64 tiles whose
    last tile row is ragged (8192 = 42 * 192 + 128), 256 resident programs in
    grouped order, so the ragged persistent edge runs at scale. Every
    element against fp64."""
    w = dataclasses.replace(configs.PERSISTENT, name="persistent_8192_192x128",
                            block=(192, 128, 64), exact_tile=False)
    print(f"workload {w.name}", flush=True)
    A, B, ref = persistent_8192_ref
    desc = tb.plan_from_mlir(w.mlir())
    cfg = desc.config
    assert (cfg.block_m, cfg.block_n, cfg.num_programs) == (192, 128, 256)
    assert cfg.mapping == tb.MAP_PERSISTENT_GROUPED
    print(f"kernel {desc.kernel_name}", flush=True)
    _check_full(run_desc(desc, A, B, device), ref)


def test_persistent_8192_f32_accumulate(device, persistent_8192_ref):
    """8192^3 in the reference's semantics, f32 C += A*B, through the plan
    (the 16x16x32 256x256x64 instance, 256 resident programs over 1024
    tiles): each program adds four tiles' prior C inside their main loops
    (128 k-tiles each) in turn. Every element against fp64 product + C."""
    w = dataclasses.replace(configs.PERSISTENT, name="persistent_8192_f32", c_f32=True)
    print(f"workload {w.name}", flush=True)
    A, B, ref = persistent_8192_ref
    desc = tb.plan_from_mlir(w.mlir())
    assert desc.kernel_name == "tb_gemm_gfx950_256x256x64_w2x2_s2_out2_16x16x32"
    assert desc.config.num_programs == 256
    init = np.random.default_rng(8192).uniform(-1, 1, (w.M, w.N)).astype(np.float32)
    got = run_desc(desc, A, B, device, c_init=init)
    _check_full(got, ref + init)


# The configurations of the reference's examples/*.mlir and contract tests
# (f32 C, 1-4 warps), which the plan maps to C += A B, the reference's
# tb.matmul semantics: C starts from a seeded non-zero value and the oracle
# adds it. Plus a serial split-k with an uneven k-tile split.
PLAN_MODULES = [
    ("smoke_64x64x32_1wave", 64, 64, 32, 64, 1, ""),
    ("smoke_128x128x32", 128, 128, 32, 128, 4, ""),
    ("smoke_96x80x32_1wave", 96, 80, 32, 64, 1, ""),
    ("grouped_192x128x32", 192, 128, 32, 64, 4, ""),
    ("two_wave_64x64x32", 64, 64, 32, 64, 2, ""),
    ("persistent_192x128x32", 192, 128, 32, 64, 4,
     ', "tb.persistent" = true, "tb.num-ctas" = 2 : i64'),
    ("splitk_atomic_64x64x64", 64, 64, 64, 64, 1,
     ', "tb.split-k" = 2 : i64, "tb.reduction-mode" = "split_k_parallel"'),
    ("splitk_serial_64x64x128", 64, 64, 128, 64, 1,
     ', "tb.split-k" = 3 : i64, "tb.reduction-mode" = "split_k_serial"'),
]


@pytest.mark.parametrize("name,M,N,K,tile,warps,extra", PLAN_MODULES,
                         ids=[p[0] for p in PLAN_MODULES])
def test_plan_module_f32_accumulate(name, M, N, K, tile, warps, extra, device):
    exact = "true" if M % tile == 0 and N % tile == 0 else "false"
    gm = ", group_m = 2 : i64" if name.startswith("grouped") else ""
    text = (
        f'module attributes {{"tb.num-warps" = {warps} : i64, '
        f'"tb.requested-stages" = 2 : i64{extra}}} {{\n'
        f"  func.func @kernel(%A: memref<{M}x{K}xf16>, %B: memref<{K}x{N}xf16>, "
        f"%C: memref<{M}x{N}xf32>) {{\n"
        f"    tb.matmul %A, %B, %C {{block_m = {tile} : i64, block_n = {tile} : i64, "
        f"block_k = 32 : i64, exact_tile = {exact}{gm}}} : memref<{M}x{K}xf16>, "
        f"memref<{K}x{N}xf16>, memref<{M}x{N}xf32>\n    return\n  }}\n}}\n")
    print(f"plan module {name}", flush=True)
    desc = tb.plan_from_mlir(text)
    assert desc.config.acc_init == tb.ACC_INIT_LOAD_C
    A, B = oracle.config_inputs(M, N, K, 0x5EED0500, oracle.UNIFORM)
    C0 = oracle.fill_f16(M, N, 0x5EED0501, oracle.UNIFORM, 4.0).astype(np.float32)
    got = run_desc(desc, A, B, device, c_init=C0.copy(), c_dtype=torch.float32)
    check(got, A, B, init=C0)


# Large shapes with edges in M, N and K, through the plan pipeline: partial
# 256x256 tiles with a ragged last k-tile, a split-K whose 157 k-tiles do not
# divide by 8 splits (5 splits take one more), and persistent order over
# ragged tiles on 7 programs. K, N and the leading dimensions stay multiples
# of 8, which the C ABI requires.
LARGE_RAGGED = [
    configs.Workload("ragged_1000x1496x712", 1000, 1496, 712, 0x5EED0200, configs.NORMAL,
                     (256, 256, 64), num_waves=4, exact_tile=False),
    configs.Workload("ragged_splitk_300x520x10000", 300, 520, 10000, 0x5EED0201,
                     configs.UNIFORM, (128, 64, 64), num_waves=4, stages=3, split_k=8,
                     exact_tile=False),
    configs.Workload("ragged_persistent_1300x904x520", 1300, 904, 520, 0x5EED0202,
                     configs.NORMAL, (256, 256, 64), num_waves=4, persistent=True,
                     num_ctas=7, exact_tile=False),
    # K a multiple of 64 (the ragged-K cases above take the same instance)
    configs.Workload("ragged16_1000x1496x768", 1000, 1496, 768, 0x5EED0203, configs.NORMAL,
                     (256, 256, 64), num_waves=4, exact_tile=False),
    configs.Workload("ragged16_persistent_1300x904x512", 1300, 904, 512, 0x5EED0204,
                     configs.NORMAL, (256, 256, 64), num_waves=4, persistent=True,
                     num_ctas=7, exact_tile=False),
    configs.Workload("ragged16_4000x4000x4096", 4000, 4000, 4096, 0x5EED0205,
                     configs.NORMAL, (256, 256, 64), num_waves=4, exact_tile=False),
]


@pytest.mark.parametrize("w", LARGE_RAGGED, ids=lambda w: w.name)
def test_large_ragged_parity(w, device):
    print(f"large ragged {w.name}", flush=True)
    A, B = oracle.config_inputs(w.M, w.N, w.K, w.seed, w.dist)
    desc = tb.plan_from_mlir(w.mlir())
    # the 16x16x32 instance takes the 256x256x64 4-wave tiles, ragged M, N
    # and K included
    assert ("16x16x32" in desc.kernel_name) == w.mfma16_supported(), desc.kernel_name
    got = run_desc(desc, A, B, device)
    check(got, A, B)


RAGGED_SHAPES = [(1, 8, 8), (33, 24, 16), (97, 88, 40), (200, 136, 72),
                 (65, 64, 32), (64, 72, 96), (130, 264, 264)]


@pytest.mark.parametrize("M,N,K", RAGGED_SHAPES)
# (block, wave grid, 16x16x32): the 256x256 tile on four waves holds its
# 128x128 wave tiles in registers only on 16x16x32 (its 32x32x16 build spills
# and is refused)
@pytest.mark.parametrize("tile", [(64, 64, 32, 2, 2, 0), (128, 128, 64, 2, 2, 0),
                                  (128, 128, 64, 2, 2, 1), (128, 128, 32, 2, 2, 1),
                                  (256, 256, 64, 2, 2, 1)])
def test_ragged_edges(M, N, K, tile, device):
    bm, bn, bk, wgm, wgn, mfma16 = tile
    print(f"ragged {M}x{N}x{K} tile {tile}", flush=True)
    A, B = oracle.config_inputs(M, N, K, 0x5EED0100 + M, oracle.UNIFORM)
    tm, tn = -(-M // bm), -(-N // bn)
    mapping = tb.MAP_GROUPED_TILE if tm > 1 and tn > 1 else tb.MAP_TILE
    cfg = tb.GemmConfig(m=M, n=N, k=K, lda=K, ldb=N, ldc=N, c_dtype=tb.DTYPE_F16,
                        acc_init=tb.ACC_INIT_ZERO, block_m=bm, block_n=bn,
                        block_k=bk, num_waves=wgm * wgn, wave_grid_m=wgm,
                        wave_grid_n=wgn, stages=2, mapping=mapping, group_m=8,
                        split_k=1, reduction=tb.RED_NONE, num_programs=tm * tn,
                        xcd_remap=8, mfma=tb.MFMA_16X16X32 if mfma16 else tb.MFMA_32X32X16)
    got = run_desc(tb.GemmDesc.from_config(cfg), A, B, device)
    check(got, A, B)


def _every_instance():
    seen = set()
    for name in tb.kernel_names():
        # tb_gemm_gfx950_{BM}x{BN}x{BK}_w{WGM}x{WGN}_s{STAGES}_out{OUT}[_16x16x32][_epi]
        body = name[len("tb_gemm_gfx950_"):]
        epi = body.endswith("_epi")
        body = body[:-4] if epi else body
        mfma16 = body.endswith("_16x16x32")
        body = body[:-len("_16x16x32")] if mfma16 else body
        shape, waves, stages, out = body.split("_")
        bm, bn, bk = map(int, shape.split("x"))
        wgm, wgn = map(int, waves[1:].split("x"))
        seen.add((bm, bn, bk, wgm, wgn, int(stages[1:]), int(out[3:]), int(epi),
                  int(mfma16)))
    return sorted(seen)


_RESOURCES = {}


def _spills(inst, partial_k: bool) -> bool:
    """The instance's build (for a partial last k-tile when partial_k) uses
    scratch, in the compiler's report the library carries."""
    bm, bn, bk, wgm, wgn, stages, out, epi, mfma16 = inst
    if partial_k not in _RESOURCES:
        _RESOURCES[partial_k] = tb.kernel_resources(partial_k=partial_k)
    name = (f"tb_gemm_gfx950_{bm}x{bn}x{bk}_w{wgm}x{wgn}_s{stages}_out{out}"
            f"{'_16x16x32' if mfma16 else ''}{'_epi' if epi else ''}")
    return _RESOURCES[partial_k][name][2] > 0


# fused steps per output mode of the `_epi` instances: (bias kind, activation,
# clamp bits, lo, hi)
EPI_STEPS = {0: (tb.EPI_BIAS_F16, tb.ACT_GELU_TANH, 3, -0.5, 1.5),
             1: (tb.EPI_BIAS_F32, tb.ACT_SILU, 0, 0.0, 0.0),
             2: (tb.EPI_BIAS_F32, tb.ACT_RELU, 2, 0.0, 2.0)}


@pytest.mark.parametrize("inst", _every_instance(), ids=lambda t: "x".join(map(str, t)))
def test_every_instance(inst, device):
    """Each compiled instance on a shape with several K tiles (more than the
    stage count, plus a ragged last tile when possible) and an M/N edge; the
    16x16x32 instance on the same shape."""
    bm, bn, bk, wgm, wgn, stages, out, epi, mfma16 = inst
    M, N, K = bm + 40, bn * 2 - 24, bk * 5 + (bk // 2 if out == 0 else 0)
    print(f"instance {inst} on {M}x{N}x{K}", flush=True)
    A, B = oracle.config_inputs(M, N, K, 0x5EED0200 + bm + bn + bk, oracle.UNIFORM)
    tm, tn = -(-M // bm), -(-N // bn)
    kw = dict(m=M, n=N, k=K, lda=K, ldb=N, ldc=N, block_m=bm, block_n=bn,
              block_k=bk, num_waves=wgm * wgn, wave_grid_m=wgm, wave_grid_n=wgn,
              stages=stages, group_m=8, xcd_remap=0,
              mfma=tb.MFMA_16X16X32 if mfma16 else tb.MFMA_32X32X16)
    rng = np.random.default_rng(out)
    init = None
    if out == 0:
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F16, acc_init=tb.ACC_INIT_ZERO,
                            mapping=tb.MAP_GROUPED_TILE, split_k=1,
                            reduction=tb.RED_NONE, num_programs=tm * tn, **kw)
        c_dtype = torch.float16
    elif out == 1 and (epi or mfma16):  # plain f32 store (fused instances, and
        # 16x16x32, which has no split-K)
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F32, acc_init=tb.ACC_INIT_ZERO,
                            mapping=tb.MAP_TILE, split_k=1, reduction=tb.RED_NONE,
                            num_programs=tm * tn, **kw)
        c_dtype = torch.float32
    elif out == 1:  # f32 partials: split-K with workspace, f16 result
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F16, acc_init=tb.ACC_INIT_ZERO,
                            mapping=tb.MAP_SPLIT_K, split_k=3,
                            reduction=tb.RED_WORKSPACE,
                            num_programs=tm * tn * 3, **kw)
        c_dtype = torch.float16
    elif out == 2:  # reference semantics: f32 C += A*B
        init = rng.uniform(-1, 1, (M, N)).astype(np.float32)
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F32, acc_init=tb.ACC_INIT_LOAD_C,
                            mapping=tb.MAP_TILE, split_k=1, reduction=tb.RED_NONE,
                            num_programs=tm * tn, **kw)
        c_dtype = torch.float32
    else:  # reference split_k_atomic: f32 C += per-split partials
        init = rng.uniform(-1, 1, (M, N)).astype(np.float32)
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F32, acc_init=tb.ACC_INIT_LOAD_C,
                            mapping=tb.MAP_SPLIT_K, split_k=2,
                            reduction=tb.RED_ATOMIC, num_programs=tm * tn * 2, **kw)
        c_dtype = torch.float32
    if epi:
        kind, act, bits, lo, hi = EPI_STEPS[out]
        cfg.epi_bias, cfg.epi_activation, cfg.epi_clamp = kind, act, bits
        cfg.clamp_min, cfg.clamp_max = lo, hi
    if _spills(inst, partial_k=K % bk != 0):
        # register truth: a build that spills to scratch is refused, with the
        # compiler's figures, and never launched
        with pytest.raises(tb.TbError, match="spills .* bytes per lane to scratch"):
            tb.GemmDesc.from_config(cfg)
        return
    if not epi:
        desc = tb.GemmDesc.from_config(cfg)
        got = run_desc(desc, A, B, device, c_init=init, c_dtype=c_dtype)
        check(got, A, B, init=init)
        return
    desc = tb.GemmDesc.from_config(cfg)
    assert desc.kernel_name.endswith(f"_out{out}{'_16x16x32' if mfma16 else ''}_epi")
    bias = oracle.fill_f16(1, N, 0x5EED0300 + N, oracle.UNIFORM, 1.0).reshape(N)
    if kind == tb.EPI_BIAS_F32:
        bias = bias.astype(np.float32)
    dA, dB = _dev(A, device), _dev(B, device)
    dC = (_dev(init, device) if init is not None else
          torch.full((M, N), float("nan"), dtype=c_dtype, device=device))
    desc.launch(dA, dB, dC, bias=_dev(bias, device))
    torch.cuda.synchronize()
    got = dC.cpu().numpy()
    ref = oracle.gemm_f64(A, B, init=init)
    oracle.epilogue_f64(ref, bias.astype(np.float64), act, bits, lo, hi)
    bad, err, worst = oracle.check_tolerance(got, ref, rtol=RTOL)
    print(f"fused steps: violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"


@pytest.mark.parametrize("mapping", [tb.MAP_PERSISTENT_TILE, tb.MAP_PERSISTENT_GROUPED])
@pytest.mark.parametrize("programs", [1, 3, 7])
def test_persistent_mappings(mapping, programs, device):
    M, N, K = 448, 320, 192
    A, B = oracle.config_inputs(M, N, K, 0x5EED0300, oracle.UNIFORM)
    cfg = tb.GemmConfig(m=M, n=N, k=K, lda=K, ldb=N, ldc=N, c_dtype=tb.DTYPE_F16,
                        acc_init=tb.ACC_INIT_ZERO, block_m=64, block_n=64,
                        block_k=64, num_waves=4, wave_grid_m=2, wave_grid_n=2,
                        stages=2, mapping=mapping, group_m=3, split_k=1,
                        reduction=tb.RED_NONE, num_programs=programs, xcd_remap=8)
    got = run_desc(tb.GemmDesc.from_config(cfg), A, B, device)
    check(got, A, B)


def test_split_k_is_deterministic(device):
    w = configs.SPLIT_K
    A, B = oracle.config_inputs(w.M, w.N, w.K, w.seed, w.dist)
    desc = tb.GemmDesc.from_config(w.direct_config())
    first = run_desc(desc, A, B, device)
    second = run_desc(desc, A, B, device)
    assert np.array_equal(first.view(np.uint16), second.view(np.uint16))


def test_leading_dimensions(device):
    """Operands embedded in wider row-major buffers (lda > K, ldb > N, ldc > N)."""
    M, N, K = 130, 72, 96
    lda, ldb, ldc = 104, 88, 80
    A, B = oracle.config_inputs(M, N, K, 0x5EED0400, oracle.UNIFORM)
    Aw = np.zeros((M, lda), np.float16); Aw[:, :K] = A
    Bw = np.zeros((K, ldb), np.float16); Bw[:, :N] = B
    Cw = np.full((M, ldc), np.float16(7.0))
    cfg = tb.GemmConfig(m=M, n=N, k=K, lda=lda, ldb=ldb, ldc=ldc,
                        c_dtype=tb.DTYPE_F16, acc_init=tb.ACC_INIT_ZERO,
                        block_m=64, block_n=64, block_k=32, num_waves=4,
                        wave_grid_m=2, wave_grid_n=2, stages=2,
                        mapping=tb.MAP_GROUPED_TILE, group_m=8, split_k=1,
                        reduction=tb.RED_NONE, num_programs=3 * 2, xcd_remap=0)
    got = run_desc(tb.GemmDesc.from_config(cfg), Aw, Bw, device, c_init=Cw, M=M, N=ldc)
    check(np.ascontiguousarray(got[:, :N]), A, B)
    assert np.all(got[:, N:] == np.float16(7.0)), "padding columns of C were written"


def test_device_fill_matches_oracle(device):
    for dist, scale in [(oracle.UNIFORM, 1.0), (oracle.NORMAL, 1.0 / 64)]:
        rows, cols = 257, 1032
        want = oracle.fill_f16(rows, cols, 0x5EED0004, dist, scale).view(np.uint16)
        d = torch.empty((rows, cols), dtype=torch.float16, device=device)
        tb.fill_seeded_f16(d, rows, cols, 0x5EED0004, dist, scale)
        torch.cuda.synchronize()
        got = d.cpu().numpy().view(np.uint16)
        same = (got == want).mean()
        print(f"dist {dist}: identical fraction {same}", flush=True)
        if dist == oracle.UNIFORM:
            assert same == 1.0  # integer + exact float ops: bit-exact
        else:
            # device log/cos may differ from libm in the last f64 bit; after
            # rounding to f16 that can flip at most a rare element by 1 ulp
            assert same > 0.9999
            assert np.all(np.abs(got.astype(np.int32) - want.astype(np.int32)) <= 1)
