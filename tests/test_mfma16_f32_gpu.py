"""GPU parity of the f32-C builds of the 16x16x32 instance.

`tb_gemm_gfx950_256x256x64_w2x2_s2_out1_16x16x32` (plain f32 C) and
`..._out2_16x16x32` (f32 C += A*B, the reference's tb.matmul semantics), with
and without the fused steps, on any M, N and K. Checks:

* against the fp64 oracle, |got - ref| <= 1e-2 * (|ref| + 1): whole and
  ragged M, N and K (K % 64 != 0 takes the partial-k-tile build), padded ldc
  whose padding columns must stay unwritten, tile / grouped / persistent
  order with more tiles than programs, and the 4096^3 headline shape as
  C += A*B;
* bit for bit against the f16 instance: all three output modes run the same
  MFMA sequence, so the f16 C equals the plain f32 C rounded to nearest even
  (with and without the fused steps), and C += A*B on a zero C equals the
  plain f32 C;
* bit for bit against the 32x32x16 general loop on the same tile (same f32
  sums in the same k order, the prior C added after the sum in both) for K
  of fewer than 18 k-tiles; from 18 k-tiles on, whole tiles add the prior C
  inside the main loop, checked against the plain f32 C plus the prior C to
  f32 rounding;
* run-to-run bit-identity.
"""
import numpy as np
import pytest
import torch

import mini_triton_nvgpu_v1_amd as tb
import oracle

pytestmark = pytest.mark.gpu
RTOL = 1e-2
NAME = "tb_gemm_gfx950_256x256x64_w2x2_s2_out{}_16x16x32{}"


def _cfg(M, N, K, out, mapping=tb.MAP_GROUPED_TILE, programs=None, ld_pad=0, epi=None,
         mfma=tb.MFMA_16X16X32):
    tiles = -(-M // 256) * -(-N // 256)
    cfg = tb.GemmConfig(
        m=M, n=N, k=K, lda=K, ldb=N, ldc=N + ld_pad,
        c_dtype=tb.DTYPE_F16 if out == 0 else tb.DTYPE_F32,
        acc_init=tb.ACC_INIT_LOAD_C if out == 2 else tb.ACC_INIT_ZERO,
        block_m=256, block_n=256, block_k=64, num_waves=4, wave_grid_m=2, wave_grid_n=2,
        stages=2, mapping=mapping,
        group_m=8 if mapping in (tb.MAP_GROUPED_TILE, tb.MAP_PERSISTENT_GROUPED) else 1,
        split_k=1, reduction=tb.RED_NONE, num_programs=programs or tiles,
        xcd_remap=8 if tiles >= 256 else 0, mfma=mfma)
    if epi:
        kind, act, bits, lo, hi = epi
        cfg.epi_bias, cfg.epi_activation, cfg.epi_clamp = kind, act, bits
        cfg.clamp_min, cfg.clamp_max = lo, hi
    return cfg


def _run(cfg, dA, dB, init=None, bias=None):
    desc = tb.GemmDesc.from_config(cfg)
    suffix = "_epi" if cfg.epi_bias or cfg.epi_activation or cfg.epi_clamp else ""
    out = {tb.DTYPE_F16: 0}.get(cfg.c_dtype, 2 if cfg.acc_init == tb.ACC_INIT_LOAD_C else 1)
    name = NAME.format(out, suffix)
    if cfg.mfma == tb.MFMA_32X32X16:
        name = name.replace("_16x16x32", "")
    assert desc.kernel_name == name, desc.kernel_name
    ct = torch.float16 if cfg.c_dtype == tb.DTYPE_F16 else torch.float32
    if init is not None:
        dC = torch.from_numpy(init).to(dA.device)
    else:
        dC = torch.full((cfg.m, cfg.ldc), float("nan"), dtype=ct, device=dA.device)
    desc.launch(dA, dB, dC, bias=bias)
    torch.cuda.synchronize()
    return dC.cpu().numpy()


# (M, N, K, mapping, programs, ld_pad)
CASES = [
    (512, 512, 256, tb.MAP_GROUPED_TILE, None, 0),
    (520, 392, 200, tb.MAP_GROUPED_TILE, None, 8),        # ragged M, N, K; padded ldc
    (1000, 776, 136, tb.MAP_PERSISTENT_GROUPED, 5, 0),    # 16 tiles on 5 programs
    (768, 1024, 512, tb.MAP_TILE, None, 0),
    (264, 272, 8, tb.MAP_PERSISTENT_TILE, 3, 16),         # K below one k step
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}_m{c[3]}")
def test_f32_c_builds(case, device):
    M, N, K, mapping, programs, pad = case
    print(f"case {case}", flush=True)
    A, B = oracle.config_inputs(M, N, K, 0x5EED0F00 + M + N + K, oracle.UNIFORM)
    dA, dB = torch.from_numpy(A).to(device), torch.from_numpy(B).to(device)
    ref = oracle.gemm_f64(A, B)

    plain = _run(_cfg(M, N, K, 1, mapping, programs, pad), dA, dB)
    bad, err, worst = oracle.check_tolerance(np.ascontiguousarray(plain[:, :N]), ref,
                                             rtol=RTOL)
    print(f"plain f32: violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"plain f32 C: {bad} elements outside tolerance; worst {err} at {worst}"
    if pad:
        assert np.isnan(plain[:, N:]).all(), "padding columns written"

    rng = np.random.default_rng(M + N + K)
    init = np.full((M, N + pad), 7.0, np.float32)
    init[:, :N] = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    acc = _run(_cfg(M, N, K, 2, mapping, programs, pad), dA, dB, init=init)
    ref_acc = oracle.gemm_f64(A, B, init=np.ascontiguousarray(init[:, :N]))
    bad, err, worst = oracle.check_tolerance(np.ascontiguousarray(acc[:, :N]), ref_acc,
                                             rtol=RTOL)
    print(f"C += A*B: violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"C += A*B: {bad} elements outside tolerance; worst {err} at {worst}"
    assert (acc[:, N:] == 7.0).all(), "padding columns written"
    again = _run(_cfg(M, N, K, 2, mapping, programs, pad), dA, dB, init=init)
    assert np.array_equal(acc.view(np.uint32), again.view(np.uint32)), "not run-to-run identical"

    zero = _run(_cfg(M, N, K, 2, mapping, programs, pad), dA, dB,
                init=np.zeros((M, N + pad), np.float32))
    assert np.array_equal(zero[:, :N], plain[:, :N]), "C += A*B on a zero C != plain f32 C"

    half = _run(_cfg(M, N, K, 0, mapping, programs, pad), dA, dB)
    same = np.array_equal(half[:, :N].view(np.uint16),
                          plain[:, :N].astype(np.float16).view(np.uint16))
    print(f"f16 C == f32 C rounded: {same}", flush=True)
    assert same

    # the 32x32x16 general loop: the same f32 sums in the same k order
    general = _run(_cfg(M, N, K, 1, mapping, programs, pad, mfma=tb.MFMA_32X32X16), dA, dB)
    assert np.array_equal(general[:, :N].view(np.uint32), plain[:, :N].view(np.uint32)), \
        "plain f32 C differs from the general loop's"
    general = _run(_cfg(M, N, K, 2, mapping, programs, pad, mfma=tb.MFMA_32X32X16), dA, dB,
                   init=init)
    assert np.array_equal(general.view(np.uint32), acc.view(np.uint32)), \
        "C += A*B differs from the general loop's"


# (bias kind, activation, clamp bits, lo, hi)
STEPS = [(tb.EPI_BIAS_F32, tb.ACT_GELU_TANH, 3, -0.5, 1.5),
         (tb.EPI_BIAS_F16, tb.ACT_SILU, 0, 0.0, 0.0),
         (tb.EPI_BIAS_NONE, tb.ACT_RELU, 2, 0.0, 2.0)]


# K = 1200 (19 k-tiles): the whole tiles add the prior C inside the main loop,
# the steps then run on C + A*B in the epilogue
@pytest.mark.parametrize("K", [200, 1200])
@pytest.mark.parametrize("steps", STEPS, ids=lambda s: f"bias{s[0]}_act{s[1]}_clamp{s[2]}")
def test_f32_c_fused_steps(steps, K, device):
    M, N = 520, 392
    kind, act, bits, lo, hi = steps
    A, B = oracle.config_inputs(M, N, K, 0x5EED0F80 + act, oracle.UNIFORM)
    dA, dB = torch.from_numpy(A).to(device), torch.from_numpy(B).to(device)
    bias = oracle.fill_f16(1, N, 0x5EED0F90 + N, oracle.UNIFORM, 1.0).reshape(N)
    if kind == tb.EPI_BIAS_F32:
        bias = bias.astype(np.float32)
    dbias = torch.from_numpy(bias).to(device) if kind != tb.EPI_BIAS_NONE else None
    b64 = bias.astype(np.float64) if kind != tb.EPI_BIAS_NONE else None

    plain = _run(_cfg(M, N, K, 1, epi=steps), dA, dB, bias=dbias)
    ref = oracle.gemm_f64(A, B)
    oracle.epilogue_f64(ref, b64, act, bits, lo, hi)
    bad, err, worst = oracle.check_tolerance(plain, ref, rtol=RTOL)
    print(f"plain f32 + steps: violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"

    init = np.random.default_rng(act).uniform(-1, 1, (M, N)).astype(np.float32)
    acc = _run(_cfg(M, N, K, 2, epi=steps), dA, dB, init=init, bias=dbias)
    ref = oracle.gemm_f64(A, B, init=init)
    oracle.epilogue_f64(ref, b64, act, bits, lo, hi)
    bad, err, worst = oracle.check_tolerance(acc, ref, rtol=RTOL)
    print(f"C += A*B + steps: violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"

    half = _run(_cfg(M, N, K, 0, epi=steps), dA, dB, bias=dbias)
    same = np.array_equal(half.view(np.uint16), plain.astype(np.float16).view(np.uint16))
    print(f"f16 C + steps == f32 C + steps rounded: {same}", flush=True)
    assert same


# K of at least 18 k-tiles: whole tiles add the prior C inside the main loop
# (during its first 16 bodies), ragged tiles and shorter K after the loop
LONG_K = [
    (520, 392, 1200, tb.MAP_GROUPED_TILE, None, 8),       # 19 k-tiles, partial last; 2 whole
    (512, 768, 1152, tb.MAP_PERSISTENT_GROUPED, 4, 0),    # exactly 18; 6 tiles on 4 programs
    (512, 512, 1088, tb.MAP_TILE, None, 0),               # 17: the prior C after the loop
    (1024, 1024, 1608, tb.MAP_PERSISTENT_TILE, 5, 0),     # 26, partial last; 16 tiles on 5
]


@pytest.mark.parametrize("case", LONG_K, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}_m{c[3]}")
def test_f32_accumulate_long_k(case, device):
    """C += A*B where the prior C joins the sum inside the main loop: against
    the fp64 oracle; against the plain f32 C plus the prior C to f32 rounding
    (a prior C added twice or not at all is off by the prior C itself);
    exactly the plain f32 C on a zero C; run-to-run identical; and, where
    the add comes after the loop (fewer than 18 k-tiles), bit for bit the
    32x32x16 general loop."""
    M, N, K, mapping, programs, pad = case
    print(f"case {case}", flush=True)
    A, B = oracle.config_inputs(M, N, K, 0x5EED1000 + M + N + K, oracle.UNIFORM)
    dA, dB = torch.from_numpy(A).to(device), torch.from_numpy(B).to(device)
    init = np.full((M, N + pad), 7.0, np.float32)
    init[:, :N] = np.random.default_rng(K).uniform(-1, 1, (M, N)).astype(np.float32)
    acc = _run(_cfg(M, N, K, 2, mapping, programs, pad), dA, dB, init=init)
    ref = oracle.gemm_f64(A, B, init=np.ascontiguousarray(init[:, :N]))
    bad, err, worst = oracle.check_tolerance(np.ascontiguousarray(acc[:, :N]), ref, rtol=RTOL)
    print(f"C += A*B: violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"
    assert (acc[:, N:] == 7.0).all(), "padding columns written"

    plain = _run(_cfg(M, N, K, 1, mapping, programs, pad), dA, dB)[:, :N]
    sum_ = plain.astype(np.float64) + init[:, :N]
    scale = np.abs(plain).astype(np.float64) + np.abs(init[:, :N]) + 1.0
    off = np.abs(acc[:, :N] - sum_) > 1e-4 * scale
    print(f"C += A*B vs plain + C: {int(off.sum())} off", flush=True)
    assert not off.any(), f"{int(off.sum())} elements differ from plain f32 C + prior C"

    again = _run(_cfg(M, N, K, 2, mapping, programs, pad), dA, dB, init=init)
    assert np.array_equal(acc.view(np.uint32), again.view(np.uint32)), "not run-to-run identical"
    zero = _run(_cfg(M, N, K, 2, mapping, programs, pad), dA, dB,
                init=np.zeros((M, N + pad), np.float32))
    assert np.array_equal(zero[:, :N], plain), "C += A*B on a zero C != plain f32 C"
    if -(-K // 64) < 18:
        general = _run(_cfg(M, N, K, 2, mapping, programs, pad, mfma=tb.MFMA_32X32X16),
                       dA, dB, init=init)
        assert np.array_equal(general.view(np.uint32), acc.view(np.uint32)), \
            "C += A*B differs from the general loop's"


def test_f32_accumulate_4096(device):
    """The 4096^3 headline shape in the reference's semantics, f32 C += A*B,
    every element against the fp64 oracle."""
    M = N = K = 4096
    A, B = oracle.config_inputs(M, N, K, 0x5EED0FF0, oracle.NORMAL)
    dA, dB = torch.from_numpy(A).to(device), torch.from_numpy(B).to(device)
    init = np.random.default_rng(4096).uniform(-1, 1, (M, N)).astype(np.float32)
    got = _run(_cfg(M, N, K, 2), dA, dB, init=init)
    ref = oracle.gemm_f64(A, B, init=init)
    bad, err, worst = oracle.check_tolerance(got, ref, rtol=RTOL)
    print(f"4096^3 C += A*B: violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"
