"""GPU parity of the 16x16x32 instance of the 4-wave 256x256x64 tile.

`256x256x64_w2x2_s2_out0_16x16x32[_epi]` runs any M, N and K (tile, grouped
or persistent order) with one wave per SIMD, 128x128 wave tiles and
v_mfma_f32_16x16x32_f16, on the same LDS ring as the general loop; ragged
edges are masked at the A and B loads (a partial last k-tile loads zeros past
K) and at the C store.
Checks:

* against the fp64 oracle, |got - ref| <= 1e-2 * (|ref| + 1), on shapes that
  cover 1, 2, odd and even k-tile counts, tile / grouped / persistent orders
  (more tiles than programs), padded leading dimensions, ragged M, N and K
  (including a problem smaller than one wave tile, a K below one k-tile, and
  padding columns that must stay unwritten) and the fused steps;
* bit-identity with the general loop (32x32x16, here on 4 waves of 64x64
  over 128x128x64 blocks: the 32x32x16 builds of the same 256x256 block,
  4 waves of 128x128 or 8 waves of 64x128 with the fused steps, spill and
  are refused) and with the 16x16x32 loop's 128x128x64 build: every output
  element is the same f32 sum of the same products in the same k order (in
  32x32x16 or 16x16x32 steps), whatever the tiling, and the test pins that
  the two MFMA shapes round it alike;
* 40 seeded random ragged shapes (any M, N and K multiples of 8, every
  program order, padded leading dimensions) against the oracle and bit for
  bit against the general loop;
* every compile-time variant of the fused steps (activation x whether a
  clamp is set), against the oracle and bit-identical between the 16x16x32
  instance and the general loop's fused instance, and the fused instance in
  persistent order.

"""
import numpy as np
import pytest
import torch

import mini_triton_nvgpu_v1_amd as tb
import oracle

pytestmark = pytest.mark.gpu
RTOL = 1e-2


def _cfg(M, N, K, waves, mapping, programs=None, ld_pad=0, xcd=0, mfma16=False, block=256):
    """The 4-wave 256x256x64 tile (block=256), or a 128x128x64 block on 4
    waves of 64x64 (block=128: the general loop, or with mfma16 the 16x16x32
    loop) for the bit-identity comparisons."""
    assert waves == 4
    tm, tn = -(-M // block), -(-N // block)
    return tb.GemmConfig(
        m=M, n=N, k=K, lda=K + ld_pad, ldb=N + ld_pad, ldc=N + ld_pad,
        c_dtype=tb.DTYPE_F16, acc_init=tb.ACC_INIT_ZERO, block_m=block, block_n=block,
        block_k=64, num_waves=waves, wave_grid_m=2, wave_grid_n=2, stages=2,
        mapping=mapping, group_m=8 if mapping != tb.MAP_TILE else 1, split_k=1,
        reduction=tb.RED_NONE, num_programs=programs or tm * tn,
        xcd_remap=xcd if (programs or tm * tn) % 8 == 0 else 0,
        mfma=tb.MFMA_16X16X32 if mfma16 else tb.MFMA_32X32X16)


def _run(cfg, A, B, device, ld_pad=0, bias=None):
    M, N, K = cfg.m, cfg.n, cfg.k
    dA = torch.zeros((M, K + ld_pad), dtype=torch.float16, device=device)
    dB = torch.zeros((K, N + ld_pad), dtype=torch.float16, device=device)
    dA[:, :K] = torch.from_numpy(A).to(device)
    dB[:, :N] = torch.from_numpy(B).to(device)
    dC = torch.full((M, N + ld_pad), float("nan"), dtype=torch.float16, device=device)
    desc = tb.GemmDesc.from_config(cfg)
    desc.launch(dA, dB, dC, bias=None if bias is None else torch.from_numpy(bias).to(device))
    torch.cuda.synchronize()
    return desc.kernel_name, dC.cpu().numpy()


# (M, N, K, mapping, programs, ld_pad, xcd_remap)
CASES = [
    (256, 256, 64, tb.MAP_TILE, None, 0, 0),             # one k-tile
    (256, 512, 128, tb.MAP_TILE, None, 0, 0),            # two k-tiles
    (512, 256, 192, tb.MAP_GROUPED_TILE, None, 0, 0),    # odd count
    (768, 512, 320, tb.MAP_GROUPED_TILE, None, 0, 0),    # 5 k-tiles, 3x2 tiles
    (512, 768, 256, tb.MAP_TILE, None, 8, 0),            # padded leading dims
    (1024, 1024, 128, tb.MAP_PERSISTENT_GROUPED, 3, 0, 0),  # 16 tiles on 3 programs
    (768, 1024, 64, tb.MAP_PERSISTENT_TILE, 5, 0, 0),    # 12 tiles on 5 programs
    (2048, 2048, 128, tb.MAP_GROUPED_TILE, None, 0, 8),  # 64 tiles, XCD order
    (300, 520, 192, tb.MAP_GROUPED_TILE, None, 0, 0),    # ragged M and N
    (100, 72, 128, tb.MAP_TILE, None, 0, 0),             # smaller than a wave tile
    (1000, 1496, 768, tb.MAP_GROUPED_TILE, None, 8, 0),  # ragged, padding untouched
    (1300, 904, 512, tb.MAP_PERSISTENT_GROUPED, 7, 0, 0),  # 24 ragged tiles on 7
    (2000, 2056, 256, tb.MAP_GROUPED_TILE, None, 0, 8),  # 72 ragged tiles, XCD order
    (512, 256, 200, tb.MAP_GROUPED_TILE, None, 0, 0),    # partial last k-tile (K % 64 = 8)
    (256, 512, 40, tb.MAP_TILE, None, 8, 0),             # K below one k-tile, padded
    (300, 520, 712, tb.MAP_GROUPED_TILE, None, 0, 0),    # ragged M, N and K (K % 64 = 8)
    (1300, 904, 520, tb.MAP_PERSISTENT_GROUPED, 7, 0, 0),  # ragged all three, persistent
    (768, 768, 1016, tb.MAP_GROUPED_TILE, None, 0, 0),   # K % 64 = 56
]


@pytest.mark.parametrize("M,N,K,mapping,programs,pad,xcd", CASES,
                         ids=[f"{c[0]}x{c[1]}x{c[2]}_map{c[3]}_p{c[4]}_pad{c[5]}"
                              for c in CASES])
def test_mfma16_matches_oracle_and_general_loop(M, N, K, mapping, programs, pad, xcd,
                                               device):
    print(f"wide {M}x{N}x{K} mapping {mapping} programs {programs} pad {pad}", flush=True)
    A, B = oracle.config_inputs(M, N, K, 0x5EED0700 + M + K, oracle.NORMAL)
    name16, got16 = _run(_cfg(M, N, K, 4, mapping, programs, pad, xcd, mfma16=True),
                         A, B, device, pad)
    assert name16 == "tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32"
    if pad:  # columns past N stay as they were (NaN)
        assert np.isnan(got16[:, N:].astype(np.float32)).all()
    got16 = got16[:, :N]
    ref = oracle.gemm_f64(A, B)
    bad, err, worst = oracle.check_tolerance(got16, ref, rtol=RTOL)
    print(f"  16x16x32: violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"
    for mfma16 in (False, True):  # 128x128x64: the general loop, the 16x16x32 loop
        name, got = _run(_cfg(M, N, K, 4, mapping, programs, pad, xcd, mfma16, block=128),
                         A, B, device, pad)
        assert name.startswith("tb_gemm_gfx950_128x128x64_w2x2_s2_out0")
        assert ("16x16x32" in name) == mfma16
        assert np.array_equal(got16.view(np.uint16), got[:, :N].view(np.uint16)), name


def test_mfma16_fused_steps(device):
    """Bias (f32), tanh GELU and a clamp on the 16x16x32 instance, against the
    oracle's epilogue, and bit-identical to the general loop's fused
    instance (128x128x64 on 4 waves)."""
    M, N, K = 512, 768, 192
    print(f"wide fused {M}x{N}x{K}", flush=True)
    A, B = oracle.config_inputs(M, N, K, 0x5EED0710, oracle.UNIFORM)
    bias = oracle.fill_f16(1, N, 0x5EED0711, oracle.UNIFORM, 1.0).reshape(N).astype(np.float32)
    outs = []
    for block in (256, 128):
        cfg = _cfg(M, N, K, 4, tb.MAP_GROUPED_TILE, mfma16=block == 256, block=block)
        cfg.epi_bias, cfg.epi_activation = tb.EPI_BIAS_F32, tb.ACT_GELU_TANH
        cfg.epi_clamp, cfg.clamp_min, cfg.clamp_max = tb.CLAMP_MIN | tb.CLAMP_MAX, -0.25, 3.0
        name, got = _run(cfg, A, B, device, bias=bias)
        assert name.endswith("_16x16x32_epi" if block == 256 else "_out0_epi")
        outs.append(got)
    ref = oracle.gemm_f64(A, B)
    oracle.epilogue_f64(ref, bias.astype(np.float64), 2, 3, -0.25, 3.0)
    bad, err, worst = oracle.check_tolerance(outs[0], ref, rtol=RTOL)
    print(f"  violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))


# (activation, clamp bits, lo, hi): every compile-time (activation, clamp)
# variant of the fused steps, with an f16 bias so that even "no activation,
# no clamp" runs the fused instance.
EPI_VARIANTS = [(act, cl, -0.25, 0.5) for act in (0, 1, 2, 3) for cl in (0, 1, 3)]


@pytest.mark.parametrize("act,clamp,lo,hi", EPI_VARIANTS,
                         ids=[f"act{v[0]}_clamp{v[1]}" for v in EPI_VARIANTS])
def test_fused_step_variants(act, clamp, lo, hi, device):
    """Each activation with no clamp, a lower clamp and both clamps, on the
    16x16x32 instance and on the general loop's fused 128x128x64 instance:
    both match the oracle's epilogue and are bit-identical to each other."""
    M, N, K = 512, 512, 128
    print(f"wide fused variant act {act} clamp {clamp}", flush=True)
    A, B = oracle.config_inputs(M, N, K, 0x5EED0720 + 4 * act + clamp, oracle.NORMAL)
    bias = oracle.fill_f16(1, N, 0x5EED0721, oracle.UNIFORM, 1.0).reshape(N)
    outs = []
    for block in (256, 128):
        cfg = _cfg(M, N, K, 4, tb.MAP_GROUPED_TILE, mfma16=block == 256, block=block)
        cfg.epi_bias, cfg.epi_activation = tb.EPI_BIAS_F16, act
        cfg.epi_clamp, cfg.clamp_min, cfg.clamp_max = clamp, lo, hi
        name, got = _run(cfg, A, B, device, bias=bias)
        assert name.endswith("_16x16x32_epi" if block == 256 else "_out0_epi")
        outs.append(got)
    ref = oracle.gemm_f64(A, B)
    oracle.epilogue_f64(ref, bias.astype(np.float64), act, clamp, lo, hi)
    bad, err, worst = oracle.check_tolerance(outs[0], ref, rtol=RTOL)
    print(f"  violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))


def test_fused_steps_persistent(device):
    """The fused 16x16x32 instance in persistent grouped order (9 tiles on 4
    programs, so a program runs its epilogue, then another tile's main
    loop): against the oracle and bit-identical to the general loop's fused
    128x128x64 instance in plain grouped order."""
    M, N, K = 768, 768, 192
    print(f"wide fused persistent {M}x{N}x{K}", flush=True)
    A, B = oracle.config_inputs(M, N, K, 0x5EED0730, oracle.NORMAL)
    bias = oracle.fill_f16(1, N, 0x5EED0731, oracle.UNIFORM, 1.0).reshape(N).astype(np.float32)
    outs = []
    for block, mapping, programs in ((256, tb.MAP_PERSISTENT_GROUPED, 4),
                                     (128, tb.MAP_GROUPED_TILE, None)):
        cfg = _cfg(M, N, K, 4, mapping, programs, mfma16=block == 256, block=block)
        cfg.epi_bias, cfg.epi_activation = tb.EPI_BIAS_F32, tb.ACT_SILU
        cfg.epi_clamp, cfg.clamp_min, cfg.clamp_max = tb.CLAMP_MIN, -0.125, 0.0
        name, got = _run(cfg, A, B, device, bias=bias)
        assert name.endswith("_16x16x32_epi" if block == 256 else "_out0_epi")
        outs.append(got)
    ref = oracle.gemm_f64(A, B)
    oracle.epilogue_f64(ref, bias.astype(np.float64), 3, 1, -0.125, 0.0)
    bad, err, worst = oracle.check_tolerance(outs[0], ref, rtol=RTOL)
    print(f"  violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))


def _random_cases(n, seed):
    """Seeded random shapes for the 16x16x32 instance: M any size, N and K
    multiples of 8 (the C ABI's transport rule), every program order, padded
    leading dimensions and the XCD order on some."""
    import random
    rng = random.Random(seed)
    maps = [tb.MAP_TILE, tb.MAP_GROUPED_TILE, tb.MAP_PERSISTENT_TILE,
            tb.MAP_PERSISTENT_GROUPED]
    out = []
    for i in range(n):
        M, N, K = rng.randint(1, 1300), 8 * rng.randint(1, 160), 8 * rng.randint(1, 160)
        mapping = rng.choice(maps)
        tiles = -(-M // 256) * -(-N // 256)
        programs = rng.randint(1, tiles) if mapping in maps[2:] else None
        pad = rng.choice([0, 0, 8, 24])
        xcd = 8 if mapping == tb.MAP_GROUPED_TILE and tiles % 8 == 0 and rng.random() < 0.5 else 0
        out.append((M, N, K, mapping, programs, pad, xcd))
    return out


RANDOM_CASES = _random_cases(40, 0x5EED0780)


@pytest.mark.parametrize("M,N,K,mapping,programs,pad,xcd", RANDOM_CASES,
                         ids=[f"r{i}_{c[0]}x{c[1]}x{c[2]}" for i, c in enumerate(RANDOM_CASES)])
def test_mfma16_random_shapes(M, N, K, mapping, programs, pad, xcd, device):
    """Random ragged shapes on the 16x16x32 instance (whole-K and partial-K
    builds): against the oracle, with padding columns untouched, and bit for
    bit against the general loop (128x128x64 on 4 waves) on the same shape."""
    print(f"wide random {M}x{N}x{K} mapping {mapping} programs {programs} pad {pad} "
          f"xcd {xcd}", flush=True)
    A, B = oracle.config_inputs(M, N, K, 0x5EED0781 + M + 3 * N + 7 * K, oracle.NORMAL)
    name16, got16 = _run(_cfg(M, N, K, 4, mapping, programs, pad, xcd, mfma16=True),
                         A, B, device, pad)
    assert name16 == "tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32"
    if pad:
        assert np.isnan(got16[:, N:].astype(np.float32)).all()
    got16 = got16[:, :N]
    bad, err, worst = oracle.check_tolerance(got16, oracle.gemm_f64(A, B), rtol=RTOL)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"
    name, got = _run(_cfg(M, N, K, 4, mapping, programs, pad, xcd, block=128), A, B, device,
                     pad)
    assert "16x16x32" not in name
    assert np.array_equal(got16.view(np.uint16), got[:, :N].view(np.uint16)), name
