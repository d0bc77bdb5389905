"""GPU parity of the exact-shape kernel of the 4-wave 256x256x64 instance.

When M and N are multiples of 256 and K of 64 (tile, grouped or persistent
order), the launcher runs a kernel of its own for the
`256x256x64_w2x2_s2_out0[_epi]` instance: one wave per SIMD, 128x128 wave
tiles, the same LDS ring and MFMA k order as the general loop. Two checks:

* against the fp64 oracle, |got - ref| <= 1e-2 * (|ref| + 1), on shapes that
  cover 1, 2, odd and even k-tile counts, tile / grouped / persistent orders
  (more tiles than programs), padded leading dimensions and the fused steps;
* bit-identity with the 8-wave instance (`w4x2`), which runs the general
  loop: both issue the same MFMAs over the same fragments in the same k
  order, so C agrees to the last bit.

Ragged shapes on the same instance take the general loop and are covered by
test_gemm_gpu.py (test_ragged_edges, test_every_instance).
"""
import numpy as np
import pytest
import torch

import mini_triton_nvgpu_v1_amd as tb
import oracle

pytestmark = pytest.mark.gpu
RTOL = 1e-2


def _cfg(M, N, K, waves, mapping, programs=None, ld_pad=0, xcd=0):
    wgm, wgn = (2, 2) if waves == 4 else (4, 2)
    tm, tn = M // 256, N // 256
    return tb.GemmConfig(
        m=M, n=N, k=K, lda=K + ld_pad, ldb=N + ld_pad, ldc=N + ld_pad,
        c_dtype=tb.DTYPE_F16, acc_init=tb.ACC_INIT_ZERO, block_m=256, block_n=256,
        block_k=64, num_waves=waves, wave_grid_m=wgm, wave_grid_n=wgn, stages=2,
        mapping=mapping, group_m=8 if mapping != tb.MAP_TILE else 1, split_k=1,
        reduction=tb.RED_NONE, num_programs=programs or tm * tn, xcd_remap=xcd)


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
]


@pytest.mark.parametrize("M,N,K,mapping,programs,pad,xcd", CASES,
                         ids=[f"{c[0]}x{c[1]}x{c[2]}_map{c[3]}_p{c[4]}_pad{c[5]}"
                              for c in CASES])
def test_wide_exact_matches_oracle_and_8_waves(M, N, K, mapping, programs, pad, xcd,
                                               device):
    print(f"wide {M}x{N}x{K} mapping {mapping} programs {programs} pad {pad}", flush=True)
    A, B = oracle.config_inputs(M, N, K, 0x5EED0700 + M + K, oracle.NORMAL)
    name4, got4 = _run(_cfg(M, N, K, 4, mapping, programs, pad, xcd), A, B, device, pad)
    assert name4 == "tb_gemm_gfx950_256x256x64_w2x2_s2_out0"
    got4 = got4[:, :N]
    ref = oracle.gemm_f64(A, B)
    bad, err, worst = oracle.check_tolerance(got4, ref, rtol=RTOL)
    print(f"  4 waves: violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"
    _, got8 = _run(_cfg(M, N, K, 8, mapping, programs, pad, xcd), A, B, device, pad)
    assert np.array_equal(got4.view(np.uint16), got8[:, :N].view(np.uint16))


def test_wide_exact_fused_steps(device):
    """Bias (f32), tanh GELU and a clamp on the exact-shape kernel, against the
    oracle's epilogue, and bit-identical to the 8-wave fused instance."""
    M, N, K = 512, 768, 192
    print(f"wide fused {M}x{N}x{K}", flush=True)
    A, B = oracle.config_inputs(M, N, K, 0x5EED0710, oracle.UNIFORM)
    bias = oracle.fill_f16(1, N, 0x5EED0711, oracle.UNIFORM, 1.0).reshape(N).astype(np.float32)
    outs = []
    for waves in (4, 8):
        cfg = _cfg(M, N, K, waves, tb.MAP_GROUPED_TILE)
        cfg.epi_bias, cfg.epi_activation = tb.EPI_BIAS_F32, tb.ACT_GELU_TANH
        cfg.epi_clamp, cfg.clamp_min, cfg.clamp_max = tb.CLAMP_MIN | tb.CLAMP_MAX, -0.25, 3.0
        name, got = _run(cfg, A, B, device, bias=bias)
        assert name.endswith("_out0_epi")
        outs.append(got)
    ref = oracle.gemm_f64(A, B)
    oracle.epilogue_f64(ref, bias.astype(np.float64), 2, 3, -0.25, 3.0)
    bad, err, worst = oracle.check_tolerance(outs[0], ref, rtol=RTOL)
    print(f"  violations={bad} max|err|={err:.3e}", flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))
