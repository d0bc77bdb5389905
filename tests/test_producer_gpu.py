"""GPU parity of the producer-wave builds (`gemm_kernel_pw`).

`tb_gemm_gfx950_128x64x64_w4x2_s3_out1` (8 load-only waves beside a 4x2
grid of MFMA waves) and `tb_gemm_gfx950_64x64x64_w2x2_s3_out1` (4 beside
2x2) serve every configuration that binds their keys: split-K f32 partials
(the first is the split-K workload's instance) and plain f32 C in tile,
grouped and persistent order. Checks, each against the fp64 oracle with
|got - ref| <= 1e-2 * (|ref| + 1):

* split-K over even and uneven k-tile partitions, a ragged last k-tile
  (K % 64 != 0), ragged M and N, more splits than k-tiles (a split with no
  k-tile stores zeros), padded leading dimensions;
* plain f32 C in every program order, with more tiles than persistent
  programs, ragged edges and padding columns that must stay unwritten;
* run-to-run bit-identity of every case (fixed k order in each split, fixed
  split order in the reduce).
"""
import numpy as np
import pytest
import torch

import mini_triton_nvgpu_v1_amd as tb
import oracle

pytestmark = pytest.mark.gpu
RTOL = 1e-2
# tile -> (wave grid, instance name)
TILES = {(128, 64): ((4, 2), "tb_gemm_gfx950_128x64x64_w4x2_s3_out1"),
         (64, 64): ((2, 2), "tb_gemm_gfx950_64x64x64_w2x2_s3_out1")}


def _cfg(M, N, K, mapping, split=1, programs=None, c_f32=False, ld_pad=0, xcd=0,
         tile=(128, 64)):
    (wm, wn), _ = TILES[tile]
    tiles = -(-M // tile[0]) * -(-N // tile[1])
    return tb.GemmConfig(
        m=M, n=N, k=K, lda=K + ld_pad, ldb=N + ld_pad, ldc=N + ld_pad,
        c_dtype=tb.DTYPE_F32 if c_f32 else tb.DTYPE_F16, acc_init=tb.ACC_INIT_ZERO,
        block_m=tile[0], block_n=tile[1], block_k=64, num_waves=wm * wn, wave_grid_m=wm,
        wave_grid_n=wn, stages=3, mapping=mapping,
        group_m=8 if mapping in (tb.MAP_GROUPED_TILE, tb.MAP_PERSISTENT_GROUPED) else 1,
        split_k=split, reduction=tb.RED_WORKSPACE if split > 1 else tb.RED_NONE,
        num_programs=programs or tiles * (split if mapping == tb.MAP_SPLIT_K else 1),
        xcd_remap=xcd, mfma=tb.MFMA_32X32X16)


def _run(desc, cfg, A, B, device, ld_pad):
    M, N, K = cfg.m, cfg.n, cfg.k
    dA = torch.zeros((M, K + ld_pad), dtype=torch.float16, device=device)
    dB = torch.zeros((K, N + ld_pad), dtype=torch.float16, device=device)
    dA[:, :K] = torch.from_numpy(A).to(device)
    dB[:, :N] = torch.from_numpy(B).to(device)
    ct = torch.float32 if cfg.c_dtype == tb.DTYPE_F32 else torch.float16
    dC = torch.full((M, N + ld_pad), float("nan"), dtype=ct, device=device)
    ws = None
    if desc.workspace_bytes:
        ws = torch.full((desc.workspace_bytes // 4,), float("nan"), dtype=torch.float32,
                        device=device)
    desc.launch(dA, dB, dC, ws)
    torch.cuda.synchronize()
    return dC.cpu().numpy()


# (M, N, K, mapping, split, programs, c_f32, ld_pad, xcd_remap)
CASES = [
    (512, 512, 4096, tb.MAP_SPLIT_K, 8, None, False, 0, 0),     # 8 k-tiles per split
    (384, 320, 1000, tb.MAP_SPLIT_K, 3, None, False, 0, 0),     # 16 k-tiles / 3, K % 64 = 40
    (200, 136, 520, tb.MAP_SPLIT_K, 5, None, False, 0, 0),      # ragged M, N and K
    (256, 128, 192, tb.MAP_SPLIT_K, 4, None, False, 0, 0),      # 3 k-tiles over 4 splits
    (640, 448, 2056, tb.MAP_SPLIT_K, 8, None, False, 8, 0),     # padded, ragged k-tile
    (1000, 520, 328, tb.MAP_GROUPED_TILE, 1, None, True, 0, 0),  # plain f32, ragged
    (768, 640, 256, tb.MAP_PERSISTENT_TILE, 1, 7, True, 0, 0),   # 60 tiles on 7 programs
    (904, 584, 136, tb.MAP_PERSISTENT_GROUPED, 1, 5, True, 8, 0),  # ragged, padded
    (1024, 1024, 128, tb.MAP_GROUPED_TILE, 1, None, True, 0, 8),   # 128 tiles, XCD order
    (128, 64, 8, tb.MAP_TILE, 1, None, True, 0, 0),              # K below one k step
]
# the 64x64 tile: split-K (even, ragged, empty splits) and plain f32 C
CASES64 = [
    (256, 256, 4096, tb.MAP_SPLIT_K, 16, None, False, 0, 0),    # 4 k-tiles per split
    (200, 136, 520, tb.MAP_SPLIT_K, 5, None, False, 8, 0),      # ragged, padded
    (128, 64, 192, tb.MAP_SPLIT_K, 4, None, False, 0, 0),       # 3 k-tiles over 4 splits
    (1000, 520, 328, tb.MAP_GROUPED_TILE, 1, None, True, 0, 0),  # plain f32, ragged
    (520, 392, 136, tb.MAP_PERSISTENT_GROUPED, 1, 5, True, 8, 0),  # 63 tiles on 5
    (1024, 1024, 128, tb.MAP_GROUPED_TILE, 1, None, True, 0, 8),   # 256 tiles, XCD order
]
ALL = [c + ((128, 64),) for c in CASES] + [c + ((64, 64),) for c in CASES64]


@pytest.mark.parametrize("case", ALL,
                         ids=lambda c: f"{c[9][0]}x{c[9][1]}_{c[0]}x{c[1]}x{c[2]}_m{c[3]}_s{c[4]}")
def test_producer_build_parity(case, device):
    M, N, K, mapping, split, programs, c_f32, ld_pad, xcd, tile = case
    cfg = _cfg(M, N, K, mapping, split, programs, c_f32, ld_pad, xcd, tile)
    desc = tb.GemmDesc.from_config(cfg)
    print(f"case {case} via {desc.kernel_name}", flush=True)
    assert desc.kernel_name == TILES[tile][1]
    A, B = oracle.config_inputs(M, N, K, 0x5EED0900 + M + N + K, oracle.UNIFORM)
    got = _run(desc, cfg, A, B, device, ld_pad)
    ref = oracle.gemm_f64(A, B)
    bad, err, worst = oracle.check_tolerance(np.ascontiguousarray(got[:, :N]), ref,
                                             rtol=RTOL)
    print(f"violations={bad} max|err|={err:.3e} at {worst}", flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"
    if ld_pad:
        assert np.isnan(got[:, N:].astype(np.float32)).all(), "padding columns written"
    again = _run(desc, cfg, A, B, device, ld_pad)
    assert np.array_equal(got.view(np.uint8), again.view(np.uint8)), "not run-to-run identical"
