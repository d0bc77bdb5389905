"""GPU parity past 2 GiB per operand.

The kernels address A, C and the split-K partial planes through buffer
windows that start at each tile's first row (32-bit offsets inside a tile, a
64-bit window base), so A, C and the workspace may exceed 2 GiB; only a
tile's rows (under 1 GiB), and B (under 2 GiB), stay bounded. Each case puts
the rows that lie past the 2^31-byte mark of the large operand under the
fp64 oracle, together with the first and last rows:

* A of 2.1 GiB through the 16x16x32 instance, the general loop and the
  producer-wave split-K build;
* f16 C of 2.1 GiB (16x16x32 instance), f32 C of 2.1 GiB as a plain store and
  as C += A*B (general loop), and as C += A*B on the 16x16x32 instance;
* a split-K workspace of 2.3 GiB (eight partial planes), producer-wave build.

Operands are filled on the device with the oracle's SplitMix64 stream (the
device fill is checked against the oracle's on B); the checked rows of A
and of the prior C are copied back for the oracle. Tolerance
|got - ref| <= 1e-2 * (|ref| + 1).
"""
import numpy as np
import pytest
import torch

import mini_triton_nvgpu_v1_amd as tb
import oracle

pytestmark = pytest.mark.gpu
RTOL = 1e-2
GIB2 = 1 << 31


def _cfg(M, N, K, tile, waves, grid, stages, c_dtype=tb.DTYPE_F16,
         acc_init=tb.ACC_INIT_ZERO, split=1, mfma=tb.MFMA_32X32X16):
    bm, bn, bk = tile
    tiles = -(-M // bm) * -(-N // bn)
    return tb.GemmConfig(
        m=M, n=N, k=K, lda=K, ldb=N, ldc=N, c_dtype=c_dtype, acc_init=acc_init,
        block_m=bm, block_n=bn, block_k=bk, num_waves=waves, wave_grid_m=grid[0],
        wave_grid_n=grid[1], stages=stages,
        mapping=tb.MAP_SPLIT_K if split > 1 else tb.MAP_GROUPED_TILE,
        group_m=1 if split > 1 else 8, split_k=split,
        reduction=tb.RED_WORKSPACE if split > 1 else tb.RED_NONE,
        num_programs=tiles * split, xcd_remap=0, mfma=mfma)


def _rows_past(nbytes_per_row, M):
    """Row blocks to check: the first rows, the rows around the 2^31-byte mark
    of an operand with `nbytes_per_row` bytes per row, and the last rows."""
    mark = GIB2 // nbytes_per_row
    assert 0 < mark < M - 64, "the operand must extend past 2 GiB"
    return [(0, 64), (mark - 64, mark + 64), (M - 64, M)]


CASES = {
    # name: (M, N, K, tile, waves, grid, stages, c_dtype, acc_init, split, mfma, big)
    "A_16x16x32": (139264, 256, 8192, (256, 256, 64), 4, (2, 2), 2, tb.DTYPE_F16,
                   tb.ACC_INIT_ZERO, 1, tb.MFMA_16X16X32, "A"),
    "A_general": (139264, 128, 8192, (128, 128, 64), 4, (2, 2), 2, tb.DTYPE_F16,
                  tb.ACC_INIT_ZERO, 1, tb.MFMA_32X32X16, "A"),
    "A_producer_splitk": (139264, 64, 8192, (128, 64, 64), 8, (4, 2), 3, tb.DTYPE_F16,
                          tb.ACC_INIT_ZERO, 2, tb.MFMA_32X32X16, "A"),
    "C16_16x16x32": (139264, 8192, 64, (256, 256, 64), 4, (2, 2), 2, tb.DTYPE_F16,
                     tb.ACC_INIT_ZERO, 1, tb.MFMA_16X16X32, "C"),
    "C32_general": (70016, 8192, 64, (128, 128, 64), 4, (2, 2), 2, tb.DTYPE_F32,
                    tb.ACC_INIT_ZERO, 1, tb.MFMA_32X32X16, "C"),
    "C32_accumulate": (70016, 8192, 64, (128, 128, 64), 4, (2, 2), 2, tb.DTYPE_F32,
                       tb.ACC_INIT_LOAD_C, 1, tb.MFMA_32X32X16, "C"),
    "C32_accumulate_16x16x32": (70016, 8192, 64, (256, 256, 64), 4, (2, 2), 2, tb.DTYPE_F32,
                                tb.ACC_INIT_LOAD_C, 1, tb.MFMA_16X16X32, "C"),
    "workspace_producer": (16384, 4608, 1024, (128, 64, 64), 8, (4, 2), 3, tb.DTYPE_F16,
                           tb.ACC_INIT_ZERO, 8, tb.MFMA_32X32X16, "ws"),
}


@pytest.mark.parametrize("name", list(CASES))
def test_operands_past_2gib(name, device):
    M, N, K, tile, waves, grid, stages, c_dtype, acc_init, split, mfma, big = CASES[name]
    cfg = _cfg(M, N, K, tile, waves, grid, stages, c_dtype, acc_init, split, mfma)
    desc = tb.GemmDesc.from_config(cfg)
    ct = torch.float16 if c_dtype == tb.DTYPE_F16 else torch.float32
    es = 2 if c_dtype == tb.DTYPE_F16 else 4
    sizes = {"A": M * K * 2, "C": M * N * es, "ws": desc.workspace_bytes}
    print(f"case {name}: {M}x{N}x{K} via {desc.kernel_name}, "
          f"{big} = {sizes[big] / 2**30:.3f} GiB", flush=True)
    assert sizes[big] > GIB2
    seed = 0x5EED0A00 + len(name)
    dA = torch.empty((M, K), dtype=torch.float16, device=device)
    dB = torch.empty((K, N), dtype=torch.float16, device=device)
    tb.fill_seeded_f16(dA, M, K, seed, oracle.UNIFORM, 1.0)
    tb.fill_seeded_f16(dB, K, N, seed ^ 0xB, oracle.UNIFORM, 1.0)
    B = oracle.fill_f16(K, N, seed ^ 0xB, oracle.UNIFORM, 1.0)
    assert np.array_equal(dB.cpu().numpy().view(np.uint16), B.view(np.uint16))
    if acc_init == tb.ACC_INIT_LOAD_C:
        gen = torch.Generator(device=device).manual_seed(seed)
        dC = torch.rand((M, N), generator=gen, device=device, dtype=torch.float32) - 0.5
    else:
        dC = torch.full((M, N), float("nan"), dtype=ct, device=device)
    if big == "ws":  # the last partial plane starts past 2 GiB: check its rows too
        blocks = [(0, 64), (M // 2 - 32, M // 2 + 32), (M - 64, M)]
    else:
        blocks = _rows_past({"A": K * 2, "C": N * es}[big], M)
    C0 = {b: dC[b[0]:b[1]].float().cpu().numpy() for b in blocks} \
        if acc_init == tb.ACC_INIT_LOAD_C else None
    ws = (torch.empty(desc.workspace_bytes, dtype=torch.uint8, device=device)
          if desc.workspace_bytes else None)
    desc.launch(dA, dB, dC, ws)
    torch.cuda.synchronize()
    for r0, r1 in blocks:
        A_rows = dA[r0:r1].cpu().numpy()
        init = None if C0 is None else np.ascontiguousarray(C0[(r0, r1)], np.float32)
        ref = oracle.gemm_f64(A_rows, B, init=init)
        got = dC[r0:r1].cpu().numpy()
        bad, err, worst = oracle.check_tolerance(got, ref, rtol=RTOL)
        print(f"rows [{r0},{r1}): violations={bad} max|err|={err:.3e} at {worst}", flush=True)
        assert bad == 0, f"rows [{r0},{r1}): {bad} elements outside tolerance; worst {err}"
    del dA, dB, dC, ws
    torch.cuda.empty_cache()
