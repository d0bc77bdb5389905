"""GPU: launches captured into a HIP graph and replayed.

A serving loop captures its GEMMs once and replays them: the C ABI's launch
entry points record only kernel launches on the caller's stream (no
allocation, no memset, no synchronisation), so they can be captured. Three
calls are captured into one graph with torch.cuda.graph: a plain f16 GEMM, a
split-K GEMM with its reduce (caller's workspace), the same split-K through
the no-allocation entry point (the library's device scratch; its one-time
set-up runs eagerly first), and an f32 C += A*B on the 16x16x32 build. The
graph is replayed five times with eager work between the replays (outputs
cleared, the prior C of C += A*B restored, an unrelated GEMM), and every
replay's outputs must be bit-identical to the eager launches'.
"""
import numpy as np
import pytest
import torch

import mini_triton_nvgpu_v1_amd as tb
import oracle
from mini_triton_nvgpu_v1_amd import configs

pytestmark = pytest.mark.gpu


def test_captured_launches_replay_bit_identically(device):
    plain = tb.GemmDesc.from_config(configs.RAGGED_128.direct_config())
    w = configs.Workload("splitk_graph", 384, 320, 2048, 1, 0, (128, 64, 64), num_waves=8,
                         stages=3, split_k=4)
    split = tb.GemmDesc.from_config(w.direct_config())

    def operands(M, N, K, seed):
        A, B = oracle.config_inputs(M, N, K, seed, oracle.UNIFORM)
        return torch.from_numpy(A).to(device), torch.from_numpy(B).to(device)

    pA, pB = operands(128, 128, 32, 0x5EED0E01)
    sA, sB = operands(384, 320, 2048, 0x5EED0E02)
    acfg = configs.ROOFLINE.direct_config()
    acfg.m, acfg.n, acfg.k, acfg.lda, acfg.ldb, acfg.ldc = 512, 768, 328, 328, 768, 768
    acfg.c_dtype, acfg.acc_init = tb.DTYPE_F32, tb.ACC_INIT_LOAD_C
    acfg.num_programs, acfg.xcd_remap = 6, 0
    accum = tb.GemmDesc.from_config(acfg)
    assert accum.kernel_name == "tb_gemm_gfx950_256x256x64_w2x2_s2_out2_16x16x32"
    aA, aB = operands(512, 768, 328, 0x5EED0E03)
    aC0 = torch.rand((512, 768), dtype=torch.float32, device=device) - 0.5
    aC = aC0.clone()
    pC = torch.empty((128, 128), dtype=torch.float16, device=device)
    sC = torch.empty((384, 320), dtype=torch.float16, device=device)
    nC = torch.empty_like(sC)
    ws = torch.empty(split.workspace_bytes, dtype=torch.uint8, device=device)

    def run():
        plain.launch(pA, pB, pC)
        split.launch(sA, sB, sC, ws)
        split.launch_noalloc(sA, sB, nC)
        accum.launch(aA, aB, aC)

    run()  # eager: the references, and the no-allocation scratch's set-up
    torch.cuda.synchronize()
    refs = [x.clone() for x in (pC, sC, nC, aC)]
    assert torch.equal(refs[1], refs[2])  # the two split-K entry points agree

    aC.copy_(aC0)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    other = torch.randn(256, 256, device=device)
    for r in range(5):
        for x in (pC, sC, nC):
            x.fill_(float("nan"))
        aC.copy_(aC0)
        other = other @ other.T / 256.0  # unrelated eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, x, ref in zip(("plain", "split-K", "split-K no-alloc", "f32 C += A*B"),
                                (pC, sC, nC, aC), refs):
            same = np.array_equal(x.cpu().numpy().view(np.uint8),
                                  ref.cpu().numpy().view(np.uint8))
            print(f"replay {r} {name}: bit-identical to eager: {same}", flush=True)
            assert same, (r, name)
