"""Randomized GPU parity: 400 seeded random cases over every plain compiled
instance, every program order and both split-K reductions, each against the
fp64 oracle (|got - ref| <= 1e-2 * (|ref| + 1)).

A case draws an instance, a shape (M any size, N and K multiples of 8, the C
ABI's transport rule; whole tiles for the 16x16x32 instance), GROUP_M, the
XCD order and, per output mode, the mapping and program count (persistent
orders get 1 .. tiles programs) or the split count (2 .. 8 with a
workspace, 2 .. 6 atomic). The seed is fixed, so a failure reproduces; its
case line is printed before the launch.
"""
import random

import numpy as np
import pytest
import torch

import mini_triton_nvgpu_v1_amd as tb
import oracle
from test_gemm_gpu import _every_instance, run_desc

pytestmark = pytest.mark.gpu
RTOL = 1e-2
CASES = 400
MAPS = [tb.MAP_TILE, tb.MAP_GROUPED_TILE, tb.MAP_PERSISTENT_TILE, tb.MAP_PERSISTENT_GROUPED]


def _case(rng, insts, case):
    bm, bn, bk, wgm, wgn, stages, out, _epi, mfma16 = rng.choice(insts)
    if mfma16:
        M, N, K = 256 * rng.randint(1, 3), 256 * rng.randint(1, 3), 64 * rng.randint(1, 12)
    else:
        M, N, K = rng.randint(1, 600), 8 * rng.randint(1, 80), 8 * rng.randint(1, 128)
    tm, tn = -(-M // bm), -(-N // bn)
    kw = dict(m=M, n=N, k=K, lda=K, ldb=N, ldc=N, block_m=bm, block_n=bn, block_k=bk,
              num_waves=wgm * wgn, wave_grid_m=wgm, wave_grid_n=wgn, stages=stages,
              group_m=rng.choice([1, 2, 8]), xcd_remap=rng.choice([0, 8]),
              mfma=tb.MFMA_16X16X32 if mfma16 else tb.MFMA_32X32X16)
    mapping = rng.choice(MAPS)
    progs = tm * tn if mapping in MAPS[:2] else rng.randint(1, tm * tn)
    init = None
    if out == 0:
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F16, acc_init=tb.ACC_INIT_ZERO, mapping=mapping,
                            split_k=1, reduction=tb.RED_NONE, num_programs=progs, **kw)
    elif out == 1:
        s = rng.randint(2, 8)
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F16, acc_init=tb.ACC_INIT_ZERO,
                            mapping=tb.MAP_SPLIT_K, split_k=s, reduction=tb.RED_WORKSPACE,
                            num_programs=tm * tn * s, **kw)
    elif out == 2:
        init = np.random.default_rng(case).uniform(-1, 1, (M, N)).astype(np.float32)
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F32, acc_init=tb.ACC_INIT_LOAD_C, mapping=mapping,
                            split_k=1, reduction=tb.RED_NONE, num_programs=progs, **kw)
    else:
        s = rng.randint(2, 6)
        init = np.random.default_rng(case).uniform(-1, 1, (M, N)).astype(np.float32)
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F32, acc_init=tb.ACC_INIT_LOAD_C,
                            mapping=tb.MAP_SPLIT_K, split_k=s, reduction=tb.RED_ATOMIC,
                            num_programs=tm * tn * s, **kw)
    return cfg, init, rng.choice([oracle.UNIFORM, oracle.NORMAL])


def test_random_parity(device):
    insts = [i for i in _every_instance() if not i[7]]  # plain (unfused) instances
    rng = random.Random(0x5EED0900)
    failures = []
    for case in range(CASES):
        cfg, init, dist = _case(rng, insts, case)
        desc = tb.GemmDesc.from_config(cfg)
        print(f"case {case}: {cfg.m}x{cfg.n}x{cfg.k} {desc.kernel_name} mapping "
              f"{cfg.mapping} programs {cfg.num_programs} split {cfg.split_k} "
              f"group_m {cfg.group_m} xcd {cfg.xcd_remap}", flush=True)
        A, B = oracle.config_inputs(cfg.m, cfg.n, cfg.k, 0x5EED0900 + case, dist)
        c_dtype = torch.float16 if cfg.c_dtype == tb.DTYPE_F16 else torch.float32
        got = run_desc(desc, A, B, device, c_init=None if init is None else init.copy(),
                       c_dtype=c_dtype)
        ref = oracle.gemm_f64(A, B, init=init)
        bad, err, worst = oracle.check_tolerance(got, ref, rtol=RTOL)
        if bad:
            failures.append(f"case {case} ({desc.kernel_name}): {bad} violations, "
                            f"worst {err} at {worst}")
    assert not failures, "\n".join(failures)
