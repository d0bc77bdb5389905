"""Randomized GPU parity: 400 seeded random cases over every plain compiled
instance, every program order and both split-K reductions, and 200 over the
fused-step (`_epi`) instances and the split-K reduction's fused steps, each
against the fp64 oracle (|got - ref| <= 1e-2 * (|ref| + 1)).

A case draws an instance, a shape (M any size, N and K multiples of 8, the C
ABI's transport rule), GROUP_M, the XCD order and, per output mode, the
mapping and program count (persistent orders get 1 .. tiles programs) or the
split count (2 .. 8 with a workspace, 2 .. 6 atomic). The seed is fixed, so a failure reproduces; its
case line is printed before the launch.
"""
import random
import re

import numpy as np
import pytest
import torch

import mini_triton_nvgpu_v1_amd as tb
import oracle
from test_gemm_gpu import _every_instance, _spills, run_desc

pytestmark = pytest.mark.gpu
RTOL = 1e-2
CASES = 400
MAPS = [tb.MAP_TILE, tb.MAP_GROUPED_TILE, tb.MAP_PERSISTENT_TILE, tb.MAP_PERSISTENT_GROUPED]


def _case(rng, insts, case):
    bm, bn, bk, wgm, wgn, stages, out, _epi, mfma16 = rng.choice(insts)
    if mfma16:
        M, N, K = rng.randint(1, 800), 8 * rng.randint(1, 100), 8 * rng.randint(1, 100)
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
    elif out == 1 and mfma16:  # plain f32 C (the 16x16x32 build has no split-K)
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F32, acc_init=tb.ACC_INIT_ZERO, mapping=mapping,
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
    # plain (unfused) instances; those whose builds spill are refused (register
    # truth) and have their own test
    insts = [i for i in _every_instance()
             if not i[7] and not _spills(i, False) and not _spills(i, True)]
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


FUSED_CASES = 200


def _fused_case(rng, insts, case):
    """A random fused-step configuration on an `_epi` instance: f16 C, plain
    f32 C, f32 C += A*B, or split-K (the steps then run in the reduction)."""
    bm, bn, bk, wgm, wgn, stages, out, _epi, mfma16 = rng.choice(insts)
    if mfma16:
        M, N, K = rng.randint(1, 600), 8 * rng.randint(1, 90), 8 * rng.randint(1, 64)
    else:
        M, N, K = rng.randint(1, 400), 8 * rng.randint(1, 64), 8 * rng.randint(1, 96)
    tm, tn = -(-M // bm), -(-N // bn)
    lo = rng.uniform(-1.0, 0.5)
    steps = dict(epi_bias=rng.choice([tb.EPI_BIAS_NONE, tb.EPI_BIAS_F16, tb.EPI_BIAS_F32]),
                 epi_activation=rng.choice([tb.ACT_RELU, tb.ACT_GELU_TANH, tb.ACT_SILU]),
                 epi_clamp=rng.randint(0, 3), clamp_min=lo, clamp_max=lo + rng.uniform(0, 2))
    kw = dict(m=M, n=N, k=K, lda=K, ldb=N, ldc=N, block_m=bm, block_n=bn, block_k=bk,
              num_waves=wgm * wgn, wave_grid_m=wgm, wave_grid_n=wgn, stages=stages,
              group_m=rng.choice([1, 8]), xcd_remap=rng.choice([0, 8]),
              mfma=tb.MFMA_16X16X32 if mfma16 else tb.MFMA_32X32X16, **steps)
    mapping = rng.choice(MAPS)
    progs = tm * tn if mapping in MAPS[:2] else rng.randint(1, tm * tn)
    init = None
    if out == 0:
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F16, acc_init=tb.ACC_INIT_ZERO, mapping=mapping,
                            split_k=1, reduction=tb.RED_NONE, num_programs=progs, **kw)
    elif out == 1 and (mfma16 or rng.random() < 0.5):  # plain f32 store (16x16x32: always)
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F32, acc_init=tb.ACC_INIT_ZERO,
                            mapping=tb.MAP_TILE, split_k=1, reduction=tb.RED_NONE,
                            num_programs=tm * tn, **kw)
    elif out == 1:  # split-K: the reduction applies the steps
        s = rng.randint(2, 8)
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F16, acc_init=tb.ACC_INIT_ZERO,
                            mapping=tb.MAP_SPLIT_K, split_k=s, reduction=tb.RED_WORKSPACE,
                            num_programs=tm * tn * s, **kw)
    else:  # f32 C += A*B, then the steps
        init = np.random.default_rng(case).uniform(-1, 1, (M, N)).astype(np.float32)
        cfg = tb.GemmConfig(c_dtype=tb.DTYPE_F32, acc_init=tb.ACC_INIT_LOAD_C, mapping=mapping,
                            split_k=1, reduction=tb.RED_NONE, num_programs=progs, **kw)
    return cfg, init


def test_random_fused_parity(device):
    insts = [i for i in _every_instance()  # `_epi` instances that hold their tile
             if i[7] and not _spills(i, False) and not _spills(i, True)]
    rng = random.Random(0x5EED0A00)
    failures = []
    for case in range(FUSED_CASES):
        cfg, init = _fused_case(rng, insts, case)
        desc = tb.GemmDesc.from_config(cfg)
        print(f"fused case {case}: {cfg.m}x{cfg.n}x{cfg.k} {desc.kernel_name} mapping "
              f"{cfg.mapping} programs {cfg.num_programs} split {cfg.split_k} bias "
              f"{cfg.epi_bias} act {cfg.epi_activation} clamp {cfg.epi_clamp}", flush=True)
        M, N, K = cfg.m, cfg.n, cfg.k
        A, B = oracle.config_inputs(M, N, K, 0x5EED0A00 + case, oracle.NORMAL)
        bias_host = None
        bias_dev = None
        if cfg.epi_bias:
            v = oracle.fill_f16(1, N, 0x5EED0B00 + case, oracle.UNIFORM, 1.0).reshape(N)
            host = v if cfg.epi_bias == tb.EPI_BIAS_F16 else v.astype(np.float32)
            bias_dev = torch.from_numpy(np.ascontiguousarray(host)).to(device)
            bias_host = host.astype(np.float64)
        c_dtype = torch.float16 if cfg.c_dtype == tb.DTYPE_F16 else torch.float32
        dA = torch.from_numpy(A).to(device)
        dB = torch.from_numpy(B).to(device)
        dC = (torch.full((M, N), float("nan"), dtype=c_dtype, device=device) if init is None
              else torch.from_numpy(init.copy()).to(device))
        ws = (torch.empty(desc.workspace_bytes, dtype=torch.uint8, device=device)
              if desc.workspace_bytes else None)
        desc.launch(dA, dB, dC, ws, bias=bias_dev)
        torch.cuda.synchronize()
        ref = oracle.gemm_f64(A, B, init=init)
        oracle.epilogue_f64(ref, bias_host, cfg.epi_activation, cfg.epi_clamp,
                            cfg.clamp_min, cfg.clamp_max)
        bad, err, worst = oracle.check_tolerance(dC.cpu().numpy(), ref, rtol=RTOL)
        if bad:
            failures.append(f"fused case {case} ({desc.kernel_name}): {bad} violations, "
                            f"worst {err} at {worst}")
    assert not failures, "\n".join(failures)


PLAN_CASES = 200
PLAN_TILES = [(64, 64, 32), (64, 64, 64), (128, 128, 32), (128, 128, 64), (128, 64, 32),
              (128, 64, 64), (64, 128, 32), (64, 128, 64), (256, 256, 32), (256, 256, 64),
              (256, 128, 32), (256, 128, 64), (128, 256, 32), (128, 256, 64),
              (64, 256, 64), (256, 64, 32), (192, 128, 64)]


def test_random_plan_pipeline_parity(device):
    """Random tb.matmul modules through the plan pipeline (tile, 1-8 waves,
    2-4 stages, GROUP_M, split-K, persistent programs) and the C ABI, against
    the oracle. A module may be refused by a plan pass (a legality rule, the
    LDS or register budget, or a wave grid with no compiled kernel); one the
    plan accepts must bind a kernel and match."""
    from mini_triton_nvgpu_v1_amd import configs
    rng = random.Random(0x5EED0C00)
    ran, failures = 0, []
    for case in range(PLAN_CASES):
        bm, bn, bk = rng.choice(PLAN_TILES)
        M, N, K = rng.randint(1, 700), 8 * rng.randint(1, 90), 8 * rng.randint(1, 160)
        split = rng.choice([1, 1, 1, 2, 4, 8])
        if split > -(-K // bk):  # the plan needs a k-tile per split
            split = 1
        persistent = split == 1 and rng.random() < 0.3
        tiles = -(-M // bm) * -(-N // bn)
        w = configs.Workload(
            f"random_{case}", M, N, K, 0x5EED0C00 + case, rng.choice([0, 1]), (bm, bn, bk),
            num_waves=rng.choice([1, 2, 4, 4, 8, 8]), stages=rng.choice([2, 3, 4]),
            group_m=rng.choice([1, 4, 8]),
            exact_tile=M % bm == 0 and N % bn == 0 and K % bk == 0, split_k=split,
            persistent=persistent, num_ctas=rng.randint(1, tiles) if persistent else 1)
        try:
            desc = tb.plan_from_mlir(w.mlir())
        except tb.TbError as e:
            # only a plan pass may refuse (its name leads the message); the
            # runtime's "no gfx950 kernel instance for tile" would mean the
            # plan accepted a configuration with no kernel
            assert re.match(r"tb_plan_from_mlir: tb-[a-z0-9-]+: ", str(e)), str(e)
            print(f"plan case {case}: {M}x{N}x{K} tile {(bm, bn, bk)} waves "
                  f"{w.num_waves} stages {w.stages} refused: {e}", flush=True)
            continue
        print(f"plan case {case}: {M}x{N}x{K} tile {(bm, bn, bk)} waves {w.num_waves} "
              f"stages {w.stages} split {split} persistent {persistent} -> "
              f"{desc.kernel_name}", flush=True)
        A, B = oracle.config_inputs(M, N, K, w.seed, w.dist)
        got = run_desc(desc, A, B, device)
        ref = oracle.gemm_f64(A, B)
        bad, err, worst = oracle.check_tolerance(got, ref, rtol=RTOL)
        ran += 1
        if bad:
            failures.append(f"plan case {case} ({desc.kernel_name}): {bad} violations, "
                            f"worst {err} at {worst}")
    assert not failures, "\n".join(failures)
    assert ran >= PLAN_CASES // 2, f"only {ran} of {PLAN_CASES} modules planned"
