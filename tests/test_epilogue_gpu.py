"""GPU parity of the fused epilogue steps (bias, activation, clamp) against
the fp64 oracle.

Each case is a tb.matmul module with `epilogue_*` attrs run through the plan
pipeline and the C ABI (tb_gemm_launch_ex with the bias vector), except the
plain-f32-store case, which only a direct descriptor reaches. The oracle
computes [C0 +] A@B in f64, then tbo_epilogue_f64 (bias, activation, clamp),
and every element must satisfy |got - ref| <= 1e-2 * (|ref| + 1). The
kernels compute the steps in f32 (GELU and SiLU as x * sigmoid(z) from the
hardware exp2 and reciprocal, about 1 ulp each), well inside that bound. The
reference declares these expr kinds but has no implementation to compare
with; the oracle's formulas are pinned to torch's CPU GELU/SiLU and to closed
forms in tests/test_oracle.py.
"""
import dataclasses

import numpy as np
import pytest
import torch

import mini_triton_nvgpu_v1_amd as tb
import oracle
from mini_triton_nvgpu_v1_amd import configs

pytestmark = pytest.mark.gpu
RTOL = 1e-2
ACT = {"": 0, "relu": 1, "gelu_tanh": 2, "silu": 3}


def _bias(N: int, kind: str, seed: int):
    """Seeded bias in [-1, 1): the device array and its exact f64 values."""
    if not kind:
        return None, None
    v = oracle.fill_f16(1, N, seed, oracle.UNIFORM, 1.0).reshape(N)
    host = v if kind == "f16" else v.astype(np.float32) * np.float32(0.75)
    return torch.from_numpy(np.ascontiguousarray(host)), host.astype(np.float64)


def _clamp_bits(w):
    return (1 if w.clamp_min is not None else 0) | (2 if w.clamp_max is not None else 0)


def _run_and_check(desc, w, A, B, device, c0=None, c_dtype=torch.float16):
    bias_dev, bias_ref = _bias(w.N, w.bias, w.seed ^ 0xB1A5)
    dA = torch.from_numpy(A).to(device)
    dB = torch.from_numpy(B).to(device)
    if c0 is None:
        dC = torch.full((w.M, w.N), float("nan"), dtype=c_dtype, device=device)
    else:
        dC = torch.from_numpy(c0.copy()).to(device)
    ws = (torch.empty(desc.workspace_bytes, dtype=torch.uint8, device=device)
          if desc.workspace_bytes else None)
    desc.launch(dA, dB, dC, ws, bias=None if bias_dev is None else bias_dev.to(device))
    torch.cuda.synchronize()
    got = dC.cpu().numpy()
    ref = oracle.gemm_f64(A, B, init=c0)
    oracle.epilogue_f64(ref, bias_ref, ACT[w.activation], _clamp_bits(w),
                        w.clamp_min or 0.0, w.clamp_max or 0.0)
    bad, err, worst = oracle.check_tolerance(got, ref, rtol=RTOL)
    print(f"{w.name} via {desc.kernel_name}: violations={bad} max|err|={err:.3e}",
          flush=True)
    assert bad == 0, f"{bad} elements outside tolerance; worst {err} at {worst}"
    return got, ref


def _w(base, name, **kw):
    return dataclasses.replace(base, name=name, **kw)


# f16 C through the plan pipeline: every epilogue store path of the kernel
# (direct 8-byte stores, the LDS-staged stores of 64- and 128-wide wave
# tiles, the exact-shape 4-wave 256x256 kernel, the split-K reduction, the
# persistent loop).
F16_CASES = [
    _w(configs.SMOKE, "smoke_bias16_relu", bias="f16", activation="relu"),
    _w(configs.RAGGED, "ragged_bias32_gelu_clamp", bias="f32", activation="gelu_tanh",
       clamp_min=-0.5, clamp_max=2.0),
    _w(configs.RAGGED_128, "tile128_bias16_silu_max", bias="f16", activation="silu",
       clamp_max=0.75),
    _w(configs.ROOFLINE, "w4x2_512x256_bias32_gelu", M=512, N=512, K=256, bias="f32",
       activation="gelu_tanh", block=(256, 128, 64), num_waves=8),
    _w(configs.ROOFLINE, "w2x2_512_bias16_silu", M=512, N=768, K=192, bias="f16",
       activation="silu", clamp_min=-0.5),
    _w(configs.RAGGED, "ragged_clamp_only", clamp_min=-0.25),
    _w(configs.SPLIT_K, "splitk_bias16_silu", M=128, N=128, K=2048, bias="f16",
       activation="silu"),
    _w(configs.SMOKE, "persistent_bias16_clamp", M=192, N=128, K=64, persistent=True,
       num_ctas=2, bias="f16", clamp_min=-1.0, clamp_max=1.0),
]


@pytest.mark.parametrize("w", F16_CASES, ids=lambda w: w.name)
def test_fused_epilogue_f16(w, device):
    print(f"case {w.name} {w.M}x{w.N}x{w.K}", flush=True)
    desc = tb.plan_from_mlir(w.mlir())
    assert desc.config == w.direct_config()
    A, B = oracle.config_inputs(w.M, w.N, w.K, w.seed, w.dist)
    _run_and_check(desc, w, A, B, device)


def test_fused_epilogue_f32_accumulate(device):
    """Reference semantics C += A*B (f32 C), then the steps on the sum."""
    w = _w(configs.RAGGED_128, "acc_bias32_relu_min", bias="f32", activation="relu",
           clamp_min=-1.0)
    text = w.mlir(c_type="f32")
    print(f"case {w.name}", flush=True)
    desc = tb.plan_from_mlir(text)
    assert desc.config.acc_init == tb.ACC_INIT_LOAD_C
    assert "_out2" in desc.kernel_name and desc.kernel_name.endswith("_epi")
    A, B = oracle.config_inputs(w.M, w.N, w.K, w.seed, w.dist)
    C0 = oracle.fill_f16(w.M, w.N, 0x5EED0601, oracle.UNIFORM, 2.0).astype(np.float32)
    _run_and_check(desc, w, A, B, device, c0=C0, c_dtype=torch.float32)


def test_fused_epilogue_f32_plain_store(device):
    """f32 C written (not accumulated): only a direct descriptor asks for it."""
    w = _w(configs.RAGGED, "plain_f32_gelu", activation="gelu_tanh", bias="f16")
    cfg = w.direct_config()
    cfg.c_dtype = tb.DTYPE_F32
    desc = tb.GemmDesc.from_config(cfg)
    assert desc.kernel_name.endswith("_out1_epi")
    print(f"case {w.name}", flush=True)
    A, B = oracle.config_inputs(w.M, w.N, w.K, w.seed, w.dist)
    _run_and_check(desc, w, A, B, device, c_dtype=torch.float32)


def test_fused_epilogue_matches_unfused_plus_steps(device):
    """The fused instance's result equals the plain instance's f32 result with
    the steps applied on the host in f32 (same accumulation; only the final
    rounding of the step arithmetic may differ)."""
    w = _w(configs.RAGGED_128, "fused_vs_host", bias="f32", activation="relu",
           clamp_max=1.5)
    A, B = oracle.config_inputs(w.M, w.N, w.K, w.seed, w.dist)
    base = dataclasses.replace(w, bias="", activation="", clamp_max=None)
    cfg_plain = base.direct_config()
    cfg_plain.c_dtype = tb.DTYPE_F32
    cfg_fused = w.direct_config()
    cfg_fused.c_dtype = tb.DTYPE_F32
    dA = torch.from_numpy(A).to(device)
    dB = torch.from_numpy(B).to(device)
    bias_dev, _ = _bias(w.N, w.bias, w.seed ^ 0xB1A5)
    outs = []
    for cfg, bias in ((cfg_plain, None), (cfg_fused, bias_dev.to(device))):
        dC = torch.full((w.M, w.N), float("nan"), dtype=torch.float32, device=device)
        tb.GemmDesc.from_config(cfg).launch(dA, dB, dC, bias=bias)
        torch.cuda.synchronize()
        outs.append(dC.cpu().numpy())
    expect = np.minimum(np.maximum(outs[0] + bias_dev.numpy()[None, :], 0.0), 1.5)
    assert np.array_equal(outs[1], expect.astype(np.float32))
