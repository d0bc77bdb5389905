"""CPU-side checks of the C ABI: the library loads, exports every symbol the
public header declares, and validates descriptors without touching a GPU."""
import ctypes
import os
import re

import pytest

import mini_triton_nvgpu_v1_amd as tb
from mini_triton_nvgpu_v1_amd import configs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tb_gfx950.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tb_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = tb.lib()
    names = declared_functions()
    assert "tb_gemm_launch" in names and "tb_plan_from_mlir" in names
    for name in names:
        assert hasattr(L, name), f"{name} declared in include/tb_gfx950.h but not exported"


def test_abi_version_and_struct_layout(tmp_path):
    """The ctypes mirror of tb_gemm_config matches the C compiler's layout."""
    assert tb.lib().tb_abi_version() == 4
    fields = [name for name, _ in tb.GemmConfig._fields_]
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "tb_gfx950.h"\n'
        "int main(void) {\n"
        '  printf("%zu\\n", sizeof(tb_gemm_config));\n'
        + "".join(f'  printf("%zu\\n", offsetof(tb_gemm_config, {f}));\n' for f in fields)
        + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    import subprocess
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    out = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True,
                                          text=True).stdout.split()]
    assert out[0] == ctypes.sizeof(tb.GemmConfig)
    assert out[1:] == [getattr(tb.GemmConfig, f).offset for f in fields]


def test_kernel_registry_names():
    names = tb.kernel_names()
    assert len(names) >= 40
    assert "tb_gemm_gfx950_256x256x64_w2x2_s2_out0" in names
    assert "tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32" in names
    assert "tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32_epi" in names
    for out in (1, 2):  # f32 C: plain store, C += A*B
        for suffix in ("", "_epi"):
            assert f"tb_gemm_gfx950_256x256x64_w2x2_s2_out{out}_16x16x32{suffix}" in names


def _wide(**kw):
    c = configs.ROOFLINE.direct_config()
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def test_mfma_16x16x32_instance_selection():
    """The 4-wave 256x256x64 f16 config binds the 16x16x32 instance when the
    config asks for it; its 32x32x16 build spills (128x128 wave tiles of 32x32
    MFMA tiles) and is refused with the compiler's figures."""
    assert configs.ROOFLINE.direct_config().mfma == tb.MFMA_16X16X32
    d16 = tb.GemmDesc.from_config(_wide())
    assert d16.kernel_name == "tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32"
    with pytest.raises(tb.TbError, match=r"_out0 spills \d+ bytes per lane to scratch"):
        tb.GemmDesc.from_config(_wide(mfma=tb.MFMA_32X32X16))
    fused = tb.GemmDesc.from_config(_wide(epi_activation=tb.ACT_RELU))
    assert fused.kernel_name.endswith("_16x16x32_epi")
    plain32 = tb.GemmDesc.from_config(_wide(c_dtype=tb.DTYPE_F32))
    assert plain32.kernel_name == "tb_gemm_gfx950_256x256x64_w2x2_s2_out1_16x16x32"
    accum = tb.GemmDesc.from_config(_wide(c_dtype=tb.DTYPE_F32,
                                          acc_init=tb.ACC_INIT_LOAD_C))
    assert accum.kernel_name == "tb_gemm_gfx950_256x256x64_w2x2_s2_out2_16x16x32"


@pytest.mark.parametrize("kw,msg", [
    (dict(mfma=2), "TB_MFMA_"),
    (dict(mapping=tb.MAP_SPLIT_K, split_k=2, reduction=tb.RED_WORKSPACE,
          num_programs=512), "no split-K"),
    (dict(stages=3), "no gfx950 kernel instance.*16x16x32"),
    (dict(c_dtype=tb.DTYPE_F32, acc_init=tb.ACC_INIT_LOAD_C, mapping=tb.MAP_SPLIT_K,
          split_k=2, reduction=tb.RED_ATOMIC, num_programs=512), "no split-K"),
])
def test_mfma_16x16x32_validation(kw, msg):
    with pytest.raises(tb.TbError, match=msg):
        tb.GemmDesc.from_config(_wide(**kw))


@pytest.mark.parametrize("w", configs.ALL, ids=lambda w: w.name)
def test_every_workload_has_an_instance(w):
    d = tb.GemmDesc.from_config(w.direct_config())
    bm, bn, bk = w.block
    assert d.kernel_name.startswith(f"tb_gemm_gfx950_{bm}x{bn}x{bk}_")
    assert d.lds_bytes == w.stages * (bm + bn) * bk * 2
    if w.split_k > 1:
        assert d.workspace_bytes == w.split_k * w.M * w.N * 4
    else:
        assert d.workspace_bytes == 0


def _cfg(**kw):
    c = configs.SMOKE.direct_config()
    for k, v in kw.items():
        setattr(c, k, v)
    return c


@pytest.mark.parametrize("kw,msg", [
    (dict(m=0), "positive"),
    (dict(k=36, lda=36), "multiples of 8"),
    (dict(lda=16), "leading dimensions"),
    (dict(wave_grid_m=1), "wave grid"),
    (dict(block_m=48, num_programs=2), "no gfx950 kernel instance"),
    (dict(mapping=tb.MAP_SPLIT_K, split_k=1), "split_k >= 2"),
    (dict(mapping=tb.MAP_SPLIT_K, split_k=2, reduction=tb.RED_NONE), "reduction"),
    (dict(mapping=tb.MAP_SPLIT_K, split_k=2, reduction=tb.RED_ATOMIC), "f32 C"),
    (dict(acc_init=tb.ACC_INIT_LOAD_C), "f32 C"),
    (dict(num_programs=7), "launch formula"),
    (dict(mapping=9), "unknown mapping"),
    (dict(epi_bias=3), "epi_bias"),
    (dict(epi_activation=4), "epi_activation"),
    (dict(epi_clamp=4), "unknown bits"),
    (dict(epi_clamp=tb.CLAMP_MIN, clamp_min=float("inf")), "finite"),
    (dict(epi_clamp=tb.CLAMP_MIN | tb.CLAMP_MAX, clamp_min=1.0, clamp_max=0.0),
     "must not exceed"),
    (dict(epi_activation=tb.ACT_RELU, c_dtype=tb.DTYPE_F32, acc_init=tb.ACC_INIT_LOAD_C,
          mapping=tb.MAP_SPLIT_K, split_k=2, reduction=tb.RED_ATOMIC, num_programs=2),
     "whole sum"),
    # 32-bit buffer offsets: B whole under 2 GiB, a tile's rows of A and C under 1 GiB
    (dict(k=32768, lda=32768, n=32768, ldb=32768, ldc=32768, num_programs=0),
     "B larger than 2 GiB"),  # B = 2 GiB
    (dict(lda=1 << 23, num_programs=0), "a tile's rows"),  # 64 rows of A = 1 GiB
    (dict(ldc=1 << 23, num_programs=0), "a tile's rows"),  # 64 rows of C = 1 GiB
])
def test_descriptor_validation_errors(kw, msg):
    with pytest.raises(tb.TbError, match=msg):
        tb.GemmDesc.from_config(_cfg(**kw))


def test_operands_past_2gib_are_accepted():
    """A, C and the split-K workspace are addressed in per-tile windows, so
    they may exceed 2 GiB: a 2 GiB A, and eight 8192^2 f32 partial planes."""
    d = tb.GemmDesc.from_config(_cfg(m=32768, k=32768, lda=32768, num_programs=0))
    assert d.config.m == 32768
    sk = tb.GemmDesc.from_config(_cfg(m=8192, n=8192, ldb=8192, ldc=8192,
                                      mapping=tb.MAP_SPLIT_K, split_k=8,
                                      reduction=tb.RED_WORKSPACE, k=256, lda=256,
                                      num_programs=0))
    assert sk.workspace_bytes == 8 * 8192 * 8192 * 4


def test_launch_argument_errors_before_any_gpu_call():
    d = tb.GemmDesc.from_config(configs.SPLIT_K.direct_config())
    with pytest.raises(tb.TbError, match="device pointers"):
        d.launch(0, 0, 0)
    with pytest.raises(tb.TbError, match="workspace"):
        d.launch(16, 16, 16, None)
    for a, b, c in ((18, 16, 16), (16, 24, 16), (16, 16, 20)):
        with pytest.raises(tb.TbError, match="A, B and C must be 16-byte aligned"):
            d.launch(a, b, c, 256)
    with pytest.raises(tb.TbError, match="workspace must be 16-byte aligned"):
        d.launch(16, 16, 16, 264)


def test_fused_epilogue_instances_and_bias_arguments():
    """A fused config binds an `_epi` instance (split-K keeps the plain GEMM
    instance and fuses the steps into its reduction); the bias pointer is
    required exactly when the config adds one, and must be vector-aligned."""
    d = tb.GemmDesc.from_config(_cfg(epi_activation=tb.ACT_RELU))
    assert d.kernel_name.endswith("_epi")
    sk = configs.SPLIT_K.direct_config()
    sk.epi_bias = tb.EPI_BIAS_F32
    assert not tb.GemmDesc.from_config(sk).kernel_name.endswith("_epi")
    plain = tb.GemmDesc.from_config(_cfg())
    assert not plain.kernel_name.endswith("_epi")
    with pytest.raises(tb.TbError, match="no bias step"):
        plain.launch(16, 16, 16, bias=256)
    biased = tb.GemmDesc.from_config(_cfg(epi_bias=tb.EPI_BIAS_F32))
    with pytest.raises(tb.TbError, match="tb_gemm_launch_ex"):
        biased.launch(16, 16, 16)
    with pytest.raises(tb.TbError, match="16-byte aligned"):
        biased.launch(16, 16, 16, bias=260)
    with pytest.raises(tb.TbError, match="device pointers"):
        biased.launch(0, 0, 0, bias=256)


def test_bound_launcher_checks_like_launch():
    """GemmDesc.bind resolves the arguments once; its calls report the same
    argument errors as launch (checked before any GPU call)."""
    biased = tb.GemmDesc.from_config(_cfg(epi_bias=tb.EPI_BIAS_F32))
    with pytest.raises(tb.TbError, match="tb_gemm_launch_ex"):
        biased.bind(16, 16, 16)()
    with pytest.raises(tb.TbError, match="16-byte aligned"):
        biased.bind(16, 16, 16, bias=260)()
    plain = tb.GemmDesc.from_config(_cfg())
    with pytest.raises(tb.TbError, match="device pointers"):
        plain.bind(0, 16, 16)()


def test_tensor_operands_checked_against_the_descriptor():
    """GemmDesc.launch / bind check torch tensors before any GPU call: the
    element type, the bytes the descriptor touches from the tensor's address,
    a 2-D tensor's row-major layout, and the device (CPU tensors of the right
    type and size get as far as the device check)."""
    import torch
    w = configs.SMOKE  # 64 x 64 x 32, f16 C
    d = tb.GemmDesc.from_config(_cfg())
    A = torch.zeros(w.M, w.K, dtype=torch.float16)
    B = torch.zeros(w.K, w.N, dtype=torch.float16)
    C = torch.zeros(w.M, w.N, dtype=torch.float16)
    with pytest.raises(tb.TbError, match="C: expected a float16 tensor"):
        d.launch(A, B, C.float())
    with pytest.raises(tb.TbError, match="A: the descriptor touches 4096 bytes"):
        d.launch(torch.zeros(w.M // 2, w.K, dtype=torch.float16), B, C)
    with pytest.raises(tb.TbError, match="at least 64 x 32"):
        d.launch(A[: w.M // 2], B, C)  # a view: storage enough, shape short
    with pytest.raises(tb.TbError, match="B: expected a float16"):
        d.bind(A, B.to(torch.bfloat16), C)
    with pytest.raises(tb.TbError, match="row-major with leading dimension"):
        d.launch(A, B, C.t())
    with pytest.raises(tb.TbError, match="storage holds"):
        d.launch(A, B, C[1:])
    with pytest.raises(tb.TbError, match="must be on a GPU"):
        d.launch(A, B, C)
    # a flat buffer of enough bytes passes the size check
    with pytest.raises(tb.TbError, match="must be on a GPU"):
        d.launch(A, B, torch.zeros(w.M * w.N, dtype=torch.float16))
    biased = tb.GemmDesc.from_config(_cfg(epi_bias=tb.EPI_BIAS_F32))
    with pytest.raises(tb.TbError, match="bias: expected a float32"):
        biased.launch(A, B, C, bias=torch.zeros(w.N, dtype=torch.float16))
    with pytest.raises(tb.TbError, match="bias: the descriptor touches 256 bytes"):
        biased.launch(A, B, C, bias=torch.zeros(w.N - 4, dtype=torch.float32))
    sk = tb.GemmDesc.from_config(configs.SPLIT_K.direct_config())
    s = configs.SPLIT_K
    As = torch.zeros(s.M, s.K, dtype=torch.float16)
    Bs = torch.zeros(s.K, s.N, dtype=torch.float16)
    Cs = torch.zeros(s.M, s.N, dtype=torch.float16)
    short = torch.zeros(sk.workspace_bytes // 4 - 1, dtype=torch.float32)
    with pytest.raises(tb.TbError, match="workspace: the descriptor touches"):
        sk.launch(As, Bs, Cs, short)


def test_descriptors_and_errors_from_many_threads():
    """Descriptor creation and the plan pipeline run concurrently from host
    threads (ctypes releases the GIL for the library's calls), and each
    thread reads its own error message: tb_last_error is thread-local. Every
    thread alternates a valid descriptor, a plan, and a refusal whose message
    is specific to that thread."""
    import threading
    bad = [(dict(wave_grid_m=1), "wave grid"), (dict(lda=16), "leading dimensions"),
           (dict(num_programs=7), "launch formula"), (dict(epi_bias=3), "epi_bias"),
           (dict(k=36, lda=36), "multiples of 8"), (dict(mapping=9), "unknown mapping"),
           (dict(epi_clamp=4), "unknown bits"), (dict(m=0), "positive")]
    good_name = tb.GemmDesc.from_config(_cfg()).kernel_name
    mlir = configs.RAGGED.mlir()
    plan_name = tb.plan_from_mlir(mlir).kernel_name
    failures = []

    def worker(i):
        kw, msg = bad[i % len(bad)]
        try:
            for _ in range(40):
                assert tb.GemmDesc.from_config(_cfg()).kernel_name == good_name
                try:
                    tb.GemmDesc.from_config(_cfg(**kw))
                    failures.append(f"thread {i}: no error for {kw}")
                except tb.TbError as e:
                    if msg not in str(e):
                        failures.append(f"thread {i}: expected '{msg}', got '{e}'")
                assert tb.plan_from_mlir(mlir).kernel_name == plan_name
        except Exception as e:  # noqa: BLE001 - reported below
            failures.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not failures, "\n".join(failures[:10])


def test_small_tile_profile_problems_bind():
    """Every single-tile problem of `profiling --small-tiles` (the command of
    the committed small-tile kernel trace) binds its instance in each output
    mode, on the MFMA shape it names."""
    from mini_triton_nvgpu_v1_amd import profiling
    for (M, N, K, bm, bn, bk, gm, gn, m16) in profiling.SMALL_TILES:
        for out in (0, 1, 2):
            d = tb.GemmDesc.from_config(tb.GemmConfig(
                m=M, n=N, k=K, lda=K, ldb=N, ldc=N,
                c_dtype=tb.DTYPE_F16 if out == 0 else tb.DTYPE_F32,
                acc_init=tb.ACC_INIT_LOAD_C if out == 2 else tb.ACC_INIT_ZERO,
                block_m=bm, block_n=bn, block_k=bk, num_waves=gm * gn, wave_grid_m=gm,
                wave_grid_n=gn, stages=2, mapping=tb.MAP_TILE, group_m=1, split_k=1,
                reduction=tb.RED_NONE, num_programs=1, xcd_remap=0,
                mfma=tb.MFMA_16X16X32 if m16 else tb.MFMA_32X32X16))
            assert d.kernel_name.endswith(f"_out{out}" + ("_16x16x32" if m16 else "")), \
                d.kernel_name
