"""Plan pipeline (tb-opt and tb_plan_from_mlir) on the CPU.

Covers: the IR text as a lossless checkpoint (pass-by-pass runs through
separate tb-opt processes equal one pipeline run; print/parse round trips),
agreement of the contract lowering with the runtime's kernel binding and
with the workloads' direct configurations, the diagnostics of every
legality rule, and the contract verifier catching a tampered mainline.
"""
import pathlib
import re
import subprocess

import pytest

import mini_triton_nvgpu_v1_amd as tb
from mini_triton_nvgpu_v1_amd import configs

ROOT = pathlib.Path(__file__).resolve().parent.parent
TB_OPT = ROOT / "mini_triton_nvgpu_v1_amd" / "bin" / "tb-opt"

STAGE1_PASSES = [
    "tb-verify-scope", "tb-attach-target-info{gpu-arch=gfx950}",
    "tb-semanticize-matmul", "tb-build-program-mapping-plan",
    "tb-build-layout-plan", "tb-build-transport-plan",
    "tb-build-c-register-plan", "tb-rewrite-matmul-mainloop",
    "tb-cleanup-layout-conversions", "tb-build-mainloop-graph",
    "tb-regularize-k-loop", "tb-assign-latencies", "tb-schedule-loops",
    "tb-derive-waits", "tb-expand-pipeline", "tb-cleanup-pipeline",
    "tb-verify-pipeline-mainline-contract"]
FULL = "builtin.module(tb-stage1-full-to-gfx950-pipeline{cubin-chip=gfx950})"
MAINLINE = "builtin.module(" + ",".join(STAGE1_PASSES) + ")"


def tb_opt(text, *args, check=True):
    if not TB_OPT.exists():
        pytest.fail("bin/tb-opt is not built (run __graft_entry__.build())")
    p = subprocess.run([str(TB_OPT), "-", *args], input=text,
                       capture_output=True, text=True, timeout=120)
    if check and p.returncode != 0:
        raise AssertionError(f"tb-opt {args} failed:\n{p.stderr}")
    return p


def matmul_module(M=64, N=64, K=32, bm=64, bn=64, bk=32, warps=4, stages=2,
                  c="f16", exact=True, extra_module="", extra_op=""):
    ex = "true" if exact else "false"
    return (
        f'module attributes {{"tb.num-warps" = {warps} : i64, '
        f'"tb.requested-stages" = {stages} : i64{extra_module}}} {{\n'
        f"  func.func @kernel(%A: memref<{M}x{K}xf16>, %B: memref<{K}x{N}xf16>,"
        f" %C: memref<{M}x{N}x{c}>) {{\n"
        f"    tb.matmul %A, %B, %C {{block_m = {bm} : i64, block_n = {bn} : i64,"
        f" block_k = {bk} : i64, exact_tile = {ex}{extra_op}}}\n"
        f"      : memref<{M}x{K}xf16>, memref<{K}x{N}xf16>, memref<{M}x{N}x{c}>\n"
        f"    func.return\n  }}\n}}\n")


@pytest.mark.parametrize("w", configs.ALL, ids=lambda w: w.name)
def test_pass_by_pass_equals_pipeline(w):
    """Every pass re-reads its inputs from the IR text: running the passes
    one process at a time gives exactly the one-shot pipeline's output."""
    text = w.mlir()
    for p in STAGE1_PASSES:
        text = tb_opt(text, f"--pass-pipeline=builtin.module({p})").stdout
    one_shot = tb_opt(w.mlir(), f"--pass-pipeline={MAINLINE}").stdout
    assert text == one_shot
    assert "tb.pipeline_mainline" in text and "tb.matmul " not in text


@pytest.mark.parametrize("w", configs.ALL, ids=lambda w: w.name)
def test_print_parse_roundtrip(w):
    sealed = tb_opt(w.mlir(), f"--pass-pipeline={MAINLINE}").stdout
    assert tb_opt(sealed).stdout == sealed
    lowered = tb_opt(w.mlir(), f"--pass-pipeline={FULL}").stdout
    assert tb_opt(lowered).stdout == lowered


@pytest.mark.parametrize("w", configs.ALL, ids=lambda w: w.name)
def test_plan_config_matches_direct_config(w):
    plan = tb.plan_from_mlir(w.mlir()).config
    direct = w.direct_config()
    for f, _ in type(plan)._fields_:
        assert getattr(plan, f) == getattr(direct, f), f


@pytest.mark.parametrize("w", configs.ALL, ids=lambda w: w.name)
def test_lowering_names_the_bound_kernel(w, tmp_path):
    lowered = tb_opt(w.mlir(), f"--pass-pipeline={FULL}").stdout
    name = re.search(r'kernel = "([^"]+)"', lowered).group(1)
    desc = tb.plan_from_mlir(w.mlir())
    assert desc.kernel_name == name
    lds = int(re.search(r"lds_bytes = (\d+)", lowered).group(1))
    assert desc.lds_bytes == lds
    ws = int(re.search(r"workspace_bytes = (\d+)", lowered).group(1))
    assert desc.workspace_bytes == ws
    # the lowered module and the sealed mainline both load as plan files
    f = tmp_path / "lowered.mlir"
    f.write_text(lowered)
    assert tb.plan_from_file(str(f)).config == desc.config
    g = tmp_path / "sealed.mlir"
    g.write_text(tb_opt(w.mlir(), f"--pass-pipeline={MAINLINE}").stdout)
    assert tb.plan_from_file(str(g)).config == desc.config


def test_schedule_window_is_bounded():
    """The buffer model covers min(k groups, stages + 1) groups, so the host
    work does not grow with K (4096 and 8192 share the same plan size)."""
    sizes = {}
    for w in (configs.ROOFLINE, configs.PERSISTENT):
        text = tb_opt(w.mlir(), f"--pass-pipeline={MAINLINE}").stdout
        window = min(-(-w.K // w.block[2]), w.stages + 1)
        assert text.count("tb.async_issue_cluster") == window
        assert text.count("tb.consumer_wait_cluster") == window
        assert text.count("tb.mma_compute_cluster") == window
        assert f"iteration_count = {-(-w.K // w.block[2])}" not in text  # loop plan dropped
        sizes[w.name] = len(text)
    assert abs(sizes["gemm_4096"] - sizes["persistent_8192"]) < 4096


def test_cluster_order_refills_after_reads():
    """Within a time slot the waits and MFMAs of the consumed group come
    before the refill of its ring slot (clusters 0, 1, 2)."""
    text = tb_opt(configs.ROOFLINE.mlir(), f"--pass-pipeline={MAINLINE}").stdout
    body = re.findall(r"tb\.(async_issue|consumer_wait|mma_compute)_cluster "
                      r"\{cluster = (\d+) : i64, k_group = (\d+) : i64.*?"
                      r"stage = (\d+) : i64", text)
    S = configs.ROOFLINE.stages
    seen = [(int(st), int(cl), k, int(g)) for k, cl, g, st in body]
    assert seen == sorted(seen)
    for st, cl, kind, g in seen:
        if kind == "async_issue":
            assert (st, cl) == (g, 2)
        else:
            assert st == g + S and cl == (0 if kind == "consumer_wait" else 1)


ERRORS = [
    ("sm86", matmul_module(), "--tb-attach-target-info=gpu-arch=sm_86",
     "supports gpu-arch `gfx950`"),
    ("no_arch", matmul_module(), "--tb-attach-target-info",
     "requires explicit `gpu-arch`"),
    ("block_m_48", matmul_module(M=96, bm=48, exact=False), FULL,
     "block_m % 32 == 0"),
    ("block_k_16", matmul_module(bk=16), FULL, "block_k in {32, 64}"),
    ("inexact", matmul_module(M=96), FULL, "exact_tile=true requires"),
    ("stages_5", matmul_module(stages=5), FULL, "num_stages in [2, 4]"),
    ("lds_budget", matmul_module(M=256, N=256, K=64, bm=256, bn=256, bk=64,
                                 stages=4), FULL, "exceed the target LDS budget"),
    ("persistent_splitk", matmul_module(
        K=64, extra_module=', "tb.persistent" = true, "tb.split-k" = 2 : i64'),
     FULL, "persistent and split-k"),
    ("bad_reduction", matmul_module(
        K=64, extra_module=', "tb.split-k" = 2 : i64, "tb.reduction-mode" = "tree"'),
     FULL, "must be `split_k_serial` or `split_k_parallel`"),
    ("atomic_f16", matmul_module(
        K=64, extra_module=', "tb.split-k" = 2 : i64, '
        '"tb.reduction-mode" = "split_k_parallel"'),
     FULL, "needs an f32 C"),
    ("wave_grid", matmul_module(warps=3), FULL, "legal wave grid"),
    ("mfma16_small_tile", matmul_module(extra_op=', mma = "mfma_f32_16x16x32_f16"'),
     FULL, "implemented for the 4-wave 256x256x64 2-stage tile"),
    ("mfma16_split_k", matmul_module(
        M=256, N=256, K=256, bm=256, bn=256, bk=64,
        extra_module=', "tb.split-k" = 2 : i64',
        extra_op=', mma = "mfma_f32_16x16x32_f16"'),
     FULL, "has no split-k instance"),
    ("bad_mma", matmul_module(extra_op=', mma = "mfma_f64"'), FULL, "mma"),
    ("f32_a", matmul_module().replace("memref<64x32xf16>", "memref<64x32xf32>"),
     FULL, "fp16 x fp16"),
    ("n_not_8", matmul_module(N=68, exact=False), FULL, "multiples of 8"),
    ("out_of_order", matmul_module(), "--tb-build-layout-plan", "tb.target"),
    ("unknown_pass", matmul_module(), "--tb-frobnicate", "unknown pass"),
    ("bad_ir", "module {", FULL, "parse error"),
]


@pytest.mark.parametrize("name,text,arg,msg", ERRORS, ids=[e[0] for e in ERRORS])
def test_diagnostics(name, text, arg, msg):
    args = [f"--pass-pipeline={arg}"] if arg.startswith("builtin") else [arg]
    p = tb_opt(text, *args, check=False)
    assert p.returncode == 1, p.stdout[:500]
    assert msg in p.stderr, p.stderr


@pytest.mark.parametrize("name,text,arg,msg",
                         [e for e in ERRORS if e[2] == FULL],
                         ids=[e[0] for e in ERRORS if e[2] == FULL])
def test_plan_from_mlir_diagnostics(name, text, arg, msg):
    with pytest.raises(tb.TbError, match=re.escape(msg)):
        tb.plan_from_mlir(text)


def test_mfma_instruction_choice():
    """Without an `mma` attribute the plan takes 16x16x32 exactly where that
    instance exists: the 4-wave 256x256x64 2-stage f16 tile on whole tiles
    without split-K. The EncodingPlan records the instruction shape."""
    def launch(text):
        return tb.plan_from_mlir(text)
    wide = dict(M=512, N=768, K=192, bm=256, bn=256, bk=64)
    assert launch(matmul_module(**wide)).config.mfma == tb.MFMA_16X16X32
    for kw in (dict(wide, warps=8), dict(wide, bk=32), dict(wide, c="f32"),
               dict(wide, M=520, exact=False),
               dict(wide, extra_module=', "tb.split-k" = 3 : i64'),
               dict(wide, extra_op=', mma = "mfma_f32_32x32x16_f16"'), {}):
        assert launch(matmul_module(**kw)).config.mfma == tb.MFMA_32X32X16, kw
    text = tb_opt(matmul_module(**wide), f"--pass-pipeline={MAINLINE}").stdout
    assert "instrShape = [16, 16, 32]" in text
    text = tb_opt(matmul_module(), f"--pass-pipeline={MAINLINE}").stdout
    assert "instrShape = [32, 32, 16]" in text


def test_verifier_catches_tampering():
    sealed = tb_opt(configs.ROOFLINE.mlir(), f"--pass-pipeline={MAINLINE}").stdout
    verify = "--tb-verify-pipeline-mainline-contract"
    assert tb_opt(sealed, verify).returncode == 0
    n = len(re.findall(r"tb\.async_issue_cluster", sealed))
    bad = sealed.replace(f"async_groups = {n} : i64", f"async_groups = {n + 1} : i64")
    p = tb_opt(bad, verify, check=False)
    assert p.returncode == 1 and "async_groups" in p.stderr
    # a refill scheduled before the last read of its slot
    bad = re.sub(r"(tb\.async_issue_cluster \{cluster = )2", r"\g<1>0", sealed, count=4)
    p = tb_opt(bad, verify, check=False)
    assert p.returncode == 1 and "contract" in p.stderr
    # the lowering refuses an LDS encoding the kernels do not implement
    bad = sealed.replace("perPhase = 2, maxPhase = 8", "perPhase = 1, maxPhase = 8")
    assert bad != sealed
    p = tb_opt(bad, "--tb-lower-pipeline-to-gfx950", check=False)
    assert p.returncode == 1 and "swizzle" in p.stderr


def test_cleanup_layout_conversions():
    text = (
        'module attributes {"tb.num-warps" = 4 : i64, "tb.requested-stages" = 2 : i64} {\n'
        "  func.func @kernel(%A: memref<64x32xf16>, %B: memref<32x64xf16>, %C: memref<64x64xf16>) {\n"
        "    %0 = tb.convert_layout %A : (memref<64x32xf16>) -> memref<64x32xf16>\n"
        "    %1 = tb.convert_layout %B : (memref<32x64xf16>) -> memref<32x64xf16, strided<[64, 1]>>\n"
        "    %2 = tb.convert_layout %1 : (memref<32x64xf16, strided<[64, 1]>>) -> memref<32x64xf16>\n"
        "    %3 = tb.convert_layout %C : (memref<64x64xf16>) -> memref<64x64xf16, strided<[64, 1]>>\n"
        "    tb.matmul %0, %2, %C {block_m = 64 : i64, block_n = 64 : i64, block_k = 32 : i64, exact_tile = true} : memref<64x32xf16>, memref<32x64xf16>, memref<64x64xf16>\n"
        "    return\n  }\n}\n")
    out = tb_opt(text, "--tb-cleanup-layout-conversions").stdout
    assert "tb.convert_layout" not in out
    assert "tb.matmul %A, %B, %C" in out


def _listed_instances():
    """tb-opt --list-instances: name -> (issue schedule, vmcnt prologue,
    vmcnt loop, lgkmcnt loop) from the host-side table."""
    p = subprocess.run([str(TB_OPT), "--list-instances"], capture_output=True,
                       text=True, timeout=60, check=True)
    out = {}
    for line in p.stdout.splitlines():
        name, issue, *kv = line.split()
        vals = dict(x.split("=") for x in kv)
        assert name not in out
        out[name] = (issue, int(vals["vmcnt_prologue"]), int(vals["vmcnt_loop"]),
                     int(vals["lgkmcnt_loop"]))
    return out


def _compiled_waits():
    """The registry of libtb_gfx950.so: name -> the s_waitcnt depths compiled
    into the kernel (the kernel template's own constants)."""
    import ctypes
    L = tb.lib()
    L.tb_kernel_waits.argtypes = [ctypes.c_int] + [ctypes.POINTER(ctypes.c_int32)] * 3
    out = {}
    for i, name in enumerate(tb.kernel_names()):
        v = [ctypes.c_int32() for _ in range(3)]
        assert L.tb_kernel_waits(i, *[ctypes.byref(x) for x in v]) == 0
        out[name] = tuple(x.value for x in v)
    return out


def test_tb_opt_instance_table_equals_the_kernel_registry():
    """tb-opt carries the instance table without the kernels; it lists
    exactly the instances compiled into libtb_gfx950.so, by the same names,
    and states for each the waits the kernel's own constants compile in
    (vmcnt at the prologue, vmcnt and lgkmcnt at the per-k-tile barrier)."""
    listed, compiled = _listed_instances(), _compiled_waits()
    assert sorted(listed) == sorted(compiled)
    for name, (issue, vmp, vml, lgkm) in listed.items():
        assert (vmp, vml, lgkm) == compiled[name], (name, issue)
    # the three issue schedules all occur, and differ in the prologue wait
    assert {v[0] for v in listed.values()} == {"slot_spread", "burst", "exact_tile_slots"}
    assert listed["tb_gemm_gfx950_256x256x64_w4x2_s2_out0"][1:] == (4, 0, -1)
    assert listed["tb_gemm_gfx950_128x64x64_w4x1_s3_out1"][:2] == ("burst", 12)
    assert listed["tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32"][1:] == (16, 0, 0)
    L = tb.lib()
    import ctypes
    x = ctypes.c_int32()
    assert L.tb_kernel_waits(-1, ctypes.byref(x), ctypes.byref(x), ctypes.byref(x)) != 0
    assert L.tb_kernel_waits(len(compiled), ctypes.byref(x), ctypes.byref(x),
                             ctypes.byref(x)) != 0


def _async_waits(text):
    """The sealed mainline's tb.async_plan: (issue_schedule, loads_per_thread,
    prologue_tail_loads, [(group, vmcnt, lgkmcnt), ...]) read from the IR."""
    out = tb_opt(text, f"--pass-pipeline={MAINLINE}").stdout
    body = out[out.index("tb.async_plan"):]
    issue = re.search(r'issue_schedule = "(\w+)"', body).group(1)
    lpt = int(re.search(r"loads_per_thread = (\d+)", body).group(1))
    tail = int(re.search(r"prologue_tail_loads = (\d+)", body).group(1))
    waits = [(int(g), int(vm), int(lg)) for g, lg, vm in re.findall(
        r"group_id = (\d+) : i64, lgkmcnt_allowance = (-?\d+) : i64.*?"
        r"vmcnt_allowance = (\d+) : i64", body)]
    return issue, lpt, tail, waits


@pytest.mark.parametrize("w", configs.ALL, ids=lambda w: w.name)
def test_async_plan_states_the_bound_kernels_waits(w):
    """The AsyncPlan's waits are those compiled into the kernel the plan
    binds: vmcnt at the prologue (k group 0), vmcnt at every later barrier,
    lgkmcnt there (reference: the lowering emits the AsyncPlan's waits,
    LowerPipelineToNVGPU.cpp:2279-2294)."""
    issue, lpt, tail, waits = _async_waits(w.mlir())
    assert waits and waits[0][0] == 0
    name = tb.plan_from_mlir(w.mlir()).kernel_name
    vmp, vml, lgkm = _compiled_waits()[name]
    assert _listed_instances()[name][0] == issue
    for g, vm, lg in waits:
        assert vm == (vmp if g == 0 else vml), (name, g, vm)
        assert lg == lgkm, (name, g, lg)
    assert vmp == (w.stages - 2) * lpt + tail


def test_lowering_refuses_waits_that_differ_from_the_kernel():
    """A sealed mainline whose AsyncPlan states another wait depth than the
    instance it binds is refused by the lowering, as is one whose lowered
    launch op carries waits the compiled kernel does not have."""
    w = configs.ROOFLINE
    sealed = tb_opt(w.mlir(), f"--pass-pipeline={MAINLINE}").stdout
    tampered = re.sub(r"vmcnt_allowance = 16 : i64", "vmcnt_allowance = 8 : i64", sealed,
                      count=1)
    assert tampered != sealed
    p = tb_opt(tampered, "--tb-lower-pipeline-to-gfx950", check=False)
    assert p.returncode == 1 and "AsyncPlan vmcnt of the wait for k group 0 (8)" in p.stderr
    with pytest.raises(tb.TbError, match="AsyncPlan vmcnt"):
        tb.plan_from_mlir(tampered)
    lowered = tb_opt(sealed, "--tb-lower-pipeline-to-gfx950").stdout
    assert "waits = array<i64: 16, 0, 0>" in lowered
    bad = lowered.replace("waits = array<i64: 16, 0, 0>", "waits = array<i64: 16, 0, -1>")
    with pytest.raises(tb.TbError, match="differ from the compiled kernel"):
        tb.plan_from_mlir(bad)


# every block shape with an instance list, 1 to 8 waves, 2 to 4 stages,
# block_k 32 and 64, f16 and f32 C, plus shapes with no list at all
SWEEP_BLOCKS = [(64, 64), (64, 128), (128, 64), (128, 128), (64, 256), (256, 64),
                (128, 256), (256, 128), (256, 256), (192, 128), (96, 64), (160, 96)]


@pytest.mark.parametrize("bm,bn", SWEEP_BLOCKS, ids=lambda v: str(v))
def test_no_plan_legal_configuration_lacks_a_kernel(bm, bn):
    """The plan either refuses a configuration (with a diagnostic) or binds
    it to a compiled kernel: nothing that passes the plan pipeline and its
    lowering fails at tb_desc_create for want of an instance. The lowering
    names exactly the instance the runtime binds."""
    bound = 0
    for bk in (32, 64):
        for warps in (1, 2, 4, 8):
            for stages in (2, 3, 4):
                for c in ("f16", "f32"):
                    M = N = 768 if max(bm, bn) <= 256 else 1536
                    text = matmul_module(M=M, N=N, K=256, bm=bm, bn=bn, bk=bk,
                                         warps=warps, stages=stages, c=c,
                                         exact=M % bm == 0 and N % bn == 0)
                    try:
                        d = tb.plan_from_mlir(text)
                    except tb.TbError as e:
                        msg = str(e)
                        # a plan refusal names the pass; the runtime's own
                        # "no gfx950 kernel instance for tile" must not occur
                        assert re.match(r"tb_plan_from_mlir: tb-[a-z0-9-]+: ", msg), msg
                        continue
                    bound += 1
                    cfg = d.config
                    grid = configs.wave_grid(bm, bn, warps)
                    assert (cfg.wave_grid_m, cfg.wave_grid_n) == grid
                    assert d.kernel_name.startswith(
                        f"tb_gemm_gfx950_{bm}x{bn}x{bk}_w{grid[0]}x{grid[1]}_s{stages}_")
    if (bm, bn) not in ((96, 64), (160, 96)):
        assert bound > 0
