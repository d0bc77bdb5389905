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


@pytest.mark.parametrize("w", configs.ALL + configs.F32_ACCUMULATE, ids=lambda w: w.name)
def test_plan_config_matches_direct_config(w):
    plan = tb.plan_from_mlir(w.mlir()).config
    direct = w.direct_config()
    for f, _ in type(plan)._fields_:
        assert getattr(plan, f) == getattr(direct, f), f


@pytest.mark.parametrize("w", configs.ALL + configs.F32_ACCUMULATE, ids=lambda w: w.name)
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
     FULL, "has no gfx950 kernel instance for this block"),
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
    instance exists: the hand-scheduled 4-wave 256x256x64 2-stage tile and
    the 16x16x32 loop's tiles (here 4 waves on 128x128 and 256x128, 2 on
    256x128), with an f16 C or an f32 C (C += A*B, the reference's
    semantics), M, N and K possibly ragged, without split-K. Elsewhere it
    takes 32x32x16, and it refuses a 32x32x16 build that spills. The
    EncodingPlan records the instruction shape."""
    def launch(text):
        return tb.plan_from_mlir(text)
    wide = dict(M=512, N=768, K=192, bm=256, bn=256, bk=64)
    assert launch(matmul_module(**wide)).config.mfma == tb.MFMA_16X16X32
    for kw in (dict(wide, M=520, N=200, exact=False), dict(wide, K=200, exact=False),
               dict(wide, c="f32"), dict(wide, c="f32", M=520, K=200, exact=False),
               dict(wide, bm=128, bn=128), dict(wide, bn=128, bk=32, stages=3),
               dict(wide, bn=128, warps=2), dict(wide, bm=128, bn=128, warps=1),
               dict(wide, bk=32)):
        assert launch(matmul_module(**kw)).config.mfma == tb.MFMA_16X16X32, kw
    f32 = tb.plan_from_mlir(matmul_module(**dict(wide, c="f32")))
    assert f32.kernel_name == "tb_gemm_gfx950_256x256x64_w2x2_s2_out2_16x16x32"
    for kw in (dict(wide, warps=8),
               dict(wide, extra_module=', "tb.split-k" = 3 : i64'),
               dict(wide, c="f32", extra_module=', "tb.split-k" = 2 : i64, '
                    '"tb.reduction-mode" = "split_k_parallel"'), {}):
        assert launch(matmul_module(**kw)).config.mfma == tb.MFMA_32X32X16, kw
    # 32x32x16 builds of 128x128 wave tiles spill: refused at KernelConfig
    # legality with the compiler's figures (4 waves on 256x256x32 take the
    # 16x16x32 loop's build above; asked for 32x32x16 they are refused)
    for kw in (dict(wide, bk=32, extra_op=', mma = "mfma_f32_32x32x16_f16"'),
               dict(wide, extra_op=', mma = "mfma_f32_32x32x16_f16"')):
        with pytest.raises(tb.TbError, match=r"tb-build-program-mapping-plan: .* spills"):
            launch(matmul_module(**kw))
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
    # a refill moved in front of the reads of its slot: the op verifier
    # (TBOps.cpp:253-258) refuses the clusters' order as the module is read
    bad = re.sub(r"(tb\.async_issue_cluster \{cluster = )2", r"\g<1>0", sealed, count=4)
    p = tb_opt(bad, verify, check=False)
    assert p.returncode == 1 and "clusters must stay ordered by stage/cluster" in p.stderr
    # the lowering refuses an LDS encoding the kernels do not implement
    bad = sealed.replace("perPhase = 2, maxPhase = 8", "perPhase = 1, maxPhase = 8")
    assert bad != sealed
    p = tb_opt(bad, "--tb-lower-pipeline-to-gfx950", check=False)
    assert p.returncode == 1 and "swizzle" in p.stderr


CGA = "#tb.cga<ctasPerCGA = [1, 1, 1], ctaSplitNum = [1, 1, 1], ctaOrder = [0, 1, 2]>"


def _memdesc(order, shape=(64, 32), space="global", alloc=None):
    enc = (f"#tb.blocked<sizePerThread = [1, 1], threadsPerWarp = [32, 1], "
           f"warpsPerCTA = [1, 1], order = [{order}], cga = {CGA}>")
    alloc = alloc or shape
    return (f"!tb.memdesc<shape = [{shape[0]}, {shape[1]}], elementType = f16, "
            f"encoding = {enc}, memorySpace = \"{space}\", mutableMemory = true, "
            f"allocShape = [{alloc[0]}, {alloc[1]}]>")


def test_cleanup_layout_conversions():
    """tb-cleanup-layout-conversions (CleanupLayoutConversions.cpp:21-54)
    folds a conversion back to its source's source: row -> col -> row is the
    source itself (the reference's examples/layout_convert_roundtrip.mlir),
    and a dead conversion goes away; a conversion to another layout stays."""
    row, col = _memdesc("1, 0"), _memdesc("0, 1")
    text = (
        "module {\n"
        f"  func.func @f(%src: {row}) -> {col} {{\n"
        f"    %0 = tb.convert_layout %src : ({row}) -> {col}\n"
        f"    %1 = tb.convert_layout %0 : ({col}) -> {row}\n"
        f"    %2 = tb.convert_layout %1 : ({row}) -> {col}\n"
        f"    %3 = tb.convert_layout %src : ({row}) -> {col}\n"
        f"    return %2 : {col}\n  }}\n}}\n")
    out = tb_opt(text, "--tb-cleanup-layout-conversions").stdout
    assert out.count("tb.convert_layout") == 1, out
    assert "%2 = tb.convert_layout %src" in out and "return %2" in out
    ex = ROOT.parent / "reference" / "examples" / "layout_convert_roundtrip.mlir"
    if ex.exists():  # the reference's example, where this container has it
        out = tb_opt(ex.read_text(), "--tb-cleanup-layout-conversions").stdout
        assert "tb.convert_layout" not in out and "return %src" in out


SHARED_OK = ("#tb.shared<order = [1, 0], perPhase = 1, maxPhase = 4, transposed = false, "
             f"swizzlingByteWidth = 64, cga = {CGA}>")
# (name, module text, expected diagnostic): each attribute, type and op rule of
# the reference's verifiers (TBAttrs.cpp:47-195, TBTypes.cpp:16-46,
# TBOps.cpp:16-60, :128-182), plus the gfx950 second XOR term.
IR_ERRORS = [
    ("shared_negative_phase",
     SHARED_OK.replace("perPhase = 1, maxPhase = 4", "perPhase = 0, maxPhase = -3"),
     "per_phase and max_phase must be non-negative"),
    ("shared_negative_width",
     SHARED_OK.replace("swizzlingByteWidth = 64", "swizzlingByteWidth = -7"),
     "swizzling_byte_width must be non-negative"),
    ("shared_no_cga",
     SHARED_OK.replace(f", cga = {CGA}", ""), "expected parameter `cga`"),
    ("shared_bad_order", SHARED_OK.replace("order = [1, 0]", "order = [1, 1]"),
     "order must not contain duplicates"),
    ("shared_empty_order", SHARED_OK.replace("order = [1, 0]", "order = []"),
     "shared encoding must have non-empty order"),
    ("shared_padding_rank",
     SHARED_OK[:-1] + ", paddingIntervals = [32, 32], paddings = [8]>",
     "padding_intervals and paddings must have same rank"),
    ("shared_second_term_too_wide",
     SHARED_OK[:-1] + ", secondPerPhase = 8, secondMaxPhase = 4, secondSwizzlingByteWidth = 32>",
     "second XOR term must permute whole 16-byte chunks"),
    ("cga_rank", CGA.replace("ctaOrder = [0, 1, 2]", "ctaOrder = [0, 1]"),
     "cga encoding must carry rank-3"),
    ("cga_positive", CGA.replace("ctasPerCGA = [1, 1, 1]", "ctasPerCGA = [1, 0, 1]"),
     "ctas_per_cga entries must be positive"),
    ("blocked_rank",
     f"#tb.blocked<sizePerThread = [1, 4], threadsPerWarp = [32], warpsPerCTA = [1, 1], "
     f"order = [1, 0], cga = {CGA}>", "size_per_thread/threads_per_warp rank mismatch"),
    ("semantic_contiguous",
     "#tb.semantic_layout<order = [1, 0], strides = [64, 1], zeroOffset = true, "
     "hasStaticStrides = true, unitStrideOnMinor = false, contiguous = true>",
     "contiguous=true requires unitStrideOnMinor=true"),
    ("semantic_static_strides",
     "#tb.semantic_layout<order = [1, 0], strides = [64, 0], zeroOffset = true, "
     "hasStaticStrides = true, unitStrideOnMinor = true, contiguous = true>",
     "static strides must be positive"),
    ("mfma_instr_rank",
     f"#tb.amd_mfma<versionMajor = 4, versionMinor = 0, warpsPerCTA = [2, 2], "
     f"instrShape = [32, 32], isTransposed = true, cga = {CGA}>",
     "instr_shape must have rank 3"),
    ("dot_operand_index",
     f"#tb.dot_operand<operandIndex = 2, parent = #tb.amd_mfma<versionMajor = 4, "
     f"versionMinor = 0, warpsPerCTA = [2, 2], instrShape = [32, 32, 16], "
     f"isTransposed = true, cga = {CGA}>, kWidth = 8>", "operand_index must be 0 or 1"),
    ("unknown_attr", "#tb.swizzled<order = [1, 0]>", "unknown tb attribute `#tb.swizzled`"),
]


@pytest.mark.parametrize("name,attr,msg", IR_ERRORS, ids=[e[0] for e in IR_ERRORS])
def test_ir_attribute_verifiers(name, attr, msg):
    """A malformed #tb attribute is refused when the module is read, by
    tb-opt and by tb_plan_from_mlir, with the reference's diagnostic."""
    text = f"#bad = {attr}\n" + matmul_module()
    p = tb_opt(text, "--tb-verify-scope", check=False)
    assert p.returncode == 1 and msg in p.stderr, p.stderr
    with pytest.raises(tb.TbError, match=re.escape(msg)):
        tb.plan_from_mlir(text)


def test_ir_type_and_op_verifiers():
    """!tb.memdesc (TBTypes.cpp:16-46) and the ops (TBOps.cpp): shapes,
    memory spaces, conversion legality, matmul operands and attributes."""
    row, col = _memdesc("1, 0"), _memdesc("0, 1")
    cases = [
        (_memdesc("1, 0", space="local"), "memory_space must be one of global/shared/registers"),
        (_memdesc("1, 0", alloc=(64, 0)), "alloc_shape dimensions must be positive"),
        (row.replace("#tb.blocked<sizePerThread = [1, 1], threadsPerWarp = [32, 1], "
                     "warpsPerCTA = [1, 1], order = [1, 0]", "#tb.shared<order = [1, 0], "
                     "perPhase = 1, maxPhase = 1, transposed = false, swizzlingByteWidth = 16")
                .replace(f", cga = {CGA}>, memorySpace", f", cga = {CGA}>, memorySpace"),
         "shared encoding requires shared memory_space"),
    ]
    for ty, msg in cases:
        text = f"module {{\n  func.func @f(%x: {ty}) {{\n    return\n  }}\n}}\n"
        p = tb_opt(text, "--tb-cleanup-layout-conversions", check=False)
        assert p.returncode == 1 and msg in p.stderr, (msg, p.stderr)
    convs = [
        (row, row, "layout conversion must change encoding or alloc_shape"),
        (row, _memdesc("0, 1", shape=(32, 64)), "logical shapes must match"),
        (row, _memdesc("0, 1", space="shared"), "memory spaces must match"),
    ]
    for src, dst, msg in convs:
        text = (f"module {{\n  func.func @f(%x: {src}) {{\n"
                f"    %0 = tb.convert_layout %x : ({src}) -> {dst}\n    return\n  }}\n}}\n")
        p = tb_opt(text, "--tb-cleanup-layout-conversions", check=False)
        assert p.returncode == 1 and msg in p.stderr, (msg, p.stderr)
    text = matmul_module().replace("tb.convert_layout", "")
    ops = [
        (text.replace("block_m = 64", "block_m = 0"), "block sizes must be positive"),
        (text.replace("exact_tile = true", "exact_tile = true, group_m = 0 : i64"),
         "group_m must be positive"),
        (text.replace("%C: memref<64x64xf16>", "%C: memref<64x64xbf16>")
             .replace("memref<64x64xf16>\n", "memref<64x64xbf16>\n"),
         "expected fp16 x fp16 -> fp32"),
        (text.replace("%B: memref<32x64xf16>", "%B: memref<16x64xf16>")
             .replace(", memref<32x64xf16>,", ", memref<16x64xf16>,"),
         "expected A:[M,K], B:[K,N], C:[M,N] operand shapes"),
    ]
    for t, msg in ops:
        p = tb_opt(t, "--tb-verify-scope", check=False)
        assert p.returncode == 1 and msg in p.stderr, (msg, p.stderr)
    # the sealed mainline keeps the reference's structural rules
    sealed = tb_opt(matmul_module(), f"--pass-pipeline={MAINLINE}").stdout
    assert '"tb.num-ctas" = 1 : i64' in sealed
    p = tb_opt(sealed.replace('"tb.num-ctas" = 1 : i64, ', ""), "--tb-verify-scope",
               check=False)
    assert p.returncode == 1 and "requires module attr `tb.num-ctas`" in p.stderr


def _listed_instances(loader_waves=False, resources=False):
    """tb-opt --list-instances: name -> (issue schedule, vmcnt prologue,
    vmcnt loop, lgkmcnt loop) from the host-side table; with loader_waves,
    name -> the load-only waves the instance adds to its wave grid; with
    resources, name -> (VGPRs, AGPRs, scratch bytes per lane) of the
    compiler's report."""
    p = subprocess.run([str(TB_OPT), "--list-instances"], capture_output=True,
                       text=True, timeout=60, check=True)
    out = {}
    for line in p.stdout.splitlines():
        name, issue, *kv = line.split()
        vals = dict(x.split("=") for x in kv)
        assert name not in out
        if resources:
            out[name] = (int(vals["vgprs"]), int(vals["agprs"]), int(vals["scratch"]))
        else:
            out[name] = int(vals["loader_waves"]) if loader_waves else (
                issue, int(vals["vmcnt_prologue"]), int(vals["vmcnt_loop"]),
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
    # the four issue schedules all occur, and differ in the prologue wait
    assert {v[0] for v in listed.values()} == {"slot_spread", "burst", "exact_tile_slots",
                                               "producer_waves", "tile16_slots"}
    assert listed["tb_gemm_gfx950_256x256x64_w4x2_s2_out0"][1:] == (4, 0, -1)
    assert listed["tb_gemm_gfx950_128x64x64_w4x1_s3_out1"][:2] == ("burst", 12)
    assert listed["tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32"][1:] == (16, 0, 0)
    # the split-K tile's partial instance: 8 load-only waves that issue all 3
    # k-tiles (3 loads per lane each) up front and wait for one at a time; its
    # other output modes keep the general loop (burst: 32x32 wave tiles)
    pw = "tb_gemm_gfx950_128x64x64_w4x2_s3_out1"
    assert listed[pw] == ("producer_waves", 6, 3, -1)
    waves = _listed_instances(loader_waves=True)
    assert waves[pw] == 8
    pw64 = "tb_gemm_gfx950_64x64x64_w2x2_s3_out1"
    assert listed[pw64][0] == "producer_waves" and waves[pw64] == 4
    assert {n for n, v in waves.items() if v} == {pw, pw64}
    assert listed["tb_gemm_gfx950_128x64x64_w4x2_s3_out0"] == ("burst", 6, 3, -1)
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


@pytest.mark.parametrize("w", configs.ALL + configs.F32_ACCUMULATE, ids=lambda w: w.name)
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


_RESOURCES = {}


@pytest.fixture(scope="module", autouse=True)
def _instance_resources():
    _RESOURCES.update(_listed_instances(resources=True))


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
                    # register truth: the bound instance's compiled build holds
                    # its wave tile in registers (no scratch)
                    assert _RESOURCES[d.kernel_name][2] == 0, (d.kernel_name,
                                                              _RESOURCES[d.kernel_name])
                    cfg = d.config
                    grid = configs.wave_grid(bm, bn, warps)
                    assert (cfg.wave_grid_m, cfg.wave_grid_n) == grid
                    assert d.kernel_name.startswith(
                        f"tb_gemm_gfx950_{bm}x{bn}x{bk}_w{grid[0]}x{grid[1]}_s{stages}_")
    if (bm, bn) not in ((96, 64), (160, 96)):
        assert bound > 0


def test_plan_over_operands_past_2gib():
    """The plan pipeline and the C ABI bind A and C of several GiB: the
    kernels address them in per-tile windows. B stays under 2 GiB."""
    w = configs.Workload("big", 262144, 32768, 8192, 1, 0, (256, 256, 64), num_waves=4)
    desc = tb.plan_from_mlir(w.mlir())
    assert desc.kernel_name == "tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32"
    cfg = desc.config
    assert (cfg.m, cfg.n, cfg.k) == (262144, 32768, 8192)
    assert cfg.m * cfg.lda * 2 > 1 << 31 and cfg.m * cfg.ldc * 2 > 1 << 31
    assert cfg.k * cfg.ldb * 2 < 1 << 31


def test_instance_resource_table_covers_every_instance():
    """Every compiled instance has the compiler's register report in the
    host-side table (generated at build time from hipcc's
    kernel-resource-usage remarks): registers within a lone wave's 512, and
    the known spilling builds read as spilling. The 32x32x16 builds of 128x128
    wave tiles hold 256 accumulator registers and spill; the 16x16x32 loop
    holds the same wave tile without scratch."""
    res = _listed_instances(resources=True)
    assert res and all(s >= 0 for _, _, s in res.values()), "instance without a report"
    for name, (v, a, s) in res.items():
        assert 0 < v <= 512 and 0 <= a <= 256 and v + a <= 512, (name, v, a)
    assert res["tb_gemm_gfx950_128x128x64_w1x1_s2_out0"][2] > 0
    assert res["tb_gemm_gfx950_256x128x32_w2x1_s2_out0"][2] > 0
    assert res["tb_gemm_gfx950_128x128x64_w1x1_s2_out0_16x16x32"][2] == 0
    assert res["tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32"] [2] == 0
    assert res["tb_gemm_gfx950_256x256x64_w2x2_s2_out0_16x16x32"][1] == 256


def test_plan_refuses_an_instance_that_spills():
    """Register truth: a configuration whose instance spills to scratch is
    refused by the lowering with the compiler's figures (here 1 wave on a
    128x128x64 block, forced onto 32x32x16), and by tb_desc_create; without
    the forced instruction the plan binds the 16x16x32 build of the same
    tile, which does not spill."""
    forced = matmul_module(M=256, N=256, K=256, bm=128, bn=128, bk=64, warps=1,
                           extra_op=', mma = "mfma_f32_32x32x16_f16"')
    p = tb_opt(forced, f"--pass-pipeline={FULL}", check=False)
    assert p.returncode == 1
    assert re.search(r"tb-build-program-mapping-plan: gfx950 kernel instance "
                     r"tb_gemm_gfx950_128x128x64_w1x1_s2_out0 spills \d+ bytes per lane "
                     r"to scratch", p.stderr), p.stderr
    with pytest.raises(tb.TbError, match="spills"):
        tb.plan_from_mlir(forced)
    d = tb.plan_from_mlir(forced.replace(', mma = "mfma_f32_32x32x16_f16"', ""))
    assert d.kernel_name == "tb_gemm_gfx950_128x128x64_w1x1_s2_out0_16x16x32"
    cfg = d.config
    cfg.mfma = tb.MFMA_32X32X16
    with pytest.raises(tb.TbError, match="spills"):
        tb.GemmDesc.from_config(cfg)
