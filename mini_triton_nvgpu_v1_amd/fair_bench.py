"""Interleaved fair benchmark of the tb.matmul gfx950 path.

The counterpart of the reference's tools/bench_stage1_fair.py: the same
case list (its CASES, :120-324, plus its large-shape cases and this build's
benchmark workloads, configs.ALL), the same CLI knobs and the same
measurement protocol:
- every case is verified once before timing;
- samples are taken in interleaved rounds, the two sides alternating who goes
  first (:750-809);
- a case whose min-to-max spread exceeds a threshold gets extra rounds
  (:1044-1083);
- an optional preheat repeats a heater case until the GPU clock reaches a
  floor (:812-877);
- the report is written as JSON and text (:1153-1236).

Differences, all forced by the platform:
- The comparison side is hipBLASLt through ``torch.matmul`` (f16 in, f16 out)
  instead of a Triton cubin; Triton has no place in this build.
- Samples are taken in-process with HIP events around ``iters`` back-to-back
  launches on one stream, instead of an external driver process per sample.
  A per-sample time cap (``--max-sample-ms``) bounds the iteration count for
  the large cases.
- Verification compares against an fp32 GEMM on the GPU (``C0 + A.float() @
  B.float()``) with the per-element tolerance |err| <= 1e-2 (|ref| + 1).
- GPU state comes from ``rocm-smi`` instead of ``nvidia-smi``.
- ``--rocprof`` re-runs each case in a child process under ``rocprofv3
  --kernel-trace --stats`` and keeps the summary beside the report.

Usage: python -m mini_triton_nvgpu_v1_amd.fair_bench [--cases all|a,b,...]
       [--rounds 5] [--warmup 500] [--iters 20000] [--compare hipblaslt|none]
       [--output-dir DIR] [--enable-preheat] [--rocprof]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import statistics
import subprocess
import sys
import time
from dataclasses import dataclass
from pathlib import Path
from typing import Any


@dataclass(frozen=True)
class FairCase:
    """One benchmark case: a tb.matmul module (shape, tile, module attrs) and
    its launch. Field meanings follow the reference's Stage1Case."""
    name: str
    m: int
    n: int
    k: int
    block_m: int
    block_n: int
    block_k: int
    num_warps: int  # wavefronts on gfx950
    num_stages: int
    exact_tile: bool
    group_m: int = 1
    c_type: str = "f32"  # f32: C += A*B (the reference's semantics); f16: C = A*B
    extra_module_attrs: tuple = ()
    compare: bool = True
    seed: int = 0x5EED0700
    normal: bool = False  # N(0,1)/sqrt(K) inputs instead of uniform[-1,1)

    def module_attr(self, name, default):
        return dict(self.extra_module_attrs).get(name, default)

    @property
    def split_k(self) -> int:
        return int(self.module_attr("tb.split-k", 1))

    @property
    def persistent(self) -> bool:
        return bool(self.module_attr("tb.persistent", False))

    @property
    def mapping_kind(self) -> str:
        if self.persistent:
            return "persistent_tile"
        if self.split_k > 1:
            return "split_k"
        if (self.group_m > 1 and math.ceil(self.m / self.block_m) > 1
                and math.ceil(self.n / self.block_n) > 1):
            return "grouped_tile"
        return "tile"

    @property
    def flops(self) -> int:
        return 2 * self.m * self.n * self.k

    def mlir(self) -> str:
        attrs = [f'"tb.num-warps" = {self.num_warps} : i64',
                 f'"tb.requested-stages" = {self.num_stages} : i64']
        for key, value in self.extra_module_attrs:
            if isinstance(value, bool):
                text = "true" if value else "false"
            elif isinstance(value, int):
                text = f"{value} : i64"
            else:
                text = f'"{value}"'
            attrs.append(f'"{key}" = {text}')
        a = f"memref<{self.m}x{self.k}xf16>"
        b = f"memref<{self.k}x{self.n}xf16>"
        c = f"memref<{self.m}x{self.n}x{self.c_type}>"
        return (
            f"module attributes {{{', '.join(attrs)}}} {{\n"
            f"  func.func @kernel(%A: {a}, %B: {b}, %C: {c}) {{\n"
            f"    tb.matmul %A, %B, %C {{block_m = {self.block_m} : i64, "
            f"block_n = {self.block_n} : i64, block_k = {self.block_k} : i64, "
            f"exact_tile = {'true' if self.exact_tile else 'false'}, "
            f"group_m = {self.group_m} : i64}} : {a}, {b}, {c}\n"
            f"    func.return\n  }}\n}}\n")


# Per-call time below which torch.matmul is bound by its host dispatch (~17 us
# per call on these boxes), not by its kernel
HOST_DISPATCH_NS = 25000.0


def _ref_case(name, m, n, k, bm, bn, bk, warps, exact, **kw):
    return FairCase(name, m, n, k, bm, bn, bk, warps, 2, exact, **kw)


# The reference's stage1 cases (tools/bench_stage1_fair.py:120-324, f32 C,
# C += A*B) and its large-shape cases
# (results/2026-04-07/large_shapes/large_shapes_report.json).
REFERENCE_CASES = (
    _ref_case("64x64x32", 64, 64, 32, 64, 64, 32, 1, True),
    _ref_case("64x128x32", 64, 128, 32, 64, 128, 32, 4, True),
    _ref_case("128x64x32", 128, 64, 32, 128, 64, 32, 4, True),
    _ref_case("64x64x64", 64, 64, 64, 64, 64, 64, 1, True),
    _ref_case("128x128x32", 128, 128, 32, 128, 128, 32, 4, True),
    _ref_case("128x128x64", 128, 128, 64, 128, 128, 64, 4, True),
    _ref_case("96x80x32_general", 96, 80, 32, 64, 64, 32, 1, False),
    _ref_case("192x128x32_grouped", 192, 128, 32, 64, 64, 32, 4, True, group_m=2),
    _ref_case("160x96x32_general", 160, 96, 32, 64, 64, 32, 4, False),
    _ref_case("224x160x64_general", 224, 160, 64, 64, 64, 64, 4, False),
    _ref_case("320x224x64_general", 320, 224, 64, 64, 64, 64, 4, False),
    _ref_case("448x288x64_general", 448, 288, 64, 64, 64, 64, 4, False),
    _ref_case("64x64x64_splitk2", 64, 64, 64, 64, 64, 32, 1, True, compare=False,
              extra_module_attrs=(("tb.split-k", 2),
                                  ("tb.reduction-mode", "split_k_parallel"))),
    _ref_case("192x128x32_persistent", 192, 128, 32, 64, 64, 32, 4, True, compare=False,
              extra_module_attrs=(("tb.persistent", True), ("tb.num-ctas", 2))),
    _ref_case("256x256x64", 256, 256, 64, 128, 128, 64, 4, True),
    _ref_case("256x256x128", 256, 256, 128, 128, 128, 64, 4, True),
)


def _baseline_cases():
    """The benchmark workloads of configs.py (f16 C = A*B, and the roofline
    GEMM as f32 C += A*B), as FairCases."""
    from . import configs
    out = []
    for w in configs.ALL + configs.F32_ACCUMULATE:
        attrs = []
        if w.split_k > 1:
            attrs += [("tb.split-k", w.split_k), ("tb.reduction-mode", "split_k_serial")]
        if w.persistent:
            attrs += [("tb.persistent", True), ("tb.num-ctas", w.num_ctas)]
        bm, bn, bk = w.block
        out.append(FairCase(w.name, w.M, w.N, w.K, bm, bn, bk, w.num_waves, w.stages,
                            w.exact_tile, group_m=w.group_m,
                            c_type="f32" if w.c_f32 else "f16",
                            extra_module_attrs=tuple(attrs), seed=w.seed,
                            normal=w.dist == configs.NORMAL))
    return tuple(out)


def all_cases():
    return REFERENCE_CASES + _baseline_cases()


# ---- statistics (the reference's summarize / spread rule, :702-720) --------
def summarize(values: list[float]) -> dict[str, float]:
    if not values:
        raise ValueError("cannot summarize an empty sample")
    s = {"min": min(values), "median": statistics.median(values), "max": max(values),
         "mean": statistics.fmean(values)}
    s["spread_pct"] = (s["max"] - s["min"]) / s["median"] * 100.0
    s["stdev"] = statistics.stdev(values) if len(values) > 1 else 0.0
    return s


def spread_exceeds(summary: dict[str, float], threshold_pct: float) -> bool:
    return summary["spread_pct"] > threshold_pct


def format_delta(mini_ns: float, other_ns: float, other: str) -> str:
    if mini_ns < other_ns:
        return f"mini faster than {other} by {(other_ns / mini_ns - 1.0) * 100.0:.2f}%"
    if mini_ns > other_ns:
        return f"mini slower than {other} by {(mini_ns / other_ns - 1.0) * 100.0:.2f}%"
    return f"mini equal to {other}"


def select_cases(selector: str) -> list[FairCase]:
    cases = all_cases()
    if selector == "all":
        return list(cases)
    if selector == "reference":
        return list(REFERENCE_CASES)
    if selector == "baseline":
        return list(_baseline_cases())
    wanted = [s.strip() for s in selector.split(",") if s.strip()]
    by_name = {c.name: c for c in cases}
    missing = [w for w in wanted if w not in by_name]
    if missing:
        raise ValueError(f"unknown case(s): {', '.join(missing)}")
    return [by_name[w] for w in wanted]


def order_cases(cases: list[FairCase], mode: str) -> list[FairCase]:
    if mode == "input":
        return list(cases)
    if mode == "hot_first":
        return sorted(cases, key=lambda c: c.flops, reverse=True)
    raise ValueError(f"unknown execution order: {mode}")


# ---- GPU state (rocm-smi) ----------------------------------------------------
def _smi_json(*flags) -> dict:
    out = subprocess.run(["rocm-smi", *flags, "--json"], capture_output=True, text=True,
                         timeout=30).stdout
    start = out.find("{")
    return next(iter(json.loads(out[start:]).values())) if start >= 0 else {}


def query_gpu_state() -> dict[str, Any]:
    """Current and maximum shader clock, memory clock, junction temperature and
    package power of GPU 0 ({"error": ...} when rocm-smi is unavailable)."""
    try:
        card = _smi_json("--showclocks", "--showtemp", "--showpower")
    except Exception as e:  # the report still stands without it
        return {"error": str(e)[:200]}

    def find(pred, conv):
        for key, value in card.items():
            if pred(key.lower()):
                try:
                    return conv(str(value))
                except ValueError:
                    pass
        return -1

    def mhz(text):
        m = re.search(r"(\d+)\s*mhz", text.lower())
        if not m:
            raise ValueError(text)
        return int(m.group(1))

    return {"sclk_mhz": find(lambda k: k.startswith("sclk clock speed"), mhz),
            "mclk_mhz": find(lambda k: k.startswith("mclk clock speed"), mhz),
            "temperature_c": find(lambda k: "temperature" in k and "junction" in k,
                                  lambda v: int(float(v))),
            "power_w": find(lambda k: "power" in k and "max" not in k,
                            lambda v: float(v)),
            "sclk_max_mhz": _max_sclk()}


_MAX_SCLK = None


def _max_sclk() -> int:
    """Highest shader clock level rocm-smi lists (-1 if unknown)."""
    global _MAX_SCLK
    if _MAX_SCLK is None:
        _MAX_SCLK = -1
        try:
            out = subprocess.run(["rocm-smi", "--showclkfrq"], capture_output=True,
                                 text=True, timeout=30).stdout
            sect = out.split("sclk", 1)[1] if "sclk" in out else ""
            sect = re.split(r"Supported \w+ frequencies|mclk|fclk|socclk", sect)[0]
            nums = [int(x) for x in re.findall(r"(\d+)\s*[Mm][Hh]z", sect)]
            _MAX_SCLK = max(nums) if nums else -1
        except Exception:
            pass
    return _MAX_SCLK


def clock_floor_mhz(state: dict[str, Any], floor_pct: float) -> int:
    top = state.get("sclk_max_mhz", -1)
    return math.floor(top * floor_pct / 100.0) if top > 0 else -1


def is_clock_hot_enough(state: dict[str, Any], floor_pct: float) -> bool:
    need = clock_floor_mhz(state, floor_pct)
    return need > 0 and state.get("sclk_mhz", -1) >= need


# ---- one case on the GPU -------------------------------------------------------
class CaseRunner:
    """Device buffers, the plan-pipeline descriptor and the comparison op of
    one case; `sample()` times `iters` back-to-back launches of one side."""

    def __init__(self, case: FairCase, device, gpu_arch: str):
        import torch
        from . import fill_seeded_f16, plan_from_mlir
        self.torch = torch
        self.case = case
        t0 = time.perf_counter()
        self.desc = plan_from_mlir(case.mlir(), gpu_arch)
        self.plan_ms = (time.perf_counter() - t0) * 1e3
        self.stream = torch.cuda.current_stream(device)
        m, n, k = case.m, case.n, case.k
        self.A = torch.empty((m, k), dtype=torch.float16, device=device)
        self.B = torch.empty((k, n), dtype=torch.float16, device=device)
        dist, scale = (1, 1.0 / math.sqrt(k)) if case.normal else (0, 1.0)
        fill_seeded_f16(self.A, m, k, case.seed, dist, scale, stream=self.stream)
        fill_seeded_f16(self.B, k, n, case.seed ^ 0xB, dist, scale, stream=self.stream)
        cdt = torch.float32 if case.c_type == "f32" else torch.float16
        self.C = torch.zeros((m, n), dtype=cdt, device=device)
        self.C16 = torch.empty((m, n), dtype=torch.float16, device=device)
        self.ws = (torch.empty(self.desc.workspace_bytes, dtype=torch.uint8, device=device)
                   if self.desc.workspace_bytes else None)
        # one C call per launch, like the reference's driver loop
        self.launch_mini = self.desc.bind(self.A, self.B, self.C, self.ws,
                                          stream=self.stream)

    def launch_other(self):
        self.torch.matmul(self.A, self.B, out=self.C16)

    def verify(self) -> dict[str, Any]:
        """One launch from a seeded C0 checked against C0 + A @ B in fp32."""
        torch = self.torch
        c0 = torch.empty((self.case.m, self.case.n), dtype=torch.float16,
                         device=self.C.device)
        if self.case.c_type == "f32":
            from . import fill_seeded_f16
            fill_seeded_f16(c0, self.case.m, self.case.n, self.case.seed ^ 0xC0, 0, 1.0,
                            stream=self.stream)
            self.C.copy_(c0.float())
        self.launch_mini()
        ref = torch.matmul(self.A.float(), self.B.float())
        if self.case.c_type == "f32":
            ref += c0.float()
        torch.cuda.synchronize()
        err = (self.C.float() - ref).abs()
        bad = int((err > 1e-2 * (ref.abs() + 1)).sum().item())
        finite = bool(torch.isfinite(self.C).all().item())
        return {"violations": bad, "max_abs_err": float(err.max().item()),
                "finite": finite, "ok": bad == 0 and finite}

    def sample(self, side: str, warmup: int, iters: int) -> dict[str, Any]:
        torch = self.torch
        fn = self.launch_mini if side == "mini" else self.launch_other
        for _ in range(warmup):
            fn()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        torch.cuda.synchronize()
        ev[0].record(self.stream)
        for _ in range(iters):
            fn()
        ev[1].record(self.stream)
        torch.cuda.synchronize()
        avg_ns = ev[0].elapsed_time(ev[1]) * 1e6 / iters
        return {"avg_ns": avg_ns, "gflops": self.case.flops / avg_ns, "iters": iters,
                "warmup": warmup}


def collect_interleaved_samples(runner: CaseRunner, compare: bool, rounds: int,
                                warmup: int, iters: int):
    mini, other = [], []
    for r in range(rounds):
        order = ("mini", "other") if r % 2 == 0 else ("other", "mini")
        for side in order:
            if side == "other" and not compare:
                continue
            (mini if side == "mini" else other).append(runner.sample(side, warmup, iters))
    return mini, other


def preheat_gpu(runner: CaseRunner, warmup: int, iters: int, max_attempts: int,
                floor_pct: float) -> dict[str, Any]:
    attempts = []
    for attempt in range(max_attempts):
        before = query_gpu_state()
        s = runner.sample("mini", warmup, iters)
        after = query_gpu_state()
        attempts.append({"attempt": attempt + 1, "before": before, "after": after,
                         "mini_avg_ns": s["avg_ns"]})
        if is_clock_hot_enough(after, floor_pct):
            break
    final = attempts[-1]["after"]
    return {"enabled": True, "heater_case": runner.case.name, "attempts": attempts,
            "target_floor_pct": floor_pct, "target_floor_mhz": clock_floor_mhz(final, floor_pct),
            "reached_hot_clock": is_clock_hot_enough(final, floor_pct)}


def rocprof_case(case: FairCase, out_dir: Path, args) -> dict[str, Any]:
    """rocprofv3 --kernel-trace --stats over one round of this case, in a child
    process (the profiler must start its own program)."""
    # absolute: the profiler runs from TMPDIR
    cdir = (out_dir / case.name / "rocprof").resolve()
    cdir.mkdir(parents=True, exist_ok=True)
    cmd = ["rocprofv3", "--kernel-trace", "--stats", "--output-format", "csv",
           "-d", str(cdir), "-o", "trace", "--", sys.executable, "-m",
           "mini_triton_nvgpu_v1_amd.fair_bench", "--cases", case.name, "--rounds", "1",
           "--warmup", str(min(args.warmup, 50)), "--iters", str(min(args.iters, 200)),
           "--extra-rounds-for-unstable", "0", "--output-dir", str(cdir / "run"),
           "--gpu-arch", args.gpu_arch, "--compare", args.compare]
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    try:
        p = subprocess.run(cmd, capture_output=True, text=True, timeout=300, env=env,
                           cwd=os.environ.get("TMPDIR", "/tmp"))
    except Exception as e:
        return {"ok": False, "error": str(e)[:300]}
    (cdir / "rocprof.log").write_text(p.stdout + p.stderr)
    stats = sorted(cdir.rglob("*kernel_stats.csv"))
    # any nonzero exit is a failure, a crash of the profiled run included
    return {"ok": p.returncode == 0 and bool(stats), "returncode": p.returncode,
            "kernel_stats": [str(s) for s in stats], "log": str(cdir / "rocprof.log")}


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(
        description="Interleaved fair benchmark of the tb.matmul gfx950 path.")
    p.add_argument("--cases", default="all",
                   help="all | reference | baseline | comma-separated case names")
    p.add_argument("--rounds", type=int, default=5)
    p.add_argument("--warmup", type=int, default=500)
    p.add_argument("--iters", type=int, default=20000)
    p.add_argument("--max-sample-ms", type=float, default=400.0,
                   help="cap a sample's timed launches at about this much GPU time")
    p.add_argument("--execution-order", choices=("input", "hot_first"), default="hot_first")
    p.add_argument("--enable-preheat", action="store_true")
    p.add_argument("--preheat-case", default="gemm_4096")
    p.add_argument("--preheat-warmup", type=int, default=50)
    p.add_argument("--preheat-iters", type=int, default=2000)
    p.add_argument("--preheat-max-attempts", type=int, default=3)
    p.add_argument("--preheat-clock-floor-pct", type=float, default=90.0)
    p.add_argument("--unstable-spread-threshold", type=float, default=10.0)
    p.add_argument("--extra-rounds-for-unstable", type=int, default=5)
    p.add_argument("--output-dir", type=Path, default=Path("fair_bench_out"))
    p.add_argument("--gpu-arch", default="gfx950")
    p.add_argument("--compare", choices=("hipblaslt", "none"), default="hipblaslt")
    p.add_argument("--rocprof", action="store_true",
                   help="also capture rocprofv3 --kernel-trace --stats per case")
    return p.parse_args(argv)


def _iters_for(runner: CaseRunner, args) -> int:
    """args.iters, capped so one sample's timed launches take about
    max_sample_ms (from a short probe of the slower side)."""
    probe = runner.sample("mini", 3, 5)["avg_ns"]
    if args.compare != "none" and runner.case.compare:
        probe = max(probe, runner.sample("other", 3, 5)["avg_ns"])
    cap = max(10, int(args.max_sample_ms * 1e6 / max(probe, 1.0)))
    return min(args.iters, cap)


def main(argv=None) -> int:
    args = parse_args(argv)
    import torch
    if not torch.cuda.is_available():
        print("fair_bench: needs an MI355X (gfx950) GPU", file=sys.stderr)
        return 2
    device = torch.device("cuda:0")
    cases = select_cases(args.cases)
    execution = order_cases(cases, args.execution_order)
    args.output_dir.mkdir(parents=True, exist_ok=True)
    compare_name = "hipblaslt" if args.compare == "hipblaslt" else None

    report: dict[str, Any] = {
        "rounds": args.rounds, "warmup": args.warmup, "iters": args.iters,
        "max_sample_ms": args.max_sample_ms, "compare": args.compare,
        "compare_op": "torch.matmul(A f16, B f16) -> f16 (hipBLASLt)" if compare_name else None,
        "gpu_state_before_all": query_gpu_state(), "cases": []}
    preheat: dict[str, Any] = {"enabled": False}
    heater = None
    if args.enable_preheat:
        heater = CaseRunner(select_cases(args.preheat_case)[0], device, args.gpu_arch)
        preheat = preheat_gpu(heater, args.preheat_warmup, args.preheat_iters,
                              args.preheat_max_attempts, args.preheat_clock_floor_pct)
    report["preheat"] = preheat
    report["gpu_state_after_preheat"] = query_gpu_state()
    report["execution_order"] = args.execution_order
    report["requested_case_order"] = [c.name for c in cases]
    report["measured_case_order"] = [c.name for c in execution]

    by_name: dict[str, dict[str, Any]] = {}
    failed = False
    for case in execution:
        print(f"fair_bench: case {case.name}", file=sys.stderr, flush=True)
        state_before = query_gpu_state()
        case_preheat = None
        if heater is not None and not is_clock_hot_enough(state_before,
                                                          args.preheat_clock_floor_pct):
            case_preheat = preheat_gpu(heater, args.preheat_warmup, args.preheat_iters,
                                       args.preheat_max_attempts,
                                       args.preheat_clock_floor_pct)
            state_before = query_gpu_state()
        runner = CaseRunner(case, device, args.gpu_arch)
        check = runner.verify()
        failed |= not check["ok"]
        compare = compare_name is not None and case.compare
        iters = _iters_for(runner, args)
        mini, other = collect_interleaved_samples(runner, compare, args.rounds,
                                                  args.warmup, iters)

        def summaries():
            ms = summarize([s["avg_ns"] for s in mini])
            mg = summarize([s["gflops"] for s in mini])
            os_ = summarize([s["avg_ns"] for s in other]) if other else None
            og = summarize([s["gflops"] for s in other]) if other else None
            return ms, mg, os_, og

        ms, mg, os_, og = summaries()
        extra = 0
        if args.extra_rounds_for_unstable > 0 and (
                spread_exceeds(ms, args.unstable_spread_threshold)
                or (os_ is not None and spread_exceeds(os_, args.unstable_spread_threshold))):
            extra = args.extra_rounds_for_unstable
            m2, o2 = collect_interleaved_samples(runner, compare, extra, args.warmup, iters)
            mini += m2
            other += o2
            ms, mg, os_, og = summaries()
        unstable = spread_exceeds(ms, args.unstable_spread_threshold) or (
            os_ is not None and spread_exceeds(os_, args.unstable_spread_threshold))
        comparison = None
        if os_ is not None:
            comparison = {
                "median_ns_delta": format_delta(ms["median"], os_["median"], compare_name),
                "mini_over_other_median_pct": os_["median"] / ms["median"] * 100.0,
                # a torch.matmul call costs ~17 us of host dispatch: below
                # HOST_DISPATCH_NS per call the ratio compares host paths
                # (ctypes against torch), not kernels
                "host_dispatch_bound": os_["median"] < HOST_DISPATCH_NS}
        cfg = runner.desc.config
        summary = {
            "shape": case.name,
            "config": {
                "m": case.m, "n": case.n, "k": case.k, "block_m": case.block_m,
                "block_n": case.block_n, "block_k": case.block_k,
                "num_warps": case.num_warps, "num_stages": case.num_stages,
                "exact_tile": case.exact_tile, "group_m": case.group_m,
                "split_k": case.split_k, "persistent": case.persistent,
                "mapping_kind": case.mapping_kind, "c_type": case.c_type,
                "block_x": case.num_warps * 64, "grid_x": cfg.num_programs,
                "compare": compare,
                "extra_module_attrs": {k: v for k, v in case.extra_module_attrs}},
            "gpu_state_before_case": state_before,
            "gpu_state_after_case": query_gpu_state(),
            "case_preheat": case_preheat,
            "verify": check,
            "mini": {"kernel": runner.desc.kernel_name,
                     "plan_pipeline_ms": round(runner.plan_ms, 3),
                     "summary_ns": ms, "summary_gflops": mg, "samples": mini},
            "other": None if os_ is None else {
                "name": compare_name, "summary_ns": os_, "summary_gflops": og,
                "samples": other},
            "comparison": comparison,
            "measurement": {"unstable": unstable,
                            "unstable_spread_threshold": args.unstable_spread_threshold,
                            "extra_rounds_run": extra, "total_rounds_run": len(mini),
                            "iters_per_sample": iters}}
        if args.rocprof:
            summary["rocprof"] = rocprof_case(case, args.output_dir, args)
        by_name[case.name] = summary
        del runner

    report["cases"] = [by_name[c.name] for c in cases]
    report["gpu_state_after_all"] = query_gpu_state()
    json_path = args.output_dir / "stage1_fair_report.json"
    json_path.write_text(json.dumps(report, indent=2))
    lines = [f"rounds={args.rounds} warmup={args.warmup} iters={args.iters} "
             f"compare={args.compare}",
             f"gpu_before={report['gpu_state_before_all']}",
             f"gpu_after_preheat={report['gpu_state_after_preheat']}", ""]
    if preheat.get("enabled"):
        status = "hot" if preheat.get("reached_hot_clock") else "not_hot_enough"
        lines += [f"preheat={preheat['heater_case']} status={status} "
                  f"target_floor={preheat['target_floor_mhz']}MHz "
                  f"attempts={len(preheat['attempts'])}", ""]
    for cs in report["cases"]:
        ms, mg = cs["mini"]["summary_ns"], cs["mini"]["summary_gflops"]
        lines.append(f"===== {cs['shape']} =====")
        lines.append(f"mini kernel={cs['mini']['kernel']} verify="
                     f"{'ok' if cs['verify']['ok'] else 'FAILED'} "
                     f"(max|err|={cs['verify']['max_abs_err']:.3e})")
        lines.append(f"mini median_ns={ms['median']:.2f} (mean={ms['mean']:.2f}, "
                     f"min={ms['min']:.2f}, max={ms['max']:.2f}, "
                     f"spread={ms['spread_pct']:.2f}%)")
        if cs["other"] is not None:
            os_, og = cs["other"]["summary_ns"], cs["other"]["summary_gflops"]
            name = cs["other"]["name"]
            lines.append(f"{name} median_ns={os_['median']:.2f} (mean={os_['mean']:.2f}, "
                         f"min={os_['min']:.2f}, max={os_['max']:.2f}, "
                         f"spread={os_['spread_pct']:.2f}%)")
            lines.append(f"mini median_gflops={mg['median']:.2f} "
                         f"{name} median_gflops={og['median']:.2f}")
            lines.append(cs["comparison"]["median_ns_delta"])
            note = (" (per call, host dispatch bound: not a kernel ratio)"
                    if cs["comparison"].get("host_dispatch_bound") else "")
            lines.append(f"mini_vs_{name}={cs['comparison']['mini_over_other_median_pct']:.2f}%"
                         f"{note}")
        else:
            lines.append(f"mini median_gflops={mg['median']:.2f}")
            lines.append("comparison=mini-only")
        lines.append(f"gpu_case=before={cs['gpu_state_before_case']} "
                     f"after={cs['gpu_state_after_case']}")
        meas = cs["measurement"]
        if meas["unstable"]:
            lines.append(f"measurement=unstable (threshold="
                         f"{meas['unstable_spread_threshold']:.2f}%, "
                         f"total_rounds={meas['total_rounds_run']})")
        elif meas["extra_rounds_run"] > 0:
            lines.append(f"measurement=restabilized (total_rounds={meas['total_rounds_run']})")
        if "rocprof" in cs:
            lines.append(f"rocprof={cs['rocprof']}")
        lines.append("")
    text_path = args.output_dir / "stage1_fair_report.txt"
    text_path.write_text("\n".join(lines))
    print("\n".join(lines))
    print(f"json_report={json_path}")
    print(f"text_report={text_path}")
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
