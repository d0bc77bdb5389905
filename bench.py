#!/usr/bin/env python3
"""Benchmark of the tb.matmul gfx950 path (one MI355X).

Headline metric: TFLOP/s and fraction of dense FP16 MFMA peak on the 4096^3
f16 GEMM (the roofline workload of configs.py); a "step" is
one GEMM launch over inputs already resident in HBM. The same JSON line also
carries microseconds per launch for the small shapes and the split-K and
persistent workloads (`extra`), the live roofline of the dominant kernel and
the host fp32 CPU baseline (the oracle's blocked OpenMP GEMM on this box's
cores, on a bounded sample of the same workload).

Timing: a clock-settle phase (--settle-s seconds of launches), W warm-up
launches, then --rounds rounds of exactly K launches, each bracketed by a
device synchronize; `value` and `ms_per_step` are the median round. The
timed output is checked against torch.matmul in f32 on every 16th row (for
f32 C += A*B, one more launch on the prior C after the timed rounds).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--rounds R]
       [--settle-s S] [--no-extra] [--no-cpu] [--workload NAME]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_TFLOPS_F16 = 2500.0  # MI355X dense FP16 MFMA (published, no sparsity)
PEAK_HBM_GBS = 8000.0
PEAK_CLOCK_MHZ = 2400.0  # the clock the dense peak is quoted at (1024 SIMDs x 1024 FLOP/clk)
XCDS = 8  # MI355X: 8 XCDs of 32 CUs
STAMP_WGS = 1024  # one-wave clock stamps per reading: about every CU is stamped


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def time_workload(w, steps: int, warmup: int, device, rounds: int = 5,
                  settle_s: float = 0.0):
    """Time `w` through the plan pipeline's kernel.

    Order: a clock-settle phase (launches back to back for `settle_s` seconds
    of wall clock, so the timed rounds run at the part's sustained clock and
    not on the ramp up from idle), `warmup` untimed launches, then `rounds`
    rounds of exactly `steps` launches, each bracketed by a device
    synchronize on both sides. Per round: the wall clock and HIP events
    recorded on the launch stream around its launches (average launch
    duration = elapsed / steps; the GPU never idles in between, so for
    kernels longer than the launch rate this is the kernel duration). The
    medians over rounds are reported (the reference's median-of-rounds
    method, tools/bench_stage1_fair.py:702-716)."""
    import torch
    import mini_triton_nvgpu_v1_amd as tb

    # the product path: tb.matmul module text -> plan pipeline -> kernel
    desc = tb.plan_from_mlir(w.mlir())
    A = torch.empty((w.M, w.K), dtype=torch.float16, device=device)
    B = torch.empty((w.K, w.N), dtype=torch.float16, device=device)
    C = torch.empty((w.M, w.N), dtype=torch.float32 if w.c_f32 else torch.float16,
                    device=device)
    ws = (torch.empty(desc.workspace_bytes, dtype=torch.uint8, device=device)
          if desc.workspace_bytes else None)
    stream = torch.cuda.current_stream(device)
    C0 = None
    if w.c_f32:  # C += A*B: a seeded prior C, uniform in [-1, 1)
        C0 = torch.empty((w.M, w.N), dtype=torch.float16, device=device)
        tb.fill_seeded_f16(C0, w.M, w.N, w.seed ^ 0xC0, 0, 1.0, stream=stream)
        C0 = C0.float()
        C.copy_(C0)
    bias = None
    if w.bias:  # fused bias step: N seeded values
        bias = torch.empty((1, w.N), dtype=torch.float16, device=device)
        tb.fill_seeded_f16(bias, 1, w.N, w.seed ^ 0xB1A5, 0, 1.0, stream=stream)
        if w.bias == "f32":
            bias = bias.float()
    tb.fill_seeded_f16(A, w.M, w.K, w.seed, w.dist, w.scale, stream=stream)
    tb.fill_seeded_f16(B, w.K, w.N, w.seed_b, w.dist, w.scale, stream=stream)
    launch = desc.bind(A, B, C, ws, stream=stream, bias=bias)
    settle_launches = 0
    if settle_s > 0:
        t_end = time.perf_counter() + settle_s
        while time.perf_counter() < t_end:
            for _ in range(50):
                launch()
            settle_launches += 50
            torch.cuda.synchronize(device)
    for _ in range(warmup):
        launch()
    walls, events, clocks = [], [], []
    # shader-clock stamps (1024 one-wave workgroups) on the launch stream
    # right before and right after each round's launches: per CU stamped
    # both times, the cycles between its two stamps over the 100 MHz ticks
    # between them is the mean clock the round's kernels ran at (the stamps
    # add a few us to a round of tens of ms); the median over CUs
    stamps = torch.zeros((rounds, 2, 3 * STAMP_WGS), dtype=torch.int64, device=device)
    for r in range(rounds):
        region = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        torch.cuda.synchronize(device)
        t0 = time.perf_counter()
        tb.clock_stamp(stamps[r, 0], STAMP_WGS, stream=stream)
        region[0].record(stream)
        for _ in range(steps):
            launch()
        region[1].record(stream)
        tb.clock_stamp(stamps[r, 1], STAMP_WGS, stream=stream)
        torch.cuda.synchronize(device)
        walls.append(time.perf_counter() - t0)
        events.append(region[0].elapsed_time(region[1]) / steps)
    for before, after in stamps.tolist():
        per_cu = tb.stamps_clock_mhz(before, after)
        clocks.append(statistics.median(per_cu.values()) if per_cu else None)
    if C0 is not None:
        # the timed launches accumulated into C: check one more launch on the
        # prior C instead
        C.copy_(C0)
        launch()
        torch.cuda.synchronize(device)
    ok = verify_output(w, A, B, C, bias, C0)
    return {"wall_s": statistics.median(walls), "avg_launch_ms": statistics.median(events),
            "round_wall_s": walls, "round_launch_ms": events, "round_clock_mhz": clocks,
            "kernel": desc.kernel_name,
            "settle_launches": settle_launches, "verified": ok}


def verify_output(w, A, B, C, bias, C0=None):
    """The timed launches' output against torch.matmul in f32 on the same
    device buffers (an independent GEMM), plus the prior C for C += A*B, with
    the fused steps applied, on every 16th row: per-element
    |err| <= 1e-2 (|ref| + 1)."""
    import torch

    rows = torch.arange(0, w.M, 16, device=A.device)
    ref = A[rows].float() @ B.float()
    if C0 is not None:
        ref += C0[rows]
    if bias is not None:
        ref += bias.float().view(1, -1)
    if w.activation == "relu":
        ref = torch.relu(ref)
    elif w.activation == "gelu_tanh":
        ref = torch.nn.functional.gelu(ref, approximate="tanh")
    elif w.activation == "silu":
        ref = torch.nn.functional.silu(ref)
    if w.clamp_min is not None or w.clamp_max is not None:
        ref = torch.clamp(ref, w.clamp_min, w.clamp_max)
    got = C[rows].float()
    err = (got - ref).abs()
    bad = int((~(err <= 1e-2 * (ref.abs() + 1))).sum().item())
    return {"rows": int(rows.numel()), "violations": bad,
            "max_abs_err": float(err.max().item()), "vs": "torch.matmul f32"}


def clock_summary(r) -> dict:
    """The shader clock the timed rounds ran at (per round: stamps on the
    launch stream right before and right after its launches, the cycles
    between them over the 100 MHz ticks between them, mean over the XCDs),
    the median round's value. The caller adds the fraction of peak the kernel
    reaches per clock cycle: the achieved rate over the peak scaled from
    2.4 GHz to that clock."""
    clk = [c for c in r["round_clock_mhz"] if c]
    if not clk:
        return {"mhz": None}
    mhz = statistics.median(clk)
    return {"mhz": round(mhz, 1), "round_mhz": [round(c, 1) for c in clk],
            "source": "s_memtime / s_memrealtime stamps (1024 one-wave workgroups) on the "
                      "launch stream right before and right after each timed round's "
                      "launches, paired per CU, median over CUs",
            "peak_clock_mhz": PEAK_CLOCK_MHZ}


def plan_time_ms(w, reps: int = 20) -> float:
    """Host time of the whole plan pipeline (parse, 17 passes, contract
    lowering, kernel binding) for the workload's tb.matmul module: the
    reference's CPU-side work on this path, single-threaded."""
    import mini_triton_nvgpu_v1_amd as tb

    text = w.mlir()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        tb.plan_from_mlir(text)
        times.append(time.perf_counter() - t0)
    return statistics.median(times) * 1e3


def cpu_baseline(w, budget_s: float = 12.0):
    """Host fp32 GEMM (oracle/oracle.c tbo_gemm_f32) on the same seeded inputs.

    Sample: the full M x N x K product of the workload when one repetition
    fits the budget, else a slab of rows; repeated until `budget_s` elapses."""
    import numpy as np
    import oracle

    threads = oracle.max_threads()
    rows = w.M
    A16, B16 = oracle.config_inputs(rows, w.N, w.K, w.seed, w.dist)
    A = A16.astype(np.float32)
    B = B16.astype(np.float32)
    flop = 2.0 * rows * w.N * w.K
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or not times:
        t0 = time.perf_counter()
        oracle.gemm_f32(A, B, threads=threads)
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    best = min(times)
    med = statistics.median(times)
    # the same GEMM on one core, over a slab of rows (a few seconds)
    rows1 = max(1, min(w.M, 256))
    flop1 = 2.0 * rows1 * w.N * w.K
    t1 = []
    t_end = time.perf_counter() + budget_s / 3
    while time.perf_counter() < t_end or not t1:
        t0 = time.perf_counter()
        oracle.gemm_f32(A[:rows1], B, threads=1)
        t1.append(time.perf_counter() - t0)
        if len(t1) >= 20:
            break
    med1 = statistics.median(t1)
    return {"value": flop / med / 1e12, "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": (f"{len(times)} x fp32 {rows}x{w.N}x{w.K} GEMM on host "
                       f"(oracle tbo_gemm_f32, OpenMP {threads} threads, median "
                       f"{med * 1e3:.1f} ms, best {best * 1e3:.1f} ms); "
                       f"{os.uname().machine} {cpu_model()}"),
            "single_core": {"value": flop1 / med1 / 1e12, "unit": "TFLOP/s", "cores": 1,
                            "sample": (f"{len(t1)} x fp32 {rows1}x{w.N}x{w.K} GEMM "
                                       f"(first {rows1} rows), 1 thread, median "
                                       f"{med1 * 1e3:.1f} ms")}}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown cpu"


def load_traffic(workload: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy-kernel calibration), committed under
    profiles/; null if no measurement exists."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    try:
        with open(path) as f:
            return json.load(f).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--rounds", type=int, default=5,
                    help="timed rounds of --steps launches; medians are reported")
    ap.add_argument("--settle-s", type=float, default=2.0,
                    help="seconds of back-to-back launches before the warm-up, so the "
                         "timed rounds see the sustained clock, not the ramp from idle")
    ap.add_argument("--workload", default="gemm_4096")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "across GPUs the GEMM would shard by output row panels with no exchange",
              file=sys.stderr)
        return 2

    import torch
    from mini_triton_nvgpu_v1_amd import configs

    device = torch.device("cuda:0")
    w = configs.BY_NAME[args.workload]
    log(f"bench: workload {w.name} {w.M}x{w.N}x{w.K} steps={args.steps} "
        f"warmup={args.warmup} rounds={args.rounds} settle={args.settle_s}s")
    r = time_workload(w, args.steps, args.warmup, device, args.rounds, args.settle_s)
    if r["verified"]["violations"]:
        log(f"bench: output check failed: {r['verified']}")
        return 1
    ms_per_step = r["wall_s"] * 1e3 / args.steps
    value = w.flop * args.steps / r["wall_s"] / 1e12
    avg_kernel_ms = r["avg_launch_ms"]
    achieved = w.flop / (avg_kernel_ms * 1e-3) / 1e12
    clock = clock_summary(r)
    if clock["mhz"]:
        # per clock cycle: the fraction of the MFMA issue rate at the clock held
        clock["frac_of_peak_at_clock"] = round(
            achieved / (PEAK_TFLOPS_F16 * clock["mhz"] / PEAK_CLOCK_MHZ), 4)
    log(f"bench: {r['kernel']} wall {ms_per_step * 1e3:.1f} us/step, "
        f"kernel avg {avg_kernel_ms * 1e3:.1f} us -> {achieved:.1f} TFLOP/s "
        f"(rounds {[round(x * 1e3, 2) for x in r['round_launch_ms']]} us, "
        f"clock {clock})")

    extra = {}
    if not args.no_extra:
        for other in configs.ALL + configs.FUSED + configs.F32_ACCUMULATE:
            if other.name == w.name:
                continue
            # a few tens of ms of GPU time per extra: long enough for a steady clock
            steps = 200 if other.flop < 1e9 else (300 if other.flop < 2e11 else 60)
            o = time_workload(other, steps, steps, device, rounds=5)
            if o["verified"]["violations"]:
                log(f"bench: {other.name} output check failed: {o['verified']}")
                return 1
            us = o["avg_launch_ms"] * 1e3
            wall_us = o["wall_s"] * 1e6 / steps
            extra[other.name] = {
                "us_per_launch": round(us, 2),
                "us_per_launch_wall": round(wall_us, 2),
                "tflops": round(other.flop / (us * 1e-6) / 1e12, 2),
                "frac_mfma_peak": round(other.flop / (us * 1e-6) / 1e12 / PEAK_TFLOPS_F16, 4),
                "frac_hbm_peak": round(other.algo_bytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                "plan_pipeline_ms": round(plan_time_ms(other), 3),
                "kernel": o["kernel"], "verified_rows": o["verified"]["rows"],
                "clock_mhz": clock_summary(o)["mhz"]}
            log(f"bench: {other.name}: {extra[other.name]}")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(w)
        log(f"bench: cpu baseline {cpu}")

    line = {
        "metric": "TFLOP/s + % FP16 MFMA peak, 4096^3 f16 GEMM; us/launch small shapes",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (device SplitMix64 seeded N(0,1)/sqrt(K) f16)",
        "frac_of_peak": round(value / PEAK_TFLOPS_F16, 4),
        "config": {"workload": w.name, "M": w.M, "N": w.N, "K": w.K,
                   "tile": list(w.block), "num_waves": w.num_waves,
                   "group_m": w.group_m, "split_k": w.split_k,
                   "persistent": w.persistent,
                   "c_dtype": "f32 (C += A*B)" if w.c_f32 else "f16",
                   "accumulate": "f32", "kernel": r["kernel"],
                   "plan_pipeline_ms": round(plan_time_ms(w), 3)},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3),
                     "peak": PEAK_TFLOPS_F16, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_TFLOPS_F16, 4),
                     "traffic": load_traffic(w.name),
                     "traffic_source": ("committed profile, not measured in this run: "
                                        f"profiles/traffic_{w.name}.json (rocprofv3 --pmc "
                                        "FETCH_SIZE + WRITE_SIZE per launch, copy-calibrated)")},
        "clock": clock,
        "timing": {"rounds": args.rounds, "statistic": "median over rounds",
                   "round_us_per_launch": [round(x * 1e3, 2) for x in r["round_launch_ms"]],
                   "round_ms_per_step_wall": [round(x * 1e3 / args.steps, 5)
                                              for x in r["round_wall_s"]],
                   "settle_s": args.settle_s, "settle_launches": r["settle_launches"]},
        "verified": r["verified"],
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
