"""The interleaved fair benchmark (mini_triton_nvgpu_v1_amd/fair_bench.py),
counterpart of the reference's tools/bench_stage1_fair.py.

CPU: every case of the reference's case list (and of the benchmark workloads)
goes through the plan pipeline and binds a compiled instance; the case
descriptors agree with the reference's launch formulas; the statistics and
case-selection rules behave like the reference's. GPU: a short run writes
both reports with verified, interleaved samples.
"""
import json
import math

import pytest

import mini_triton_nvgpu_v1_amd as tb
from mini_triton_nvgpu_v1_amd import fair_bench as fb


@pytest.mark.parametrize("case", fb.all_cases(), ids=lambda c: c.name)
def test_every_case_binds_an_instance(case):
    d = tb.plan_from_mlir(case.mlir())
    cfg = d.config
    assert (cfg.m, cfg.n, cfg.k) == (case.m, case.n, case.k)
    tiles = math.ceil(case.m / case.block_m) * math.ceil(case.n / case.block_n)
    # the reference's grid formula (bench_stage1_fair.py:65-71)
    if case.persistent:
        assert cfg.num_programs == min(case.module_attr("tb.num-ctas", 1), tiles)
    else:
        assert cfg.num_programs == tiles * case.split_k
    kinds = {"tile": tb.MAP_TILE, "grouped_tile": tb.MAP_GROUPED_TILE,
             "split_k": tb.MAP_SPLIT_K}
    if case.persistent:
        assert cfg.mapping in (tb.MAP_PERSISTENT_TILE, tb.MAP_PERSISTENT_GROUPED)
    else:
        assert cfg.mapping == kinds[case.mapping_kind]
    assert cfg.acc_init == (tb.ACC_INIT_LOAD_C if case.c_type == "f32" else tb.ACC_INIT_ZERO)


def test_reference_case_list():
    names = [c.name for c in fb.REFERENCE_CASES]
    assert len(names) == 16 and len(set(names)) == 16
    assert {"64x64x64_splitk2", "192x128x32_persistent", "448x288x64_general"} <= set(names)
    no_compare = {c.name for c in fb.REFERENCE_CASES if not c.compare}
    assert no_compare == {"64x64x64_splitk2", "192x128x32_persistent"}


def test_summarize_and_spread():
    s = fb.summarize([10.0, 12.0, 11.0])
    assert (s["min"], s["median"], s["max"]) == (10.0, 11.0, 12.0)
    assert s["spread_pct"] == pytest.approx(2.0 / 11.0 * 100.0)
    assert s["stdev"] == pytest.approx(1.0)
    assert fb.summarize([5.0])["stdev"] == 0.0
    assert fb.spread_exceeds(s, 10.0) and not fb.spread_exceeds(s, 20.0)
    with pytest.raises(ValueError):
        fb.summarize([])
    assert "faster" in fb.format_delta(1.0, 2.0, "x")
    assert "slower" in fb.format_delta(2.0, 1.0, "x")


def test_select_and_order():
    assert [c.name for c in fb.select_cases("64x64x32,gemm_4096")] == [
        "64x64x32", "gemm_4096"]
    assert len(fb.select_cases("reference")) == len(fb.REFERENCE_CASES)
    with pytest.raises(ValueError, match="unknown case"):
        fb.select_cases("nope")
    cases = fb.select_cases("64x64x32,gemm_4096,128x128x64")
    hot = fb.order_cases(cases, "hot_first")
    assert [c.name for c in hot] == ["gemm_4096", "128x128x64", "64x64x32"]
    assert fb.order_cases(cases, "input") == cases


def test_clock_floor_rule():
    st = {"sclk_mhz": 2200, "sclk_max_mhz": 2400}
    assert fb.clock_floor_mhz(st, 90.0) == 2160
    assert fb.is_clock_hot_enough(st, 90.0)
    assert not fb.is_clock_hot_enough({"sclk_mhz": 2000, "sclk_max_mhz": 2400}, 90.0)
    assert not fb.is_clock_hot_enough({"error": "no rocm-smi"}, 90.0)


@pytest.mark.gpu
def test_short_run_writes_reports(tmp_path):
    out = tmp_path / "fair"
    rc = fb.main(["--cases", "64x64x32,192x128x32_persistent,tile_128x128x32",
                  "--rounds", "2", "--warmup", "5", "--iters", "50",
                  "--extra-rounds-for-unstable", "1", "--output-dir", str(out)])
    assert rc == 0
    report = json.loads((out / "stage1_fair_report.json").read_text())
    assert [c["shape"] for c in report["cases"]] == [
        "64x64x32", "192x128x32_persistent", "tile_128x128x32"]
    for c in report["cases"]:
        assert c["verify"]["ok"], c["verify"]
        assert c["measurement"]["total_rounds_run"] >= 2
        assert len(c["mini"]["samples"]) == c["measurement"]["total_rounds_run"]
        assert c["mini"]["summary_ns"]["median"] > 0
        if c["config"]["compare"]:
            assert len(c["other"]["samples"]) == len(c["mini"]["samples"])
        else:
            assert c["other"] is None
    text = (out / "stage1_fair_report.txt").read_text()
    assert "===== 64x64x32 =====" in text and "mini_vs_hipblaslt=" in text


@pytest.mark.parametrize("rc,ok", [(0, True), (139, False), (1, False)])
def test_rocprof_capture_counts_any_nonzero_exit_as_failure(tmp_path, monkeypatch, rc, ok):
    """A profiled run that crashes (139 = SIGSEGV) is a failed capture, even
    when it left a kernel-stats file behind; the code and the log path are
    recorded."""
    import subprocess
    import types

    case = fb.select_cases("gemm_4096")[0]

    def fake_run(cmd, **kw):
        d = tmp_path / case.name / "rocprof"
        (d / "x").mkdir(parents=True, exist_ok=True)
        (d / "x" / "trace_kernel_stats.csv").write_text("Name,Calls\n")
        return types.SimpleNamespace(returncode=rc, stdout="", stderr="")

    monkeypatch.setattr(subprocess, "run", fake_run)
    args = fb.parse_args(["--cases", case.name])
    r = fb.rocprof_case(case, tmp_path, args)
    assert r["ok"] is ok and r["returncode"] == rc
    assert r["log"].endswith("rocprof.log")
