"""The 16x16x32 instance's slot schedule and MFMA hazard rules are checked at
compile time (mini_triton_nvgpu_v1_amd/csrc/kernels/mfma16_schedule.h): the
kernel takes its fragment-read slots and accumulator wait from
Mfma16Schedule, whose static_asserts encode (a) one first MFMA (srcC = 0) per
accumulator tile, (b) 24 wait states (3 per MFMA pass) before accumulator
reads, (c) fragment registers rewritten at least 8 MFMA slots after their
last read, and the barrier's read ordering. Here the header is compiled on
the CPU with the kernel's parameters (it builds) and with edits that break
each rule (each fails to build, naming the rule)."""
import pathlib
import subprocess

import pytest

HDR = (pathlib.Path(__file__).resolve().parent.parent / "mini_triton_nvgpu_v1_amd" /
       "csrc" / "kernels")


def _compile(tmp_path, params):
    src = tmp_path / "sched.cpp"
    src.write_text('#include "mfma16_schedule.h"\n'
                   f"template struct tbk::Mfma16Schedule<{params}>;\n"
                   "int main() { return 0; }\n")
    return subprocess.run(["g++", "-std=c++17", "-fsyntax-only", f"-I{HDR}", str(src)],
                          capture_output=True, text=True, timeout=60)


def test_kernel_schedule_builds(tmp_path):
    p = _compile(tmp_path, "")  # the defaults the kernel instantiates
    assert p.returncode == 0, p.stderr
    p = _compile(tmp_path, "16, 8, 3, 24, 2, 1")
    assert p.returncode == 0, p.stderr
    # the earlier schedule (barrier at slot 40, one read per slot after it)
    # keeps the rules too
    p = _compile(tmp_path, "40, 8, 3, 24, 1, 1")
    assert p.returncode == 0, p.stderr


@pytest.mark.parametrize("params,rule", [
    # (b) two s_nop 7 instead of three
    ("16, 8, 3, 16, 2, 1", "(b) accumulator reads need 3 wait states per MFMA pass"),
    # (c) k step 1's reads bunched at the start of k step 0: A7's buffer-1
    # register rewritten 6 slots after the previous k step's last read of it
    ("16, 1, 4, 24, 2, 1", "(c) a fragment register rewritten too soon"),
    # the next k-tile's reads would run past the k step
    ("24, 8, 3, 24, 2, 1", "the next k-tile's reads must fit after the barrier"),
    # k step 1's reads spread past the end of k step 0
    ("16, 3, 1, 24, 2, 1", "fragment reads must fall inside their k step"),
])
def test_schedule_edits_that_break_a_rule_do_not_build(tmp_path, params, rule):
    p = _compile(tmp_path, params)
    assert p.returncode != 0
    assert rule in p.stderr, p.stderr[-2000:]
