"""FileCheck tests of tb-opt (tests/lit/*.mlir).

Each file carries `// RUN:` lines in the reference's lit style
(test/Transforms/*.mlir, run there by lit.cfg.py with %tb-opt substituted);
this runner substitutes %tb-opt, %s and FileCheck and runs the line under
bash -o pipefail, with lit's `not` (succeeds when its command fails) as a
shell function. The CHECK lines are the gfx950 contract: where the
reference checks a target-independent fact (mapping kinds, reduction kinds,
wave grids, persistent residency) the check is the same; where it checks an
NVIDIA-specific choice (LDS swizzle, epilogue reorder, NVGPU lowering) the
file checks the gfx950 choice and says why.
"""
import os
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
TB_OPT = ROOT / "mini_triton_nvgpu_v1_amd" / "bin" / "tb-opt"
FILECHECK = pathlib.Path("/opt/rocm/lib/llvm/bin/FileCheck")
LIT_FILES = sorted((ROOT / "tests" / "lit").glob("*.mlir"))


def run_lines(path):
    lines, cur = [], None
    for raw in path.read_text().splitlines():
        if "RUN:" not in raw:
            continue
        body = raw.split("RUN:", 1)[1].strip()
        if cur is not None:
            cur += " " + body
        else:
            cur = body
        if cur.endswith("\\"):
            cur = cur[:-1]
            continue
        lines.append(cur)
        cur = None
    return lines


@pytest.mark.parametrize("path", LIT_FILES, ids=[p.name for p in LIT_FILES])
def test_lit(path):
    if not TB_OPT.exists():
        pytest.fail("bin/tb-opt is not built (run __graft_entry__.build())")
    if not FILECHECK.exists():
        pytest.skip("FileCheck not available")
    runs = run_lines(path)
    assert runs, f"{path.name} has no RUN line"
    for cmd in runs:
        cmd = (cmd.replace("%tb-opt", str(TB_OPT)).replace("%s", str(path))
               .replace("FileCheck", str(FILECHECK)))
        cmd = 'not() { if "$@"; then return 1; else return 0; fi; }; ' + cmd
        proc = subprocess.run(["bash", "-o", "pipefail", "-c", cmd],
                              capture_output=True, text=True, timeout=120,
                              env=dict(os.environ))
        assert proc.returncode == 0, (
            f"{path.name}: `{cmd}` failed ({proc.returncode})\n"
            f"stdout:\n{proc.stdout[-4000:]}\nstderr:\n{proc.stderr[-4000:]}")
