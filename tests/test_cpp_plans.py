"""C++ unit tests of the plan derivations (tests/cpp/test_plans.cpp): the
derive* functions of csrc/plan called directly, built here with g++ from the
plan, IR and pass sources (no GPU, no HIP), and run."""
import pathlib
import subprocess

PKG = pathlib.Path(__file__).resolve().parent.parent / "mini_triton_nvgpu_v1_amd"
SRC = pathlib.Path(__file__).resolve().parent / "cpp" / "test_plans.cpp"


def test_plan_derivations(tmp_path):
    sources = sorted(str(p) for d in ("ir", "plan", "passes")
                     for p in (PKG / "csrc" / d).glob("*.cpp"))
    exe = tmp_path / "test_plans"
    # instances.cpp includes the build's instance resource table (_build/)
    build = subprocess.run(["g++", "-std=c++17", "-O0", f"-I{PKG / 'csrc'}",
                            f"-I{PKG / '_build'}", f"-I{PKG.parent / 'include'}", str(SRC),
                            *sources, "-o", str(exe)],
                           capture_output=True, text=True, timeout=600)
    assert build.returncode == 0, build.stderr[-3000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(run.stdout)
    assert run.returncode == 0, run.stdout[-3000:]
    assert "0 failures" in run.stdout
