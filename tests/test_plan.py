"""CPU check of the GEMV grid plans (one-shot tiling and persistent plan): builds
tests/cpp/plan_check.hip (host code only) and runs it.  Guards the wave -> matrix -> tile mapping against out-of-range
loads (a surplus wave once selected a matrix slot that did not exist)."""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_gemv_grid_plans(tmp_path):
    exe = tmp_path / "plan_check"
    subprocess.run(["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O1", "-std=c++17",
                    str(ROOT / "tests" / "cpp" / "plan_check.hip"), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
