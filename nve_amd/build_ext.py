"""Build libnve_hip.so (gfx950) in-tree with hipcc.

The library is compiled from nve_amd/csrc/*.hip: one hipcc job per translation unit
(run in parallel), then one link step.  Output: nve_amd/libnve_hip.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libnve_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-command-line-argument",
    # Packed-FP32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Correctly rounded f32 division / sqrt (the quantizers depend on it).
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-fast-math",
    # Kernel arguments preloaded into SGPRs by the dispatch (as many as the free user
    # SGPRs hold): the first scalar load of each launch's arguments leaves the critical
    # path of the decode chain (3B decode 1163.5 against 1158.5 tok/s).
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


INCLUDE = PKG.parent / "include"


def source_id() -> str:
    """Hash of everything the library is built from: every file under csrc/ and
    include/ (name and bytes, in sorted order) and the compile flags.  The build embeds
    it (nve_hip_build_id), and the loader refuses a library whose id differs from the
    tree's, so a stale prebuilt .so can never be what runs."""
    h = hashlib.sha256()
    h.update(" ".join(CFLAGS).encode())
    for d in (CSRC, INCLUDE):
        for f in sorted(p for p in d.iterdir() if p.is_file() and p.suffix in (".hip", ".h", ".cpp")):
            h.update(f"{d.name}/{f.name}\0".encode())
            h.update(f.read_bytes())
            h.update(b"\0")
    return h.hexdigest()[:32]


def _compile(src: Path, build_id: str) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, f'-DNVE_BUILD_ID="{build_id}"', "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OBJ.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    bid = source_id()
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda f: _compile(f, bid), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    # hipBLASLt: the dense GEMM of the large-M prefill path (gemm_blas.hip)
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-lhipblaslt", "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
