"""Builds libjeeves_fp8.so (the gfx950 kernels and their C ABI) in-tree with hipcc.

    python -m jeeves_amd.build            # product library
    python -m jeeves_amd.build --tests    # also the test-hook library under tests/

Every HIP source is compiled for gfx950 only, with packed-fp32 instruction
selection turned off and IEEE fp32 division, then linked into one shared
object next to this file.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libjeeves_fp8.so"
TEST_CSRC = ROOT / "tests" / "csrc"
TEST_LIB = ROOT / "tests" / "libjeeves_fp8_testhooks.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 VALU ops stay off: plain fp32 code only
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the quantizer's division must be the IEEE one
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-ffp-contract=off",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the FP8 library needs ROCm's hipcc to build")
    return path


def _compile(src: Path, obj: Path, include: list[Path]) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *[f"-I{p}" for p in include], "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr[-8000:]}")


def _build(sources: list[Path], out: Path, include: list[Path], build_dir: Path) -> Path:
    build_dir.mkdir(parents=True, exist_ok=True)
    objs = [build_dir / (s.stem + ".o") for s in sources]
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")), 16)
    with ThreadPoolExecutor(max_workers=max(jobs, 1)) as pool:
        list(pool.map(lambda so: _compile(*so, include), zip(sources, objs)))
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link of {out.name} failed:\n{r.stderr[-8000:]}")
    os.replace(tmp, out)
    return out


def build(tests: bool = False) -> Path:
    """Compile the product library (and, with tests=True, the test hooks)."""
    _build(sorted(CSRC.glob("*.hip")), LIB, [CSRC, ROOT / "include"], PKG / "_build")
    if tests and TEST_CSRC.is_dir():
        _build(sorted(TEST_CSRC.glob("*.hip")), TEST_LIB, [CSRC, ROOT / "include"], ROOT / "tests" / "_build")
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--tests", action="store_true", help="also build the test-hook library")
    a = ap.parse_args()
    print(build(tests=a.tests))


if __name__ == "__main__":
    sys.exit(main())
