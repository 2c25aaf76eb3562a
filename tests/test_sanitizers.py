"""The library's host-side C++ under AddressSanitizer and UndefinedBehaviour-
Sanitizer (CPU only, no GPU code is built here):

* the host quantizer of GPU-less exports (``jeeves_amd/csrc/quant_host.hip``,
  the counterpart of ``quantize_row_blocks_on_cpu``,
  ``inference/fp8_weights.py:22-26``) compiled host-only with amdclang++
  ``-fsanitize=address,undefined``, driven by ``tests/csrc/host_quant_driver.cpp``
  over the torch fixtures and over odd row strides (input padding holding
  NaN, which any read past a row's columns would turn into a NaN scale; code
  padding holding a sentinel, which any write past them would change) on odd
  thread counts; codes and scales must equal the fixtures and the oracle bit
  for bit;
* the exhaustive fast-quotient check (``tests/csrc/quotient_check.c``) built
  with gcc ``-fsanitize=address,undefined``: same counts as the plain build.

Any sanitizer report aborts the program (``-fno-sanitize-recover=all``), which
fails the test."""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from tests import helpers

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "jeeves_amd" / "csrc"
AMDCLANG = shutil.which("amdclang++") or "/opt/rocm/bin/amdclang++"
SAN_ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")


@pytest.fixture(scope="module")
def host_quant_driver(tmp_path_factory) -> Path:
    if not Path(AMDCLANG).exists():
        pytest.skip("amdclang++ not found")
    exe = tmp_path_factory.mktemp("asan") / "host_quant_driver"
    cmd = [AMDCLANG, "-x", "hip", "--offload-host-only", "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined",
           "-fno-gpu-sanitize", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", f"-I{CSRC}",
           f"-I{ROOT / 'include'}", str(CSRC / "quant_host.hip"), "-x", "c++",
           str(ROOT / "tests" / "csrc" / "host_quant_driver.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    return exe


def run_host_quantizer(exe: Path, tmp: Path, w: np.ndarray, ldw: int, ldc: int, threads: int):
    rows, cols = w.shape
    buf = np.full((rows, ldw), np.nan, dtype=np.float32)
    buf[:, :cols] = w
    src, dst = tmp / "in.bin", tmp / "out.bin"
    buf.tofile(src)
    r = subprocess.run([str(exe), str(src), str(dst), str(rows), str(cols), str(ldw), str(ldc), str(threads)],
                       capture_output=True, text=True, timeout=300, env=SAN_ENV)
    assert r.returncode == 0, r.stderr[-4000:]
    raw = np.fromfile(dst, dtype=np.uint8)
    codes = raw[:rows * ldc].reshape(rows, ldc)
    scales = raw[rows * ldc:].view(np.float32)
    assert (codes[:, cols:] == 0xAB).all(), "a code was written past its row's columns"
    return codes[:, :cols], scales


@pytest.mark.parametrize("name", ["edge", "cfg0_x", "cfg0_w64"])
@pytest.mark.parametrize("threads", [1, 3])
def test_host_quantizer_under_asan_matches_fixtures(host_quant_driver, tmp_path, name, threads):
    g = helpers.golden("quantize_rows.npz")
    x = oracle.bf16_to_f32(g["edge_x" if name == "edge" else name]).astype(np.float32)
    codes, scales = run_host_quantizer(host_quant_driver, tmp_path, x, x.shape[1], x.shape[1], threads)
    want_codes, want_scales = g[f"{name}_codes"], g[f"{name}_scales"]
    assert helpers.same_codes(codes, want_codes).all()
    assert helpers.same_f32(scales, want_scales).all()


@pytest.mark.parametrize("rows,cols,ldw,ldc,threads", [(37, 200, 203, 205, 3), (11, 4100, 4107, 4113, 7),
                                                       (5, 8, 13, 9, 5), (64, 1024, 1031, 1040, 16)])
def test_host_quantizer_under_asan_odd_strides_and_threads(host_quant_driver, tmp_path, rows, cols, ldw, ldc, threads):
    rng = np.random.default_rng(rows * 1000 + cols)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[0, cols // 2] = 3.0
    if rows > 2:
        w[1] = 0.0
        w[2, 0] = np.inf
    codes, scales = run_host_quantizer(host_quant_driver, tmp_path, w, ldw, ldc, threads)
    want_codes, want_scales = oracle.quantize_rows(w)
    assert helpers.same_codes(codes, want_codes).all()
    assert helpers.same_f32(scales, want_scales).all()


def test_quotient_check_under_asan(tmp_path):
    exe = tmp_path / "quotient_check_asan"
    subprocess.run(["gcc", "-O1", "-g", "-fopenmp", "-ffp-contract=off", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=all", str(ROOT / "tests" / "csrc" / "quotient_check.c"), "-o", str(exe),
                    "-lm"], check=True, capture_output=True, timeout=300)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, env=SAN_ENV)
    assert r.returncode == 0, r.stderr[-4000:]
    pairs, bad_code, bad_big, _ = map(int, r.stdout.split())
    assert pairs == 1065402240 and bad_code == 0 and bad_big == 0
