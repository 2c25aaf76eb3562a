"""Device conformance of the building blocks the kernels rely on:
the hardware e4m3 converter vs the OCP spec encoder, the quantizer's fast
quotient over every bf16 input pair, and the FP8 MFMA lane layouts."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from tests import helpers

pytestmark = pytest.mark.gpu


def _check(rc: int) -> None:
    assert rc == 0, f"hook returned {rc}"


def test_device_encoders_on_golden_inputs(hooks_lib):
    g = helpers.golden("e4m3_encode.npz")
    inp = torch.from_numpy(g["inputs"]).cuda()
    n = inp.numel()
    hw = torch.empty(n, dtype=torch.uint8, device="cuda")
    sw = torch.empty(n, dtype=torch.uint8, device="cuda")
    _check(hooks_lib.th_encode(inp.data_ptr(), hw.data_ptr(), sw.data_ptr(), n, helpers.stream()))
    torch.cuda.synchronize()
    sw_np, hw_np = sw.cpu().numpy(), hw.cpu().numpy()
    # the device spec encoder equals torch's cast everywhere
    assert helpers.same_codes(sw_np, g["codes"]).all()
    # the hardware converter equals it on the quantizer's domain |f| <= 449
    domain = np.abs(g["inputs"]) <= 449.0
    assert domain.sum() > 1000
    assert helpers.same_codes(hw_np[domain], g["codes"][domain]).all()


def _sweep(hooks_lib, start: int, n: int) -> np.ndarray:
    counts = torch.zeros(3, dtype=torch.int64, device="cuda")
    first = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    _check(hooks_lib.th_encode_sweep(start, n, counts.data_ptr(), first.data_ptr(), helpers.stream()))
    torch.cuda.synchronize()
    return counts.cpu().numpy()


def test_hardware_encoder_equals_spec_on_whole_domain(hooks_lib):
    top = int(np.float32(449.0).view(np.uint32))
    pos = _sweep(hooks_lib, 0, top + 1)
    neg = _sweep(hooks_lib, 0x80000000, top + 1)
    assert pos[2] == top + 1 and neg[2] == top + 1   # every float with |f| <= 449 was checked
    assert pos[0] == 0 and neg[0] == 0
    # outside the domain (NaN, inf, overflow band) the hardware may differ; report it
    rest = _sweep(hooks_lib, top + 1, 0x80000000 - top - 1)
    print(f"hardware vs spec encoder outside |f|<=449: {int(rest[1])} differing positive patterns")


def test_fast_quotient_exhaustive_on_device(hooks_lib):
    counts = torch.zeros(3, dtype=torch.int64, device="cuda")
    first = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    for begin in range(0, 0x7F80, 8160):
        _check(hooks_lib.th_quotient_sweep(begin, min(8160, 0x7F80 - begin), counts.data_ptr(), first.data_ptr(),
                                           helpers.stream()))
    torch.cuda.synchronize()
    quotient_bits, code_mismatch, pairs = counts.cpu().numpy().tolist()
    assert pairs == 1065402240
    assert code_mismatch == 0, hex(first.item() & 0xFFFFFFFF)
    # the CPU check bounds these to |q| < 2^-11, where both codes are signed zeros
    assert quotient_bits <= 1969204


def _lane_operands(rows: int, kper: int, mat: np.ndarray) -> np.ndarray:
    """Pack a [rows, 64*32/rows] code matrix into 64 lanes x 32 bytes: lane l holds
    row l % rows, k bytes 32*(l // rows) .. +32 (the layout the kernels load)."""
    out = np.zeros((64, 32), np.uint8)
    for l in range(64):
        out[l] = mat[l % rows, 32 * (l // rows): 32 * (l // rows) + 32]
    return out


def _random_codes(rng, shape) -> np.ndarray:
    c = rng.integers(0, 256, shape, dtype=np.uint8)
    c[np.isnan(oracle.e4m3_decode(c))] = 0x38
    # keep magnitudes moderate so every fp32 sum is exact
    c[np.abs(oracle.e4m3_decode(c)) > 8] = 0x40
    return c


@pytest.mark.parametrize("shape", ["32x32x64", "16x16x128"])
def test_mfma_output_layout(hooks_lib, shape):
    rows, k = (32, 64) if shape == "32x32x64" else (16, 128)
    regs = 16 if rows == 32 else 4
    rng = np.random.default_rng(9)
    A = _random_codes(rng, (rows, k))
    B = _random_codes(rng, (rows, k))   # B[j, k]: column j of the MFMA's B operand
    a = torch.from_numpy(_lane_operands(rows, k, A)).cuda()
    b = torch.from_numpy(_lane_operands(rows, k, B)).cuda()
    d = torch.zeros(64, regs, dtype=torch.float32, device="cuda")
    fn = hooks_lib.th_mfma32 if rows == 32 else hooks_lib.th_mfma16
    _check(fn(a.data_ptr(), b.data_ptr(), d.data_ptr(), helpers.stream()))
    torch.cuda.synchronize()
    D = oracle.e4m3_decode(A).astype(np.float64) @ oracle.e4m3_decode(B).astype(np.float64).T
    got = d.cpu().numpy()
    for l in range(64):
        for r in range(regs):
            if rows == 32:
                i, j = 8 * (r // 4) + 4 * (l // 32) + (r % 4), l % 32
            else:
                i, j = 4 * (l // 16) + r, l % 16
            assert got[l, r] == D[i, j], (l, r)
