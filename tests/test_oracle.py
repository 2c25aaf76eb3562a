"""Pins the CPU oracle (oracle/fp8_ref.py) before it is trusted as the checker:
against torch's own e4m3fn cast and decode (the library the reference calls),
the committed golden fixtures, known answers from the OCP FP8 spec and the
reference's constants, invariants, and brute force on tiny shapes."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests import helpers

FP8 = torch.float8_e4m3fn


# ----------------------------------------------------------------- e4m3 codec

def test_decode_matches_torch_and_golden():
    g = helpers.golden("e4m3_decode.npz")
    assert np.array_equal(oracle.e4m3_decode(g["codes"]), g["values"], equal_nan=True)
    live = torch.arange(256, dtype=torch.uint8).view(FP8).float().numpy()
    assert np.array_equal(oracle.E4M3_TABLE, live, equal_nan=True)


def test_decode_known_answers_from_ocp_spec():
    t = oracle.E4M3_TABLE
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0          # largest finite, S.1111.110
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])          # the only NaNs, S.1111.111
    assert np.isnan(t).sum() == 2
    assert t[0x08] == 2.0 ** -6                              # smallest normal
    assert t[0x01] == 2.0 ** -9 and t[0x07] == 7 * 2.0 ** -9  # subnormals m * 2^-9
    assert t[0x38] == 1.0 and t[0x39] == 1.125               # bias 7, 3 mantissa bits
    assert t[0x00] == 0.0 and np.signbit(t[0x80])
    finite = t[np.isfinite(t)]
    assert len(np.unique(finite)) == 253                     # +0 and -0 equal, 2 NaNs


def test_encode_matches_golden():
    g = helpers.golden("e4m3_encode.npz")
    got = oracle.e4m3_encode(g["inputs"])
    assert helpers.same_codes(got, g["codes"]).all()
    # NaN positions equal (the sign of a NaN may differ between platforms)
    assert np.array_equal(np.isnan(oracle.e4m3_decode(got)), np.isnan(oracle.e4m3_decode(g["codes"])))


def test_encode_dense_sweep_matches_torch_cast():
    rng = np.random.default_rng(1)
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    f = np.concatenate([hi, hi | rng.integers(0, 1 << 16, 1 << 16, dtype=np.uint32), hi | 0x8000, hi | 0x7FFF]).view(np.float32)
    want = torch.from_numpy(f.copy()).to(FP8).view(torch.uint8).numpy()
    assert helpers.same_codes(oracle.e4m3_encode(f), want).all()


def test_encode_known_answers():
    cases = {448.0: 0x7E, 456.0: 0x7E, 464.0: 0x7E, 480.0: 0x7F, 1e9: 0x7F, float("inf"): 0x7F, 2.0 ** -9: 0x01,
             2.0 ** -10: 0x00, 3 * 2.0 ** -11: 0x01, 1.0: 0x38, 1.0625: 0x38, 1.1875: 0x3A, -2.0 ** -10: 0x80, -0.0: 0x80}
    for v, c in cases.items():
        assert oracle.e4m3_encode(np.float32(v)) == c, v
    nxt = np.nextafter(np.float32(464.0), np.float32(1e9))
    assert oracle.e4m3_encode(nxt) == 0x7F                   # just above the 448/480 midpoint -> NaN
    assert oracle.e4m3_encode(np.float32(-np.inf)) == 0xFF


def test_encode_decode_round_trip_on_every_finite_code():
    codes = np.arange(256, dtype=np.uint8)
    finite = codes[np.isfinite(oracle.e4m3_decode(codes))]
    assert np.array_equal(oracle.e4m3_encode(oracle.e4m3_decode(finite)), finite)


# ----------------------------------------------------------------- bf16 rounding

def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(2)
    f = np.concatenate([rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32),
                        np.array([np.inf, -np.inf, 3.4e38, -3.4e38, 1e-45, 0.0, -0.0], np.float32)])
    want = helpers.bits(torch.from_numpy(f.copy()))
    got = oracle.f32_to_bf16(f)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.isnan(oracle.bf16_to_f32(got[nan])).all()
    # double -> bf16 goes through float, as torch does (double rounding)
    d = np.array([1 + 2.0 ** -8 + 2.0 ** -40, -(1 + 2.0 ** -8 + 2.0 ** -40), 1e300])
    assert np.array_equal(oracle.f64_to_bf16(d), helpers.bits(torch.from_numpy(d).to(torch.bfloat16)))


# ----------------------------------------------------------------- quantize_rows

def test_reciprocal_constant():
    # inference/fp8_weights.py:10: float(torch.tensor(1/448, float32)) == 0x1.24924ap-9
    assert oracle.FP8_MAX_RECIPROCAL.view(np.uint32) == 0x3B124925
    assert float(oracle.FP8_MAX_RECIPROCAL) == float.fromhex("0x1.24924ap-9")


def test_quantize_rows_matches_golden_edge_rows():
    g = helpers.golden("quantize_rows.npz")
    codes, scales = oracle.quantize_rows(oracle.bf16_to_f32(g["edge_x"]))
    assert helpers.same_f32(scales, g["edge_scales"]).all()
    assert helpers.same_codes(codes, g["edge_codes"]).all()


def test_quantize_rows_matches_golden_workload_rows():
    g = helpers.golden("quantize_rows.npz")
    for tag in ("cfg0_x", "cfg0_w64"):
        codes, scales = oracle.quantize_rows(oracle.bf16_to_f32(g[tag]))
        assert np.array_equal(scales.view(np.uint32), g[f"{tag}_scales"].view(np.uint32)), tag
        assert np.array_equal(codes, g[f"{tag}_codes"]), tag


def test_quantize_rows_known_answers():
    codes, scales = oracle.quantize_rows(np.array([[1.0, 0.5, -0.25, 0.0]], np.float32))
    assert scales[0] == oracle.FP8_MAX_RECIPROCAL
    assert list(codes[0]) == [0x7E, 0x76, 0xEE, 0x00]  # 448, 224, -112, 0
    # all-zero row: scale is the clamp times the reciprocal, codes zero
    codes, scales = oracle.quantize_rows(np.zeros((1, 8), np.float32))
    assert scales[0] == np.float32(np.float32(1e-12) * oracle.FP8_MAX_RECIPROCAL)
    assert not codes.any()
    # a row holding inf: scale inf, finite entries -> 0, inf entries -> NaN
    codes, scales = oracle.quantize_rows(np.array([[1.0, np.inf, -2.0, -np.inf]], np.float32))
    assert np.isinf(scales[0])
    assert codes[0, 0] == 0x00 and codes[0, 2] == 0x80
    assert np.isnan(oracle.e4m3_decode(codes[0, [1, 3]])).all()
    # a NaN anywhere makes the whole row NaN
    codes, scales = oracle.quantize_rows(np.array([[1.0, np.nan, 3.0]], np.float32))
    assert np.isnan(scales[0]) and np.isnan(oracle.e4m3_decode(codes[0])).all()
    # multiply by the float32 reciprocal, not divide by 448: these maxima differ
    amax = np.float32(3.0)
    assert np.float32(amax * oracle.FP8_MAX_RECIPROCAL) != np.float32(amax / np.float32(448.0))
    _, s = oracle.quantize_rows(np.array([[3.0, -1.0]], np.float32))
    assert s[0] == np.float32(amax * oracle.FP8_MAX_RECIPROCAL)


def test_quantize_rows_invariants():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((256, 1024)) * np.logspace(-20, 20, 256)[:, None]).astype(np.float32)
    w = oracle.bf16_to_f32(oracle.f32_to_bf16(w))
    codes, scales = oracle.quantize_rows(w)
    arg = np.abs(w).argmax(axis=1)
    top = codes[np.arange(256), arg]
    unclamped = np.abs(w).max(axis=1) >= np.float32(1e-12)
    assert unclamped.sum() > 100 and (~unclamped).sum() > 10
    assert np.isin(top[unclamped], [0x7E, 0xFE]).all()     # the amax element encodes to +-448
    clamp_scale = np.float32(np.float32(1e-12) * oracle.FP8_MAX_RECIPROCAL)
    assert (scales[~unclamped] == clamp_scale).all()        # rows below the clamp share one scale
    assert not np.isnan(oracle.e4m3_decode(codes)).any()    # finite rows never produce NaN
    deq = oracle.e4m3_decode(codes).astype(np.float64) * scales[:, None]
    # half an e4m3 step: 2^-4 relative for normals, 2^-10 * scale in the subnormal range
    bound = np.maximum(np.abs(w) * 2.0 ** -4, scales[:, None].astype(np.float64) * 2.0 ** -10) * (1 + 1e-6)
    assert (np.abs(deq - w) <= bound).all()


def test_quantize_rows_live_torch_on_random_rows():
    g = torch.Generator().manual_seed(4)
    w = (torch.randn(300, 640, generator=g) * torch.logspace(-30, 30, 300)[:, None]).to(torch.bfloat16)
    wf = w.float()
    scale = wf.abs().amax(1).clamp(min=1e-12) * float(torch.tensor(1 / 448, dtype=torch.float32))
    want = (wf / scale[:, None]).to(FP8).view(torch.uint8).numpy()
    codes, scales = oracle.quantize_rows(wf.numpy())
    assert np.array_equal(scales.view(np.uint32), scale.numpy().view(np.uint32))
    assert np.array_equal(codes, want)


def test_quantize_row_blocks():
    w = np.random.default_rng(5).standard_normal((oracle.QUANTIZE_BLOCK_ROWS + 3, 16)).astype(np.float32)
    blocks = list(oracle.quantize_row_blocks_on_cpu(w))
    assert [b[0] for b in blocks] == [slice(0, 16384), slice(16384, 32768)]
    c, s = oracle.quantize_rows(w)
    assert np.array_equal(np.concatenate([b[1] for b in blocks]), c)
    assert np.array_equal(np.concatenate([b[2] for b in blocks]), s)


def test_quantizable_rule():
    assert oracle.quantizable(4096, 4096) and oracle.quantizable(256, 1024)
    assert not oracle.quantizable(4096, 1008) and not oracle.quantizable(4096, 1030) and not oracle.quantizable(4100, 4096)


# ----------------------------------------------------------------- fast quotient (device algorithm)

def test_fast_quotient_exhaustive_on_cpu(tmp_path: Path):
    """The device quantizer's one-multiply-two-FMA quotient, for every bf16 x and
    bf16 row maximum, gives the IEEE quotient's e4m3 code (tests/csrc/quotient_check.c)."""
    src = Path(__file__).with_name("csrc") / "quotient_check.c"
    exe = tmp_path / "quotient_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", str(src), "-o", str(exe), "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    pairs, bad_code, bad_big, _ = map(int, r.stdout.split())
    assert pairs == 1065402240
    assert bad_code == 0 and bad_big == 0 and r.returncode == 0


# ----------------------------------------------------------------- GEMM oracles

def test_gemm_exact_matches_golden():
    g = helpers.golden("gemm_small.npz")
    for tag in ("a", "b"):
        out = oracle.gemm_exact_bf16(g[f"{tag}_xq"], g[f"{tag}_xs"], g[f"{tag}_wq"], g[f"{tag}_ws"])
        assert np.array_equal(out, g[f"{tag}_exact"]), tag


def test_gemm_exact_brute_force():
    rng = np.random.default_rng(6)
    xq = rng.integers(0, 256, (3, 8), dtype=np.uint8)
    wq = rng.integers(0, 256, (4, 8), dtype=np.uint8)
    xq[np.isnan(oracle.e4m3_decode(xq))] = 0
    wq[np.isnan(oracle.e4m3_decode(wq))] = 0
    sx = rng.random(3).astype(np.float32)
    sw = rng.random(4).astype(np.float32)
    got = oracle.gemm_exact_f64(xq, sx, wq, sw)
    for m in range(3):
        for n in range(4):
            acc = sum(float(oracle.E4M3_TABLE[xq[m, k]]) * float(oracle.E4M3_TABLE[wq[n, k]]) for k in range(8))
            assert got[m, n] == acc * float(sx[m]) * float(sw[n])


def test_gemm_exact_identity_decodes_every_code():
    # check_kernel_on_every_code (inference/fp8_metal.py:38-46) restated: an
    # identity activation picks every finite code of a permuted table.
    codes = np.arange(256, dtype=np.uint8)
    finite = codes[np.isfinite(oracle.e4m3_decode(codes))]
    table = finite[(np.arange(256)[:, None] + np.arange(256)[None]) % len(finite)]
    eye = np.full((256, 256), 0x00, np.uint8)
    eye[np.arange(256), np.arange(256)] = 0x38  # 1.0
    picked = oracle.gemm_exact_f64(eye, np.ones(256, np.float32), table, np.ones(256, np.float32))
    assert np.array_equal(picked, oracle.e4m3_decode(table).astype(np.float64).T)


def test_w8a16_math_matches_golden():
    g = helpers.golden("gemm_small.npz")
    for tag in ("a", "b"):
        out = oracle.w8a16_math(g[f"{tag}_x"], g[f"{tag}_wq"], g[f"{tag}_ws"])
        assert oracle.bitwise_equal_fraction(out, g[f"{tag}_w8a16"]) >= 0.999, tag


def test_dequant_matmul_linearity_and_agreement():
    rng = np.random.default_rng(7)
    xq = rng.integers(0, 0x7E, (5, 128), dtype=np.uint8)
    wq = rng.integers(0, 0x7E, (6, 128), dtype=np.uint8)
    sx, sw = rng.random(5).astype(np.float32), rng.random(6).astype(np.float32)
    a = oracle.dequant_matmul_f64(xq, sx, wq, sw)
    assert np.allclose(a, oracle.gemm_exact_f64(xq, sx, wq, sw), rtol=1e-12)
    assert np.allclose(oracle.dequant_matmul_f64(xq, 2 * sx, wq, sw), 2 * a, rtol=1e-12)
    assert oracle.rel_l2(oracle.dequant_matmul_f32(xq, sx, wq, sw), a) < 1e-6


def test_lora_and_swiglu_closed_forms():
    rng = np.random.default_rng(8)
    x, a, b = rng.standard_normal((2, 6)), rng.standard_normal((3, 6)), rng.standard_normal((4, 3))
    got = oracle.lora_f64(x, a, b, 2.0)
    for m in range(2):
        for n in range(4):
            want = sum(sum(x[m, k] * a[r, k] for k in range(6)) * b[n, r] * 2.0 for r in range(3))
            assert abs(got[m, n] - want) < 1e-12


def test_swiglu_on_every_bf16_gate_value():
    """``F.silu(gate) * up`` (model/model.py:583) on all 65536 bf16 gate
    patterns, against torch's bf16 ops: silu alone (up = 1) and with random
    bf16 ups of both signs and wide exponent range. NaN results compare by
    position. (A float64 silu rounded once to bf16 would differ on 17 gates
    below -88.5, where torch's float32 exp overflows and silu gives -0.)"""
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    rng = np.random.default_rng(9)
    ups = [np.full(65536, 0x3F80, np.uint16),
           oracle.f32_to_bf16((rng.standard_normal(65536) * 2.0 ** rng.integers(-20, 20, 65536)).astype(np.float32))]
    for u in ups:
        want = helpers.bits(torch.nn.functional.silu(helpers.from_bits(g)) * helpers.from_bits(u))
        got = oracle.swiglu_bf16(g, u)
        assert oracle.bitwise_equal_fraction(got, want) == 1.0


def test_add_bias_matches_torch_bf16_add():
    """FP8Linear.forward's ``y + bias`` (inference/fp8.py:183-184) on bf16:
    random pairs over a wide exponent range, cancellations, ties and
    specials, against torch's bf16 add."""
    rng = np.random.default_rng(10)
    y = oracle.f32_to_bf16((rng.standard_normal((64, 512)) * 2.0 ** rng.integers(-30, 30, (64, 512))).astype(np.float32))
    b = oracle.f32_to_bf16((rng.standard_normal(512) * 2.0 ** rng.integers(-30, 30, 512)).astype(np.float32))
    y[0] = b ^ 0x8000  # exact cancellation
    y[1] = b  # doubling
    y[2, :8] = oracle.f32_to_bf16(np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 3e38, 1e-40, 1.0], np.float32))
    want = helpers.bits(helpers.from_bits(y) + helpers.from_bits(b))
    assert oracle.bitwise_equal_fraction(oracle.add_bias_bf16(y, b), want) == 1.0


def test_acceptance_helpers():
    a = oracle.f32_to_bf16(np.array([1.0, 2.0, np.nan], np.float32))
    b = oracle.f32_to_bf16(np.array([1.0, 2.5, np.nan], np.float32))
    assert oracle.bitwise_equal_fraction(a, b) == pytest.approx(2 / 3)
    assert oracle.within_metal_bound(np.array([1.0]), np.array([1.0 + 2.0 ** -9]), np.array([1.0]))
    assert not oracle.within_metal_bound(np.array([1.0]), np.array([1.0 + 2.0 ** -6]), np.array([1.0]))
