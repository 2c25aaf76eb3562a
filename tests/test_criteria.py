"""The FP8 GEMM acceptance criteria of tests/helpers.py on the CPU: the exact
product rounded once passes them, and planted mistakes fail them -- one bf16
unit on 2.5 % of the outputs fails the equal-share bar, and an error of
magnitude * 2^-11.5 on a single output (inside the 2^-11 allowance the bound
used before) fails the bound."""

from __future__ import annotations

import numpy as np

import oracle
from tests import helpers


def _case(M=64, N=512, K=512, seed=5):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[:, rng.choice(K, 4, replace=False)] *= 20
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    xq, sx = oracle.quantize_rows(x)
    wq, sw = oracle.quantize_rows(w)
    return xq, sx, wq, sw


def test_equal_floor_values():
    assert abs(helpers.equal_floor(1 << 18, 0.98) - 0.97917) < 1e-5
    assert abs(helpers.equal_floor(1024, 0.98) - 0.96688) < 1e-5
    assert helpers.equal_floor(0, 0.98) == 0.0


def test_exact_rounding_passes_and_one_unit_on_a_few_percent_fails():
    xq, sx, wq, sw = _case()
    exact_bits = oracle.f64_to_bf16(oracle.gemm_exact_f64(xq, sx, wq, sw))
    c = helpers.gemm_criteria(exact_bits, xq, sx, wq, sw)
    assert c["equal"] == 1.0 and c["bound"] and c["finite_match"] and c["n"] == exact_bits.size
    rng = np.random.default_rng(6)
    flat = exact_bits.reshape(-1).copy()
    flat[rng.choice(flat.size, int(0.025 * flat.size), replace=False)] += np.uint16(1)
    c = helpers.gemm_criteria(flat.reshape(exact_bits.shape), xq, sx, wq, sw)
    assert c["equal"] < helpers.equal_floor(c["n"], helpers.EQUAL_MIN), c["equal"]
    # the same share of errors stays inside the previous flat 97 % bar
    assert c["equal"] >= 0.97


def test_error_of_magnitude_2_pow_minus_11_5_fails_the_bound():
    xq, sx, wq, sw = _case()
    exact = oracle.gemm_exact_f64(xq, sx, wq, sw)
    mag = helpers.gemm_magnitude(xq, sx, wq, sw)
    # the output with the most cancellation, where the magnitude term dominates
    m, n = np.unravel_index(np.argmin(np.abs(exact) / mag), exact.shape)
    out = exact.copy()
    out[m, n] = exact[m, n] + mag[m, n] * 2.0 ** -11.5
    out_bits = oracle.f64_to_bf16(out)
    got = oracle.bf16_to_f32(out_bits).astype(np.float64)
    assert abs(got[m, n] - exact[m, n]) <= abs(exact[m, n]) * 2.0 ** -8 + mag[m, n] * 2.0 ** -11  # the old bound
    assert not helpers.gemm_criteria(out_bits, xq, sx, wq, sw)["bound"]
