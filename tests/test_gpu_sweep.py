"""A seeded sweep of random GEMM shapes over every kernel regime: decode
(1-16 tokens, split-K on narrow weights, 8-wave bursts for K > 4096), 17-64
tokens on either kernel, and each prefill tile form (64x64 up to the 256x256
ping-pong tiles), with ragged N (row-major weights take any N, tiled ones
multiples of 16), K from 128 to 16384, bias, LoRA, and the reference's outlier
and tiny rows (inference/cuda_test.py:83-85). Each case checks:

* both quantizers bit-exact with the oracle (inference/fp8_weights.py:16-19):
  the weight's codes and scales, and the activation rows' codes and scales;
* the GEMM output against the oracle: finite where the exact result is and
  within the per-element bound of tests/helpers.py everywhere; the share
  bitwise equal to the exact result and the rel-L2 (the reference's
  aggregate acceptance numbers) once the output holds at least 4096 values,
  since a few dozen values leave too few for a 3 % rate (two or three
  one-ulp MFMA roundings out of 66 outputs would cross either threshold);
* tiled weights giving the same bits as row-major ones.

The oracle's float64 product bounds the sizes (M*N*K <= 6e9 per case)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jeeves_amd import synthetic
from jeeves_amd.fp8 import fp8_matmul, tile_weight
from jeeves_amd.fp8_weights import quantize_rows
from tests import helpers

pytestmark = pytest.mark.gpu

CASES = 40
MAX_MNK = 6e9
AGGREGATE_MIN_OUTPUTS = 4096


def sweep_shapes() -> list[tuple[int, int, int]]:
    rng = np.random.default_rng(20261202)
    # Forced first: 17-64 tokens on wide weights (64x64 prefill tiles, one
    # ragged), split-K decode with 8-wave bursts, a narrow split-K weight.
    shapes = [(24, 24592, 1024), (64, 24576, 1152), (16, 96, 12288), (9, 336, 2048)]
    buckets = [(1, 16), (17, 64), (65, 512), (513, 2304)]
    while len(shapes) < CASES:
        lo, hi = buckets[int(rng.integers(len(buckets)))]
        M = int(rng.integers(lo, hi + 1))
        N = int(np.exp(rng.uniform(np.log(3), np.log(32768))))
        if rng.integers(3):  # two in three take tiled weights too
            N = max(16, N // 16 * 16)
        K = 128 * int(np.exp(rng.uniform(0.0, np.log(128.0))))
        if M * N * K <= MAX_MNK:
            shapes.append((M, N, K))
    return shapes


SHAPES = sweep_shapes()


def same_bits_f32(a: np.ndarray, b: np.ndarray) -> bool:
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("case", range(CASES), ids=[f"M{m}-N{n}-K{k}" for m, n, k in SHAPES])
def test_random_shape(case):
    M, N, K = SHAPES[case]
    g = torch.Generator().manual_seed(7000 + case)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    if case % 4 == 1:
        x[1::2, 0] = 1e5
        x[2::4] *= 2 ** -20
    bias = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16).cuda() if case % 3 == 0 else None
    lora = None
    if case % 5 == 0:
        a, b = synthetic.lora_factors(N, K, 7100 + case)
        lora = (a.cuda(), b.cuda(), synthetic.LORA_SCALING)
    print(f"sweep case {case}: M={M} N={N} K={K} bias={bias is not None} lora={lora is not None}", flush=True)

    wq, sw = quantize_rows(w.cuda())
    codes_o, scales_o = oracle.quantize_rows(w.float().numpy())
    assert np.array_equal(helpers.codes_np(wq), codes_o), "weight codes differ from the oracle"
    assert same_bits_f32(sw.cpu().numpy(), scales_o), "weight scales differ from the oracle"
    xq_d, sx_d = quantize_rows(x.cuda())
    xq_o, sx_o = oracle.quantize_rows(x.float().numpy())
    assert np.array_equal(helpers.codes_np(xq_d), xq_o), "activation codes differ from the oracle"
    assert same_bits_f32(sx_d.cpu().numpy(), sx_o), "activation scales differ from the oracle"

    xc = x.cuda()
    y = fp8_matmul(xc, wq, sw, bias=bias, lora=lora)
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    lora_term = None
    if lora is not None:
        a, b, s = lora
        lora_term = oracle.lora_f64(oracle.bf16_to_f32(helpers.bits(xc)), oracle.bf16_to_f32(helpers.bits(a)),
                                    oracle.bf16_to_f32(helpers.bits(b)), s)
    c = helpers.gemm_criteria(helpers.bits(y), xq_o, sx_o, codes_o, scales_o,
                              bias_bits=helpers.bits(bias) if bias is not None else None, lora_term=lora_term)
    assert c["finite_match"], c
    assert c["bound"], c
    if M * N >= AGGREGATE_MIN_OUTPUTS:
        assert c["equal"] >= helpers.equal_floor(c["n"], helpers.EQUAL_MIN), c
        assert c["rel_l2"] <= helpers.REL_L2_MAX, c
    if N % 16 == 0:
        assert torch.equal(fp8_matmul(xc, tile_weight(wq), sw, bias=bias, lora=lora, tiled=True), y), "tiled differs"
