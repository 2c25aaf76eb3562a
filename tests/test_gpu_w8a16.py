"""Parity of the W8A16 parity mode (bf16 activations x e4m3 weights, the
reference's own arithmetic) with the oracle, under the reference's two
acceptance tests for that arithmetic:

* model/metal_test.py:202-224 -- at least 99.9% of outputs bitwise equal to
  ``((x.float() @ w8.float().t()) * scale).to(bf16)`` (``oracle.w8a16_math``)
  and every output within ``|exact| 2^-8 + magnitude 2^-20`` of the float64
  result, on its six shapes; a bias is ``bf16(y + bias)``; every e4m3 code;
* inference/cuda_test.py:74-94 -- at least 99.5% of outputs bitwise equal to
  the float64 product rounded once to bf16, finite, and identical on a second
  call, on its four weights and nine row counts with outliers and tiny rows.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jeeves_amd import _lib
from jeeves_amd.fp8 import FP8Linear, FP8SwiGLU, fp8_matmul_w8a16, tile_weight
from jeeves_amd.fp8_weights import FP8, quantize_rows
from tests import helpers

pytestmark = pytest.mark.gpu

MATH_EQUAL_MIN = 0.999   # model/metal_test.py:219
EXACT_EQUAL_MIN = 0.995  # inference/cuda_test.py:90
BOUND_MAGNITUDE = 2.0 ** -20  # model/metal_test.py:220


def f64_parts(x: torch.Tensor, wq: torch.Tensor, sw: torch.Tensor, cols=None):
    """(exact, magnitude) in float64 on the host for the chosen columns."""
    xd = oracle.bf16_to_f32(helpers.bits(x)).astype(np.float64)
    w = oracle.e4m3_decode(helpers.codes_np(wq)).astype(np.float64) * sw.cpu().numpy().astype(np.float64)[:, None]
    if cols is not None:
        w = w[cols]
    return xd @ w.T, np.abs(xd) @ np.abs(w).T


def columns(N: int, limit: int = 1536) -> np.ndarray | None:
    """All columns for small N; otherwise a fixed spread including both ends
    (the float64 reference at N=17408 would dominate the test's time)."""
    if N <= limit:
        return None
    return np.unique(np.concatenate([np.arange(256), np.linspace(0, N - 1, limit - 512).astype(np.int64), np.arange(N - 256, N)]))


# model/metal_test.py:208: (activation shape, K, N)
METAL_SHAPES = [((1,), 256, 16), ((3,), 4096, 1024), ((12,), 4096, 4096), ((2, 8), 12288, 4096), ((37,), 4096, 8192),
                ((300,), 1024, 2048)]


@pytest.mark.parametrize("shape,K,N", METAL_SHAPES)
def test_w8a16_matches_reference_math(shape, K, N):
    g = torch.Generator().manual_seed(6 + K + N)
    wq, sw = quantize_rows((torch.randn(N, K, generator=g) * 0.02).cuda())
    x = torch.randn(*shape, K, generator=g).to(torch.bfloat16)
    x2 = x.reshape(-1, K).cuda()
    out = helpers.bits(fp8_matmul_w8a16(x2, wq, sw))
    math = oracle.w8a16_math(helpers.bits(x2), helpers.codes_np(wq), sw.cpu().numpy())
    equal = oracle.bitwise_equal_fraction(out, math)
    exact, magnitude = f64_parts(x2, wq, sw)
    assert equal >= MATH_EQUAL_MIN, (shape, K, N, equal)
    assert oracle.within_metal_bound(oracle.bf16_to_f32(out), exact, magnitude * (BOUND_MAGNITUDE / 2.0 ** -20)), (shape, K, N)


# inference/cuda_test.py:78-82: weights and row counts
CUDA_WEIGHTS = [(4096, 4096), (1024, 12288), (1040, 4096), (17408, 4096)]
CUDA_ROWS = (1, 4, 12, 16, 17, 48, 256, 300, 1024)


@pytest.mark.parametrize("N,K", CUDA_WEIGHTS)
def test_w8a16_exact_rounding(N, K):
    g = torch.Generator().manual_seed(1 + N + K)
    wq, sw = quantize_rows((torch.randn(N, K, generator=g) * (1.0 / K ** 0.5)).cuda())
    cols = columns(N)
    for M in CUDA_ROWS:
        x = torch.randn(M, K, generator=g).to(torch.bfloat16)
        # outliers in odd rows, tiny rows (inference/cuda_test.py:83-85)
        x[1::2, 0] = 1e5
        x[2::4] *= 2 ** -20
        x = x.cuda()
        y = fp8_matmul_w8a16(x, wq, sw)
        again = fp8_matmul_w8a16(x, wq, sw)
        assert torch.equal(y, again), (N, K, M, "second call differs")
        out = helpers.bits(y if cols is None else y[:, torch.from_numpy(cols).cuda()])
        exact, _ = f64_parts(x, wq, sw, cols)
        exact_bits = oracle.f64_to_bf16(exact)
        assert np.isfinite(oracle.bf16_to_f32(out)).all(), (N, K, M)
        same = oracle.bitwise_equal_fraction(out, exact_bits)
        assert same >= EXACT_EQUAL_MIN, (N, K, M, same)


# The FP8 decode kernel's short-tail cases (tests/test_gpu_gemm.py): k ranges
# whose length leaves 1-3 steps after a wave's full bursts of U steps, with and
# without split-K.
SHORT_TAILS = [(7, 16, 6656), (7, 4096, 6656), (16, 96, 6656), (7, 16, 4224), (7, 16, 4608), (7, 4096, 6528),
               (7, 4096, 5632), (7, 4096, 3968), (7, 4096, 1152), (33, 4096, 6656), (31, 16, 2688), (3, 1040, 2432)]


@pytest.mark.parametrize("M,N,K", SHORT_TAILS)
def test_w8a16_k_ranges_with_short_tails(M, N, K):
    """The W8A16 decode kernel's guarded last burst of 1-3 steps: the
    reference's Metal acceptance (>= 99.9% equal to the fp32 math, the float64
    bound with magnitude 2^-20) and a bitwise-equal second call."""
    g = torch.Generator().manual_seed(M + N + K)
    wq, sw = quantize_rows((torch.randn(N, K, generator=g) * 0.02).cuda())
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
    y = fp8_matmul_w8a16(x, wq, sw)
    assert torch.equal(y, fp8_matmul_w8a16(x, wq, sw)), (M, N, K)
    assert torch.equal(fp8_matmul_w8a16(x, tile_weight(wq), sw, tiled=True), y) if N % 16 == 0 else True
    out = helpers.bits(y)
    math = oracle.w8a16_math(helpers.bits(x), helpers.codes_np(wq), sw.cpu().numpy())
    exact, magnitude = f64_parts(x, wq, sw)
    assert oracle.bitwise_equal_fraction(out, math) >= MATH_EQUAL_MIN, (M, N, K)
    assert oracle.within_metal_bound(oracle.bf16_to_f32(out), exact, magnitude * (BOUND_MAGNITUDE / 2.0 ** -20)), (M, N, K)


@pytest.mark.parametrize("M", [5, 64, 65, 2048])
def test_w8a16_large_tiles_and_bias(M):
    """The 256x256 prefill tile (M=2048 over 16384 channels), decode and the
    smallest prefill; with a bias the output is bf16(bf16(acc*s) + bias)
    bitwise (the reference adds its bias to the bf16 GEMM output,
    inference/fp8.py:183-184; model/metal_test.py:240)."""
    N, K = 16384, 4096
    g = torch.Generator().manual_seed(M)
    wq, sw = quantize_rows((torch.randn(N, K, generator=g) * 0.02).cuda())
    bias = (torch.randn(N, generator=g) * 0.5).to(torch.bfloat16).cuda()
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
    y = fp8_matmul_w8a16(x, wq, sw)
    yb = fp8_matmul_w8a16(x, wq, sw, bias=bias)
    assert torch.equal(yb, y + bias)
    cols = columns(N)
    sel = torch.from_numpy(cols).cuda()
    out = helpers.bits(y[:, sel])
    math = oracle.w8a16_math(helpers.bits(x), helpers.codes_np(wq)[cols], sw.cpu().numpy()[cols])
    assert oracle.bitwise_equal_fraction(out, math) >= MATH_EQUAL_MIN


@pytest.mark.parametrize("N", [24576, 24592])
def test_w8a16_wide_small_batches_take_64x64_prefill_tiles(N):
    """32-64 tokens over a weight wide enough for 1.5 rounds of 64-channel
    tiles (the fused gate+up, 24576 channels; 24592 leaves a ragged last
    tile) run on the 64x64 prefill tiles, 17 tokens on the decode kernel;
    neither needs a workspace. The exact-rounding acceptance
    (inference/cuda_test.py:83-90) with outliers and tiny rows, tiled weights
    equal to row-major ones, the bias bitwise."""
    K = 4096
    g = torch.Generator().manual_seed(N)
    wq, sw = quantize_rows((torch.randn(N, K, generator=g) * (1.0 / K ** 0.5)).cuda())
    wt = tile_weight(wq)
    bias = (torch.randn(N, generator=g) * 0.5).to(torch.bfloat16).cuda()
    cols = columns(N)
    sel = torch.from_numpy(cols).cuda()
    for M in (17, 32, 40, 64):
        assert _lib.lib().jv_w8a16_workspace_bytes(M, N, K) == 0, (N, M)
        x = torch.randn(M, K, generator=g).to(torch.bfloat16)
        x[1::2, 0] = 1e5
        x[2::4] *= 2 ** -20
        x = x.cuda()
        y = fp8_matmul_w8a16(x, wq, sw)
        assert torch.equal(fp8_matmul_w8a16(x, wt, sw, tiled=True), y), (N, M)
        assert torch.equal(fp8_matmul_w8a16(x, wq, sw, bias=bias), y + bias), (N, M)
        out = helpers.bits(y[:, sel])
        exact, _ = f64_parts(x, wq, sw, cols)
        assert np.isfinite(oracle.bf16_to_f32(out)).all(), (N, M)
        assert oracle.bitwise_equal_fraction(out, oracle.f64_to_bf16(exact)) >= EXACT_EQUAL_MIN, (N, M)


# 17-128 tokens that take the W8A16 batch-decode plan: k/v (1024 x 4096),
# q/o (4096 x 4096), a ragged 1040 channels; token counts whose last tile is
# partly outside.
@pytest.mark.parametrize("N,K,M", [(1024, 4096, 17), (1024, 4096, 48), (1024, 4096, 64), (1024, 4096, 80),
                                   (1024, 4096, 128), (4096, 4096, 32), (4096, 4096, 64), (4096, 4096, 96),
                                   (4096, 4096, 128), (1040, 4096, 40)])
def test_w8a16_batch_decode(N, K, M):
    """The batch-decode form: the reference's Metal acceptance (>= 99.9% equal
    to the fp32 math, the float64 bound), every output bitwise equal to its
    16-token slice on the W8A16 decode kernel (same waves per row), tiled
    weights equal to row-major ones, the bias bitwise, no workspace."""
    print(f"w8a16 batch N={N} K={K} M={M}", flush=True)
    assert _lib.lib().jv_w8a16_workspace_bytes(M, N, K) == 0
    g = torch.Generator().manual_seed(N + M)
    wq, sw = quantize_rows((torch.randn(N, K, generator=g) * 0.02).cuda())
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
    bias = (torch.randn(N, generator=g) * 0.5).to(torch.bfloat16).cuda()
    y = fp8_matmul_w8a16(x, wq, sw)
    assert torch.equal(y, torch.cat([fp8_matmul_w8a16(x[i:i + 16], wq, sw) for i in range(0, M, 16)])), (N, M)
    if N % 16 == 0:
        assert torch.equal(fp8_matmul_w8a16(x, tile_weight(wq), sw, tiled=True), y), (N, M)
    assert torch.equal(fp8_matmul_w8a16(x, wq, sw, bias=bias), y + bias), (N, M)
    out = helpers.bits(y)
    math = oracle.w8a16_math(helpers.bits(x), helpers.codes_np(wq), sw.cpu().numpy())
    exact, magnitude = f64_parts(x, wq, sw)
    assert oracle.bitwise_equal_fraction(out, math) >= MATH_EQUAL_MIN, (N, M)
    assert oracle.within_metal_bound(oracle.bf16_to_f32(out), exact, magnitude * (BOUND_MAGNITUDE / 2.0 ** -20)), (N, M)


# K split across workgroups on the prefill kernel's 64x64 tiles (at most a
# third of a round of them): k/v at 129-320 tokens, a ragged 1040 channels,
# a short k range (8 stages per split).
@pytest.mark.parametrize("N,K,M", [(1024, 4096, 130), (1024, 4096, 256), (1024, 4096, 300), (1040, 4096, 200),
                                   (1040, 4096, 300), (1024, 2048, 192)])
def test_w8a16_split_prefill(N, K, M):
    """The split form: the reference's Metal acceptance (>= 99.9% equal to the
    fp32 math, the float64 bound), identical on a second call, tiled weights
    equal to row-major ones, the bias bitwise."""
    print(f"w8a16 split prefill N={N} K={K} M={M}", flush=True)
    assert _lib.lib().jv_w8a16_workspace_bytes(M, N, K) > 0
    g = torch.Generator().manual_seed(N + M + 1)
    wq, sw = quantize_rows((torch.randn(N, K, generator=g) * 0.02).cuda())
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
    bias = (torch.randn(N, generator=g) * 0.5).to(torch.bfloat16).cuda()
    y = fp8_matmul_w8a16(x, wq, sw)
    assert torch.equal(fp8_matmul_w8a16(x, wq, sw), y), (N, M)
    if N % 16 == 0:
        assert torch.equal(fp8_matmul_w8a16(x, tile_weight(wq), sw, tiled=True), y), (N, M)
    assert torch.equal(fp8_matmul_w8a16(x, wq, sw, bias=bias), y + bias), (N, M)
    out = helpers.bits(y)
    math = oracle.w8a16_math(helpers.bits(x), helpers.codes_np(wq), sw.cpu().numpy())
    exact, magnitude = f64_parts(x, wq, sw)
    assert oracle.bitwise_equal_fraction(out, math) >= MATH_EQUAL_MIN, (N, M)
    assert oracle.within_metal_bound(oracle.bf16_to_f32(out), exact, magnitude * (BOUND_MAGNITUDE / 2.0 ** -20)), (N, M)


@pytest.mark.parametrize("M", [16, 64, 256])
def test_w8a16_every_code(M):
    """Every e4m3 code through the in-kernel widening: weight row n holds code
    n in every column, x is one-hot, so y[m,n] is the code's value (NaN codes
    give NaN) -- the role of model/metal_test.py:205's check on every code."""
    K, N = 256, 256
    codes = torch.arange(N, dtype=torch.uint8)[:, None].expand(N, K).contiguous()
    wq = codes.view(FP8).cuda()
    sw = torch.ones(N, dtype=torch.float32, device="cuda")
    x = torch.zeros(M, K, dtype=torch.bfloat16)
    x[torch.arange(M), (torch.arange(M) * 7) % K] = 1.0
    y = fp8_matmul_w8a16(x.cuda(), wq, sw).float().cpu().numpy()
    want = np.broadcast_to(oracle.e4m3_decode(np.arange(256, dtype=np.uint8)), (M, N))
    nan = np.isnan(want)
    assert (np.isnan(y) == nan).all()
    assert (y[~nan] == want[~nan]).all()  # every finite e4m3 value is a bf16 value: exact


def test_w8a16_module_mode():
    """FP8Linear.set_activations("bf16") runs the parity mode with its bias;
    the SwiGLU block in that mode feeds bf16 silu(gate)*up to the down GEMM."""
    K, N = 1024, 2048
    g = torch.Generator().manual_seed(11)
    lin = FP8Linear(K, N, bias=True, device="cuda")
    lin.load_weight((torch.randn(N, K, generator=g) * 0.02).cuda())
    lin.bias.copy_((torch.randn(N, generator=g) * 0.1).to(torch.bfloat16))
    lin.set_activations("bf16")
    x = torch.randn(3, 5, K, generator=g).to(torch.bfloat16).cuda()
    assert torch.equal(lin(x), (fp8_matmul_w8a16(x.reshape(-1, K), lin.weight, lin.scale) + lin.bias).view(3, 5, N))
    with pytest.raises(ValueError):
        lin.set_lora(torch.zeros(16, K), torch.zeros(N, 16), 1.0)

    inter = 1024
    gate_up = FP8Linear(K, 2 * inter, device="cuda")
    gate_up.load_weight((torch.randn(2 * inter, K, generator=g) * 0.02).cuda())
    down = FP8Linear(inter, K, device="cuda")
    down.load_weight((torch.randn(K, inter, generator=g) * 0.02).cuda())
    gate_up.set_activations("bf16")
    down.set_activations("bf16")
    block = FP8SwiGLU(gate_up, down)
    for M in (4, 100):
        xm = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
        gu = fp8_matmul_w8a16(xm, gate_up.weight, gate_up.scale)
        h = oracle.swiglu_bf16(helpers.bits(gu[:, :inter]), helpers.bits(gu[:, inter:]))
        want = fp8_matmul_w8a16(helpers.from_bits(h, "cuda"), down.weight, down.scale)
        assert torch.equal(block(xm), want)


def test_w8a16_rejects_bad_k():
    """K not a multiple of 128 or not the weight's raises ValueError
    (inference/fp8.py:115-117; model/metal_test.py:225-231)."""
    x = torch.zeros(4, 4096 + 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        fp8_matmul_w8a16(x, torch.zeros(1024, 4096 + 64, dtype=torch.uint8, device="cuda").view(FP8),
                         torch.ones(1024, device="cuda"))
    with pytest.raises(ValueError):
        fp8_matmul_w8a16(torch.zeros(4, 4096, dtype=torch.bfloat16, device="cuda"),
                         torch.zeros(1024, 4096 + 128, dtype=torch.uint8, device="cuda").view(FP8), torch.ones(1024, device="cuda"))
