"""The batch-decode kernel (17-128 tokens on K = 4096 and K = 12288 weights
whose 16-row tiles fill at most one round of workgroups; the 9B model's q/o,
k/v, merged q/k/v and 8192-wide projections, and down up to 32 tokens):
* the oracle criteria (tests/helpers.py) on heavy-tailed activations, with
  bias and LoRA in the epilogue;
* every operand layout (packed or row-major codes, tiled or row-major
  weights) bitwise equal;
* every output bitwise equal to the decode kernel's on 16-token slices of the
  batch: both kernels give each output the same k order (the same waves per
  row, each wave's steps in order, waves summed in order), so the decode
  kernel's oracle parity carries over bit for bit, whatever the batch's token
  split across workgroups;
* writes confined to [M, N] of a strided output;
* the fused SwiGLU epilogue on a batch plan equal to the unfused steps, its
  per-16-channel maxima those of h."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from jeeves_amd import _lib, synthetic
from jeeves_amd.device import sm_count
from jeeves_amd.fp8 import fp8_matmul, fp8_matmul_quantized, gate_up_swiglu, swiglu_quantize, tile_weight
from jeeves_amd.fp8_weights import quantize_rows
from tests import helpers

pytestmark = pytest.mark.gpu


def launch_shape(M, N, K):
    shape = (ctypes.c_int32 * 4)()
    _lib.check(_lib.lib().jv_fp8_launch_shape(M, N, K, sm_count(torch.device("cuda:0")), shape))
    return list(shape)


def check(y, x, wq, sw, bias=None, lora=None):
    xq, sx = oracle.quantize_rows(x.float().cpu().numpy())
    lora_term = None
    if lora is not None:
        a, b, s = lora
        lora_term = oracle.lora_f64(oracle.bf16_to_f32(helpers.bits(x)), oracle.bf16_to_f32(helpers.bits(a)),
                                    oracle.bf16_to_f32(helpers.bits(b)), s)
    c = helpers.gemm_criteria(helpers.bits(y), xq, sx, helpers.codes_np(wq), sw.cpu().numpy(),
                              bias_bits=helpers.bits(bias) if bias is not None else None, lora_term=lora_term)
    assert c["finite_match"] and c["bound"], c
    assert c["equal"] >= helpers.equal_floor(c["n"], helpers.EQUAL_MIN) and c["rel_l2"] <= helpers.REL_L2_MAX, c
    return c


# (N, K, M): k/v, q/o, merged q/k/v, the 8192-wide projection, down; ragged
# token counts (last token tile partly outside) and a ragged channel count
# (1036: row-major weights only, the last 16-row tile partly outside).
CASES = [(1024, 4096, 17), (1024, 4096, 32), (1024, 4096, 64), (1024, 4096, 100), (1024, 4096, 128),
         (4096, 4096, 33), (4096, 4096, 64), (4096, 4096, 96), (4096, 4096, 128), (6144, 4096, 50),
         (6144, 4096, 64), (8192, 4096, 64), (4096, 12288, 17), (4096, 12288, 32), (1036, 4096, 48)]


@pytest.mark.parametrize("N,K,M", CASES)
def test_batch_kernel_oracle_and_layouts(N, K, M):
    print(f"batch kernel N={N} K={K} M={M}", flush=True)
    assert launch_shape(M, N, K)[0] == 3
    x = synthetic.activations_heavy_tail(M, K, 9100 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 9101 + N % 13).cuda())
    y = fp8_matmul(x, wq, sw)
    check(y, x, wq, sw)
    xq, sx = quantize_rows(x)
    assert torch.equal(fp8_matmul_quantized(xq, sx, wq, sw), y), "row-major codes differ"
    if N % 16 == 0:
        wt = tile_weight(wq)
        assert torch.equal(fp8_matmul(x, wt, sw, tiled=True), y), "tiled weights differ"
        assert torch.equal(fp8_matmul_quantized(xq, sx, wt, sw, tiled=True), y), "row-major codes, tiled weights differ"
    assert torch.equal(fp8_matmul(x, wq, sw), y), "second call differs"


@pytest.mark.parametrize("N,K,M", [(1024, 4096, 64), (1024, 4096, 100), (4096, 4096, 128), (4096, 4096, 96),
                                   (4096, 12288, 32), (1036, 4096, 48)])
def test_batch_rows_equal_decode_kernel_slices(N, K, M):
    """The decode kernel at 16 tokens runs these weights with the same waves
    per row and no K split, so every output of the batch equals, bit for bit,
    the output of its 16-token slice; with bias and LoRA too (the GEMM on
    quantized codes with one set of low-rank activations t = x A^T: the
    quantizer of more than 64 rows sums t in another order than that of 16)."""
    print(f"batch vs decode slices N={N} K={K} M={M}", flush=True)
    assert launch_shape(M, N, K)[0] == 3
    assert launch_shape(16, N, K)[0] == 0 and launch_shape(16, N, K)[3] == 1
    x = synthetic.activations_outliers(M, K, 9200 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 9201).cuda())
    y = fp8_matmul(x, wq, sw)
    assert torch.equal(y, torch.cat([fp8_matmul(x[i:i + 16], wq, sw) for i in range(0, M, 16)]))
    a, b = synthetic.lora_factors(N, K, 9202)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(9203)) * 0.1).to(torch.bfloat16).cuda()
    lora = (a.cuda(), b.cuda(), synthetic.LORA_SCALING)
    yb = fp8_matmul(x, wq, sw, bias=bias, lora=lora)
    check(yb, x, wq, sw, bias=bias, lora=lora)
    if N % 16 == 0:
        assert torch.equal(fp8_matmul(x, tile_weight(wq), sw, bias=bias, lora=lora, tiled=True), yb)
    xq, sx = quantize_rows(x)
    t = x.float() @ lora[0].float().t()
    lb, s = lora[1], lora[2]
    yt = fp8_matmul_quantized(xq, sx, wq, sw, bias=bias, lora_t=t, lora_b=lb, lora_scaling=s)
    assert torch.equal(yt, torch.cat([fp8_matmul_quantized(xq[i:i + 16], sx[i:i + 16], wq, sw, bias=bias,
                                                           lora_t=t[i:i + 16].contiguous(), lora_b=lb, lora_scaling=s)
                                      for i in range(0, M, 16)]))


@pytest.mark.parametrize("N,K", [(1024, 4096), (4096, 4096), (6144, 4096), (4096, 12288)])
def test_batch_every_token_count(N, K):
    """Every token count of 17-128 that takes a batch plan on these weights
    (each token split and tile shape the plan picks): the batch equals its
    16-token slices on the decode kernel bit for bit where the decode kernel
    runs the same waves per row (one 16-row tile per wave), else the oracle
    criteria on the first and last rows."""
    wq, sw = quantize_rows(synthetic.weight(N, K, 9250).cuda())
    wt = tile_weight(wq)
    x_all = synthetic.activations_heavy_tail(128, K, 9251).cuda()
    same_waves = N <= 4096  # the decode plan takes one tile per wave here (merged q/k/v: two, eight waves)
    ran = 0
    for M in range(17, 129):
        if launch_shape(M, N, K)[0] != 3:
            continue
        ran += 1
        x = x_all[:M]
        y = fp8_matmul(x, wt, sw, tiled=True)
        if same_waves:
            assert torch.equal(y, torch.cat([fp8_matmul(x[i:i + 16], wt, sw, tiled=True) for i in range(0, M, 16)])), M
        else:
            rows = torch.tensor([0, M - 1], device="cuda")
            check(y[rows], x[rows], wq, sw)
    assert ran >= 16, ran


@pytest.mark.parametrize("N,K,M", [(1036, 4096, 40), (1024, 4096, 100), (4096, 12288, 20)])
def test_batch_writes_stay_inside_the_output(N, K, M):
    """Through the C ABI with a row stride past N and a sentinel-filled guard
    band: nothing outside [M, N] changes."""
    assert launch_shape(M, N, K)[0] == 3
    x = synthetic.activations_heavy_tail(M, K, 9300 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 9301).cuda())
    ldy = N + 40
    y = torch.full((M + 2, ldy), -3.0, dtype=torch.bfloat16, device="cuda")
    guard = y.clone()
    L = _lib.lib()
    ws_bytes = L.jv_fp8_linear_workspace_bytes(M, N, K, 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    _lib.check(L.jv_fp8_linear(x.data_ptr(), K, wq.data_ptr(), K, sw.data_ptr(), None, None, None, 0, 0.0, y.data_ptr(),
                               ldy, M, N, K, ws.data_ptr(), ws_bytes, None, 0, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(y[:M, N:], guard[:M, N:]) and torch.equal(y[M:], guard[M:])
    assert torch.equal(y[:M, :N], fp8_matmul(x, wq, sw))


def amax_of(h: torch.Tensor) -> np.ndarray:
    b = helpers.bits(h).astype(np.uint32) & 0x7FFF
    return b.reshape(h.shape[0], -1, 16).max(axis=2).astype(np.uint16)


# (I, K, M): gate+up weights of 2I rows that take batch plans
@pytest.mark.parametrize("I,K,M", [(512, 4096, 64), (512, 4096, 128), (2048, 4096, 96), (2048, 4096, 128),
                                   (3072, 4096, 40), (2048, 12288, 32)])
def test_batch_fused_swiglu_equals_unfused(I, K, M):
    print(f"batch swiglu I={I} K={K} M={M}", flush=True)
    N = 2 * I
    assert launch_shape(M, N, K)[0] == 3
    x = synthetic.activations_heavy_tail(M, K, 9400 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 9401 + I).cuda())
    a, b = synthetic.lora_factors(N, K, 9402)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(9403)) * 0.1).to(torch.bfloat16).cuda()
    for kw in ({}, {"bias": bias, "lora": (a.cuda(), b.cuda(), synthetic.LORA_SCALING)}):
        gu = fp8_matmul(x, wq, sw, **kw)
        want = swiglu_quantize(gu[:, :I], gu[:, I:], return_h=True)[-1]
        h, parts = gate_up_swiglu(x, wq, sw, amax=True, **kw)
        assert torch.equal(h, want), kw.keys()
        assert np.array_equal(parts.cpu().numpy().view(np.uint16), amax_of(want))
        assert torch.equal(gate_up_swiglu(x, tile_weight(wq), sw, tiled=True, **kw), want)
