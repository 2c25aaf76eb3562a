"""The 128x384 ping-pong prefill tiles (plans where 256x256 tiles would leave
part of a round empty: gate+up at 512-1536 tokens, the 6144-, 10240- and
12288-wide merges, the lm_head past 64 tokens):
* the oracle criteria on sampled token rows (heavy-tailed activations), with
  bias and LoRA in the epilogue;
* every output bitwise equal to the same rows under the plan of a shorter
  batch (lockstep or 256x256 tiles): without a K split every FP8 prefill
  plan sums each output's k range in the same order;
* ragged token and channel counts (last tiles partly outside), writes
  confined to [M, N] of a strided output;
* the fused SwiGLU epilogue (h and its per-16-channel maxima) equal to the
  unfused steps."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jeeves_amd import _lib, synthetic
from jeeves_amd.fp8 import fp8_matmul, fp8_matmul_quantized, gate_up_swiglu, swiglu_quantize, tile_weight
from jeeves_amd.fp8_weights import quantize_rows
from tests import helpers
from tests.test_gpu_batch import amax_of, check, launch_shape
from tests.test_gpu_swiglu_oracle import H_EQUAL_MIN

pytestmark = pytest.mark.gpu


def takes_128x384(M: int, N: int, K: int) -> bool:
    kind, wgs, threads, splits = launch_shape(M, N, K)
    return kind == 2 and wgs == -(-M // 128) * -(-N // 384) and threads == 512 and splits == 1


def sample_rows(M: int) -> torch.Tensor:
    return torch.cat([torch.arange(0, 16), torch.arange(M // 2 - 8, M // 2 + 8), torch.arange(M - 16, M)]).cuda()


# (N, K, M): the 12288-wide merge (whole and ragged token counts), gate+up,
# the 10240-wide merge (last channel tile 256 of 384 wide), merged q/k/v
# (ragged tokens), K = 8192 and 2048
CASES = [(12288, 4096, 768), (12288, 4096, 777), (24576, 4096, 1000), (10240, 4096, 2048), (6144, 4096, 2900),
         (12288, 8192, 640), (12288, 2048, 768)]


@pytest.mark.parametrize("N,K,M", CASES)
def test_128x384_tiles_oracle_and_other_plans(N, K, M):
    print(f"128x384 tiles N={N} K={K} M={M}", flush=True)
    assert takes_128x384(M, N, K)
    x = synthetic.activations_heavy_tail(M, K, 9600 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 9601 + N % 11).cuda())
    wt = tile_weight(wq)
    y = fp8_matmul(x, wt, sw, tiled=True)
    rows = sample_rows(M)
    check(y[rows], x[rows], wq, sw)
    assert torch.equal(fp8_matmul(x, wq, sw), y), "row-major weights differ"
    xq, sx = quantize_rows(x)  # row-major activation codes (the kernel's unpacked token rows)
    assert torch.equal(fp8_matmul_quantized(xq, sx, wt, sw, tiled=True), y), "row-major codes differ"
    assert torch.equal(fp8_matmul_quantized(xq, sx, wq, sw), y), "row-major codes and weights differ"
    for short in (256, 384, 512, 192):  # a shorter batch on another plan without a K split
        kind, _, _, splits = launch_shape(short, N, K)
        if kind in (1, 2) and splits == 1 and not takes_128x384(short, N, K):
            break
    else:
        pytest.fail("no shorter batch without a K split")
    assert torch.equal(fp8_matmul(x[:short], wt, sw, tiled=True), y[:short]), "differs from the shorter batch's plan"
    assert torch.equal(fp8_matmul(x[M - short:], wt, sw, tiled=True), y[M - short:])


@pytest.mark.parametrize("N,K,M", [(12288, 4096, 777), (10240, 4096, 2048)])
def test_128x384_tiles_bias_lora_and_strided_output(N, K, M):
    print(f"128x384 tiles with bias and LoRA N={N} K={K} M={M}", flush=True)
    assert takes_128x384(M, N, K)
    x = synthetic.activations_outliers(M, K, 9700 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 9701).cuda())
    a, b = synthetic.lora_factors(N, K, 9702)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(9703)) * 0.1).to(torch.bfloat16).cuda()
    lora = (a.cuda(), b.cuda(), synthetic.LORA_SCALING)
    y = fp8_matmul(x, tile_weight(wq), sw, bias=bias, lora=lora, tiled=True)
    rows = sample_rows(M)
    check(y[rows], x[rows], wq, sw, bias=bias, lora=lora)
    # through the C ABI into a strided output with a guard band
    L = _lib.lib()
    ldy = N + 24
    out = torch.full((M + 3, ldy), -5.0, dtype=torch.bfloat16, device="cuda")
    guard = out.clone()
    ws_bytes = L.jv_fp8_linear_workspace_bytes(M, N, K, 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    _lib.check(L.jv_fp8_linear(x.data_ptr(), K, wq.data_ptr(), K, sw.data_ptr(), None, None, None, 0, 0.0, out.data_ptr(),
                               ldy, M, N, K, ws.data_ptr(), ws_bytes, None, 0, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(out[:M, N:], guard[:M, N:]) and torch.equal(out[M:], guard[M:])
    assert torch.equal(out[:M, :N], fp8_matmul(x, wq, sw))


# (I, K, M): gate+up weights of 2I rows on 128x384 tiles
@pytest.mark.parametrize("I,K,M", [(6144, 4096, 768), (6144, 4096, 777), (12288, 4096, 1000), (5120, 4096, 2048)])
def test_128x384_fused_swiglu_equals_unfused(I, K, M):
    print(f"128x384 swiglu I={I} K={K} M={M}", flush=True)
    N = 2 * I
    assert takes_128x384(M, N, K)
    x = synthetic.activations_heavy_tail(M, K, 9800 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 9801 + I % 7).cuda())
    wt = tile_weight(wq)
    a, b = synthetic.lora_factors(N, K, 9802)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(9803)) * 0.1).to(torch.bfloat16).cuda()
    for kw in ({}, {"bias": bias, "lora": (a.cuda(), b.cuda(), synthetic.LORA_SCALING)}):
        gu = fp8_matmul(x, wt, sw, tiled=True, **kw)
        want = swiglu_quantize(gu[:, :I], gu[:, I:], return_h=True)[-1]
        h, parts = gate_up_swiglu(x, wt, sw, amax=True, tiled=True, **kw)
        assert torch.equal(h, want), kw.keys()
        assert np.array_equal(parts.cpu().numpy().view(np.uint16), amax_of(want))
        assert torch.equal(gate_up_swiglu(x, wq, sw, **kw), want)
    # the SwiGLU criteria against the oracle on sampled rows
    rows = sample_rows(M)
    h = gate_up_swiglu(x, wt, sw, tiled=True)
    xq, sx = oracle.quantize_rows(x[rows].float().cpu().numpy())
    c = helpers.swiglu_criteria(helpers.bits(h[rows]), xq, sx, helpers.codes_np(wq), sw.cpu().numpy())
    assert c["bound"] and c["equal"] >= helpers.equal_floor(len(rows) * I, H_EQUAL_MIN), (c["outside"], c["equal"])
