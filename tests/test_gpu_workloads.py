"""Model-scale workloads through the FP8 path:
* lm_head, N = 248320 x K = 4096 (1.02 GB of e4m3 weights; inference/engine.py:293-297): decode and
  prefill batches, checked against the oracle on sampled output channels;
* the ragged request mix (64 log-uniform sequence lengths packed into one token batch through a
  32-layer stack of the 9B layer shapes, then decode steps at batch 64): oracle checks on sampled
  rows of the first and last layer, and packed rows equal to each sequence computed alone wherever
  both batches run unsplit prefill plans (per-token scales make rows independent; an unsplit
  prefill tile sums every output in the same k order whatever its shape). A plan that splits K
  sums the splits' partials at the end, a different fp32 order, so those rows are held to the
  oracle criteria instead."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jeeves_amd import _lib, synthetic
from jeeves_amd.device import sm_count
from jeeves_amd.fp8 import fp8_matmul, fp8_matmul_quantized, swiglu_quantize
from jeeves_amd.fp8_weights import quantize_rows
from tests import helpers

pytestmark = pytest.mark.gpu


def check_rows(y, x, wq, sw, rows=None, cols=None, bar=None):
    """Oracle criteria (tests/helpers.py) on a sample of token rows and output
    channels; `bar`: the equal-share bar of the input family (default
    helpers.EQUAL_MIN)."""
    if rows is not None:
        x, y = x[rows], y[rows]
    if cols is not None:
        wq, sw, y = wq[cols], sw[cols], y[:, cols]
    xq, sx = oracle.quantize_rows(x.float().cpu().numpy())
    c = helpers.gemm_criteria(helpers.bits(y), xq, sx, helpers.codes_np(wq), sw.cpu().numpy())
    assert c["finite_match"] and c["bound"], c
    assert c["equal"] >= helpers.equal_floor(c["n"], bar or helpers.EQUAL_MIN) and c["rel_l2"] <= helpers.REL_L2_MAX, c
    return c


def device_weight(N, K, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(N, K, device="cuda", generator=g) * synthetic.WEIGHT_STD).to(torch.bfloat16)


@pytest.fixture(scope="module")
def lm_head():
    w = device_weight(synthetic.VOCAB, synthetic.HIDDEN, 600)
    wq, sw = quantize_rows(w)
    del w
    torch.cuda.empty_cache()
    yield wq, sw
    del wq, sw
    torch.cuda.empty_cache()


@pytest.mark.parametrize("M", [1, 16, 64, 200])
def test_lm_head_vocab_logits(lm_head, M):
    wq, sw = lm_head
    x = synthetic.activations_outliers(M, 4096, 610 + M).cuda()
    y = fp8_matmul(x, wq, sw)
    assert y.shape == (M, synthetic.VOCAB)
    cols = torch.randperm(synthetic.VOCAB, generator=torch.Generator().manual_seed(M))[:2048].sort().values.cuda()
    check_rows(y, x, wq, sw, cols=cols)
    assert torch.equal(y[:, -16:], fp8_matmul(x, wq[-16:], sw[-16:])) if M > 64 else True
    assert torch.equal(y, fp8_matmul(x, wq, sw))


def rms_normalize(h):
    hf = h.float()
    return (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)


LAYERS = 32


@pytest.fixture(scope="module")
def stack():
    layers = []
    for layer in range(LAYERS):
        weights = {}
        for i, (name, (N, K)) in enumerate(synthetic.SHAPES.items()):
            weights[name] = quantize_rows(device_weight(N, K, 700 + 10 * layer + i))
        layers.append(weights)
    torch.cuda.empty_cache()
    yield layers
    layers.clear()
    torch.cuda.empty_cache()


def run_layer(weights, h):
    """q, k, v, o and gate+up on the layer input, SwiGLU, down; returns every projection's output."""
    out = {name: fp8_matmul(h, *weights[name]) for name in ("q", "k", "v", "o", "gate_up")}
    inter = synthetic.INTERMEDIATE
    codes, scales, hmid = swiglu_quantize(out["gate_up"][:, :inter], out["gate_up"][:, inter:], return_h=True)
    out["down"] = fp8_matmul_quantized(codes, scales, *weights["down"])
    out["h_mid"] = hmid
    return out


def unsplit_prefill(M, N, K):
    """True when the (M, N, K) GEMM runs on prefill tiles without a K split on
    this device (the batch-decode kernel, for 17-128 tokens on some weights,
    sums in another k order)."""
    import ctypes
    shape = (ctypes.c_int32 * 4)()
    _lib.check(_lib.lib().jv_fp8_launch_shape(M, N, K, sm_count(torch.device("cuda:0")), shape))
    return shape[0] in (1, 2) and shape[3] == 1


def test_ragged_prefill_then_decode(stack):
    lengths = synthetic.ragged_lengths()
    assert len(lengths) == 64 and min(lengths) >= 64 and max(lengths) <= 2048
    g = torch.Generator().manual_seed(500)
    seqs = [synthetic.activations_heavy_tail(n, synthetic.HIDDEN, 5000 + i) for i, n in enumerate(lengths)]
    h = torch.cat(seqs).cuda()
    T = h.shape[0]
    rows = torch.randperm(T, generator=g)[:12].sort().values.cuda()
    starts = np.cumsum([0] + lengths)
    for layer, weights in enumerate(stack):
        out = run_layer(weights, h)
        if layer in (0, LAYERS - 1):
            for name in ("q", "k", "v", "o", "gate_up"):
                check_rows(out[name], h, *weights[name], rows=rows)
            check_rows(out["down"], out["h_mid"], *weights["down"], rows=rows, bar=helpers.EQUAL_MIN_SWIGLU_H)
        if layer == 0:
            # packed rows equal each sequence alone (sequences longer than 64 tokens: prefill kernel)
            for i in (0, 17, 63):
                a, b = int(starts[i]), int(starts[i + 1])
                if b - a > 64:
                    alone = run_layer(weights, h[a:b].contiguous())
                    for name in ("q", "k", "o", "gate_up", "down"):
                        N, K = synthetic.SHAPES[name]
                        if unsplit_prefill(T, N, K) and unsplit_prefill(b - a, N, K):
                            assert torch.equal(out[name][a:b], alone[name]), (i, name)
                        else:
                            x_in = alone["h_mid"] if name == "down" else h[a:b]
                            check_rows(alone[name], x_in, *weights[name], rows=torch.arange(0, b - a, 29, device="cuda"),
                                       bar=helpers.EQUAL_MIN_SWIGLU_H if name == "down" else None)
        h = rms_normalize(out["down"])
        assert torch.isfinite(h.float()).all()
    # decode: 64 steps at batch 64 through the whole stack
    x = rms_normalize(synthetic.activations_outliers(64, synthetic.HIDDEN, 5500).cuda())
    first = None
    for step in range(64):
        hs = x
        for layer, weights in enumerate(stack):
            out = run_layer(weights, hs)
            if step == 0 and layer == 0:
                first = out
                for name in ("q", "k", "v", "o", "gate_up"):
                    check_rows(out[name], hs, *weights[name])
                check_rows(out["down"], out["h_mid"], *weights["down"], bar=helpers.EQUAL_MIN_SWIGLU_H)
            hs = rms_normalize(out["down"])
        x = hs
    again = run_layer(stack[0], rms_normalize(synthetic.activations_outliers(64, synthetic.HIDDEN, 5500).cuda()))
    for name in ("q", "k", "v", "o", "gate_up", "down"):
        assert torch.equal(again[name], first[name]), name
