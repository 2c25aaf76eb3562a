"""The gate+up GEMM with SwiGLU in its epilogue (model/model.py:581-584):
``gate_up_swiglu`` must give, bit for bit, what the unfused steps give -- the
fused gate+up FP8 GEMM's bf16 output, then ``F.silu(gate) * up`` on bf16
(the fused SwiGLU-quantizer kernel's ``h``, itself pinned to the oracle's
``swiglu_bf16`` in tests/test_gpu_quant.py) -- on every kernel regime
(decode kernel at 1-64 tokens, 64x64 prefill tiles for 17-64 tokens on wide
weights, the lockstep and ping-pong prefill tiles), tiled and row-major
weights, with bias and LoRA; its per-16-channel |h| maxima must be those of
h; the down projection's quantization of h must equal quantize_rows(h); and
FP8SwiGLU must equal the composition of its steps."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jeeves_amd import synthetic
from jeeves_amd.fp8 import (FP8Linear, FP8SwiGLU, fp8_matmul, fp8_matmul_quantized, gate_up_swiglu,
                            quantize_swiglu_output, swiglu_quantize, tile_weight)
from jeeves_amd.fp8_weights import quantize_rows
from tests import helpers

pytestmark = pytest.mark.gpu


def unfused_h(x, wq, sw, bias=None, lora=None, tiled=False):
    gu = fp8_matmul(x, wq, sw, bias=bias, lora=lora, tiled=tiled)
    inter = gu.shape[1] // 2
    return swiglu_quantize(gu[:, :inter], gu[:, inter:], return_h=True)[-1]


def amax_of(h: torch.Tensor) -> np.ndarray:
    b = helpers.bits(h).astype(np.uint32) & 0x7FFF
    return b.reshape(h.shape[0], -1, 16).max(axis=2).astype(np.uint16)


# (I, K): the 9B MLP (gate+up 24576 x 4096), a narrower one, a ragged count of
# 16-channel pairs (last 256-wide prefill tile partly outside), a long K.
SHAPES = [(12288, 4096), (1024, 4096), (1040, 2048), (2048, 12288)]


@pytest.mark.parametrize("I,K", SHAPES)
@pytest.mark.parametrize("M", [1, 5, 16, 33, 64, 65, 300, 2048])
def test_fused_swiglu_equals_unfused(I, K, M):
    print(f"fused swiglu I={I} K={K} M={M}", flush=True)
    N = 2 * I
    x = synthetic.activations_heavy_tail(M, K, 8000 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 8001 + I).cuda())
    want = unfused_h(x, wq, sw)
    h, parts = gate_up_swiglu(x, wq, sw, amax=True)
    assert torch.equal(h, want), (I, K, M)
    assert np.array_equal(parts.cpu().numpy().view(np.uint16), amax_of(want)), (I, K, M)
    assert torch.equal(gate_up_swiglu(x, tile_weight(wq), sw, tiled=True), want), (I, K, M)


@pytest.mark.parametrize("M", [4, 48, 512])
def test_fused_swiglu_with_bias_and_lora(M):
    I, K = 12288, 4096
    N = 2 * I
    x = synthetic.activations_outliers(M, K, 8100 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 8101).cuda())
    a, b = synthetic.lora_factors(N, K, 8102)
    lora = (a.cuda(), b.cuda(), synthetic.LORA_SCALING)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(8103)) * 0.1).to(torch.bfloat16).cuda()
    want = unfused_h(x, wq, sw, bias=bias, lora=lora)
    assert torch.equal(gate_up_swiglu(x, wq, sw, bias=bias, lora=lora), want)
    assert torch.equal(gate_up_swiglu(x, tile_weight(wq), sw, bias=bias, lora=lora, tiled=True), want)


def test_fused_swiglu_nan_and_inf_rows():
    """An inf activation row gives NaN or inf gate/up outputs; h, its maxima
    (NaN sorting above inf) and the quantized codes follow the unfused path."""
    I, K, M = 1024, 4096, 8
    x = synthetic.activations_outliers(M, K, 8200)
    x[3, 5] = float("inf")
    x = x.cuda()
    wq, sw = quantize_rows(synthetic.weight(2 * I, K, 8201).cuda())
    want = unfused_h(x, wq, sw)
    h, parts = gate_up_swiglu(x, wq, sw, amax=True)
    assert helpers.same_f32(h.float().cpu().numpy(), want.float().cpu().numpy()).all()
    assert np.array_equal(parts.cpu().numpy().view(np.uint16), amax_of(h))


@pytest.mark.parametrize("M", [1, 16, 40, 300])
@pytest.mark.parametrize("rank", [0, 16])
def test_quantize_swiglu_output_equals_quantize_rows(M, rank):
    I = 12288
    h = synthetic.activations_heavy_tail(M, I, 8300 + M).cuda()
    a = synthetic.lora_factors(4096, I, 8301)[0].cuda() if rank else None
    out = quantize_swiglu_output(h, lora_a=a, packed=False)
    codes, scales = quantize_rows(h)
    assert torch.equal(out[0].view(torch.uint8), codes.view(torch.uint8)) and torch.equal(out[1], scales)
    # packed codes: the down GEMM on them equals the GEMM on the row-major codes
    packed = quantize_swiglu_output(h, lora_a=a, packed=True)
    assert torch.equal(packed[1], scales)
    wq, sw = quantize_rows(synthetic.weight(4096, I, 8302).cuda())
    assert torch.equal(fp8_matmul_quantized(packed[0], packed[1], wq, sw, packed_rows=M),
                       fp8_matmul_quantized(codes, scales, wq, sw))
    if rank:
        xq_t = oracle.lora_f64(oracle.bf16_to_f32(helpers.bits(h)), oracle.bf16_to_f32(helpers.bits(a)),
                               np.eye(rank), 1.0)
        assert np.allclose(out[2].cpu().numpy(), xq_t, rtol=1e-5, atol=1e-5)
        assert torch.equal(packed[2], out[2])


@pytest.mark.parametrize("I", [128, 1024, 4096, 12288, 16384])
@pytest.mark.parametrize("M", [1, 5, 16, 17, 40, 64, 96, 128])
def test_quantize_h_from_maxima_equals_one_pass(I, M):
    """Decode batches (up to 128 tokens) quantize h from the epilogue's
    per-16-channel maxima,
    each row split over workgroups: codes (padding rows included) and scales
    are the bits of the one-pass quantizer, which takes each row's maximum
    from h. Rows whose maximum sits in the first or last 16 channels, an inf,
    a NaN and an all-zero row."""
    print(f"h from maxima I={I} M={M}", flush=True)
    h = synthetic.activations_heavy_tail(M, I, 8500 + M + I)
    h[0, -1] = 300.0
    if M > 1:
        h[1, 0] = -300.0
    if M > 4:
        h[2, I // 2] = float("inf")
        h[3, 7] = float("nan")
        h[4] = 0.0
    h = h.cuda()
    parts = torch.from_numpy(amax_of(h).view(np.int16)).cuda()
    want = quantize_swiglu_output(h, packed=True)
    got = quantize_swiglu_output(h, parts, packed=True)
    assert torch.equal(got[0], want[0]), (I, M)
    assert helpers.same_f32(got[1].cpu().numpy(), want[1].cpu().numpy()).all(), (I, M)
    codes, scales = quantize_rows(h)
    assert helpers.same_f32(got[1].cpu().numpy(), scales.cpu().numpy()).all(), (I, M)


@pytest.mark.parametrize("M", [1, 64, 65, 128, 129, 300])
def test_maxima_are_read_only_for_decode_batches(M):
    """The dispatch: maxima that understate every row (all zero) change the
    scales exactly where the quantizer reads them (M <= 128, packed, no LoRA)
    and nowhere else, so the decode path really takes its maximum from them."""
    I = 4096
    h = synthetic.activations_heavy_tail(M, I, 8700 + M).cuda()
    zeros = torch.zeros(M, I // 16, dtype=torch.int16, device="cuda")
    want = quantize_swiglu_output(h, packed=True)
    got = quantize_swiglu_output(h, zeros, packed=True)
    read = M <= 128
    assert torch.equal(got[1], want[1]) != read, M
    # LoRA and row-major codes never read the maxima
    a = synthetic.lora_factors(4096, I, 8701)[0].cuda()
    assert torch.equal(quantize_swiglu_output(h, zeros, lora_a=a, packed=True)[1], want[1])
    assert torch.equal(quantize_swiglu_output(h, zeros, packed=False)[1], want[1])


@pytest.mark.parametrize("M", [1, 16, 64, 96, 128])
def test_quantize_h_from_epilogue_maxima(M):
    """The maxima gate_up_swiglu stores, fed to the quantizer of h, give the
    bits of the quantizer that reads h alone; also through a misaligned view
    of the maxima (not 8-byte aligned: the one-pass path)."""
    I, K = 12288, 4096
    x = synthetic.activations_outliers(M, K, 8600 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(2 * I, K, 8601).cuda())
    h, parts = gate_up_swiglu(x, tile_weight(wq), sw, tiled=True, amax=True)
    want = quantize_swiglu_output(h, packed=True)
    got = quantize_swiglu_output(h, parts, packed=True)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
    shifted = torch.empty(M * (I // 16) + 1, dtype=torch.int16, device="cuda")[1:].view(M, I // 16)
    shifted.copy_(parts)
    got = quantize_swiglu_output(h, shifted, packed=True)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


@pytest.mark.parametrize("M", [1, 16, 64, 512])
def test_fp8_swiglu_module_fused_equals_steps(M):
    """FP8SwiGLU's fused forward equals gate+up (FP8Linear), SwiGLU on bf16 and
    down (FP8Linear) run one after another, bitwise; with LoRA on both."""
    K, I = 4096, 12288
    gu = FP8Linear(K, 2 * I, device="cuda")
    gu.load_weight(synthetic.weight(2 * I, K, 8400).cuda())
    down = FP8Linear(I, K, device="cuda")
    down.load_weight(synthetic.weight(K, I, 8401).cuda())
    block = FP8SwiGLU(gu, down)
    assert block.fused()
    x = synthetic.activations_heavy_tail(M, K, 8402 + M).cuda()
    g = gu(x)
    h = swiglu_quantize(g[:, :I], g[:, I:], return_h=True)[-1]
    assert torch.equal(block(x), down(h))
    a, b = synthetic.lora_factors(2 * I, K, 8403)
    gu.set_lora(a.cuda(), b.cuda(), synthetic.LORA_SCALING)
    a2, b2 = synthetic.lora_factors(K, I, 8404)
    down.set_lora(a2.cuda(), b2.cuda(), synthetic.LORA_SCALING)
    g = gu(x)
    h = swiglu_quantize(g[:, :I], g[:, I:], return_h=True)[-1]
    assert torch.equal(block(x), down(h))


@pytest.mark.parametrize("M", [16, 65, 300])
def test_fused_swiglu_writes_stay_inside_h_and_amax(M):
    """Through the C ABI with sentinel-filled guard bands after h's rows and
    after the maxima (I = 1040: the last 64- or 256-wide prefill tile reaches
    past the last h channel): nothing outside [M, I] and [M, I/16] changes."""
    from jeeves_amd import _lib

    I, K = 1040, 2048
    N = 2 * I
    x = synthetic.activations_heavy_tail(M, K, 8500 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 8501).cuda())
    ldh = I + 64
    h = torch.full((M + 1, ldh), -7.0, dtype=torch.bfloat16, device="cuda")
    parts = torch.full((M * (I // 16) + 4096,), 0x5A5A, dtype=torch.int32, device="cuda").view(torch.int16)
    guard_h, guard_p = h.clone(), parts.clone()
    L = _lib.lib()
    ws_bytes = L.jv_fp8_linear_workspace_bytes(M, N, K, 0)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    counters = torch.zeros(65536, dtype=torch.int32, device="cuda")
    _lib.check(L.jv_fp8_linear_swiglu(x.data_ptr(), K, wq.data_ptr(), K, sw.data_ptr(), None, None, None, 0, 0.0,
                                      h.data_ptr(), ldh, parts.data_ptr(), M, I, K, ws.data_ptr(), ws_bytes,
                                      _lib.counters_ptr(counters), counters.numel(),
                                      torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(h[:M, I:], guard_h[:M, I:]) and torch.equal(h[M:], guard_h[M:])
    n = M * (I // 16)
    assert torch.equal(parts[n:], guard_p[n:])
    assert torch.equal(h[:M, :I], unfused_h(x, wq, sw))
