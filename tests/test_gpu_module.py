"""The drop-in module API on the device: FP8Linear.load_weight / load_codes /
concatenated / forward with bias, warm, FP8SwiGLU, and the decoder-layer
linear stack with LoRA adapters (9B shapes at M = 512)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from jeeves_amd import synthetic
from jeeves_amd.fp8 import FP8Linear, FP8SwiGLU, fp8_matmul, swiglu_quantize, warm
from jeeves_amd.fp8_weights import FP8, quantize_rows
from tests import helpers

pytestmark = pytest.mark.gpu


def quantized(linear: nn.Linear) -> FP8Linear:
    # inference/cuda_test.py:17-20
    fp8 = FP8Linear(linear.in_features, linear.out_features, bias=linear.bias is not None, device=linear.weight.device)
    fp8.load_weight(linear.weight)
    if linear.bias is not None:
        with torch.no_grad():
            fp8.bias.copy_(linear.bias)
    return fp8


def test_load_weight_equals_quantize_rows_and_load_codes():
    w = synthetic.weight(1040, 4096, 21).cuda()
    m = FP8Linear(4096, 1040, device="cuda")
    m.load_weight(w)
    codes, scale = quantize_rows(w)
    assert torch.equal(m.codes().view(torch.uint8), codes.view(torch.uint8)) and torch.equal(m.scale, scale)
    n = FP8Linear(4096, 1040, device="cuda")
    n.load_codes(codes, scale)
    assert torch.equal(n.weight.view(torch.uint8), m.weight.view(torch.uint8)) and torch.equal(n.scale, m.scale)
    want_c, want_s = oracle.quantize_rows(w.float().cpu().numpy())
    assert np.array_equal(helpers.codes_np(m.codes()), want_c)


def test_forward_shapes_bias_and_dtype():
    torch.manual_seed(0)
    lin = nn.Linear(4096, 1024, bias=True, device="cuda", dtype=torch.bfloat16)
    m = quantized(lin)
    x = torch.randn(3, 16, 4096, device="cuda")  # float32 input is cast to bf16 as the reference does
    y = m(x)
    assert y.shape == (3, 16, 1024) and y.dtype == torch.bfloat16
    x2 = x.reshape(-1, 4096).to(torch.bfloat16)
    nobias = fp8_matmul(x2, m.weight, m.scale)
    # the bias is added to the bf16 GEMM output in bf16, as FP8Linear.forward
    # does (inference/fp8.py:183-184): bitwise nobias + bias
    assert torch.equal(y.reshape(-1, 1024), nobias + lin.bias)
    # non-contiguous last dimension is made contiguous
    xt = torch.randn(4096, 8, device="cuda").to(torch.bfloat16).t()
    assert torch.equal(m(xt), m(xt.contiguous()))


def test_merged_fp8_projections():
    # inference/cuda_test.py:38-46: merged parts keep codes, views share storage, outputs match
    torch.manual_seed(0)
    x = torch.randn(3, 16, 4096, device="cuda", dtype=torch.bfloat16)
    parts = [quantized(nn.Linear(4096, n, bias=False, device="cuda", dtype=torch.bfloat16)) for n in (4096, 1024, 1024)]
    codes, scales = [p.weight.clone() for p in parts], [p.scale.clone() for p in parts]
    merged = FP8Linear.concatenated(parts)
    for p, c, s in zip(parts, codes, scales):
        assert torch.equal(p.weight.view(torch.uint8), c.view(torch.uint8)) and torch.equal(p.scale, s)
        assert p.weight.untyped_storage().data_ptr() == merged.weight.untyped_storage().data_ptr()
    for a, p in zip(merged(x).split([p.out_features for p in parts], dim=-1), parts):
        assert torch.allclose(a.float(), p(x).float(), rtol=2 ** -7, atol=1e-2)


def test_warm_counts_distinct_shapes():
    mods = nn.ModuleList([FP8Linear(4096, 1024, device="cuda"), FP8Linear(4096, 1024, device="cuda"),
                          FP8Linear(12288, 4096, device="cuda")])
    for m in mods:
        m.load_weight(synthetic.weight(m.out_features, m.in_features, 3).cuda())
    assert warm(mods) == 2


def test_fp8_swiglu_module_equals_composition():
    x = synthetic.activations_heavy_tail(48, 4096, 31).cuda()
    gu = FP8Linear(4096, 2 * 12288, device="cuda")
    gu.load_weight(synthetic.weight(2 * 12288, 4096, 104).cuda())
    down = FP8Linear(12288, 4096, device="cuda")
    down.load_weight(synthetic.weight(4096, 12288, 105).cuda())
    y = FP8SwiGLU(gu, down)(x)
    g = gu(x)
    h = (torch.nn.functional.silu(g[:, :12288]) * g[:, 12288:])
    ref = down(h)
    # h from the fused kernel may differ from torch's silu in rare last bits
    assert torch.allclose(y.float(), ref.float(), rtol=2 ** -6, atol=2e-2)
    assert (y == ref).float().mean().item() > 0.95


def test_decoder_layer_stack_with_lora():
    """q, k, v, o, gate_up -> SwiGLU -> down at M = 512, each with a rank-16
    LoRA adapter (scaling 2) fused into the FP8 epilogue; every projection is
    checked against the float64 oracle on the same FP8 inputs."""
    M = 512
    x = synthetic.activations_heavy_tail(M, synthetic.HIDDEN, 400).cuda()
    xq, sx = oracle.quantize_rows(x.float().cpu().numpy())
    xf = oracle.bf16_to_f32(helpers.bits(x)).astype(np.float64)
    outs = {}
    for i, (name, (N, K)) in enumerate(synthetic.SHAPES.items()):
        m = FP8Linear(K, N, device="cuda")
        m.load_weight(synthetic.weight(N, K, 400 + i).cuda())
        a, b = synthetic.lora_factors(N, K, 410 + i)
        m.set_lora(a.cuda(), b.cuda(), synthetic.LORA_SCALING)
        af = oracle.bf16_to_f32(helpers.bits(a)).astype(np.float64)
        bf = oracle.bf16_to_f32(helpers.bits(b)).astype(np.float64)
        if name != "down":
            y = m(x)
            exact = oracle.gemm_exact_f64(xq, sx, helpers.codes_np(m.codes()), m.scale.cpu().numpy()) + \
                oracle.lora_f64(xf, af, bf, synthetic.LORA_SCALING)
        else:
            inter = synthetic.INTERMEDIATE
            gu = outs["gate_up"]
            codes, scales, t, h = swiglu_quantize(gu[:, :inter], gu[:, inter:], lora_a=m.lora[0], return_h=True)
            from jeeves_amd.fp8 import fp8_matmul_quantized
            y = fp8_matmul_quantized(codes, scales, m.weight, m.scale, lora_t=t, lora_b=m.lora[1],
                                     lora_scaling=m.lora[2])
            hq, hs = oracle.quantize_rows(h.float().cpu().numpy())
            assert np.array_equal(hq, helpers.codes_np(codes))
            hf = oracle.bf16_to_f32(helpers.bits(h)).astype(np.float64)
            exact = oracle.gemm_exact_f64(hq, hs, helpers.codes_np(m.codes()), m.scale.cpu().numpy()) + \
                oracle.lora_f64(hf, af, bf, synthetic.LORA_SCALING)
        outs[name] = y
        got = oracle.bf16_to_f32(helpers.bits(y)).astype(np.float64)
        exact_bits = oracle.f64_to_bf16(exact)
        assert oracle.rel_l2(got, oracle.bf16_to_f32(exact_bits)) <= helpers.REL_L2_MAX, name
        bar = helpers.EQUAL_MIN_SWIGLU_H if name == "down" else helpers.EQUAL_MIN
        assert oracle.bitwise_equal_fraction(helpers.bits(y), exact_bits) >= helpers.equal_floor(y.numel(), bar), name
