"""FP8 checkpoint round trip with the device quantizer: the exporter's codes
and scales are quantize_rows' (bit-exact with the oracle), and a module
loaded from the FP8 file computes exactly what a module loaded from the bf16
file (quantized while loading) computes."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import oracle
from jeeves_amd import fp8_checkpoint
from jeeves_amd.fp8 import FP8Linear
from jeeves_amd.fp8_weights import replace_linears
from tests import helpers
from tests.test_checkpoint import Block, make_checkpoint

pytestmark = pytest.mark.gpu


def cuda_block():
    m = Block().to(torch.bfloat16)
    replace_linears(m, lambda lin: FP8Linear(lin.in_features, lin.out_features, bias=lin.bias is not None, device="cuda"))
    return m.cuda()


def test_export_then_load_equals_quantize_on_load(tmp_path):
    src, dst = tmp_path / "in.safetensors", tmp_path / "out.safetensors"
    tensors = make_checkpoint(src, 3)
    fp8_checkpoint.write_quantized(src, dst, fp8_checkpoint.quantized_linears(Block()))
    from_fp8, from_bf16 = cuda_block(), cuda_block()
    _, unexpected = fp8_checkpoint.load_tensors(from_fp8, [dst], FP8Linear)
    assert unexpected == []
    _, unexpected = fp8_checkpoint.load_tensors(from_bf16, [src], FP8Linear)
    assert unexpected == []
    for name in ("q", "o"):
        a, b = getattr(from_fp8, name), getattr(from_bf16, name)
        assert torch.equal(a.weight.view(torch.uint8), b.weight.view(torch.uint8)) and torch.equal(a.scale, b.scale)
        codes, scale = oracle.quantize_rows(tensors[f"{name}.weight"].float().numpy())
        assert np.array_equal(helpers.codes_np(a.codes()), codes)
        assert np.array_equal(a.scale.cpu().numpy(), scale)
    x = torch.randn(20, 256, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).cuda()
    assert torch.equal(from_fp8.q(x), from_bf16.q(x))
    x2 = torch.randn(300, 512, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).cuda()
    assert torch.equal(from_fp8.o(x2), from_bf16.o(x2))


def test_cpu_quantizer_blocks_match_one_pass():
    w = (torch.randn(20000, 256, generator=torch.Generator().manual_seed(6)) * 0.02).to(torch.bfloat16)
    codes, scale = fp8_checkpoint.quantize_on_cpu(w)   # two blocks of QUANTIZE_BLOCK_ROWS
    assert codes.device.type == "cpu" and scale.device.type == "cpu"
    want_codes, want_scale = oracle.quantize_rows(w.float().numpy())
    assert np.array_equal(codes.view(torch.uint8).numpy(), want_codes)
    assert np.array_equal(scale.numpy(), want_scale)
