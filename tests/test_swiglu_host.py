"""Host-side checks of the SwiGLU binding and of its oracle criteria (no GPU):

* ``fuse_swiglus`` on a module shaped like the reference's ``SwiGLU``
  (``model/model.py:574-584``) after ``replace_linears``: the block becomes an
  ``FP8SwiGLU`` whose gate and up are views of one merged gate+up linear, the
  reference's state-dict keys and values are unchanged, the merged linear stays
  outside the module tree, and blocks whose gate or up carries its own LoRA
  adapter stay unfused;
* ``helpers.swiglu_criteria`` accepts SwiGLU of the exact-rounded GEMM outputs
  and rejects planted mistakes: gate and up swapped, a sign error, silu
  rounded once with the product (the other SwiGLU rounding), and a one-unit
  error on a few percent of the outputs."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn

import oracle
from jeeves_amd.fp8 import FP8Linear, FP8SwiGLU, fuse_swiglus
from jeeves_amd.fp8_weights import FP8
from tests import helpers


def _fp8(in_f: int, out_f: int, g: torch.Generator, bias: bool = False) -> FP8Linear:
    m = FP8Linear(in_f, out_f, bias=bias, device="cpu")
    m.weight.copy_(torch.randint(0, 0x7E, (out_f, in_f), generator=g, dtype=torch.uint8).view(FP8))
    m.scale.copy_(torch.rand(out_f, generator=g))
    if bias:
        m.bias.data.copy_(torch.randn(out_f, generator=g).to(torch.bfloat16))
    return m


class Block(nn.Module):
    def __init__(self, hidden: int, inter: int, g: torch.Generator, bias: bool = False):
        super().__init__()
        self.gate_proj, self.up_proj = _fp8(hidden, inter, g, bias), _fp8(hidden, inter, g, bias)
        self.down_proj = _fp8(inter, hidden, g)


def test_fuse_swiglus_keeps_reference_names_and_views():
    g = torch.Generator().manual_seed(0)
    model = nn.ModuleDict({"a": nn.ModuleDict({"mlp": Block(256, 64, g)}), "b": nn.ModuleDict({"mlp": Block(256, 64, g)})})
    before = {k: v.clone() for k, v in model.state_dict().items()}
    gate = model["a"]["mlp"].gate_proj
    assert fuse_swiglus(model) == 2
    mlp = model["a"]["mlp"]
    assert isinstance(mlp, FP8SwiGLU) and mlp.gate_proj is gate
    after = model.state_dict()
    assert set(after) == set(before)
    for k, v in before.items():
        assert torch.equal(after[k].view(torch.uint8), v.view(torch.uint8)) if v.dtype == FP8 else torch.equal(after[k], v), k
    # gate and up are views of the merged codes, scales and tiled copy, gate rows first
    merged = mlp.gate_up
    assert merged.out_features == 128 and merged not in list(mlp.modules())
    assert mlp.gate_proj.weight.data_ptr() == merged.weight.data_ptr()
    assert mlp.up_proj.weight.data_ptr() == merged.weight.data_ptr() + 64 * 256
    assert mlp.up_proj.scale.data_ptr() == merged.scale.data_ptr() + 64 * 4
    assert mlp.up_proj.tiled_codes.data_ptr() == merged.tiled_codes.data_ptr() + 64 * 256
    assert mlp.down is mlp.down_proj
    # already fused blocks are left alone
    assert fuse_swiglus(model) == 0


def test_fuse_swiglus_bias_views_and_lora_blocks():
    g = torch.Generator().manual_seed(1)
    holder = nn.ModuleDict({"mlp": Block(256, 32, g, bias=True)})
    gb, ub = holder["mlp"].gate_proj.bias.clone(), holder["mlp"].up_proj.bias.clone()
    assert fuse_swiglus(holder) == 1
    mlp = holder["mlp"]
    assert torch.equal(mlp.gate_up.bias, torch.cat([gb, ub]))
    assert mlp.up_proj.bias.data_ptr() == mlp.gate_up.bias.data_ptr() + 32 * 2
    lora_holder = nn.ModuleDict({"mlp": Block(256, 32, g)})
    a = torch.zeros(16, 256, dtype=torch.bfloat16)
    b = torch.zeros(32, 16, dtype=torch.bfloat16)
    lora_holder["mlp"].up_proj.set_lora(a, b, 2.0)
    assert fuse_swiglus(lora_holder) == 0 and not isinstance(lora_holder["mlp"], FP8SwiGLU)


def _case(M=6, I=48, K=256, seed=3):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[:, rng.choice(K, 3, replace=False)] *= 20
    w = (rng.standard_normal((2 * I, K)) * 0.02).astype(np.float32)
    xq, sx = oracle.quantize_rows(x)
    wq, sw = oracle.quantize_rows(w)
    exact = oracle.gemm_exact_f64(xq, sx, wq, sw)
    g_bits, u_bits = oracle.f64_to_bf16(exact[:, :I]), oracle.f64_to_bf16(exact[:, I:])
    return xq, sx, wq, sw, g_bits, u_bits


def test_swiglu_criteria_accept_the_oracle_and_reject_planted_mistakes():
    xq, sx, wq, sw, g_bits, u_bits = _case()
    h = oracle.swiglu_bf16(g_bits, u_bits)
    c = helpers.swiglu_criteria(h, xq, sx, wq, sw)
    assert c["equal"] == 1.0 and c["bound"]
    # gate and up swapped
    c = helpers.swiglu_criteria(oracle.swiglu_bf16(u_bits, g_bits), xq, sx, wq, sw)
    assert not c["bound"] and c["equal"] < 0.5
    # a sign error
    c = helpers.swiglu_criteria(h ^ np.uint16(0x8000), xq, sx, wq, sw)
    assert not c["bound"]
    # silu not rounded to bf16 before the product (one rounding instead of two)
    one = oracle.f32_to_bf16(oracle.silu_f32(oracle.bf16_to_f32(g_bits)) * oracle.bf16_to_f32(u_bits))
    c = helpers.swiglu_criteria(one, xq, sx, wq, sw)
    assert c["equal"] < 0.95, c["equal"]
    # one bf16 unit on 6 % of the outputs: inside the bound, below the equality bar
    rng = np.random.default_rng(4)
    bumped = h.copy().reshape(-1)
    bumped[rng.choice(bumped.size, int(np.ceil(0.06 * bumped.size)), replace=False)] += np.uint16(1)
    bumped = bumped.reshape(h.shape)
    c = helpers.swiglu_criteria(bumped, xq, sx, wq, sw)
    assert c["bound"] and c["equal"] < 0.95
