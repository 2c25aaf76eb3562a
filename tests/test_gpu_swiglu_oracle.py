"""The fused SwiGLU against the oracle alone (model/model.py:574-584).

* ``gate_up_swiglu``'s h is compared with ``oracle.swiglu_bf16`` of the exact
  gate and up products (``oracle.gemm_exact_f64`` on the same FP8 inputs)
  rounded to bf16, and must lie inside the interval SwiGLU maps the GEMM
  criteria's per-output allowance to (``helpers.swiglu_criteria``); its
  per-16-channel maxima must be those of h.
* A module shaped like the reference's ``SwiGLU`` (``gate_proj``,
  ``up_proj``, ``down_proj``; ``F.silu(gate) * up``), its linears swapped for
  ``FP8Linear`` by ``replace_linears``, is fused by ``fuse_swiglus``: it then
  runs ``FP8SwiGLU`` (the SwiGLU epilogue, the quantization of h, the down
  GEMM), keeps the reference's state-dict keys, and its output meets the GEMM
  criteria against the oracle on the oracle's quantization of that h.

Rows are sampled (16 per batch) so the float64 oracle stays fast."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import oracle
from jeeves_amd import synthetic
from jeeves_amd.fp8 import FP8Linear, FP8SwiGLU, fp8_matmul, fuse_swiglus, gate_up_swiglu, tile_weight
from jeeves_amd.fp8_weights import quantize_rows, replace_linears
from tests import helpers

pytestmark = pytest.mark.gpu

# Share of h bitwise equal to SwiGLU of the exact-rounded gate and up values
# (less three binomial standard deviations for the outputs checked): h differs
# where either GEMM output differs from its exact rounding (about 1-2 % each
# on these inputs, tests/helpers.py; measured 0.976-0.983 for h), and a
# differing gate or up value moves h by at most a few bf16 units, which the
# bound checks.
H_EQUAL_MIN = 0.97

SHAPES = [(12288, 4096), (1024, 4096), (1040, 2048), (2048, 12288)]


def sample_rows(M: int) -> np.ndarray:
    return np.arange(M) if M <= 16 else np.unique(np.linspace(0, M - 1, 16).astype(np.int64))


def amax_of(h_bits: np.ndarray) -> np.ndarray:
    return (h_bits.astype(np.uint32) & 0x7FFF).reshape(h_bits.shape[0], -1, 16).max(axis=2).astype(np.uint16)


@pytest.mark.parametrize("I,K", SHAPES)
@pytest.mark.parametrize("M", [1, 16, 64, 512, 2048])
def test_gate_up_swiglu_h_against_oracle(I, K, M):
    print(f"swiglu vs oracle I={I} K={K} M={M}", flush=True)
    N = 2 * I
    x = synthetic.activations_heavy_tail(M, K, 9000 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 9001 + I).cuda())
    h, parts = gate_up_swiglu(x, tile_weight(wq), sw, tiled=True, amax=True)
    rows = sample_rows(M)
    h_bits = helpers.bits(h)
    xq, sx = oracle.quantize_rows(x[torch.from_numpy(rows).cuda()].float().cpu().numpy())
    c = helpers.swiglu_criteria(h_bits[rows], xq, sx, helpers.codes_np(wq), sw.cpu().numpy())
    print(f"  h equal {c['equal']:.5f} outside {c['outside']}", flush=True)
    assert c["bound"], (I, K, M, c["outside"])
    assert c["equal"] >= helpers.equal_floor(len(rows) * I, H_EQUAL_MIN), (I, K, M, c["equal"])
    assert np.array_equal(parts.cpu().numpy().view(np.uint16), amax_of(h_bits)), (I, K, M)


def test_gate_up_swiglu_h_with_bias_against_oracle():
    I, K, M = 12288, 4096, 64
    N = 2 * I
    x = synthetic.activations_outliers(M, K, 9100).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 9101).cuda())
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(9102)) * 0.1).to(torch.bfloat16).cuda()
    h = gate_up_swiglu(x, wq, sw, bias=bias)
    rows = sample_rows(M)
    xq, sx = oracle.quantize_rows(x[torch.from_numpy(rows).cuda()].float().cpu().numpy())
    c = helpers.swiglu_criteria(helpers.bits(h)[rows], xq, sx, helpers.codes_np(wq), sw.cpu().numpy(),
                                bias_bits=helpers.bits(bias))
    assert c["bound"] and c["equal"] >= helpers.equal_floor(len(rows) * I, H_EQUAL_MIN), (c["outside"], c["equal"])


class ReferenceSwiGLU(nn.Module):
    """The reference's ``SwiGLU`` block (``model/model.py:574-584``) on its
    ``F.silu(gate) * up`` branch."""

    def __init__(self, hidden: int, inter: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden, inter, bias=False, dtype=torch.bfloat16)
        self.up_proj = nn.Linear(hidden, inter, bias=False, dtype=torch.bfloat16)
        self.down_proj = nn.Linear(inter, hidden, bias=False, dtype=torch.bfloat16)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, up = self.gate_proj(x), self.up_proj(x)
        return self.down_proj(F.silu(gate) * up)


class Layer(nn.Module):
    def __init__(self, hidden: int, inter: int):
        super().__init__()
        self.mlp = ReferenceSwiGLU(hidden, inter)


def fp8_layer(hidden: int, inter: int, seed: int) -> Layer:
    layer = Layer(hidden, inter)
    with torch.no_grad():
        for i, lin in enumerate((layer.mlp.gate_proj, layer.mlp.up_proj, layer.mlp.down_proj)):
            lin.weight.copy_(synthetic.weight(lin.out_features, lin.in_features, seed + i))
    layer = layer.cuda()

    def make(linear: nn.Linear) -> FP8Linear:  # inference/cuda_test.py:17-20
        m = FP8Linear(linear.in_features, linear.out_features, device=linear.weight.device)
        m.load_weight(linear.weight)
        return m

    assert replace_linears(layer, make) == 3
    return layer


@pytest.mark.parametrize("M", [1, 16, 64, 512, 2048])
def test_reference_mlp_fused_by_fuse_swiglus(M):
    print(f"reference MLP fused M={M}", flush=True)
    hidden, inter = synthetic.HIDDEN, synthetic.INTERMEDIATE
    layer = fp8_layer(hidden, inter, 9200)
    keys = {k: v.clone() for k, v in layer.state_dict().items()}
    x = synthetic.activations_heavy_tail(M, hidden, 9210 + M).cuda()
    unfused = layer.mlp(x)  # two FP8 GEMMs, torch's silu * up, the down FP8 GEMM
    gate, up, down = layer.mlp.gate_proj, layer.mlp.up_proj, layer.mlp.down_proj
    assert fuse_swiglus(layer) == 1 and isinstance(layer.mlp, FP8SwiGLU) and layer.mlp.fused()
    mlp = layer.mlp
    assert mlp.gate_proj is gate and mlp.up_proj is up and mlp.down_proj is down
    # the reference's state-dict keys and values, unchanged
    sd = layer.state_dict()
    assert set(sd) == set(keys)
    for k, v in keys.items():
        assert torch.equal(sd[k].view(torch.uint8) if v.dtype == torch.float8_e4m3fn else sd[k],
                           v.view(torch.uint8) if v.dtype == torch.float8_e4m3fn else v), k
    # gate and up are views of the merged gate+up codes, gate rows first
    assert gate.weight.untyped_storage().data_ptr() == mlp.gate_up.weight.untyped_storage().data_ptr()
    assert up.weight.data_ptr() == mlp.gate_up.weight.data_ptr() + inter * hidden

    y = layer.mlp(x)
    # the block is the fused gate+up GEMM's h fed to the down FP8Linear, bit for bit
    w, tiled = mlp.gate_up.kernel_weight()
    h = gate_up_swiglu(x, w, mlp.gate_up.scale, tiled=tiled)
    assert torch.equal(y, down(h))
    rows = sample_rows(M)
    sel = torch.from_numpy(rows).cuda()
    xq, sx = oracle.quantize_rows(x[sel].float().cpu().numpy())
    wcodes = helpers.codes_np(mlp.gate_up.weight)
    c = helpers.swiglu_criteria(helpers.bits(h)[rows], xq, sx, wcodes, mlp.gate_up.scale.cpu().numpy())
    assert c["bound"] and c["equal"] >= helpers.equal_floor(len(rows) * inter, H_EQUAL_MIN), (M, c["outside"], c["equal"])
    hq, hs = oracle.quantize_rows(h[sel].float().cpu().numpy())
    g = helpers.gemm_criteria(helpers.bits(y)[rows], hq, hs, helpers.codes_np(down.weight), down.scale.cpu().numpy())
    assert g["bound"] and g["finite_match"] and g["rel_l2"] <= helpers.REL_L2_MAX, g
    assert g["equal"] >= helpers.equal_floor(g["n"], helpers.EQUAL_MIN_SWIGLU_H), g
    # against the unfused module: torch's silu on the device may round a rare
    # h differently, so the outputs agree closely rather than bitwise
    assert oracle.rel_l2(oracle.bf16_to_f32(helpers.bits(y)), oracle.bf16_to_f32(helpers.bits(unfused))) <= 2e-3


def test_fuse_swiglus_leaves_lora_blocks_and_runs_under_inference_mode():
    """Blocks whose gate or up carries its own LoRA stay unfused; a block built,
    merged and run entirely under torch.inference_mode() (inference tensors
    keep no version counter) gives the result of the same block built outside
    it."""
    hidden, inter, M = 4096, 1024, 16
    x = synthetic.activations_outliers(M, hidden, 9300).cuda()
    layer = fp8_layer(hidden, inter, 9310)
    a, b = synthetic.lora_factors(inter, hidden, 9320)
    layer.mlp.gate_proj.set_lora(a.cuda(), b.cuda(), synthetic.LORA_SCALING)
    assert fuse_swiglus(layer) == 0 and not isinstance(layer.mlp, FP8SwiGLU)

    want_layer = fp8_layer(hidden, inter, 9330)
    fuse_swiglus(want_layer)
    want = want_layer.mlp(x)
    with torch.inference_mode():
        layer = fp8_layer(hidden, inter, 9330)
        assert torch.is_inference(layer.mlp.gate_proj.weight)
        assert fuse_swiglus(layer) == 1
        got = layer.mlp(x)
        got_again = layer.mlp(x)
    assert torch.equal(got, want) and torch.equal(got_again, want)


def test_retile_after_writes_the_version_counter_misses():
    """A write through weight.data bypasses the version counter; retile()
    rebuilds the tiled copy the kernels read."""
    K, N, M = 4096, 1024, 16
    m = FP8Linear(K, N, device="cuda")
    m.load_weight(synthetic.weight(N, K, 9400).cuda())
    other = FP8Linear(K, N, device="cuda")
    other.load_weight(synthetic.weight(N, K, 9401).cuda())
    x = synthetic.activations_outliers(M, K, 9402).cuda()
    before = m(x)
    m.weight.data.copy_(other.weight)
    m.scale.copy_(other.scale)
    m.retile()
    assert torch.equal(m(x), other(x)) and not torch.equal(m(x), before)
    assert torch.equal(m(x), fp8_matmul(x, m.weight, m.scale))
