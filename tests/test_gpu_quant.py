"""Bit-exact parity of the gfx950 quantizer with the reference quantizer
(quantize_rows, inference/fp8_weights.py:16-19) as restated by the oracle:
golden fixtures, workload activations, every row length the kernel
specialises on, strided rows, fp32 inputs, special values, NaN-poisoned
outputs, and the fused SwiGLU variant."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jeeves_amd import _lib, synthetic
from jeeves_amd.fp8 import swiglu_quantize
from jeeves_amd.fp8_weights import quantize_row_blocks_on_cpu, quantize_rows
from tests import helpers

pytestmark = pytest.mark.gpu


def assert_matches_oracle(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor) -> None:
    xf = x.detach().float().cpu().numpy()
    want_c, want_s = oracle.quantize_rows(xf)
    got_s = scales.cpu().numpy()
    got_c = helpers.codes_np(codes)
    assert helpers.same_f32(got_s, want_s).all(), "scales differ"
    bad = ~helpers.same_codes(got_c, want_c)
    assert not bad.any(), f"{bad.sum()} codes differ, first at {np.argwhere(bad)[0]}"


def test_golden_edge_rows():
    g = helpers.golden("quantize_rows.npz")
    x = helpers.from_bits(g["edge_x"], "cuda")
    codes, scales = quantize_rows(x)
    assert helpers.same_f32(scales.cpu().numpy(), g["edge_scales"]).all()
    assert helpers.same_codes(helpers.codes_np(codes), g["edge_codes"]).all()


def test_golden_workload_rows():
    g = helpers.golden("quantize_rows.npz")
    for tag in ("cfg0_x", "cfg0_w64"):
        codes, scales = quantize_rows(helpers.from_bits(g[tag], "cuda"))
        assert np.array_equal(scales.cpu().numpy().view(np.uint32), g[f"{tag}_scales"].view(np.uint32)), tag
        assert np.array_equal(helpers.codes_np(codes), g[f"{tag}_codes"]), tag


@pytest.mark.parametrize("K", [128, 256, 1024, 2048, 2176, 4096, 6144, 8192, 10240, 12288, 14336, 16384, 16512, 24576])
def test_every_row_length(K):
    g = torch.Generator().manual_seed(K)
    x = torch.randn(7, K, generator=g) * torch.logspace(-12, 12, 7)[:, None]
    x[0, K // 3] = 5e4
    x[2, :] = 0
    x[3, 5] = float("inf")
    x[4, 7] = float("nan")
    x = x.to(torch.bfloat16).cuda()
    codes, scales = quantize_rows(x)
    assert codes.dtype == torch.float8_e4m3fn and codes.shape == (7, K)
    assert_matches_oracle(x, codes, scales)


# Packed codes of prefill batches (the rows of a 16-token tile on one XCD):
# every row length class, special rows (huge, zero, inf, NaN, tiny) spread
# over the tiles, a partial last tile, the prefill step's shapes, and a long
# batch of long rows (1024-thread workgroups).
@pytest.mark.parametrize("M, K", [(M, K) for M in (65, 200) for K in (128, 1024, 2048, 4096, 6144, 12288, 16384)]
                         + [(2048, 4096), (2048, 12288), (1000, 8192), (4100, 12288)])
def test_packed_prefill_rows(M, K):
    from jeeves_amd.fp8 import packed_codes_bytes, tile_weight

    g = torch.Generator().manual_seed(M * 7 + K)
    x = torch.randn(M, K, generator=g) * torch.logspace(-12, 12, M)[:, None]
    x[0, K // 3] = 5e4
    x[17, :] = 0
    x[33, 5] = float("inf")
    x[50, 7] = float("nan")
    x = x.to(torch.bfloat16).cuda()
    want_codes, want_scales = quantize_rows(x)
    assert_matches_oracle(x, want_codes, want_scales)
    padded = torch.zeros((M + 15) // 16 * 16, K, dtype=torch.uint8, device="cuda")
    padded[:M] = want_codes.view(torch.uint8)
    want = tile_weight(padded).view(torch.uint8).reshape(-1)
    packed = torch.full((packed_codes_bytes(M, K),), 0xAA, dtype=torch.uint8, device="cuda")
    scales = torch.full((M,), float("nan"), device="cuda")
    _lib.check(_lib.lib().jv_fp8_quantize_rows_bf16(x.data_ptr(), K, M, K, packed.data_ptr(), 0, scales.data_ptr(),
                                                    helpers.stream()))
    assert helpers.same_f32(scales.cpu().numpy(), want_scales.cpu().numpy()).all()
    same = helpers.same_codes(packed.cpu().numpy(), want.cpu().numpy())
    assert same.all(), f"{(~same).sum()} packed codes differ"


def test_workload_activations():
    cases = [synthetic.single_linear()[0]]
    cases += [synthetic.decode_case(n, M)[0] for n in ("q", "down") for M in synthetic.DECODE_ROWS]
    cases += [synthetic.activations_heavy_tail(512, K, 812) for K in (4096, 12288)]
    for x in cases:
        x = x.cuda()
        assert_matches_oracle(x, *quantize_rows(x))


def test_weight_rows_of_every_projection_shape():
    for name, (N, K) in synthetic.SHAPES.items():
        w = synthetic.weight(N, K, 100 + synthetic.SHAPE_INDEX[name])[:512].cuda()
        assert_matches_oracle(w, *quantize_rows(w))


def test_strided_rows():
    big = (torch.randn(9, 8192 + 64) * 3).to(torch.bfloat16).cuda()
    x = big[:, 64:64 + 4096]
    assert x.stride(0) == 8192 + 64
    assert_matches_oracle(x, *quantize_rows(x))


def test_float32_rows():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(33, 4100, generator=g) * torch.logspace(-20, 20, 33)[:, None]
    x[1, 2] = float("inf")
    x[2, 3] = float("nan")
    x[4] = 0
    x[5, 9] = 3.4e38
    x = x.cuda()
    assert_matches_oracle(x, *quantize_rows(x))
    odd = torch.randn(5, 7).cuda()  # width not a multiple of 4: padded internally
    assert_matches_oracle(odd, *quantize_rows(odd))


def test_cpu_tensors_round_trip_through_the_device():
    x = synthetic.weight(1024, 4096, 5)
    codes, scales = quantize_rows(x)
    assert codes.device.type == "cpu" and scales.device.type == "cpu"
    assert_matches_oracle(x, codes, scales)
    blocks = list(quantize_row_blocks_on_cpu(x))
    assert len(blocks) == 1 and torch.equal(blocks[0][1].view(torch.uint8), codes.view(torch.uint8))


def test_every_output_written_and_deterministic():
    # NaN-poisoned outputs catch elements a kernel never writes
    x = synthetic.activations_heavy_tail(300, 12288, 77).cuda()
    codes = torch.full((300, 12288), 0x7F, dtype=torch.uint8, device="cuda")
    scales = torch.full((300,), float("nan"), device="cuda")
    _lib.check(_lib.lib().jv_fp8_quantize_rows_bf16(x.data_ptr(), 12288, 300, 12288, codes.data_ptr(), 12288,
                                                    scales.data_ptr(), helpers.stream()))
    assert_matches_oracle(x, codes, scales)
    again, s2 = quantize_rows(x)
    assert torch.equal(again.view(torch.uint8), codes) and torch.equal(s2, scales)


def test_swiglu_quantize_matches_oracle():
    g = torch.Generator().manual_seed(12)
    M, I = 96, 12288
    gu = (torch.randn(M, 2 * I, generator=g) * 2).to(torch.bfloat16).cuda()
    gate, up = gu[:, :I], gu[:, I:]
    a = (torch.randn(16, I, generator=g) * 0.01).to(torch.bfloat16).cuda()
    codes, scales, t, h = swiglu_quantize(gate, up, lora_a=a, return_h=True)
    want_h = oracle.swiglu_bf16(helpers.bits(gate), helpers.bits(up))
    got_h = helpers.bits(h)
    assert oracle.bitwise_equal_fraction(got_h, want_h) == 1.0
    # the codes are exactly the reference quantizer applied to the device's h
    assert_matches_oracle(h, codes, scales)
    # the fused LoRA down-projection t = h A^T
    want_t = oracle.bf16_to_f32(got_h).astype(np.float64) @ oracle.bf16_to_f32(helpers.bits(a)).astype(np.float64).T
    assert np.allclose(t.cpu().numpy(), want_t, rtol=1e-4, atol=1e-5)


def test_swiglu_on_every_bf16_gate_value():
    """h = bf16(bf16(silu(gate)) * up) bitwise against the oracle (torch's bf16
    F.silu(gate) * up) with the gate running over all 65536 bf16 patterns and
    random bf16 ups; the codes follow the reference quantizer on h."""
    gate = torch.from_numpy(np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.int16)).view(torch.bfloat16)
    gate = gate.reshape(16, 4096).cuda()
    up = (torch.randn(16, 4096, generator=torch.Generator().manual_seed(13)) * 3).to(torch.bfloat16).cuda()
    codes, scales, h = swiglu_quantize(gate, up, return_h=True)
    want_h = oracle.swiglu_bf16(helpers.bits(gate), helpers.bits(up))
    assert oracle.bitwise_equal_fraction(helpers.bits(h), want_h) == 1.0
    assert_matches_oracle(h, codes, scales)
