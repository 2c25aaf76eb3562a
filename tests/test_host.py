"""Host-side logic of the drop-in module that runs without a GPU: the
quantizability rule, module replacement, FP8Linear buffers and merges,
argument validation, the host quantizer of GPU-less exports, and the
synthetic workload generators."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import jeeves_amd
import oracle
from jeeves_amd import synthetic
from tests import helpers
from jeeves_amd.fp8 import FP8Linear, fp8_matmul
from jeeves_amd.fp8_weights import FP8, FP8_MAX, FP8_MAX_RECIPROCAL, QUANTIZE_BLOCK_ROWS, SCALE_SUFFIX, quantizable, replace_linears


def test_constants_match_reference():
    assert FP8 is torch.float8_e4m3fn and FP8_MAX == 448.0
    assert FP8_MAX_RECIPROCAL == float.fromhex("0x1.24924ap-9")
    assert SCALE_SUFFIX == "_scale" and QUANTIZE_BLOCK_ROWS == 16384
    assert jeeves_amd.BLOCK_K == 128 and jeeves_amd.TILE_COUNTER_SLOTS == 1 << 16


def test_quantizable_and_replace_linears():
    with torch.device("meta"):
        model = nn.Sequential(nn.Linear(4096, 4096), nn.Sequential(nn.Linear(4096, 1024), nn.Linear(4096, 32)),
                              nn.Linear(100, 2048), nn.Linear(4096, 1040))
    assert quantizable(model[0]) and not quantizable(model[1][1]) and not quantizable(model[2])
    n = replace_linears(model, lambda l: FP8Linear(l.in_features, l.out_features, bias=l.bias is not None, device="meta"))
    assert n == 3
    assert isinstance(model[0], FP8Linear) and isinstance(model[1][0], FP8Linear) and isinstance(model[3], FP8Linear)
    assert isinstance(model[1][1], nn.Linear) and isinstance(model[2], nn.Linear)


def test_fp8_linear_buffers_and_state_dict():
    m = FP8Linear(256, 1024, bias=True, device="meta")
    assert m.weight.dtype == FP8 and m.weight.shape == (1024, 256)
    assert m.scale.dtype == torch.float32 and m.scale.shape == (1024,)
    assert m.bias.dtype == torch.bfloat16 and not m.bias.requires_grad
    assert set(m.state_dict()) == {"weight", "scale", "bias"}
    assert set(FP8Linear(256, 1024).state_dict()) == {"weight", "scale"}


def test_concatenated_parts_become_views():
    # inference/cuda_test.py:38-46: merging keeps codes and scales and the parts view the merged storage
    g = torch.Generator().manual_seed(0)
    parts = []
    for n in (64, 16, 16):
        p = FP8Linear(128, n, device="cpu")
        p.weight.copy_(torch.randint(0, 0x7E, (n, 128), generator=g, dtype=torch.uint8).view(FP8))
        p.scale.copy_(torch.rand(n, generator=g))
        parts.append(p)
    codes = [p.weight.clone() for p in parts]
    scales = [p.scale.clone() for p in parts]
    merged = FP8Linear.concatenated(parts)
    assert merged.out_features == 96 and merged.in_features == 128
    for p, c, s in zip(parts, codes, scales):
        assert torch.equal(p.weight.view(torch.uint8), c.view(torch.uint8)) and torch.equal(p.scale, s)
        assert p.weight.untyped_storage().data_ptr() == merged.weight.untyped_storage().data_ptr()
        assert p.scale.untyped_storage().data_ptr() == merged.scale.untyped_storage().data_ptr()
        assert p.tiled_codes.untyped_storage().data_ptr() == merged.tiled_codes.untyped_storage().data_ptr()
    from jeeves_amd.fp8 import tile_weight
    assert torch.equal(merged.kernel_weight()[0], tile_weight(torch.cat(codes)).view(torch.uint8))


def test_tiled_layout_on_host():
    """tile_weight's byte order is the C ABI's (fragment of 16 rows x 128 k:
    two 1 KB halves of 64 lanes x 16 bytes, lane = n%16 + 16*((k%128)/32)),
    untile_weight inverts it, and FP8Linear keeps the reference's row-major
    codes in ``weight`` (and its state dict) with the kernels' tiled copy in a
    non-persistent ``tiled_codes`` buffer, rebuilt when ``weight`` changes."""
    from jeeves_amd.fp8 import tile_weight, tileable, untile_weight

    g = torch.Generator().manual_seed(3)
    N, K = 48, 384
    codes = torch.randint(0, 256, (N, K), generator=g, dtype=torch.uint8)
    tiled = tile_weight(codes).view(-1)
    for n, k in ((0, 0), (5, 17), (31, 127), (37, 300), (47, 383)):
        kk = k % 128
        off = ((n // 16 * (K // 128) + k // 128) * 2 + (kk // 16) % 2) * 1024 + (n % 16 + 16 * (kk // 32)) * 16 + k % 16
        assert tiled[off] == codes[n, k]
    assert torch.equal(untile_weight(tiled.view(N, K)), codes)
    assert tileable(1024, 4096) and not tileable(1000, 4096) and not tileable(1024, 4000)
    m = FP8Linear(K, N)
    assert m.tiled
    m.load_codes(codes.view(FP8), torch.ones(N))
    assert m.weight.dtype == FP8 and torch.equal(m.weight.view(torch.uint8), codes)
    w, is_tiled = m.kernel_weight()
    assert is_tiled and torch.equal(w.view(-1), tiled)
    assert set(m.state_dict()) == {"weight", "scale"}
    assert torch.equal(m.state_dict()["weight"].view(torch.uint8), codes)
    assert torch.equal(m.codes().view(torch.uint8), codes)
    other = FP8Linear(K, N)
    other.load_state_dict(m.state_dict())
    assert torch.equal(other.weight.view(torch.uint8), codes)
    assert torch.equal(other.kernel_weight()[0].view(-1), tiled)
    # an in-place write to weight (the reference's load_codes does weight.copy_)
    # is picked up by the next kernel_weight
    flipped = codes.flip(0).contiguous()
    with torch.no_grad():
        m.weight.copy_(flipped.view(FP8))
    assert torch.equal(m.kernel_weight()[0], tile_weight(flipped))
    FP8Linear.TILED_COPY = False
    try:
        plain = FP8Linear(K, N)
        assert not plain.tiled and plain.tiled_codes is None and plain.kernel_weight()[0] is plain.weight
    finally:
        FP8Linear.TILED_COPY = True
    assert not FP8Linear(K, 1000, device="meta").tiled


def test_fp8_matmul_validates_before_launch():
    x = torch.zeros(4, 100, dtype=torch.bfloat16)
    w = torch.zeros(64, 100, dtype=torch.uint8).view(FP8)
    with pytest.raises(ValueError, match="divisible by 128"):
        fp8_matmul(x, w, torch.ones(64))
    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="equal to the weight's"):
        fp8_matmul(x, torch.zeros(64, 128, dtype=torch.uint8).view(FP8), torch.ones(64))
    w = torch.zeros(64, 256, dtype=torch.uint8).view(FP8)
    with pytest.raises(ValueError, match="LoRA"):
        fp8_matmul(x, w, torch.ones(64), lora=(torch.zeros(8, 256), torch.zeros(64, 8), 2.0))


def test_operands_must_sit_on_a_hip_device():
    """A host pointer passed to a kernel is a GPU memory fault, so host tensors
    are refused before anything is enqueued (as the reference's Triton
    launcher refuses them), and so are weights that are not one-byte codes and
    scales or biases of the wrong length."""
    from jeeves_amd.fp8 import fp8_matmul_quantized, fp8_matmul_w8a16, swiglu_quantize

    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    w = torch.zeros(64, 256, dtype=torch.uint8).view(FP8)
    with pytest.raises(ValueError, match="HIP device"):
        fp8_matmul(x, w, torch.ones(64))
    with pytest.raises(ValueError, match="HIP device"):
        fp8_matmul_w8a16(x, w, torch.ones(64))
    with pytest.raises(ValueError, match="HIP device"):
        fp8_matmul_quantized(torch.zeros(4, 256, dtype=torch.uint8), torch.ones(4), w, torch.ones(64))
    with pytest.raises(ValueError, match="HIP device"):
        swiglu_quantize(torch.zeros(4, 256, dtype=torch.bfloat16), torch.zeros(4, 256, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="x_scale"):
        fp8_matmul_quantized(torch.zeros(4, 256, dtype=torch.uint8), torch.ones(3), w, torch.ones(64))
    with pytest.raises(ValueError, match="activation codes"):
        fp8_matmul_quantized(torch.zeros(4, 256, dtype=torch.bfloat16), torch.ones(4), w, torch.ones(64))


def test_set_lora_validates_shapes():
    m = FP8Linear(256, 1024, device="meta")
    with pytest.raises(ValueError):
        m.set_lora(torch.zeros(16, 128), torch.zeros(1024, 16), 2.0)
    m.set_lora(torch.zeros(16, 256), torch.zeros(1024, 16), 2.0)
    assert m.lora[2] == 2.0 and m.lora[0].dtype == torch.bfloat16


def test_synthetic_generators_are_seeded():
    x1, w1 = synthetic.single_linear()
    x2, w2 = synthetic.single_linear()
    assert torch.equal(x1, x2) and torch.equal(w1, w2)
    assert x1.shape == (16, 4096) and w1.shape == (4096, 4096) and x1.dtype == torch.bfloat16
    # 8 outlier channels scaled x20
    col_std = x1.float().std(0)
    assert (col_std > 5).sum() == 8
    assert abs(w1.float().std().item() - 0.02) < 1e-3
    xh = synthetic.activations_heavy_tail(512, 4096, 300 + 512).float()
    kurt = ((xh - xh.mean(0)) ** 4).mean(0) / xh.var(0) ** 2
    assert (kurt > 6).sum() >= 20  # the Student-t channels
    lens = synthetic.ragged_lengths()
    assert len(lens) == 64 and min(lens) >= 64 and max(lens) <= 2048
    assert synthetic.SHAPES["gate_up"] == (24576, 4096) and synthetic.SHAPES["down"] == (4096, 12288)
    a, b = synthetic.lora_factors(1024, 4096, 400)
    assert a.shape == (16, 4096) and b.shape == (1024, 16)
    assert abs(a.float().std().item() - 0.01) < 1e-3


def test_decode_case_seeds_are_distinct():
    xa, wa = synthetic.decode_case("q", 16)
    xb, wb = synthetic.decode_case("o", 16)
    assert torch.equal(xa, xb) and not torch.equal(wa, wb)
    assert np.isfinite(xa.float().numpy()).all()


def test_host_quantizer_matches_golden_fixtures_and_oracle():
    """The library's host quantizer (the exporter's path on a machine without a
    GPU) against torch's own quantize_rows outputs (tests/golden) and the
    oracle on rows with zeros, subnormals, huge values, inf and NaN, on 1 and
    several threads."""
    from jeeves_amd import _lib

    L = _lib.lib()

    def host(w: np.ndarray, threads: int):
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = w.shape
        codes = np.empty((rows, cols), np.uint8)
        scales = np.empty(rows, np.float32)
        _lib.check(L.jv_fp8_quantize_rows_host(w.ctypes.data, cols, rows, cols, codes.ctypes.data, cols,
                                               scales.ctypes.data, threads))
        return codes, scales

    g = helpers.golden("quantize_rows.npz")
    for name in ("edge", "cfg0_x", "cfg0_w64"):
        x = g[f"{name}_x" if name == "edge" else name]
        codes, scales = host(oracle.bf16_to_f32(x), 3)
        want_codes = g[f"{name}_codes"]
        nan = (want_codes & 0x7F) == 0x7F
        assert np.array_equal(codes[~nan], want_codes[~nan]) and np.all((codes[nan] & 0x7F) == 0x7F), name
        assert np.array_equal(scales.view(np.uint32), g[f"{name}_scales"].view(np.uint32)), name
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((257, 999)) * rng.choice([1e-40, 1e-30, 1e-3, 1.0, 1e4, 3e38], (257, 1))).astype(np.float32)
    w[5, 3], w[6], w[7, 2], w[8], w[9, 1::2] = np.inf, 0.0, np.nan, -np.inf, 1e-45
    want_codes, want_scales = oracle.quantize_rows(w)
    for threads in (1, 4, 0):
        codes, scales = host(w, threads)
        assert np.array_equal(codes, want_codes.view(np.uint8)), threads
        assert np.array_equal(scales.view(np.uint32), want_scales.view(np.uint32)), threads
    # argument errors, no HIP call
    bad = np.zeros((2, 4), np.float32)
    out = np.zeros((2, 4), np.uint8)
    sc = np.zeros(2, np.float32)
    assert L.jv_fp8_quantize_rows_host(bad.ctypes.data, 2, 2, 4, out.ctypes.data, 4, sc.ctypes.data, 1) == 1
    assert L.jv_fp8_quantize_rows_host(bad.ctypes.data, 4, 2, 0, out.ctypes.data, 4, sc.ctypes.data, 1) == 1


@pytest.mark.skipif(torch.cuda.is_available(), reason="the path for hosts without a GPU")
def test_quantize_row_blocks_on_cpu_without_a_gpu(monkeypatch):
    """inference/fp8_weights.py:22-26 on a host without a GPU: CPU blocks in
    order, bitwise the oracle's; quantize_rows itself still refuses to run
    without a HIP device."""
    from jeeves_amd import fp8_weights

    monkeypatch.setattr(fp8_weights, "QUANTIZE_BLOCK_ROWS", 48)
    w = (torch.randn(100, 256, generator=torch.Generator().manual_seed(3)) * 0.05).to(torch.bfloat16)
    blocks = list(fp8_weights.quantize_row_blocks_on_cpu(w))
    assert [b[0] for b in blocks] == [slice(0, 48), slice(48, 96), slice(96, 144)]
    codes = torch.cat([b[1] for b in blocks]).view(torch.uint8).numpy()
    scales = torch.cat([b[2] for b in blocks]).numpy()
    want_codes, want_scales = oracle.quantize_rows(w.float().numpy())
    assert all(b[1].device.type == "cpu" and b[1].dtype == fp8_weights.FP8 for b in blocks)
    assert np.array_equal(codes, want_codes.view(np.uint8)) and np.array_equal(scales, want_scales)
    with pytest.raises(RuntimeError, match="HIP device"):
        fp8_weights.quantize_rows(w)
