"""The tiled weight layout (ldw = 0, ``tile_weight``) against row-major
weights: every kernel reads the same codes from it, so outputs are bitwise
identical on every regime -- decode (1-4 token tiles, 4 and 8 waves, split K),
prefill (each tile shape the dispatcher picks), the W8A16 parity mode, packed
activation codes, bias and LoRA -- and FP8Linear, which keeps a tiled copy of its weights
tiled, keeps the reference's row-major state dict and concatenation."""

from __future__ import annotations

import pytest
import torch

from jeeves_amd import _lib, synthetic
from jeeves_amd.fp8 import (FP8Linear, fp8_matmul, fp8_matmul_quantized, fp8_matmul_w8a16, swiglu_quantize,
                            tile_weight, untile_weight)
from jeeves_amd.fp8_weights import FP8, quantize_rows

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def weights():
    cache = {}

    def get(N: int, K: int):
        if (N, K) not in cache:
            wq, sw = quantize_rows(synthetic.weight(N, K, 5000 + N + K).cuda())
            cache[(N, K)] = (wq, sw, tile_weight(wq))
        return cache[(N, K)]

    return get


def test_tile_kernel_matches_layout_and_round_trips():
    """The device conversion equals the host one (the byte-offset formula of
    the C ABI) and untiling restores the codes."""
    g = torch.Generator().manual_seed(1)
    for N, K in ((16, 128), (48, 384), (1040, 4096), (4096, 12288)):
        codes = torch.randint(0, 256, (N, K), dtype=torch.uint8, generator=g)
        dev = tile_weight(codes.cuda()).cpu()
        assert torch.equal(dev, tile_weight(codes))
        assert torch.equal(untile_weight(dev.cuda()).cpu(), codes)
    with pytest.raises(ValueError):
        tile_weight(torch.zeros(40, 128, dtype=torch.uint8, device="cuda"))
    L = _lib.lib()
    buf = torch.zeros(40 * 128, dtype=torch.uint8, device="cuda")
    assert L.jv_fp8_tile_weight(buf.data_ptr(), 128, 40, 128, buf.data_ptr(), None) == _lib.JV_ERR_VALUE


DECODE_SHAPES = [(4096, 4096), (1024, 4096), (24576, 4096), (4096, 12288), (256, 4096), (128, 12288), (144, 1024),
                 (1040, 4224)]


@pytest.mark.parametrize("N,K", DECODE_SHAPES)
@pytest.mark.parametrize("M", [1, 5, 16, 33, 64])
def test_decode_tiled_equals_row_major(weights, N, K, M):
    wq, sw, wt = weights(N, K)
    x = synthetic.activations_outliers(M, K, 5100 + M).cuda()
    assert torch.equal(fp8_matmul(x, wt, sw, tiled=True), fp8_matmul(x, wq, sw))


@pytest.mark.parametrize("N,K", [(24576, 4096), (4096, 4096), (1024, 4096), (4096, 12288), (2048, 1024)])
@pytest.mark.parametrize("M", [65, 300, 2048])
def test_prefill_tiled_equals_row_major(weights, N, K, M):
    wq, sw, wt = weights(N, K)
    x = synthetic.activations_heavy_tail(M, K, 5200 + M).cuda()
    assert torch.equal(fp8_matmul(x, wt, sw, tiled=True), fp8_matmul(x, wq, sw))


@pytest.mark.parametrize("M", [1, 16, 64, 65, 512])
def test_bias_lora_packed_and_w8a16_tiled(weights, M):
    N, K = 4096, 4096
    wq, sw, wt = weights(N, K)
    g = torch.Generator().manual_seed(5300 + M)
    x = synthetic.activations_heavy_tail(M, K, 5301 + M).cuda()
    bias = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16).cuda()
    a, b = synthetic.lora_factors(N, K, 5302)
    lora = (a.cuda(), b.cuda(), synthetic.LORA_SCALING)
    assert torch.equal(fp8_matmul(x, wt, sw, bias=bias, lora=lora, tiled=True), fp8_matmul(x, wq, sw, bias=bias, lora=lora))
    assert torch.equal(fp8_matmul_w8a16(x, wt, sw, bias=bias, tiled=True), fp8_matmul_w8a16(x, wq, sw, bias=bias))
    if M <= 64:
        codes, scales = swiglu_quantize(x[:, :2048], x[:, 2048:], packed=True)
        wq2, sw2, wt2 = weights(N, 2048)
        assert torch.equal(fp8_matmul_quantized(codes, scales, wt2, sw2, packed_rows=M, tiled=True),
                           fp8_matmul_quantized(codes, scales, wq2, sw2, packed_rows=M))


def test_module_keeps_row_major_weight_and_merges():
    """FP8Linear.weight, its state dict, load_state_dict, load_codes and
    codes() all hold the reference's row-major codes; the kernels read the
    tiled copy. Tiled parts concatenate as they are (the parts' copies become
    views of the merged copy), a part that cannot tile makes the merge
    row-major, every part's output is unchanged by the merge, and an in-place
    write to a part's weight reaches the merged module's kernels too."""
    K = 4096
    parts = [FP8Linear(K, n, device="cuda") for n in (2048, 1024, 1024)]
    for i, p in enumerate(parts):
        p.load_weight(synthetic.weight(p.out_features, K, 5400 + i).cuda())
        assert p.tiled
    codes = [quantize_rows(synthetic.weight(p.out_features, K, 5400 + i).cuda())[0] for i, p in enumerate(parts)]
    for p, c in zip(parts, codes):
        assert torch.equal(p.weight.view(torch.uint8), c.view(torch.uint8))
        assert torch.equal(p.state_dict()["weight"].view(torch.uint8), c.view(torch.uint8))
        assert torch.equal(p.kernel_weight()[0], tile_weight(c).view(torch.uint8))
    x = synthetic.activations_outliers(16, K, 5410).cuda()
    before = [p(x) for p in parts]
    merged = FP8Linear.concatenated(parts)
    assert merged.tiled and all(p.tiled for p in parts)
    y = merged(x)
    for p, b, yy in zip(parts, before, y.split([p.out_features for p in parts], dim=1)):
        assert torch.equal(p(x), b) and torch.equal(yy, b)
        assert p.tiled_codes.untyped_storage().data_ptr() == merged.tiled_codes.untyped_storage().data_ptr()
    # a fresh module loaded from the state dict gives the same outputs
    fresh = FP8Linear(K, merged.out_features, device="cuda")
    fresh.load_state_dict(merged.state_dict())
    assert torch.equal(fresh.weight.view(torch.uint8), merged.weight.view(torch.uint8))
    assert torch.equal(fresh(x), y)
    # the reference's load_codes writes weight in place: the kernels follow
    with torch.no_grad():
        parts[1].weight.copy_(codes[2])
        parts[1].scale.copy_(parts[2].scale)
    assert torch.equal(parts[1](x), before[2])
    assert torch.equal(merged(x)[:, 2048:3072], before[2])
    # a part that cannot tile (N % 16 != 0) turns the merge row-major
    odd = FP8Linear(K, 1000, device="cuda")
    odd.load_weight(synthetic.weight(1000, K, 5420).cuda())
    even = FP8Linear(K, 1024, device="cuda")
    even.load_weight(synthetic.weight(1024, K, 5421).cuda())
    want = [odd(x), even(x)]
    mixed = FP8Linear.concatenated([odd, even])
    assert not mixed.tiled and not even.tiled and even.tiled_codes is None
    assert torch.equal(odd(x), want[0]) and torch.equal(even(x), want[1])
    assert torch.equal(mixed(x), torch.cat(want, dim=1))


def test_tiled_graph_replays():
    """A captured decode call on tiled weights replays with new inputs to the
    eager result."""
    N, K, M = 24576, 4096, 16
    wq, sw = quantize_rows(synthetic.weight(N, K, 5500).cuda())
    wt = tile_weight(wq)
    static_x = torch.zeros(M, K, dtype=torch.bfloat16, device="cuda")
    fp8_matmul(static_x, wt, sw, tiled=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fp8_matmul(static_x, wt, sw, tiled=True)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            static_y = fp8_matmul(static_x, wt, sw, tiled=True)
    torch.cuda.current_stream().wait_stream(s)
    for seed in range(3):
        static_x.copy_(synthetic.activations_outliers(M, K, 5510 + seed).cuda())
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_y, fp8_matmul(static_x, wq, sw)), seed
