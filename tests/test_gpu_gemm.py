"""Parity of the FP8 x FP8 GEMM (decode and prefill kernels, fused epilogue)
with the oracle, under the reference's own acceptance criteria
(inference/cuda_test.py:74-94, model/metal_test.py:202-243):
rel-L2 <= 1e-3 against the bf16 dequantize-then-matmul output on the same FP8
inputs, outputs bitwise equal to the exact result rounded once to bf16 (at
least 98% per call, less three binomial standard deviations for the call's
output count: the FP8 MFMA's in-instruction alignment moves ~1-2% of outputs
to the neighbouring bf16 value, where the reference's fp16 MMA gets 99.5%), the
float64 error bound |out - exact| <= |exact| 2^-8 + magnitude 2^-12 (the form
of model/metal_test.py:219-221), finite outputs, and bitwise-identical repeat
calls. The tolerances live in tests/helpers.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from jeeves_amd import _lib, synthetic
from jeeves_amd.fp8 import fp8_matmul, fp8_matmul_quantized, swiglu_quantize, tile_weight
from jeeves_amd.fp8_weights import FP8, quantize_rows
from tests import helpers

pytestmark = pytest.mark.gpu

EQUAL_MIN, REL_L2_MAX = helpers.EQUAL_MIN, helpers.REL_L2_MAX


def check(y: torch.Tensor, x: torch.Tensor, wq: torch.Tensor, sw: torch.Tensor, bias=None, lora=None, equal_min=EQUAL_MIN):
    xq, sx = oracle.quantize_rows(x.float().cpu().numpy())
    lora_term = None
    if lora is not None:
        a, b, s = lora
        lora_term = oracle.lora_f64(oracle.bf16_to_f32(helpers.bits(x)), oracle.bf16_to_f32(helpers.bits(a)),
                                    oracle.bf16_to_f32(helpers.bits(b)), s)
    c = helpers.gemm_criteria(helpers.bits(y), xq, sx, helpers.codes_np(wq), sw.cpu().numpy(),
                              bias_bits=helpers.bits(bias) if bias is not None else None, lora_term=lora_term)
    assert c["finite_match"], ("non-finite outputs where the exact result is finite (or the reverse)", c)
    assert c["equal"] >= helpers.equal_floor(c["n"], equal_min), c
    assert c["rel_l2"] <= REL_L2_MAX, c
    assert c["bound"], c
    return c


@pytest.fixture(scope="module")
def weights():
    cache = {}

    def get(N: int, K: int):
        if (N, K) not in cache:
            g = torch.Generator().manual_seed(N * 7 + K)
            w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).cuda()
            cache[(N, K)] = quantize_rows(w)
        return cache[(N, K)]

    return get


# inference/cuda_test.py:79-85: shapes, rows, outliers in odd rows and tiny rows
@pytest.mark.parametrize("N,K", [(4096, 4096), (1024, 12288), (1040, 4096), (17408, 4096)])
@pytest.mark.parametrize("M", [1, 4, 12, 16, 17, 48, 256, 300, 1024])
def test_reference_acceptance_cases(weights, N, K, M):
    wq, sw = weights(N, K)
    g = torch.Generator().manual_seed(1000 + M)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    x[1::2, 0] = 1e5
    x[2::4] *= 2 ** -20
    x = x.cuda()
    y = fp8_matmul(x, wq, sw)
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    check(y, x, wq, sw)
    assert torch.equal(y, fp8_matmul(x, wq, sw)), "second call differs"


@pytest.mark.parametrize("name", list(synthetic.SHAPES))
@pytest.mark.parametrize("M", synthetic.DECODE_ROWS + (64,))
def test_decode_workload_shapes(name, M):
    """Both decode entry points: fp8_matmul (activation codes packed in MFMA
    fragment order by the quantizer) and the GEMM on row-major codes. Without
    split-K both sum every output in the same order, so they agree bitwise."""
    x, w = synthetic.decode_case(name, M)
    wq, sw = quantize_rows(w.cuda())
    x = x.cuda()
    y = fp8_matmul(x, wq, sw)
    check(y, x, wq, sw)
    xq, sx = quantize_rows(x)
    yq = fp8_matmul_quantized(xq, sx, wq, sw)
    check(yq, x, wq, sw)
    N, K = wq.shape
    if _lib.lib().jv_fp8_split_for(M, N, K, torch.cuda.get_device_properties(0).multi_processor_count) == 1:
        assert torch.equal(y, yq)


# The 9B model's merged projections on K = 4096 (inference/engine.py:154-165):
# an attention layer's q+gate, k and v (N = 10240), a DeltaNet layer's qkv
# (8192), the drafter's q/k/v (drafter/view.py:41-53, 12288); tiled as
# FP8Linear.concatenated keeps them, across the decode and prefill plans.
# Sampled token rows against the oracle, and every output equal to the same
# GEMM on row-major codes.
@pytest.mark.parametrize("N", [8192, 10240, 12288])
@pytest.mark.parametrize("M", [1, 16, 64, 128, 2048])
def test_9b_merged_projection_widths(weights, N, M):
    K = 4096
    wq, sw = weights(N, K)
    x = synthetic.activations_outliers(M, K, 9000 + M).cuda()
    y = fp8_matmul(x, tile_weight(wq), sw, tiled=True)
    rows = torch.arange(0, M, max(1, M // 16), device="cuda")
    check(y[rows], x[rows], wq, sw)
    assert torch.equal(y, fp8_matmul(x, wq, sw))


@pytest.mark.parametrize("N", [24576, 24592])
@pytest.mark.parametrize("M", [17, 24, 40, 64])
def test_wide_small_batches_take_64x64_prefill_tiles(N, M):
    """17-64 tokens on weights wide enough for 1.5 rounds of 64-channel
    tiles (gate+up, the lm_head) run on the prefill kernel's 64x64 tiles:
    oracle criteria, packed and row-major codes bitwise equal, row-major and
    tiled weights bitwise equal, bias and LoRA in the same epilogue."""
    K = 4096
    x = synthetic.activations_heavy_tail(M, K, 140 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 141).cuda())
    y = fp8_matmul(x, wq, sw)
    check(y, x, wq, sw)
    assert torch.equal(y, fp8_matmul(x, tile_weight(wq), sw, tiled=True))
    xq, sx = quantize_rows(x)
    assert torch.equal(y, fp8_matmul_quantized(xq, sx, wq, sw))
    a, b = synthetic.lora_factors(N, K, 142)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(143)) * 0.1).to(torch.bfloat16).cuda()
    lora = (a.cuda(), b.cuda(), synthetic.LORA_SCALING)
    check(fp8_matmul(x, wq, sw, bias=bias, lora=lora), x, wq, sw, bias=bias, lora=lora)


@pytest.mark.parametrize("M", [17, 48])
def test_reference_acceptance_inputs_on_64x64_prefill_tiles(weights, M):
    """The acceptance inputs of inference/cuda_test.py:79-85 (outliers in odd
    rows, tiny rows) at batch sizes that take the 64x64 prefill tiles on a
    wide weight; oracle criteria on 4096 sampled output channels, repeat
    calls bitwise equal."""
    N, K = 24576, 4096
    wq, sw = weights(N, K)
    g = torch.Generator().manual_seed(2000 + M)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    x[1::2, 0] = 1e5
    x[2::4] *= 2 ** -20
    x = x.cuda()
    y = fp8_matmul(x, wq, sw)
    cols = torch.randperm(N, generator=g)[:4096].sort().values.cuda()
    check(y[:, cols], x, wq[cols], sw[cols])
    assert torch.equal(y, fp8_matmul(x, wq, sw)), "second call differs"


@pytest.mark.parametrize("N,K", [(256, 4096), (128, 12288), (144, 1024), (144, 2048)])
@pytest.mark.parametrize("M", [1, 16, 33, 64])
def test_split_k_decode_path(N, K, M):
    """Narrow weights (N < 512) split K across workgroups; the last workgroup of
    each tile sums the partials in split order and leaves the counters zero.
    Both entry points (fp8_matmul on bf16 activations, and the GEMM on
    activations already quantized) take the split path."""
    from jeeves_amd import TILE_COUNTERS
    from jeeves_amd.device import sm_count

    assert _lib.lib().jv_fp8_split_for(M, N, K, sm_count(torch.device("cuda"))) > 1
    x = synthetic.activations_heavy_tail(M, K, 70 + M)
    w = synthetic.weight(N, K, 71)
    wq, sw = quantize_rows(w.cuda())
    x = x.cuda()
    xq, sx = quantize_rows(x)
    y = fp8_matmul_quantized(xq, sx, wq, sw)
    check(y, x, wq, sw)
    assert torch.equal(y, fp8_matmul_quantized(xq, sx, wq, sw)), "split-K result is not deterministic"
    y2 = fp8_matmul(x, wq, sw)
    check(y2, x, wq, sw)
    assert torch.equal(y2, fp8_matmul(x, wq, sw))
    torch.cuda.synchronize()
    assert all(int(c.abs().sum()) == 0 for c in TILE_COUNTERS.values())


@pytest.mark.parametrize("N,K,M", [(4096, 8192, 96), (4096, 12288, 128), (1024, 8192, 65), (1024, 4096, 512),
                                   (128, 4096, 2048), (1040, 4096, 200), (4096, 12288, 256), (4096, 12288, 512),
                                   (4112, 12288, 300), (2064, 12288, 333)])
def test_split_k_prefill_path(N, K, M):
    """Batches past the decode kernel whose lockstep tiles cannot fill the
    CUs (64x64 tiles; 128x128 tiles on long k ranges, 2-5 splits, ragged M
    and N) split K across workgroups (the reference splits K below 256 rows,
    inference/fp8.py:118-123); the last workgroup of each tile adds the
    partials in split order: within the GEMM criteria, deterministic, counters
    left zero, on row-major and tiled weights, with bias and LoRA."""
    from jeeves_amd import TILE_COUNTERS
    from jeeves_amd.device import sm_count

    assert _lib.lib().jv_fp8_split_for(M, N, K, sm_count(torch.device("cuda"))) > 1
    x = synthetic.activations_heavy_tail(M, K, 170 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 171).cuda())
    xq, sx = quantize_rows(x)
    y = fp8_matmul_quantized(xq, sx, wq, sw)
    check(y, x, wq, sw)
    assert torch.equal(y, fp8_matmul_quantized(xq, sx, wq, sw)), "split-K result is not deterministic"
    assert torch.equal(fp8_matmul(x, wq, sw), y)
    assert torch.equal(fp8_matmul(x, tile_weight(wq), sw, tiled=True), y)
    a, b = synthetic.lora_factors(N, K, 172)
    lora = (a.cuda(), b.cuda(), synthetic.LORA_SCALING)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(173)) * 0.1).to(torch.bfloat16).cuda()
    got = fp8_matmul(x, wq, sw, bias=bias, lora=lora)
    check(got, x, wq, sw, bias=bias, lora=lora)
    assert torch.equal(got, (fp8_matmul(x, wq, sw, lora=lora).float() + bias.float()).to(torch.bfloat16))
    torch.cuda.synchronize()
    assert all(int(c.abs().sum()) == 0 for c in TILE_COUNTERS.values())


@pytest.mark.parametrize("N,K", [(144, 1024), (160, 384), (48, 128), (4112, 256)])
@pytest.mark.parametrize("M", [1, 5, 16, 40])
def test_decode_short_k(N, K, M):
    """K below 4 steps of 128 per wave (some waves of the decode workgroup get
    no k step), odd tile counts, both decode entry points."""
    x = synthetic.activations_heavy_tail(M, K, 90 + M)
    wq, sw = quantize_rows(synthetic.weight(N, K, 91).cuda())
    x = x.cuda()
    check(fp8_matmul(x, wq, sw), x, wq, sw)
    xq, sx = quantize_rows(x)
    check(fp8_matmul_quantized(xq, sx, wq, sw), x, wq, sw)


@pytest.mark.parametrize("M,N,K", [(7, 16, 6656), (7, 4096, 6656), (16, 96, 6656), (7, 16, 4224), (7, 16, 4608),
                                   (7, 4096, 6528), (7, 4096, 5632), (7, 4096, 3968), (7, 4096, 1152), (33, 4096, 6656),
                                   (31, 16, 2688), (3, 1040, 2432)])
def test_decode_k_ranges_with_short_tails(M, N, K):
    """k ranges whose length leaves 1-3 steps after the full bursts of a wave
    (K = 6656 over 8 waves: 6 or 7 steps, bursts of 4), with and without
    split-K, both decode entry points. The last, partial burst guards its
    steps with scalar branches; when the k bounds sat in vector registers the
    guards were EXEC-masked and a guarded-off step's MFMA still added its
    unloaded operand registers (a seeded shape sweep found M=7, N=16,
    K=6656)."""
    x = synthetic.activations_heavy_tail(M, K, 95 + M)
    wq, sw = quantize_rows(synthetic.weight(N, K, 96).cuda())
    x = x.cuda()
    check(fp8_matmul(x, wq, sw), x, wq, sw)
    xq, sx = quantize_rows(x)
    check(fp8_matmul_quantized(xq, sx, wq, sw), x, wq, sw)


@pytest.mark.parametrize("name", list(synthetic.SHAPES))
@pytest.mark.parametrize("M", [512, 2048])
def test_prefill_workload_shapes(name, M):
    x, w = synthetic.prefill_case(name, M)
    wq, sw = quantize_rows(w.cuda())
    x = x.cuda()
    check(fp8_matmul(x, wq, sw), x, wq, sw)


@pytest.mark.parametrize("name", ["q", "k", "gate_up", "down"])
def test_prefill_8192_rows_by_sampled_rows_and_slices(name):
    """M = 8192 is too large for a float64 oracle of every row: check 96
    sampled rows against the oracle, and that row slices computed alone are
    bitwise equal (the prefill kernel's per-element k order does not depend
    on the tile it lands in)."""
    x, w = synthetic.prefill_case(name, 8192)
    wq, sw = quantize_rows(w.cuda())
    x = x.cuda()
    y = fp8_matmul(x, wq, sw)
    rows = torch.randperm(8192, generator=torch.Generator().manual_seed(5))[:96].sort().values
    check(y[rows.cuda()], x[rows.cuda()], wq, sw)
    for a, b in ((0, 512), (4096, 4096 + 300), (8192 - 65, 8192)):
        assert torch.equal(y[a:b], fp8_matmul(x[a:b].contiguous(), wq, sw)), (a, b)


def test_bias_and_lora_epilogue():
    for M in (16, 48, 512):
        N, K = 1024, 4096
        x, w = synthetic.prefill_case("k", M)
        wq, sw = quantize_rows(w.cuda())
        a, b = synthetic.lora_factors(N, K, 400)
        bias = (torch.randn(N, generator=torch.Generator().manual_seed(2)) * 0.1).to(torch.bfloat16).cuda()
        x, a, b = x.cuda(), a.cuda(), b.cuda()
        y = fp8_matmul(x, wq, sw, bias=bias, lora=(a, b, synthetic.LORA_SCALING))
        check(y, x, wq, sw, bias=bias, lora=(a, b, synthetic.LORA_SCALING))


@pytest.mark.parametrize("M,N", [(2048, 24576), (1000, 5120)])
def test_lora_prefill_on_every_tile_form(M, N):
    """Bias + LoRA on the ping-pong 256x256 tiles (the LoRA term of each 32x32
    block by fp32 MFMAs in the epilogue) against the oracle on sampled rows,
    and row slices that land on the lockstep tile forms give the same bits."""
    K = 4096
    x = synthetic.activations_heavy_tail(M, K, 160 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 161).cuda())
    a, b = synthetic.lora_factors(N, K, 162)
    a, b = a.cuda(), b.cuda()
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(3)) * 0.1).to(torch.bfloat16).cuda()
    lora = (a, b, synthetic.LORA_SCALING)
    y = fp8_matmul(x, wq, sw, bias=bias, lora=lora)
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(4))[:32].sort().values.cuda()
    check(y[rows], x[rows], wq, sw, bias=bias, lora=lora)
    for lo, hi in ((0, 300), (M - 129, M)):
        assert torch.equal(y[lo:hi], fp8_matmul(x[lo:hi].contiguous(), wq, sw, bias=bias, lora=lora)), (lo, hi)


def test_every_code_decodes_through_both_kernels():
    # check_kernel_on_every_code (inference/fp8_metal.py:38-46): identity
    # activations pick every finite code of a permuted weight table.
    codes = torch.arange(256, dtype=torch.uint8)
    finite = codes[~codes.view(FP8).float().isnan()]
    table = finite[(torch.arange(256)[:, None] + torch.arange(256)[None]) % len(finite)].cuda()
    eye = torch.zeros(256, 256, dtype=torch.uint8)
    eye[torch.arange(256), torch.arange(256)] = 0x38
    eye = eye.cuda()
    ones = torch.ones(256, device="cuda")
    want = table.view(FP8).float().t().cpu()
    for rows in (slice(0, 256), slice(0, 64), slice(64, 80), slice(200, 201)):
        picked = fp8_matmul_quantized(eye[rows], ones[rows], table.view(FP8), ones)
        assert torch.equal(picked.float().cpu(), want[rows]), rows


def test_nan_poisoned_output_is_fully_written():
    for M, N, K in ((16, 1024, 4096), (300, 1040, 4096), (33, 4096, 12288)):
        x, w = synthetic.activations_heavy_tail(M, K, 3), synthetic.weight(N, K, 9)
        wq, sw = quantize_rows(w.cuda())
        x = x.cuda()
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        L = _lib.lib()
        ws_bytes = L.jv_fp8_linear_workspace_bytes(M, N, K, 0)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
        counters = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
        _lib.check(L.jv_fp8_linear(x.data_ptr(), K, wq.data_ptr(), K, sw.data_ptr(), None, None, None, 0, 0.0, y.data_ptr(),
                                   N, M, N, K, ws.data_ptr(), ws_bytes, _lib.counters_ptr(counters), counters.numel(),
                                   helpers.stream()))
        check(y, x, wq, sw)
        # split-K tile counters are left zero for the next launch
        assert int(counters.abs().sum()) == 0


def test_row_strided_input_and_zero_rows():
    wq, sw = quantize_rows(synthetic.weight(1024, 4096, 4).cuda())
    big = synthetic.activations_heavy_tail(40, 8192, 6).cuda()
    x = big[:, 4096:]
    check(fp8_matmul(x, wq, sw), x, wq, sw)
    y0 = fp8_matmul(torch.zeros(0, 4096, dtype=torch.bfloat16, device="cuda"), wq, sw)
    assert y0.shape == (0, 1024)
    zeros = fp8_matmul(torch.zeros(20, 4096, dtype=torch.bfloat16, device="cuda"), wq, sw)
    assert not zeros.float().abs().sum().item()


def test_operands_on_another_device_or_of_the_wrong_size_are_refused():
    """Weights, scales, biases and LoRA factors left on the host (their
    pointers would fault the GPU) and per-channel vectors of the wrong length
    raise ValueError before any launch; the stream stays usable."""
    from jeeves_amd.fp8 import fp8_matmul_w8a16

    M, N, K = 16, 1024, 4096
    x = synthetic.activations_heavy_tail(M, K, 130).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 131).cuda())
    bias = torch.zeros(N, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="operands must all be on"):
        fp8_matmul(x, wq.cpu(), sw)
    with pytest.raises(ValueError, match="operands must all be on"):
        fp8_matmul(x, wq, sw.cpu())
    with pytest.raises(ValueError, match="operands must all be on"):
        fp8_matmul(x, wq, sw, bias=bias.cpu())
    with pytest.raises(ValueError, match="operands must all be on"):
        fp8_matmul(x, wq, sw, lora=(torch.zeros(16, K), torch.zeros(N, 16), 2.0))
    with pytest.raises(ValueError, match="operands must all be on"):
        fp8_matmul_w8a16(x, wq.cpu(), sw)
    with pytest.raises(ValueError, match="one value per output channel"):
        fp8_matmul(x, wq, sw[: N - 1])
    with pytest.raises(ValueError, match="one value per output channel"):
        fp8_matmul(x, wq, sw, bias=bias[:16])
    with pytest.raises(ValueError, match="weight codes"):
        fp8_matmul(x, wq.to(torch.bfloat16), sw)
    check(fp8_matmul(x, wq, sw), x, wq, sw)


def test_graph_capture_and_replay():
    """Both kernels under HIP graph capture: replays after new inputs match eager
    calls (the split-K counters are created outside the capture), including
    the split-K paths of the decode kernel (N = 256) and of the 64x64 prefill
    tiles (M = 96), whose counters every replay must leave at zero."""
    for M, (N, K) in ((16, (1024, 4096)), (256, (4096, 4096)), (16, (256, 4096)), (96, (4096, 4096))):
        wq, sw = quantize_rows(synthetic.weight(N, K, 8).cuda())
        static_x = torch.zeros(M, K, dtype=torch.bfloat16, device="cuda")
        fp8_matmul(static_x, wq, sw)  # warm: tile counters exist
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fp8_matmul(static_x, wq, sw)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=s):
                static_y = fp8_matmul(static_x, wq, sw)
        torch.cuda.current_stream().wait_stream(s)
        for seed in range(4):
            x = synthetic.activations_heavy_tail(M, K, 50 + seed).cuda()
            static_x.copy_(x)
            graph.replay()
            torch.cuda.synchronize()
            eager = fp8_matmul(x, wq, sw)
            torch.cuda.synchronize()
            assert torch.equal(static_y, eager), (M, seed)


@pytest.mark.parametrize("M", [1, 5, 16, 33, 64])
@pytest.mark.parametrize("N,K", [(1024, 4096), (4096, 12288), (256, 384)])
def test_packed_activation_codes(M, N, K):
    """Codes written in the decode GEMM's packed fragment order (ldc = 0) and
    consumed with ldxq = 0 give the same output, bit for bit, as row-major
    codes; the scales are the row-major quantizer's."""
    from jeeves_amd.fp8 import packed_codes_bytes

    x = synthetic.activations_heavy_tail(M, K, 120 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 121).cuda())
    xq, sx = quantize_rows(x)
    packed = torch.full((packed_codes_bytes(M, K),), 0xAA, dtype=torch.uint8, device="cuda")
    psx = torch.full((M,), float("nan"), device="cuda")
    L = _lib.lib()
    _lib.check(L.jv_fp8_quantize_rows_bf16(x.data_ptr(), K, M, K, packed.data_ptr(), 0, psx.data_ptr(), helpers.stream()))
    assert helpers.same_f32(psx.cpu().numpy(), sx.cpu().numpy()).all()
    y_row = fp8_matmul_quantized(xq, sx, wq, sw)
    y_packed = fp8_matmul_quantized(packed, psx, wq, sw, packed_rows=M)
    assert torch.equal(y_row, y_packed)
    check(y_packed, x, wq, sw)
    # padding rows of the last 16-token tile hold zero codes
    assert int(packed.long().sum().item()) == int(xq.view(torch.uint8).long().sum().item())


# Prefill batches over every prefill kernel form: 256x256 tiles (ping-pong
# form; M = 1993 leaves a partial last 16-token tile), 256x128 and 128x128.
@pytest.mark.parametrize("M,N,K", [(2048, 24576, 4096), (1993, 24576, 4096), (2048, 4096, 12288), (300, 1024, 4096),
                                   (65, 4096, 4096)])
def test_packed_activation_codes_prefill(M, N, K):
    """Packed codes (ldc = 0, ldxq = 0) through the prefill kernels give the
    row-major codes' output bit for bit; sampled rows meet the oracle."""
    from jeeves_amd.fp8 import packed_codes_bytes

    x = synthetic.activations_heavy_tail(M, K, 140 + M).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 141).cuda())
    xq, sx = quantize_rows(x)
    packed = torch.full((packed_codes_bytes(M, K),), 0xAA, dtype=torch.uint8, device="cuda")
    psx = torch.empty(M, device="cuda")
    _lib.check(_lib.lib().jv_fp8_quantize_rows_bf16(x.data_ptr(), K, M, K, packed.data_ptr(), 0, psx.data_ptr(),
                                                    helpers.stream()))
    assert torch.equal(psx, sx)
    # the packed order is the tiled weight order applied to token rows, with
    # zero codes in the padding rows of the last 16-token tile
    padded = torch.zeros((M + 15) // 16 * 16, K, dtype=torch.uint8, device="cuda")
    padded[:M] = xq.view(torch.uint8)
    assert torch.equal(tile_weight(padded).view(torch.uint8).reshape(-1), packed)
    for tiled in (False, True):
        w = tile_weight(wq) if tiled else wq
        y_row = fp8_matmul_quantized(xq, sx, w, sw, tiled=tiled)
        y_packed = fp8_matmul_quantized(packed, psx, w, sw, packed_rows=M, tiled=tiled)
        assert torch.equal(y_row, y_packed), tiled
    assert torch.equal(fp8_matmul(x, wq, sw), y_packed)
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(M))[:48].sort().values.cuda()
    check(y_packed[rows], x[rows], wq, sw)


# Short K on every prefill form: the ping-pong 256x256 tile (M = 2048, N = 5120
# gives 160 tiles), 256x128, 128x128 and 64x64, including K = 128 (two 64-deep
# steps: the pipelines' shortest case) and a partial last token tile.
@pytest.mark.parametrize("K", [128, 256, 384])
@pytest.mark.parametrize("M,N", [(2048, 5120), (2000, 4096), (1024, 2048), (300, 1040)])
def test_prefill_short_k(M, N, K):
    x = synthetic.activations_heavy_tail(M, K, 150 + K).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, K, 151).cuda())
    y = fp8_matmul(x, wq, sw)
    if N % 16 == 0:
        assert torch.equal(y, fp8_matmul(x, tile_weight(wq), sw, tiled=True))
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(K))[:64].sort().values.cuda()
    check(y[rows], x[rows], wq, sw)


@pytest.mark.parametrize("M", [1, 16, 40, 300, 2048])
def test_swiglu_packed_codes_feed_down_projection(M):
    I, N = 4096, 1024
    g = torch.Generator().manual_seed(130 + M)
    gate = (torch.randn(M, I, generator=g) * 2).to(torch.bfloat16).cuda()
    up = torch.randn(M, I, generator=g).to(torch.bfloat16).cuda()
    wq, sw = quantize_rows(synthetic.weight(N, I, 131).cuda())
    codes, scales, h = swiglu_quantize(gate, up, return_h=True)
    pcodes, pscales, ph = swiglu_quantize(gate, up, return_h=True, packed=True)
    assert torch.equal(scales, pscales) and torch.equal(h, ph)
    y_row = fp8_matmul_quantized(codes, scales, wq, sw)
    y_packed = fp8_matmul_quantized(pcodes, pscales, wq, sw, packed_rows=M)
    assert torch.equal(y_row, y_packed)
    check(y_packed, h, wq, sw, equal_min=helpers.EQUAL_MIN_SWIGLU_H)
