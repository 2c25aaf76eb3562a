"""jv_fp8_linear_noalloc, the entry point that allocates nothing (its scratch
is a library-owned device array per GPU), against jv_fp8_linear with a
caller-provided workspace and tile counters: bitwise-equal outputs on two
calls in a row, the second with a smaller input, on the decode kernel with
split-K (tile counters and partials in the scratch), the decode kernel
without, the prefill kernels with and without split-K, tiled and row-major
weights, bias and LoRA; and
sizes beyond the scratch are refused with a ValueError-class status before
any launch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from jeeves_amd import _lib, synthetic
from jeeves_amd.fp8 import tile_weight
from jeeves_amd.fp8_weights import quantize_rows

pytestmark = pytest.mark.gpu


def _ptr(t):
    return t.data_ptr() if t is not None else None


def with_workspace(x, w, ldw, sw, bias, lora, N):
    M, K = x.shape
    L = _lib.lib()
    rank = 0 if lora is None else lora[0].shape[0]
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=x.device)
    ws_bytes = L.jv_fp8_linear_workspace_bytes(M, N, K, rank)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    counters = torch.zeros(65536, dtype=torch.int32, device=x.device)
    _lib.check(L.jv_fp8_linear(x.data_ptr(), x.stride(0), w.data_ptr(), ldw, sw.data_ptr(), _ptr(bias),
                               _ptr(lora[0]) if lora else None, _ptr(lora[1]) if lora else None, rank,
                               lora[2] if lora else 0.0, y.data_ptr(), N, M, N, K, ws.data_ptr(), ws_bytes,
                               _lib.counters_ptr(counters), counters.numel(), torch.cuda.current_stream().cuda_stream))
    return y


def without_workspace(x, w, ldw, sw, bias, lora, N):
    M, K = x.shape
    rank = 0 if lora is None else lora[0].shape[0]
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=x.device)
    _lib.check(_lib.lib().jv_fp8_linear_noalloc(x.data_ptr(), x.stride(0), w.data_ptr(), ldw, sw.data_ptr(), _ptr(bias),
                                                _ptr(lora[0]) if lora else None, _ptr(lora[1]) if lora else None, rank,
                                                lora[2] if lora else 0.0, y.data_ptr(), N, M, N, K,
                                                torch.cuda.current_stream().cuda_stream))
    return y


def test_first_noalloc_call_captured_in_a_graph():
    """The first call of the no-allocation entry point in this process (this
    test comes first in the file, and nothing else calls it) made inside a
    captured graph: the graph holds only the call's own launches (the scratch's
    tile counters are zero from the code object's load, with no clear on the
    stream), and every replay -- with eager work and a new input between
    replays -- equals the workspace entry point on the split-K decode path,
    whose tile counters live in the scratch."""
    N, K, M = 256, 4096, 16
    wq, sw = quantize_rows(synthetic.weight(N, K, 7000).cuda())
    w = wq.view(torch.uint8)
    x = synthetic.activations_outliers(M, K, 7001).cuda()
    assert _lib.lib().jv_fp8_split_for(M, N, K, torch.cuda.get_device_properties(0).multi_processor_count) > 1
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = without_workspace(x, w, K, sw, None, None, N)
    for rep in range(4):
        x.copy_(synthetic.activations_outliers(M, K, 7002 + rep).cuda())
        want = with_workspace(x, w, K, sw, None, None, N)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), rep


# (N, K, first M, second M, tiled, bias, lora): split-K decode, batch-decode
# then plain decode, 64x64 prefill tiles on a wide weight, split-K 64x64
# prefill tiles (4 splits), split-K 128x128 prefill tiles (2 and 4 splits,
# 16 MiB of partials), lockstep and ping-pong prefill tiles, batch-decode on
# row-major weights with LoRA.
CASES = [(256, 4096, 16, 5, False, False, False), (4096, 4096, 64, 1, True, True, False),
         (24576, 4096, 48, 17, True, False, False), (1024, 4096, 300, 65, True, True, True),
         (4096, 12288, 96, 128, False, False, False), (4096, 12288, 512, 256, True, False, True),
         (24576, 4096, 2048, 256, True, False, True), (4096, 12288, 33, 16, False, True, False),
         (1024, 4096, 100, 40, False, True, True)]


@pytest.mark.parametrize("N,K,M1,M2,tiled,use_bias,use_lora", CASES)
def test_noalloc_equals_workspace_entry(N, K, M1, M2, tiled, use_bias, use_lora):
    print(f"noalloc case N={N} K={K} M={M1},{M2} tiled={tiled} bias={use_bias} lora={use_lora}", flush=True)
    wq, sw = quantize_rows(synthetic.weight(N, K, 7100 + N % 97).cuda())
    w = tile_weight(wq).view(torch.uint8) if tiled else wq.view(torch.uint8)
    ldw = 0 if tiled else K
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(7101)) * 0.1).to(torch.bfloat16).cuda() if use_bias else None
    lora = None
    if use_lora:
        a, b = synthetic.lora_factors(N, K, 7102)
        lora = (a.to(torch.bfloat16).cuda().contiguous(), b.to(torch.bfloat16).cuda().contiguous(), synthetic.LORA_SCALING)
    for M in (M1, M2):  # two calls in a row, the second smaller: the scratch keeps the first call's contents
        x = synthetic.activations_outliers(M, K, 7103 + M).cuda()
        want = with_workspace(x, w, ldw, sw, bias, lora, N)
        got = without_workspace(x, w, ldw, sw, bias, lora, N)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (N, K, M)
        assert got.isfinite().all(), (N, K, M)


def test_noalloc_refuses_sizes_beyond_its_scratch():
    L = _lib.lib()
    limit = 32 << 20
    for M, K in ((8192, 4096), (2736, 12288), (16384, 4096)):
        assert L.jv_fp8_linear_workspace_bytes(M, 4096, K, 0) > limit - 16384
        rc = L.jv_fp8_linear_noalloc(16, K, 16, 0, 16, None, None, None, 0, 0.0, 16, 4096, M, 4096, K,
                                     torch.cuda.current_stream().cuda_stream)
        assert rc == _lib.JV_ERR_VALUE and b"needs" in L.jv_fp8_last_error(), (M, K)
    assert L.jv_fp8_linear_workspace_bytes(8176, 4096, 4096, 0) <= limit - 16384
    assert L.jv_fp8_linear_workspace_bytes(2720, 4096, 12288, 0) <= limit - 16384
