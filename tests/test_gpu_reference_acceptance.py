"""The reference's own FP8 acceptance checks, ``inference/cuda_test.py:17-49``
(``quantized``, ``merges``) and ``:74-94`` (``fp8_matmuls``), restated against
``jeeves_amd.fp8.FP8Linear`` the way the reference runs them: the expected
result is computed on the device from ``linear.weight`` and ``linear.scale``
as the module holds them (row-major e4m3 codes and float32 scales).

``fp8_matmuls`` runs twice:

* in the W8A16 parity mode (``set_activations("bf16")``), the reference's own
  arithmetic, with the reference's bar unchanged: at least 99.5% of outputs
  bitwise equal to the float64 product rounded once to bf16, all finite, and
  a second call bitwise identical;
* in the FP8 x FP8 mode, where the activations are quantized per token first:
  the float64 product of the same quantized activations and ``linear.weight``
  is the exact result, and the bar is the FP8 path's (``tests/helpers.py``:
  at least 99% bitwise equal over the nine row counts of each weight and 98%
  per call, each less three binomial standard deviations -- gfx950's FP8 MFMA
  aligns each group of products to a ~13-bit window -- and rel-L2 <= 1e-3),
  finite, deterministic.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn as nn

from jeeves_amd.fp8 import FP8Linear
from jeeves_amd.fp8_weights import quantize_rows
from tests import helpers

pytestmark = pytest.mark.gpu

CUDA = torch.device("cuda")
WEIGHTS = ((4096, 4096), (1024, 12288), (1040, 4096), (17408, 4096))  # inference/cuda_test.py:79
ROWS = (1, 4, 12, 16, 17, 48, 256, 300, 1024)  # inference/cuda_test.py:81


def quantized(linear: nn.Linear) -> FP8Linear:
    """inference/cuda_test.py:17-20."""
    fp8 = FP8Linear(linear.in_features, linear.out_features, device=linear.weight.device)
    fp8.load_weight(linear.weight)
    return fp8


def merge(linears: tuple[nn.Module, ...]) -> nn.Module | None:
    """The FP8 branch of the engine's merge_linears_in_place
    (inference/engine.py:56-68), which hands FP8 parts to FP8Linear.concatenated."""
    if any(linear.bias is not None for linear in linears):
        return None
    if all(type(linear) is FP8Linear for linear in linears):
        return FP8Linear.concatenated(list(linears))
    return None


@torch.no_grad()
def test_merges():
    """inference/cuda_test.py:38-48: merging FP8 projections keeps every part's
    codes and scales bitwise, the parts become views of the merged buffers,
    the merged output equals the separate GEMMs up to bf16 rounding, and FP8
    parts do not merge with bf16 ones."""
    torch.manual_seed(0)
    x = torch.randn(3, 16, 4096, device=CUDA, dtype=torch.bfloat16)
    fp8_parts = [quantized(nn.Linear(4096, n, bias=False, device=CUDA, dtype=torch.bfloat16)) for n in (4096, 1024, 1024)]
    codes, scales = [p.weight.clone() for p in fp8_parts], [p.scale.clone() for p in fp8_parts]
    separate = [p(x) for p in fp8_parts]
    fp8_merged = merge(tuple(fp8_parts))
    for i, (p, c, s) in enumerate(zip(fp8_parts, codes, scales)):
        assert torch.equal(p.weight.view(torch.uint8), c.view(torch.uint8)) and torch.equal(p.scale, s), i
        assert p.weight.untyped_storage().data_ptr() == fp8_merged.weight.untyped_storage().data_ptr(), i
    for i, (a, p, b) in enumerate(zip(fp8_merged(x).split([p.out_features for p in fp8_parts], dim=-1), fp8_parts, separate)):
        assert torch.allclose(a.float(), p(x).float(), rtol=2 ** -7, atol=1e-2), i
        assert torch.equal(p(x), b), i  # and the parts' own outputs are unchanged by the merge
    assert merge((fp8_parts[0], nn.Linear(4096, 32, bias=False, device=CUDA, dtype=torch.bfloat16))) is None


def _inputs(M: int, K: int) -> torch.Tensor:
    x = torch.randn(M, K, device=CUDA, dtype=torch.bfloat16)
    # outliers in odd rows only, tiny rows (inference/cuda_test.py:83-85)
    x[1::2, 0] = 1e5
    x[2::4] *= 2 ** -20
    return x


@torch.no_grad()
@pytest.mark.parametrize("N,K", WEIGHTS)
def test_fp8_matmuls_w8a16_parity_mode(N, K):
    """inference/cuda_test.py:74-94 verbatim in its arithmetic: the module in
    the reference's W8A16 mode against the float64 product of x and
    linear.weight, rounded once to bf16."""
    torch.manual_seed(1 + N + K)
    linear = quantized(nn.Linear(K, N, bias=False, device=CUDA, dtype=torch.bfloat16))
    linear.set_activations("bf16")
    for M in ROWS:
        x = _inputs(M, K)
        exact = ((x.double() @ linear.weight.double().t()) * linear.scale.double()).to(torch.bfloat16)
        out = linear(x)
        same = (out == exact).double().mean().item()
        assert out.isfinite().all() and same >= 0.995, (N, K, M, same)
        assert torch.equal(out, linear(x)), (N, K, M, "second call differs")


@torch.no_grad()
@pytest.mark.parametrize("N,K", WEIGHTS)
def test_fp8_matmuls_fp8_mode(N, K):
    """The same inputs through the FP8 x FP8 path: the exact result is the
    float64 product of the per-token quantized activations and linear.weight
    (codes as the module holds them), times both scales, rounded to bf16."""
    torch.manual_seed(2 + N + K)
    linear = quantized(nn.Linear(K, N, bias=False, device=CUDA, dtype=torch.bfloat16))
    equal_total = outputs = 0
    for M in ROWS:
        x = _inputs(M, K)
        xq, sx = quantize_rows(x)
        exact = ((xq.double() @ linear.weight.double().t()) * sx.double()[:, None] * linear.scale.double()).to(torch.bfloat16)
        out = linear(x)
        equal = (out == exact).sum().item()
        same = equal / out.numel()
        rel = ((out.double() - exact.double()).norm() / exact.double().norm()).item()
        assert out.isfinite().all() and rel <= helpers.REL_L2_MAX, (N, K, M, same, rel)
        assert same >= helpers.equal_floor(out.numel(), helpers.EQUAL_MIN), (N, K, M, same)
        assert torch.equal(out, linear(x)), (N, K, M, "second call differs")
        equal_total += equal
        outputs += out.numel()
    pooled = equal_total / outputs
    print(f"{N}x{K}: {pooled:.5f} of {outputs} outputs bitwise equal to the exact product", flush=True)
    assert pooled >= helpers.equal_floor(outputs, helpers.EQUAL_MIN_REFERENCE), (N, K, pooled)
