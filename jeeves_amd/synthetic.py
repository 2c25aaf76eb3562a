"""Seeded synthetic inputs for the FP8 linear workloads (no datasets or
checkpoints are available offline, so weights are random-init with the
distributions below). Generated on the CPU with ``torch.Generator`` so the
parity tests and the benchmark see identical values; callers move them to the
device.

Workloads (9B-class projection shapes, K -> N):
  * single linear: x bf16 [16,4096] ~ N(0,1) with 8 random outlier channels
    scaled x20, W bf16 [4096,4096] ~ N(0,0.02), per-channel e4m3 weights,
    per-token e4m3 activations, bf16 out (seeds: W 0, x 1);
  * decode: M in {1,4,16,32} over q/o 4096->4096, k/v 4096->1024, fused
    gate+up 4096->24576, down 12288->4096, same distributions (seeds: W
    100 + shape index, x 200 + M);
  * prefill: M in {512,2048,8192} over the same shapes, x ~ N(0,1) except 1%
    of the channels drawn Student-t (df 3) as Z / sqrt((Z1^2+Z2^2+Z3^2)/3)
    (seed 300 + M);
  * decoder layer at M=512: q, k, v, o, gate_up -> SwiGLU -> down, each with a
    rank-16 bf16 LoRA adapter, A, B ~ N(0, 0.01), scaling alpha/r = 32/16 = 2
    (model/lora.py:16-17, :33-34) (seed 400);
  * ragged mix: 64 sequence lengths round(exp(U(ln 64, ln 2048))) packed into
    one token batch, then 64 decode steps at batch 64 (seed 500).
"""

from __future__ import annotations

import math

import torch

HIDDEN, INTERMEDIATE = 4096, 12288
# (N, K) per projection, in layer order.
SHAPES: dict[str, tuple[int, int]] = {
    "q": (4096, HIDDEN),
    "k": (1024, HIDDEN),
    "v": (1024, HIDDEN),
    "o": (4096, HIDDEN),
    "gate_up": (2 * INTERMEDIATE, HIDDEN),
    "down": (HIDDEN, INTERMEDIATE),
}
SHAPE_INDEX = {name: i for i, name in enumerate(SHAPES)}
# lm_head (inference/engine.py:293-297): the 9B vocabulary x hidden, 1.02 GB of e4m3 codes.
VOCAB = 248320
DECODE_ROWS = (1, 4, 16, 32)
PREFILL_ROWS = (512, 2048, 8192)
LORA_RANK, LORA_ALPHA = 16, 32.0
LORA_SCALING = LORA_ALPHA / LORA_RANK
OUTLIER_CHANNELS, OUTLIER_SCALE = 8, 20.0
WEIGHT_STD, LORA_STD = 0.02, 0.01


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def weight(N: int, K: int, seed: int) -> torch.Tensor:
    """bf16 [N,K] ~ N(0, 0.02)."""
    return (torch.randn(N, K, generator=gen(seed)) * WEIGHT_STD).to(torch.bfloat16)


def activations_outliers(M: int, K: int, seed: int) -> torch.Tensor:
    """bf16 [M,K] ~ N(0,1) with 8 channels (randperm(K)[:8]) scaled x20."""
    g = gen(seed)
    x = torch.randn(M, K, generator=g)
    ch = torch.randperm(K, generator=g)[:OUTLIER_CHANNELS]
    x[:, ch] *= OUTLIER_SCALE
    return x.to(torch.bfloat16)


def activations_heavy_tail(M: int, K: int, seed: int) -> torch.Tensor:
    """bf16 [M,K] ~ N(0,1) with 1% of channels Student-t(3)."""
    g = gen(seed)
    x = torch.randn(M, K, generator=g)
    n = max(1, round(K * 0.01))
    ch = torch.randperm(K, generator=g)[:n]
    z = torch.randn(M, n, generator=g)
    chi = torch.randn(3, M, n, generator=g).pow(2).sum(0) / 3.0
    x[:, ch] = z / chi.sqrt()
    return x.to(torch.bfloat16)


def lora_factors(N: int, K: int, seed: int, rank: int = LORA_RANK) -> tuple[torch.Tensor, torch.Tensor]:
    """(A bf16 [r,K], B bf16 [N,r]), both ~ N(0, 0.01)."""
    g = gen(seed)
    a = (torch.randn(rank, K, generator=g) * LORA_STD).to(torch.bfloat16)
    b = (torch.randn(N, rank, generator=g) * LORA_STD).to(torch.bfloat16)
    return a, b


def single_linear() -> tuple[torch.Tensor, torch.Tensor]:
    """(x [16,4096], W [4096,4096]) of the single-linear workload."""
    return activations_outliers(16, HIDDEN, 1), weight(4096, HIDDEN, 0)


def decode_case(name: str, M: int) -> tuple[torch.Tensor, torch.Tensor]:
    N, K = SHAPES[name]
    return activations_outliers(M, K, 200 + M), weight(N, K, 100 + SHAPE_INDEX[name])


def prefill_case(name: str, M: int) -> tuple[torch.Tensor, torch.Tensor]:
    N, K = SHAPES[name]
    return activations_heavy_tail(M, K, 300 + M), weight(N, K, 100 + SHAPE_INDEX[name])


def ragged_lengths(seed: int = 500, count: int = 64, lo: int = 64, hi: int = 2048) -> list[int]:
    g = gen(seed)
    u = torch.rand(count, generator=g, dtype=torch.float64)
    return [int(round(math.exp(math.log(lo) + float(v) * (math.log(hi) - math.log(lo))))) for v in u]
