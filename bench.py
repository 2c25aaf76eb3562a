#!/usr/bin/env python3
"""Benchmark of the MI355X FP8 linear path on one GPU.

A step is one decoder layer's FP8 linears at M = 16 decode tokens, run the way
the reference engine runs them: q, k and v merged into one projection
(4096 -> 6144, inference/engine.py:154-165, :272-284), o (4096 -> 4096), the
gate+up (4096 -> 24576) as one GEMM with SwiGLU in its epilogue, the down
projection's quantization of h, and down (12288 -> 4096). Each distinct input is
quantized once (four per-token e4m3 quantizer launches), every GEMM applies the
scale epilogue -> bf16. As in the reference engine, which replays its decode
passes as CUDA graphs (inference/engine.py:351-360), each step is a captured
HIP graph replay. Weights are in FP8Linear's tiled layout and rotate over enough
copies (>= 512 MB) that every step reads them from HBM, not the 256 MB
Infinity Cache. Inputs are resident in HBM before timing starts.

value        algorithmic bytes of the layer's linears / step time (GB/s), with
             bytes per linear = N*K (e4m3 W) + 4N (scales) + 2MK (bf16 x) + 2MN (bf16 y)
roofline     the dominant kernel (the gate+up decode GEMM) alone: graphs of
             back-to-back launches on rotated weights, timed with HIP events
             on their stream; algorithmic bytes / average launch time vs
             8 TB/s; `traffic` is copied from the committed rocprofv3 PMC
             summary (profiles/), not measured in this run
decode       the layer step, the six separate projections each with its own
             quantizer (q, k, v, o, gate+up, down), per-kernel GEMM times at
             M = 16 including the merged q/k/v, and per-kernel GEMM times at
             M = 1, 4, 32 (the other decode batch sizes) and 64, 96, 128 (the
             engine's decode row counts, inference/engine.py:299-306)
prefill      the same layer and the six projections at M = 2048 (TFLOP/s,
             2*M*N*K per linear), per-kernel times at M = 512, 2048, 8192, and
             the gate+up prefill GEMM's roofline vs 5.0 PFLOP/s
workloads    the decoder layer's linear stack at M = 512 with a rank-16 LoRA
             on every projection (q, k, v separate: each has its own adapter),
             the ragged request mix (64 log-uniform sequence lengths packed
             into one batch through 32 layers of random weights, then 64
             decode steps at batch 64), and the lm_head (248320 x 4096) at
             M = 1 and 16: time, TFLOP/s or GB/s and roofline fraction
cpu_baseline the CPU oracle's quantize + dequantize-then-matmul (numpy float32,
             BLAS threads) on the same decode layer step for a bounded number
             of steps, and the single linear (16 x 4096 -> 4096) on its own

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "FP8 linear TFLOP/s (M=2048) and HBM GB/s (M<=16) on 1 MI355X; % of roofline"
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 512 << 20
LAUNCHES_PER_GRAPH = 24
# Decode batch sizes besides 16: the other decode rows of the decode workload,
# then the engine's decode row counts above 64 (4B, 12B and 16B tokens rounded
# to a power of two, inference/engine.py:299-306).
DECODE_SWEEP_ROWS = (1, 4, 32, 64, 96, 128)
PREFILL_SWEEP_ROWS = (512, 8192)
W8A16_ROWS = (1, 16, 64, 2048)
PMC_SUMMARY = "profiles/gemm_decode_prefill_pmc.md"


def measured_counter(kind: str, key: str):
    """A per-launch figure measured with rocprofv3 PMC counters (HBM bytes,
    MFMA busy %, counter-window clock), copied from the committed summary
    (None when absent)."""
    path = ROOT / PMC_SUMMARY
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.split()
        if len(parts) == 3 and parts[0] == kind and parts[1] == key:
            return int(parts[2]) if kind == "traffic_bytes_per_launch" else float(parts[2])
    return None


def measured_traffic(key: str):
    return measured_counter("traffic_bytes_per_launch", key)


def linear_bytes(M: int, N: int, K: int) -> int:
    return N * K + 4 * N + 2 * M * K + 2 * M * N


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Bench:
    def __init__(self, torch):
        self.torch = torch
        self.stream = torch.cuda.Stream()

    def capture(self, fn):
        """Capture fn() into a HIP graph on the bench stream (after one eager run
        on that stream, which creates its tile counters outside the capture)."""
        torch = self.torch
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self.stream):
            fn()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=self.stream):
                fn()
        torch.cuda.current_stream().wait_stream(self.stream)
        torch.cuda.synchronize()
        return g

    def time_graphs(self, graphs, replays: int, warmup: int) -> float:
        """ms per replay, HIP events recorded on the stream the graphs replay on."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for i in range(warmup):
                graphs[i % len(graphs)].replay()
            self.stream.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(self.stream)
            for i in range(replays):
                graphs[i % len(graphs)].replay()
            end.record(self.stream)
            end.synchronize()
        return start.elapsed_time(end) / replays


def layer_shapes(synthetic) -> dict[str, tuple[int, int]]:
    """(N, K) of the layer's linears as the engine holds them: q/k/v merged."""
    s = synthetic.SHAPES
    return {"qkv": (s["q"][0] + s["k"][0] + s["v"][0], s["q"][1]), "o": s["o"], "gate_up": s["gate_up"], "down": s["down"]}


# The 9B model's merged projections on K = 4096 (inference/engine.py:154-165):
# an attention layer's q+gate, k and v (10240), a DeltaNet layer's qkv (8192),
# and the drafter's q/k/v (drafter/view.py:41-53, 12288).
MERGED_9B = {"qkv_attention_10240": 10240, "qkv_deltanet_8192": 8192, "qkv_drafter_12288": 12288}


def merged_9b_weights(torch, synthetic, quantize_rows) -> dict:
    from jeeves_amd.fp8 import tile_weight

    w = {}
    for i, (name, N) in enumerate(MERGED_9B.items()):
        wq, sw = quantize_rows(synthetic.weight(N, synthetic.HIDDEN, 900 + i).cuda())
        w[name] = (tile_weight(wq), sw)
    return w


def make_weights(torch, synthetic, quantize_rows) -> dict:
    """Tiled e4m3 codes and scales of the six projections (the decode and
    prefill workloads' weights), plus q/k/v merged the way FP8Linear.concatenated
    merges them (whole 16-row tiles: the merged tiled copy is the parts' copies
    one after another)."""
    from jeeves_amd.fp8 import tile_weight

    w = {}
    for name in synthetic.SHAPES:
        wq, sw = quantize_rows(synthetic.decode_case(name, 1)[1].cuda())
        w[name] = (tile_weight(wq), sw)
    w["qkv"] = (torch.cat([w[n][0] for n in ("q", "k", "v")]), torch.cat([w[n][1] for n in ("q", "k", "v")]))
    return w


class Rotation:
    """Copies of each weight totalling at least ROTATE_BYTES, so back-to-back
    launches read their weights from HBM rather than the Infinity Cache."""

    def __init__(self, weights):
        self.weights, self.cache = weights, {}

    def copies(self, name: str):
        if name not in self.cache:
            wq, sw = self.weights[name]
            n = max(2, -(-ROTATE_BYTES // wq.numel()) + 1)
            self.cache[name] = [(wq, sw)] + [(wq.clone(), sw) for _ in range(n - 1)]
        return self.cache[name]

    def drop(self):
        self.cache.clear()


def quantized_operands(torch, fp8, x):
    """Activation codes as fp8_matmul hands them to its GEMM: the packed
    fragment order (rows of up to 16384 channels, as in every workload here)."""
    from jeeves_amd import _lib

    M, K = x.shape
    sx = torch.empty(M, dtype=torch.float32, device=x.device)
    codes = torch.empty(fp8.packed_codes_bytes(M, K), dtype=torch.uint8, device=x.device)
    _lib.check(_lib.lib().jv_fp8_quantize_rows_bf16(x.data_ptr(), x.stride(0), M, K, codes.data_ptr(), 0, sx.data_ptr(),
                                                    torch.cuda.current_stream().cuda_stream))
    return codes, sx, M


def launches_ms(b: Bench, copies, launch, replays: int, graphs: int = 4) -> float:
    """Average time (ms) of one launch(wq, sw), from graphs of
    LAUNCHES_PER_GRAPH back-to-back launches on the bench stream over rotated
    weight copies."""
    gs = []
    for c in range(min(len(copies), graphs)):
        def launches(c=c):
            for j in range(LAUNCHES_PER_GRAPH):
                launch(*copies[(c * LAUNCHES_PER_GRAPH + j) % len(copies)])
        gs.append(b.capture(launches))
    ms = b.time_graphs(gs, replays, 3) / LAUNCHES_PER_GRAPH
    del gs
    return ms


def kernel_ms(b: Bench, fp8, copies, operands, replays: int, graphs: int = 4, tiled: bool = True) -> float:
    """Average time (ms) of one GEMM kernel launch on the activation codes
    fp8_matmul would produce, from graphs of back-to-back launches on the bench
    stream over rotated weight copies (tiled: FP8Linear's tiled copy; else the
    row-major codes, the layout FP8Linear.TILED_COPY = False reads)."""
    xq, sx, packed_rows = operands
    return launches_ms(b, copies, lambda wq, sw: fp8.fp8_matmul_quantized(xq, sx, wq, sw, packed_rows=packed_rows,
                                                                             tiled=tiled), replays, graphs)


def layer_inputs(synthetic, M: int, K: int, case) -> dict:
    """Distinct bf16 inputs of the layer's linears: the attention input (for
    q/k/v), the attention output (o) and the MLP input (gate+up)."""
    x = case("q", M)[0]
    g = synthetic.gen(900 + M)
    import torch

    return {"attn": x, "o": x[:, torch.randperm(K, generator=g)].contiguous(),
            "mlp": x[:, torch.randperm(K, generator=g)].contiguous()}


def layer_linears(fp8, synthetic, xs, weights, lora=None):
    """One decoder layer's linear stack. With `xs` a dict (attention input,
    attention output, MLP input) and merged q/k/v weights: the engine's merged
    qkv projection, o, gate+up with SwiGLU in its epilogue (h, and at decode
    sizes its per-16-channel maxima), the down projection's quantization of
    h, down. With `xs` one tensor: q, k, v
    (separate, each with its own LoRA adapter when `lora` is given), o and
    gate+up all on it, then the same SwiGLU and down."""
    if isinstance(xs, dict):
        wq, sw = weights["qkv"]
        fp8.fp8_matmul(xs["attn"], wq, sw, tiled=True)
        wq, sw = weights["o"]
        fp8.fp8_matmul(xs["o"], wq, sw, tiled=True)
        h = xs["mlp"]
    else:
        h = xs
        for name in ("q", "k", "v", "o"):
            wq, sw = weights[name]
            fp8.fp8_matmul(h, wq, sw, tiled=True, lora=lora[name] if lora else None)
    wq, sw = weights["gate_up"]
    # Decode batches without LoRA quantize h from the epilogue's maxima (as FP8SwiGLU does).
    amax = not lora and h.shape[0] <= fp8.DECODE_MAX_ROWS
    out = fp8.gate_up_swiglu(h, wq, sw, tiled=True, lora=lora["gate_up"] if lora else None, amax=amax)
    hh, parts = out if amax else (out, None)
    res = fp8.quantize_swiglu_output(hh, parts, lora_a=lora["down"][0] if lora else None, packed=True)
    wq, sw = weights["down"]
    return fp8.fp8_matmul_quantized(res[0], res[1], wq, sw, lora_t=res[2] if lora else None,
                                    lora_b=lora["down"][1] if lora else None,
                                    lora_scaling=lora["down"][2] if lora else 0.0, packed_rows=h.shape[0], tiled=True)


def layer_bytes(synthetic, M: int) -> int:
    return sum(linear_bytes(M, N, K) for N, K in layer_shapes(synthetic).values())


def layer_flops(synthetic, M: int, rank: int = 0) -> int:
    return sum(2 * M * N * K + 2 * M * rank * (K + N) for N, K in synthetic.SHAPES.values())


def layer_step_ms(b: Bench, torch, fp8, synthetic, weights, xs, replays: int, warmup: int) -> tuple[float, int]:
    """ms per layer step (HIP graph replay) over rotated copies of the layer's
    weights, and the number of copies."""
    names = tuple(layer_shapes(synthetic))
    per_copy = sum(weights[n][0].numel() for n in names)
    n = max(2, -(-ROTATE_BYTES // per_copy) + 1)
    sets = [{k: weights[k] for k in names}] + [{k: (weights[k][0].clone(), weights[k][1]) for k in names}
                                               for _ in range(n - 1)]
    graphs = [b.capture(lambda s=s: layer_linears(fp8, synthetic, xs, s)) for s in sets]
    ms = b.time_graphs(graphs, replays, warmup)
    del graphs, sets
    torch.cuda.empty_cache()
    return ms, n


def six_step_ms(b: Bench, torch, fp8, synthetic, weights, case, M: int, replays: int, warmup: int) -> float:
    """ms per step of the six separate projections (q, k, v, o, gate+up, down),
    each quantizing its own input, over rotated weight copies."""
    names = tuple(synthetic.SHAPES)
    xs = {name: case(name, M)[0].cuda() for name in names}
    per_copy = sum(weights[n][0].numel() for n in names)
    n = max(2, -(-ROTATE_BYTES // per_copy) + 1)
    sets = [{k: weights[k] for k in names}] + [{k: (weights[k][0].clone(), weights[k][1]) for k in names}
                                               for _ in range(n - 1)]

    def step(s):
        for name in names:
            fp8.fp8_matmul(xs[name], s[name][0], s[name][1], tiled=True)

    graphs = [b.capture(lambda s=s: step(s)) for s in sets]
    ms = b.time_graphs(graphs, replays, warmup)
    del graphs, sets
    torch.cuda.empty_cache()
    return ms


def rate(M: int, N: int, K: int, ms: float, bound: str, mfma_peak: float = None) -> dict:
    """Time, throughput and roofline fraction of one linear call: GB/s of its
    algorithmic bytes against 8 TB/s ("hbm"), or TFLOP/s against the MFMA
    peak ("mfma"; FP8 unless given)."""
    if bound == "hbm":
        gbs = linear_bytes(M, N, K) / (ms * 1e-3) / 1e9
        return {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    tf = 2 * M * N * K / (ms * 1e-3) / 1e12
    peak = mfma_peak or FP8_PEAK_TFLOPS
    key = "frac_of_fp8_peak" if peak == FP8_PEAK_TFLOPS else "frac_of_bf16_peak"
    return {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1), key: round(tf / peak, 4)}


def per_kernel(b, torch, fp8, synthetic, rot, M: int, case, replays: int, bound: str, shapes: dict | None = None,
               tiled: bool = True) -> dict:
    """GEMM kernel time per projection at M tokens (and the merged q/k/v), with
    GB/s or TFLOP/s and the fraction of the bound's peak; `shapes` ({name:
    (N, K)}, K = 4096 activations) replaces the projection list; `tiled`
    False times the row-major weights of `rot`."""
    out = {}
    if shapes is None:
        shapes = dict(synthetic.SHAPES, **{"qkv": layer_shapes(synthetic)["qkv"]})
    for name, (N, K) in shapes.items():
        x = case(name if name in synthetic.SHAPES else "q", M)[0].cuda()
        ms = kernel_ms(b, fp8, rot.copies(name), quantized_operands(torch, fp8, x), replays, tiled=tiled)
        out[name] = rate(M, N, K, ms, bound)
    return out


def per_kernel_w8a16(b, torch, fp8, synthetic, rot, M: int, case, replays: int) -> dict:
    """The W8A16 parity mode (the reference's own arithmetic: bf16 activations
    times e4m3 weights widened to bf16, bf16 MFMA, fp32 sums) per projection at
    M tokens: GB/s against 8 TB/s at decode sizes (M <= 64), TFLOP/s against
    the dense bf16 MFMA peak (2.5 PFLOP/s) above."""
    out = {}
    for name, (N, K) in synthetic.SHAPES.items():
        x = case(name, M)[0].cuda()
        ms = launches_ms(b, rot.copies(name), lambda wq, sw: fp8.fp8_matmul_w8a16(x, wq, sw, tiled=True), replays)
        out[name] = rate(M, N, K, ms, "hbm" if M <= 64 else "mfma", BF16_PEAK_TFLOPS)
    return out


def mlp_steps(b: Bench, torch, fp8, synthetic, weights, M: int, replays: int) -> dict:
    """The MLP block (gate, up, SwiGLU, down) at M tokens, two ways, over rotated
    weight copies (HIP graph replay):
    * reference_shaped: what the reference's SwiGLU.forward runs after the
      import swap alone (model/model.py:581-584): gate and up as two FP8Linear
      calls (N = 12288 each, each quantizing x), torch's F.silu(gate) * up on
      bf16, then down (quantizing h);
    * fused: FP8SwiGLU, which fuse_swiglus puts in its place: one gate+up GEMM
      with SwiGLU in its epilogue, the quantization of h from the epilogue's
      maxima, the down GEMM.
    GB/s counts the same algorithmic bytes for both (gate+up and down linears)."""
    import torch.nn.functional as F

    I = synthetic.INTERMEDIATE
    x = synthetic.decode_case("gate_up", M)[0].cuda()
    gu, sgu = weights["gate_up"]
    dw, sd = weights["down"]
    per_copy = gu.numel() + dw.numel()
    n = max(2, -(-ROTATE_BYTES // per_copy) + 1)
    sets = [(gu, sgu, dw, sd)] + [(gu.clone(), sgu, dw.clone(), sd) for _ in range(n - 1)]

    def reference_shaped(s):
        g_, sg_, d_, sd_ = s
        # the tiled layout keeps whole 16-row tiles in row order: the first I rows are gate_proj's tiled codes
        gate = fp8.fp8_matmul(x, g_[:I], sg_[:I], tiled=True)
        up = fp8.fp8_matmul(x, g_[I:], sg_[I:], tiled=True)
        h = F.silu(gate) * up
        fp8.fp8_matmul(h, d_, sd_, tiled=True)

    def fused(s):
        g_, sg_, d_, sd_ = s
        amax = M <= fp8.DECODE_MAX_ROWS
        out = fp8.gate_up_swiglu(x, g_, sg_, tiled=True, amax=amax)
        hh, parts = out if amax else (out, None)
        res = fp8.quantize_swiglu_output(hh, parts, packed=True)
        fp8.fp8_matmul_quantized(res[0], res[1], d_, sd_, packed_rows=M, tiled=True)

    nbytes = linear_bytes(M, 2 * I, synthetic.HIDDEN) + linear_bytes(M, synthetic.HIDDEN, I)
    out = {}
    for name, fn in (("reference_shaped", reference_shaped), ("fused", fused)):
        graphs = [b.capture(lambda s=s, fn=fn: fn(s)) for s in sets]
        ms = b.time_graphs(graphs, replays, 3)
        del graphs
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    del sets
    torch.cuda.empty_cache()
    return out


def host_description() -> dict:
    model = platform.processor() or ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    import numpy
    import torch

    return {"cpu_model": model, "host_cores": os.cpu_count(), "torch": torch.__version__, "numpy": numpy.__version__}


def cpu_threads() -> int:
    """BLAS threads for the CPU baseline: the cores this process may run on,
    capped by OMP_NUM_THREADS when the environment sets it (the GPU box gives
    each GPU's jobs a share of its cores and says so there)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(n, 1)


def cpu_baseline(synthetic, M: int, budget_s: float) -> dict:
    """The oracle on the host: per-token quantization of x, per-call weight
    dequantization, float32 sgemm (numpy BLAS), scale epilogue, bf16 rounding.
    The decode layer step (the four linears of the GPU step, q/k/v merged) for
    up to `budget_s` seconds, then the single linear (16 x 4096 -> 4096) alone."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    import oracle

    threads = cpu_threads()
    shapes = layer_shapes(synthetic)
    ops = []
    for i, (name, (N, K)) in enumerate(shapes.items()):
        x = synthetic.activations_outliers(M, K, 950 + i).float().numpy()
        w = synthetic.weight(N, K, 960 + i).float().numpy()
        ops.append((x, *oracle.quantize_rows(w)))
    step_bytes = layer_bytes(synthetic, M)

    def linear(xf, wq, sw):
        xq, sx = oracle.quantize_rows(xf)
        return oracle.f32_to_bf16(oracle.dequant_matmul_f32(xq, sx, wq, sw))

    with threadpool_limits(limits=threads):
        for op in ops:  # warm-up: BLAS thread pool and page faults
            linear(*op)
        steps, t0 = 0, time.perf_counter()
        while True:
            for op in ops:
                linear(*op)
            steps += 1
            elapsed = time.perf_counter() - t0
            if elapsed >= budget_s or steps >= 50:
                break
        x1, w1 = synthetic.single_linear()
        op1 = (x1.float().numpy(), *oracle.quantize_rows(w1.float().numpy()))
        linear(*op1)
        times = []
        for _ in range(7):
            t = time.perf_counter()
            linear(*op1)
            times.append(time.perf_counter() - t)
        single_ms = float(np.median(times)) * 1e3
    return {"value": round(step_bytes * steps / elapsed / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{steps} decode layer steps (M={M}; q/k/v merged, o, gate+up, down: per-token quant, per-call "
                      f"weight dequant, float32 sgemm, bf16 rounding) in {elapsed:.1f} s on {threads} BLAS threads",
            "single_linear_16x4096x4096": {"ms": round(single_ms, 3),
                                           "GB/s": round(linear_bytes(16, 4096, 4096) / (single_ms * 1e-3) / 1e9, 4),
                                           "note": "median of 7 calls, same pipeline"},
            **host_description()}


def pmc_driver(torch, fp8, synthetic, quantize_rows, launches: int = 6) -> None:
    """Workload for the hardware-counter runs (rocprofv3 --pmc, one counter set
    per run): a 256 MiB device copy of known size (reads and writes 256 MiB;
    it calibrates FETCH_SIZE and WRITE_SIZE), then `launches` GEMM launches of
    every decode shape at M=16 (q, k, v, o, gate+up, down and the merged
    q/k/v) and of the prefill shapes at M=2048 (q, k, gate+up, down, merged
    q/k/v, and gate+up with the SwiGLU epilogue), each on one of four weight
    copies in the tiled layout, each launch one dispatch record. The GEMMs run
    on activations quantized beforehand (the SwiGLU launches include their
    quantizer)."""
    copy_src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    copy_dst = torch.empty_like(copy_src)
    copy_dst.copy_(copy_src)
    torch.cuda.synchronize()
    weights = make_weights(torch, synthetic, quantize_rows)
    del copy_src, copy_dst
    for M, case, names in ((16, synthetic.decode_case, ("q", "k", "v", "o", "gate_up", "down", "qkv")),
                           (2048, synthetic.prefill_case, ("q", "k", "gate_up", "down", "qkv"))):
        for name in names:
            wq, sw = weights[name]
            x = case("q" if name == "qkv" else name, M)[0].cuda()
            ops = quantized_operands(torch, fp8, x)
            copies = [wq] + [wq.clone() for _ in range(3)]
            torch.cuda.synchronize()
            for i in range(launches):
                fp8.fp8_matmul_quantized(ops[0], ops[1], copies[i % len(copies)], sw, packed_rows=ops[2], tiled=True)
            torch.cuda.synchronize()
            del copies
    x = synthetic.prefill_case("gate_up", 2048)[0].cuda()
    wq, sw = weights["gate_up"]
    copies = [wq] + [wq.clone() for _ in range(3)]
    for i in range(launches):
        fp8.gate_up_swiglu(x, copies[i % len(copies)], sw, tiled=True)
    torch.cuda.synchronize()
    print("pmc driver done", flush=True)


def read_probe(torch, fp8, synthetic, quantize_rows) -> dict:
    """The decode ceiling at M = 16: for every decode shape (the six
    projections, the merged q/k/v and the 9B model's merged widths), the GEMM
    kernel's time next to the time a pure streaming read of the same codes
    takes (tests/csrc/read_probe.hip: each wave issues all its 1 KB loads at
    once, then folds them into one stored word), in the GEMM's own launch
    shape (workgroups and threads from jv_fp8_launch_shape) and in the fastest
    of a sweep of shapes (256 or 512 threads, 4-32 KB per wave). Same harness
    as the GEMM lines: graphs of back-to-back launches over weight copies
    rotated through >= 512 MB."""
    import ctypes

    from jeeves_amd import _lib, device

    hooks_path = ROOT / "tests" / "libjeeves_fp8_testhooks.so"
    if not hooks_path.exists():
        raise RuntimeError("the read probe is in the test-hook library: run `python -m jeeves_amd.build --tests`")
    hooks = ctypes.CDLL(str(hooks_path))
    probe = hooks.th_read_probe
    probe.restype = ctypes.c_int
    probe.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                      ctypes.c_void_p]
    b = Bench(torch)
    M = 16
    cus = device.sm_count(torch.device("cuda", 0))
    weights = make_weights(torch, synthetic, quantize_rows)
    weights.update(merged_9b_weights(torch, synthetic, quantize_rows))
    rot = Rotation(weights)
    shapes = dict(synthetic.SHAPES, qkv=layer_shapes(synthetic)["qkv"],
                  **{name: (N, synthetic.HIDDEN) for name, N in MERGED_9B.items()})
    sink = torch.empty(1 << 20, dtype=torch.int32, device="cuda")
    out = {}
    for name, (N, K) in shapes.items():
        nbytes = N * K
        x = synthetic.decode_case(name if name in synthetic.SHAPES else "q", M)[0].cuda()
        gemm_ms = kernel_ms(b, fp8, rot.copies(name), quantized_operands(torch, fp8, x), 40)
        shape = (ctypes.c_int32 * 4)()
        _lib.check(_lib.lib().jv_fp8_launch_shape(M, N, K, cus, shape))
        wg, threads = shape[1], shape[2]

        def probe_ms(wg_, threads_, lpw):
            def launch(wq, sw):
                rc = probe(wq.data_ptr(), nbytes, wg_, threads_, lpw, sink.data_ptr(), torch.cuda.current_stream().cuda_stream)
                if rc:
                    raise RuntimeError(f"read probe refused {wg_} x {threads_} x {lpw} KB for {nbytes} bytes")
            return launches_ms(b, rot.copies(name), launch, 40)

        per_wave = nbytes / (wg * (threads // 64) * 1024)
        in_shape = None
        if per_wave == int(per_wave) and int(per_wave) in (4, 8, 16, 24, 32):
            in_shape = {"us": round(probe_ms(wg, threads, int(per_wave)) * 1e3, 2),
                        "shape": [wg, threads, int(per_wave)]}
        best = None
        for threads_ in (256, 512):
            for lpw in (4, 8, 16, 32):
                wg_ = nbytes // ((threads_ // 64) * lpw * 1024)
                if wg_ * (threads_ // 64) * lpw * 1024 != nbytes or wg_ * (threads_ // 64) > (1 << 20):
                    continue
                us = probe_ms(wg_, threads_, lpw) * 1e3
                if best is None or us < best["us"]:
                    best = {"us": round(us, 2), "shape": [wg_, threads_, lpw]}
        out[name] = {"N": N, "K": K, "code_bytes": nbytes,
                     "gemm": dict(rate(M, N, K, gemm_ms, "hbm"), shape=[wg, threads]),
                     "read_in_gemm_shape": in_shape, "read_fastest": best}
        log(f"bench: read probe {name}: {out[name]}")
    rot.drop()
    return {"note": "M=16 decode GEMM vs a pure streaming read of its codes; shapes are [workgroups, threads, "
                    "KB per wave] for reads and [workgroups, threads] for the GEMM; every time includes its launch",
            "shapes": out}


def device_weight(torch, synthetic, N: int, K: int, seed: int):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(N, K, device="cuda", generator=g) * synthetic.WEIGHT_STD).to(torch.bfloat16)


def workloads(torch, b: Bench, fp8, synthetic, quantize_rows) -> dict:
    """The decoder layer with LoRA at M = 512 and the ragged request mix through
    32 layers (prefill of the packed batch, then 64 decode steps at batch 64):
    linear-layer time, throughput and roofline fraction of each phase."""
    out = {}
    # decoder layer, M = 512, rank-16 LoRA on every projection; 4 weight copies (772 MB) rotate
    M = 512
    x = synthetic.activations_heavy_tail(M, synthetic.HIDDEN, 400).cuda()
    copies, lora = [], {}
    for c in range(4):
        weights = {}
        for i, (name, (N, K)) in enumerate(synthetic.SHAPES.items()):
            wq, sw = quantize_rows(device_weight(torch, synthetic, N, K, 410 + i + 10 * c))
            weights[name] = (fp8.tile_weight(wq), sw)
            if c == 0:
                a, bb = synthetic.lora_factors(N, K, 420 + i)
                lora[name] = (a.cuda(), bb.cuda(), synthetic.LORA_SCALING)
        copies.append(weights)
    graphs = [b.capture(lambda c=c: layer_linears(fp8, synthetic, x, copies[c], lora)) for c in range(len(copies))]
    ms = b.time_graphs(graphs, 40, 4)
    fl = layer_flops(synthetic, M, synthetic.LORA_RANK)
    tf = fl / (ms * 1e-3) / 1e12
    out["decoder_layer_lora_m512"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1), "frac_of_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4),
                                      "flops": fl, "note": "q, k, v, o, gate+up with SwiGLU in its epilogue, quantization of h, down, rank-16 LoRA on each; "
                                                           "HIP graph replay over 4 weight copies (772 MB)"}
    del graphs, copies
    torch.cuda.empty_cache()
    log(f"bench: decoder layer (LoRA, M=512) {ms * 1e3:.1f} us, {tf:.0f} TFLOP/s")

    # ragged mix: 32 layers of random weights (6.2 GB of e4m3 codes), q/k/v merged as the engine merges them
    layers = []
    for layer in range(32):
        w = {}
        for i, (name, (N, K)) in enumerate(synthetic.SHAPES.items()):
            wq, sw = quantize_rows(device_weight(torch, synthetic, N, K, 700 + 10 * layer + i))
            w[name] = (fp8.tile_weight(wq), sw)
        w["qkv"] = (torch.cat([w[n][0] for n in ("q", "k", "v")]), torch.cat([w[n][1] for n in ("q", "k", "v")]))
        for n in ("q", "k", "v"):
            del w[n]
        layers.append(w)
    torch.cuda.empty_cache()
    lengths = synthetic.ragged_lengths()
    h = torch.cat([synthetic.activations_heavy_tail(n, synthetic.HIDDEN, 5000 + i) for i, n in enumerate(lengths)]).cuda()
    T = h.shape[0]
    g = torch.Generator().manual_seed(5001)
    xs = {"attn": h, "o": h[:, torch.randperm(synthetic.HIDDEN, generator=g).cuda()].contiguous(),
          "mlp": h[:, torch.randperm(synthetic.HIDDEN, generator=g).cuda()].contiguous()}
    with torch.cuda.stream(b.stream):
        for w in layers[:2]:
            layer_linears(fp8, synthetic, xs, w)
        b.stream.synchronize()
        best = None
        for _ in range(2):
            st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            st.record(b.stream)
            for w in layers:
                layer_linears(fp8, synthetic, xs, w)
            en.record(b.stream)
            en.synchronize()
            t = st.elapsed_time(en)
            best = t if best is None else min(best, t)
    pre_ms = best
    pre_fl = 32 * layer_flops(synthetic, T)
    pre_tf = pre_fl / (pre_ms * 1e-3) / 1e12
    del h, xs
    torch.cuda.empty_cache()
    xd = synthetic.activations_outliers(64, synthetic.HIDDEN, 5500).cuda()
    g = torch.Generator().manual_seed(5501)
    xds = {"attn": xd, "o": xd[:, torch.randperm(synthetic.HIDDEN, generator=g).cuda()].contiguous(),
           "mlp": xd[:, torch.randperm(synthetic.HIDDEN, generator=g).cuda()].contiguous()}

    def decode_step():
        for w in layers:
            layer_linears(fp8, synthetic, xds, w)

    graph = b.capture(decode_step)
    step_ms = b.time_graphs([graph], 64, 2)
    dec_bytes = 32 * layer_bytes(synthetic, 64)
    dec_gbs = dec_bytes / (step_ms * 1e-3) / 1e9
    out["ragged_32_layers"] = {
        "tokens_prefill": T, "sequences": len(lengths),
        "prefill_ms": round(pre_ms, 3), "prefill_TFLOP/s": round(pre_tf, 1),
        "prefill_frac_of_fp8_peak": round(pre_tf / FP8_PEAK_TFLOPS, 4),
        "decode_steps": 64, "decode_batch": 64, "decode_ms_total": round(64 * step_ms, 3),
        "decode_us_per_step": round(step_ms * 1e3, 1), "decode_GB/s": round(dec_gbs, 1),
        "decode_frac_of_hbm_peak": round(dec_gbs / HBM_PEAK_GBS, 4),
        "linear_ms_total": round(pre_ms + 64 * step_ms, 3),
        "note": "linear layers only (q/k/v merged, o, gate+up with SwiGLU epilogue, quantization of h, down per layer, no LoRA), random-init "
                "weights; prefill eager on the packed batch, each decode step one HIP graph of 32 layers",
    }
    log(f"bench: ragged prefill {T} tokens {pre_ms:.2f} ms ({pre_tf:.0f} TFLOP/s), decode step {step_ms * 1e3:.0f} us "
        f"({dec_gbs:.0f} GB/s)")
    del graph, layers
    torch.cuda.empty_cache()

    # lm_head, N = 248320 x K = 4096 (inference/engine.py:293-297): 1.02 GB of tiled e4m3 codes, more
    # than the rotation size, so every call reads its weights from HBM; quantizer + GEMM per call
    N, K = synthetic.VOCAB, synthetic.HIDDEN
    wq, sw = quantize_rows(device_weight(torch, synthetic, N, K, 600))
    wq = fp8.tile_weight(wq)
    torch.cuda.empty_cache()
    heads = {}
    for M in (1, 16):
        x = synthetic.activations_outliers(M, K, 610 + M).cuda()
        g = b.capture(lambda x=x: [fp8.fp8_matmul(x, wq, sw, tiled=True) for _ in range(4)])
        ms = b.time_graphs([g], 10, 2) / 4
        gbs = linear_bytes(M, N, K) / (ms * 1e-3) / 1e9
        heads[f"m{M}"] = {"us": round(ms * 1e3, 1), "GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        del g
    out["lm_head_decode"] = dict(heads, note="N=248320 K=4096 (1.02 GB e4m3, tiled), per-token quantizer + GEMM per "
                                             "call, HIP graph of 4 calls")
    log(f"bench: lm_head decode {heads}")
    del wq, sw
    torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--rows", type=int, default=16, help="decode tokens per step")
    ap.add_argument("--prefill-rows", type=int, default=2048)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-sweep", action="store_true", help="skip the per-kernel lines at the other batch sizes")
    ap.add_argument("--no-workloads", action="store_true",
                    help="skip the decoder-layer (LoRA, M=512), 32-layer ragged-mix and lm_head measurements")
    ap.add_argument("--pmc-driver", action="store_true",
                    help="run only the hardware-counter workload (copy calibration + gate+up GEMMs), no timing")
    ap.add_argument("--read-probe", action="store_true",
                    help="run only the decode ceiling table: each M=16 decode GEMM vs a pure read of its codes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the FP8 linear path on one GPU; runs on more than one GPU are not part of this build",
              file=sys.stderr)
        return 2

    import torch

    from jeeves_amd import fp8, synthetic
    from jeeves_amd.fp8_weights import quantize_rows

    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        return 2
    if args.pmc_driver:
        pmc_driver(torch, fp8, synthetic, quantize_rows)
        return 0
    if args.read_probe:
        print(json.dumps(read_probe(torch, fp8, synthetic, quantize_rows)), flush=True)
        return 0
    b = Bench(torch)
    dev_name = torch.cuda.get_device_name(0)
    M = args.rows
    log(f"bench: decode M={M} on {dev_name}")
    weights = make_weights(torch, synthetic, quantize_rows)
    rot = Rotation(weights)
    K = synthetic.HIDDEN

    # the headline: one decoder layer's linears, engine-style
    xs = {k: v.cuda() for k, v in layer_inputs(synthetic, M, K, synthetic.decode_case).items()}
    ms, n_sets = layer_step_ms(b, torch, fp8, synthetic, weights, xs, args.steps, args.warmup)
    step_bytes = layer_bytes(synthetic, M)
    value = step_bytes / (ms * 1e-3) / 1e9
    log(f"bench: decode layer step {ms * 1e3:.1f} us, {value:.0f} GB/s")
    six_ms = six_step_ms(b, torch, fp8, synthetic, weights, synthetic.decode_case, M, max(args.steps // 2, 20), 5)
    six_bytes = sum(linear_bytes(M, *synthetic.SHAPES[n]) for n in synthetic.SHAPES)
    log(f"bench: six-projection step {six_ms * 1e3:.1f} us")

    kernels = per_kernel(b, torch, fp8, synthetic, rot, M, synthetic.decode_case, 40, "hbm")
    N, Kg = synthetic.SHAPES["gate_up"]
    k_ms = kernels["gate_up"]["us"] * 1e-3
    k_bytes = linear_bytes(M, N, Kg)
    k_gbs = k_bytes / (k_ms * 1e-3) / 1e9
    log(f"bench: decode GEMM kernels {kernels}")
    merged_shapes = {name: (N9, synthetic.HIDDEN) for name, N9 in MERGED_9B.items()}
    merged = {}
    if not args.no_sweep:
        weights.update(merged_9b_weights(torch, synthetic, quantize_rows))
        merged = per_kernel(b, torch, fp8, synthetic, rot, M, synthetic.decode_case, 40, "hbm", merged_shapes)
        log(f"bench: 9B merged projections {merged}")
    sweep = {}
    rowmajor, w8a16, mlp = {}, {}, {}
    if not args.no_sweep:
        for m in DECODE_SWEEP_ROWS:
            sweep[f"m{m}"] = per_kernel(b, torch, fp8, synthetic, rot, m, synthetic.decode_case, 16, "hbm")
        log(f"bench: decode sweep done ({', '.join(sweep)})")
        for m in (16, 64):
            mlp[f"m{m}"] = mlp_steps(b, torch, fp8, synthetic, weights, m, 40)
        log(f"bench: MLP block, reference-shaped vs fused {mlp}")
        # the single-copy layout (FP8Linear.TILED_COPY = False): the kernels read the row-major codes
        rot_rm = Rotation({name: (fp8.untile_weight(weights[name][0]), weights[name][1])
                           for name in (*synthetic.SHAPES, "qkv")})
        for m in (16, 64):
            rowmajor[f"m{m}"] = per_kernel(b, torch, fp8, synthetic, rot_rm, m, synthetic.decode_case, 16, "hbm",
                                           tiled=False)
        rot_rm.drop()
        del rot_rm
        torch.cuda.empty_cache()
        log(f"bench: row-major weights {rowmajor}")
        for m in W8A16_ROWS:
            case = synthetic.decode_case if m <= 64 else synthetic.prefill_case
            w8a16[f"m{m}"] = per_kernel_w8a16(b, torch, fp8, synthetic, rot, m, case, 16 if m <= 64 else 4)
        log(f"bench: W8A16 parity mode {w8a16}")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (fp32 accumulate)",
        "data": "synthetic (seeded random-init weights and activations)",
        "config": {
            "workload": f"decode M={M}: one 9B-class decoder layer's FP8 linears with q/k/v merged as the engine "
                        f"merges them (4096->6144), o 4096->4096, and the MLP as FP8SwiGLU runs it after "
                        f"fuse_swiglus: gate+up 4096->24576 as one GEMM with SwiGLU in its epilogue, the "
                        f"quantization of h, down 12288->4096 (the reference-shaped MLP is decode.mlp_m16); each "
                        f"distinct input quantized once (4 quantizer + 4 GEMM launches), HIP graph replay, weights "
                        f"in FP8Linear's tiled layout rotated over {n_sets} copies",
            "tokens": M,
            "device": dev_name,
        },
        "roofline": {"bound": "hbm", "kernel": "gemm_decode_kernel (gate+up, N=24576 K=4096, M=16)",
                     "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(k_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(f"decode_gate_up_m{M}"),
                     "traffic_source": f"copied from {PMC_SUMMARY} (rocprofv3 PMC FETCH_SIZE + WRITE_SIZE), not measured "
                                       "in this run",
                     "avg_launch_us": round(k_ms * 1e3, 3), "bytes_per_launch": k_bytes},
        "decode": {
            "layer_step": {"us": round(ms * 1e3, 2), "GB/s": round(value, 1), "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
                           "bytes": step_bytes},
            "six_projections_step": {"us": round(six_ms * 1e3, 2),
                                     "GB/s": round(six_bytes / (six_ms * 1e-3) / 1e9, 1),
                                     "note": "q, k, v, o, gate+up, down each with its own quantizer launch"},
            "kernels_m16": kernels,
            "kernels_m16_9b_merged": merged,
            "kernels_sweep": sweep,
            "mlp": dict(mlp, note="the MLP block at decode sizes: reference_shaped = gate and up as two FP8Linear "
                                  "calls, torch's F.silu(gate) * up, down (model/model.py:581-584 after the import "
                                  "swap alone); fused = FP8SwiGLU after fuse_swiglus"),
            "kernels_rowmajor": dict(rowmajor, note="GEMM kernels on the row-major codes (FP8Linear.TILED_COPY = "
                                                    "False: one copy of the codes in HBM), same harness as "
                                                    "kernels_m16 / kernels_sweep"),
        },
        "w8a16": dict(w8a16, note="W8A16 parity mode (fp8_matmul_w8a16, the reference's arithmetic): GB/s vs "
                                  "8 TB/s at M <= 64, TFLOP/s vs the dense bf16 MFMA peak 2.5 PFLOP/s at M = 2048"),
    }

    if not args.no_prefill:
        Mp = args.prefill_rows
        log(f"bench: prefill M={Mp}")
        pxs = {k: v.cuda() for k, v in layer_inputs(synthetic, Mp, K, synthetic.prefill_case).items()}
        pms, _ = layer_step_ms(b, torch, fp8, synthetic, weights, pxs, max(args.steps // 8, 20), 3)
        lflops = sum(2 * Mp * n_ * k_ for n_, k_ in layer_shapes(synthetic).values())
        six_pms = six_step_ms(b, torch, fp8, synthetic, weights, synthetic.prefill_case, Mp, max(args.steps // 8, 20), 3)
        six_flops = sum(2 * Mp * n_ * k_ for n_, k_ in synthetic.SHAPES.values())
        pk = per_kernel(b, torch, fp8, synthetic, rot, Mp, synthetic.prefill_case, 8, "mfma")
        pk_us = pk["gate_up"]["us"]
        pk_tf = 2 * Mp * N * Kg / (pk_us * 1e-6) / 1e12
        psweep = {}
        if not args.no_sweep:
            for m in PREFILL_SWEEP_ROWS:
                psweep[f"m{m}"] = per_kernel(b, torch, fp8, synthetic, rot, m, synthetic.prefill_case, 4, "mfma")
            psweep[f"m{Mp}_9b_merged"] = per_kernel(b, torch, fp8, synthetic, rot, Mp, synthetic.prefill_case, 8, "mfma",
                                                     merged_shapes)
        result["prefill"] = {
            "tokens": Mp, "ms_per_step": round(pms, 4), "TFLOP/s": round(lflops / (pms * 1e-3) / 1e12, 1),
            "step": "the decode step's layer (q/k/v merged, o, gate+up with SwiGLU epilogue, quantization of h, down) at M=2048",
            "six_projections_step": {"ms": round(six_pms, 4), "TFLOP/s": round(six_flops / (six_pms * 1e-3) / 1e12, 1)},
            "roofline": {"bound": "mfma", "kernel": "gemm_prefill_pp_kernel (gate+up, N=24576 K=4096, M=2048)",
                         "achieved": round(pk_tf, 1), "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pk_tf / FP8_PEAK_TFLOPS, 4), "avg_launch_us": round(pk_us, 2),
                         "traffic": measured_traffic(f"prefill_gate_up_m{Mp}"),
                         "traffic_source": f"copied from {PMC_SUMMARY}, not measured in this run",
                         "flops_per_launch": 2 * Mp * N * Kg,
                         "mfma_busy_pct": measured_counter("mfma_busy_pct", f"prefill_gate_up_m{Mp}"),
                         "window_clock_ghz": measured_counter("window_clock_ghz", f"prefill_gate_up_m{Mp}"),
                         "counters_source": f"copied from {PMC_SUMMARY} (SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE), "
                                            "not measured in this run"},
            "kernels": pk,
            "kernels_sweep": psweep,
        }
        log(f"bench: prefill layer step {pms:.3f} ms, six projections {six_pms:.3f} ms, kernels {pk}")
    rot.drop()
    del weights
    torch.cuda.empty_cache()

    if not args.no_workloads:
        result["workloads"] = workloads(torch, b, fp8, synthetic, quantize_rows)

    if not args.no_cpu_baseline:
        log("bench: cpu baseline")
        result["cpu_baseline"] = cpu_baseline(synthetic, M, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
