#!/usr/bin/env python3
"""Benchmark of the MI355X FP8 linear path on one GPU.

A step is one pass of the decode workload: the six 9B-class projections
(q, k, v: 4096->4096/1024/1024, o: 4096->4096, fused gate+up: 4096->24576,
down: 12288->4096) each applied once to M = 16 tokens through the full path
(per-token e4m3 quantization of the bf16 activations + FP8 x FP8 GEMM + scale
epilogue -> bf16). As in the reference engine, which replays its decode passes
as CUDA graphs (inference/engine.py:351-360), each step is a captured HIP graph
replay, so host launch overhead is not measured. Weights rotate over enough
copies (>= 512 MB) that every step reads them from HBM, not the 256 MB
Infinity Cache. Inputs are resident in HBM before timing starts.

value        algorithmic bytes of the six linears / step time (GB/s), with
             bytes per linear = N*K (e4m3 W) + 4N (scales) + 2MK (bf16 x) + 2MN (bf16 y)
roofline     the dominant kernel (the fused gate+up decode GEMM) alone: a graph
             of back-to-back launches on rotated weights, timed with HIP events
             on its stream; algorithmic bytes / average launch time vs 8 TB/s
prefill      the same six projections at M = 2048 (TFLOP/s, 2*M*N*K per
             linear), with the gate+up prefill GEMM's roofline vs 5.0 PFLOP/s
workloads    the decoder layer's linear stack at M = 512 with a rank-16 LoRA
             on every projection, the ragged request mix (64 log-uniform
             sequence lengths packed into one batch through 32 layers of
             random weights, then 64 decode steps at batch 64), and the
             lm_head (248320 x 4096) at M = 1 and 16: time, TFLOP/s or GB/s
             and roofline fraction per phase
cpu_baseline the CPU oracle's dequantize-then-matmul (numpy float32, BLAS
             threads) on the same decode step, timed on the host for a bounded
             number of steps

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "FP8 linear TFLOP/s (M=2048) and HBM GB/s (M<=16) on 1 MI355X; % of roofline"
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
ROTATE_BYTES = 512 << 20
LAUNCHES_PER_GRAPH = 24


def measured_traffic(key: str):
    """HBM bytes per launch measured with rocprofv3 PMC counters, from the
    committed summary (None when absent)."""
    path = ROOT / "profiles" / "gate_up_hbm_traffic_pmc.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.split()
        if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == key:
            return int(parts[2])
    return None


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


def build_set(torch, synthetic, quantize_rows, M: int, case):
    """Quantized weights (rotated copies) and bf16 activations for one
    workload. The codes are stored as FP8Linear stores them for these shapes:
    in the tiled layout (tile_weight)."""
    from jeeves_amd.fp8 import tile_weight

    weights, xs = {}, {}
    for name in synthetic.SHAPES:
        x, w = case(name, M)
        wq, sw = quantize_rows(w.cuda())
        weights[name] = (tile_weight(wq), sw)
        xs[name] = x.cuda()
    per_copy = sum(wq.numel() for wq, _ in weights.values())
    copies = max(2, -(-ROTATE_BYTES // per_copy) + 1)
    rot = [weights] + [{n: (wq.clone(), sw.clone()) for n, (wq, sw) in weights.items()} for _ in range(copies - 1)]
    return rot, xs, copies, per_copy


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


def kernel_ms(b: Bench, fp8, rot, operands, name: str, replays: int) -> float:
    """Average time (ms) of one GEMM kernel launch for projection `name` on the
    activation codes fp8_matmul would produce, from graphs of back-to-back
    launches on the bench stream. The launches rotate over copies of this
    projection's weights totalling at least ROTATE_BYTES, so each launch reads
    its weights from HBM rather than the Infinity Cache."""
    xq, sx, packed_rows = operands
    wq0, sw0 = rot[0][name]
    n_copies = max(2, -(-ROTATE_BYTES // wq0.numel()) + 1)
    copies = [(wq0, sw0)] + [(wq0.clone(), sw0) for _ in range(n_copies - 1)]
    graphs = []
    for c in range(min(len(copies), 4)):
        def launches(c=c):
            for j in range(LAUNCHES_PER_GRAPH):
                wq, sw = copies[(c * LAUNCHES_PER_GRAPH + j) % len(copies)]
                fp8.fp8_matmul_quantized(xq, sx, wq, sw, packed_rows=packed_rows, tiled=True)
        graphs.append(b.capture(launches))
    ms = b.time_graphs(graphs, replays, 3) / LAUNCHES_PER_GRAPH
    del graphs, copies
    return ms


def cpu_baseline(synthetic, M: int, budget_s: float) -> dict:
    from threadpoolctl import threadpool_limits

    import oracle

    cores = min(os.cpu_count() or 1, 16)
    ops = []
    total_bytes = 0
    for name, (N, K) in synthetic.SHAPES.items():
        x, w = synthetic.decode_case(name, M)
        wq, sw = oracle.quantize_rows(w.float().numpy())
        ops.append((x.float().numpy(), wq, sw))
        total_bytes += linear_bytes(M, N, K)
    with threadpool_limits(limits=cores):
        steps, t0 = 0, time.perf_counter()
        while True:
            for xf, wq, sw in ops:
                xq, sx = oracle.quantize_rows(xf)
                oracle.f32_to_bf16(oracle.dequant_matmul_f32(xq, sx, wq, sw))
            steps += 1
            elapsed = time.perf_counter() - t0
            if elapsed >= budget_s or steps >= 50:
                break
    return {"value": round(total_bytes * steps / elapsed / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{steps} decode steps (M={M}, the six projections: per-token quant, per-call weight dequant, "
                      f"float32 sgemm, bf16 rounding) in {elapsed:.1f} s"}


def pmc_driver(torch, fp8, synthetic, quantize_rows, launches: int = 10) -> None:
    """Workload for the hardware-counter runs (rocprofv3 --pmc FETCH_SIZE, then
    WRITE_SIZE): a 256 MiB device copy of known size (reads and writes 256 MiB;
    it calibrates the counters), then `launches` launches each of the gate+up
    decode GEMM (M=16, packed codes) and the gate+up prefill GEMM (M=2048),
    each on a fresh weight copy, one launch per dispatch record."""
    copy_src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    copy_dst = torch.empty_like(copy_src)
    copy_dst.copy_(copy_src)
    torch.cuda.synchronize()
    for M, case in ((16, synthetic.decode_case), (2048, synthetic.prefill_case)):
        x, w = case("gate_up", M)
        x = x.cuda()
        wq, sw = quantize_rows(w.cuda())
        wq = fp8.tile_weight(wq)
        ops = quantized_operands(torch, fp8, x)
        copies = [wq] + [wq.clone() for _ in range(3)]
        torch.cuda.synchronize()
        for i in range(launches):
            fp8.fp8_matmul_quantized(ops[0], ops[1], copies[i % len(copies)], sw, packed_rows=ops[2], tiled=True)
        torch.cuda.synchronize()
        del copies
    print("pmc driver done", flush=True)


def device_weight(torch, synthetic, N: int, K: int, seed: int):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(N, K, device="cuda", generator=g) * synthetic.WEIGHT_STD).to(torch.bfloat16)


def layer_linears(fp8, synthetic, h, weights, lora=None):
    """One decoder layer's linear stack on h: q, k, v, o and gate+up, SwiGLU
    fused with the down projection's activation quantization, down (the same
    input feeds every projection: only the linear layers are timed)."""
    for name in ("q", "k", "v", "o"):
        wq, sw = weights[name]
        fp8.fp8_matmul(h, wq, sw, tiled=True, lora=lora[name] if lora else None)
    wq, sw = weights["gate_up"]
    gu = fp8.fp8_matmul(h, wq, sw, tiled=True, lora=lora["gate_up"] if lora else None)
    inter = synthetic.INTERMEDIATE
    res = fp8.swiglu_quantize(gu[:, :inter], gu[:, inter:], lora_a=lora["down"][0] if lora else None, packed=True)
    wq, sw = weights["down"]
    return fp8.fp8_matmul_quantized(res[0], res[1], wq, sw, lora_t=res[2] if lora else None,
                                    lora_b=lora["down"][1] if lora else None,
                                    lora_scaling=lora["down"][2] if lora else 0.0, packed_rows=h.shape[0], tiled=True)


def layer_flops(synthetic, M: int, rank: int = 0) -> int:
    return sum(2 * M * N * K + 2 * M * rank * (K + N) for N, K in synthetic.SHAPES.values())


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
                                      "flops": fl, "note": "q, k, v, o, gate+up, SwiGLU-quant, down with rank-16 LoRA each; "
                                                           "HIP graph replay over 4 weight copies (772 MB)"}
    del graphs, copies
    torch.cuda.empty_cache()
    log(f"bench: decoder layer (LoRA, M=512) {ms * 1e3:.1f} us, {tf:.0f} TFLOP/s")

    # ragged mix: 32 layers of random weights (6.2 GB of e4m3 codes)
    layers = []
    for layer in range(32):
        weights = {}
        for i, (name, (N, K)) in enumerate(synthetic.SHAPES.items()):
            wq, sw = quantize_rows(device_weight(torch, synthetic, N, K, 700 + 10 * layer + i))
            weights[name] = (fp8.tile_weight(wq), sw)
        layers.append(weights)
    torch.cuda.empty_cache()
    lengths = synthetic.ragged_lengths()
    h = torch.cat([synthetic.activations_heavy_tail(n, synthetic.HIDDEN, 5000 + i) for i, n in enumerate(lengths)]).cuda()
    T = h.shape[0]
    with torch.cuda.stream(b.stream):
        for weights in layers[:2]:
            layer_linears(fp8, synthetic, h, weights)
        b.stream.synchronize()
        best = None
        for _ in range(2):
            st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            st.record(b.stream)
            for weights in layers:
                layer_linears(fp8, synthetic, h, weights)
            en.record(b.stream)
            en.synchronize()
            t = st.elapsed_time(en)
            best = t if best is None else min(best, t)
    pre_ms = best
    pre_fl = 32 * layer_flops(synthetic, T)
    pre_tf = pre_fl / (pre_ms * 1e-3) / 1e12
    del h
    torch.cuda.empty_cache()
    xd = synthetic.activations_outliers(64, synthetic.HIDDEN, 5500).cuda()

    def decode_step():
        for weights in layers:
            layer_linears(fp8, synthetic, xd, weights)

    g = b.capture(decode_step)
    step_ms = b.time_graphs([g], 64, 2)
    dec_bytes = 32 * sum(linear_bytes(64, N, K) for N, K in synthetic.SHAPES.values())
    dec_gbs = dec_bytes / (step_ms * 1e-3) / 1e9
    out["ragged_32_layers"] = {
        "tokens_prefill": T, "sequences": len(lengths),
        "prefill_ms": round(pre_ms, 3), "prefill_TFLOP/s": round(pre_tf, 1),
        "prefill_frac_of_fp8_peak": round(pre_tf / FP8_PEAK_TFLOPS, 4),
        "decode_steps": 64, "decode_batch": 64, "decode_ms_total": round(64 * step_ms, 3),
        "decode_us_per_step": round(step_ms * 1e3, 1), "decode_GB/s": round(dec_gbs, 1),
        "decode_frac_of_hbm_peak": round(dec_gbs / HBM_PEAK_GBS, 4),
        "linear_ms_total": round(pre_ms + 64 * step_ms, 3),
        "note": "linear layers only (q, k, v, o, gate+up, SwiGLU-quant, down per layer, no LoRA), random-init "
                "weights; prefill eager on the packed batch, each decode step one HIP graph of 32 layers",
    }
    log(f"bench: ragged prefill {T} tokens {pre_ms:.2f} ms ({pre_tf:.0f} TFLOP/s), decode step {step_ms * 1e3:.0f} us "
        f"({dec_gbs:.0f} GB/s)")
    del g, layers
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
    ap.add_argument("--no-workloads", action="store_true",
                    help="skip the decoder-layer (LoRA, M=512) and 32-layer ragged-mix measurements")
    ap.add_argument("--pmc-driver", action="store_true",
                    help="run only the hardware-counter workload (copy calibration + gate+up GEMMs), no timing")
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
    b = Bench(torch)
    dev_name = torch.cuda.get_device_name(0)
    M = args.rows
    log(f"bench: decode M={M} on {dev_name}")
    rot, xs, copies, per_copy = build_set(torch, synthetic, quantize_rows, M, synthetic.decode_case)
    step_bytes = sum(linear_bytes(M, *synthetic.SHAPES[n]) for n in synthetic.SHAPES)

    def step(c):
        for name in synthetic.SHAPES:
            wq, sw = rot[c][name]
            fp8.fp8_matmul(xs[name], wq, sw, tiled=True)

    graphs = [b.capture(lambda c=c: step(c)) for c in range(copies)]
    ms = b.time_graphs(graphs, args.steps, args.warmup)
    value = step_bytes / (ms * 1e-3) / 1e9
    log(f"bench: decode step {ms * 1e3:.1f} us, {value:.0f} GB/s")

    per_shape = {}
    for name, (n_, k_) in synthetic.SHAPES.items():
        t = kernel_ms(b, fp8, rot, quantized_operands(torch, fp8, xs[name]), name, 40)
        per_shape[name] = {"us": round(t * 1e3, 2), "GB/s": round(linear_bytes(M, n_, k_) / (t * 1e-3) / 1e9, 1)}
    N, K = synthetic.SHAPES["gate_up"]
    k_ms = per_shape["gate_up"]["us"] * 1e-3
    k_bytes = linear_bytes(M, N, K)
    k_gbs = k_bytes / (k_ms * 1e-3) / 1e9
    log(f"bench: decode GEMM kernels {per_shape}")

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
            "workload": f"decode M={M}: 9B-class FP8 linears q 4096->4096, k/v 4096->1024, o 4096->4096, gate+up "
                        f"4096->24576, down 12288->4096, one pass each per step (quant + GEMM + epilogue) replayed as "
                        f"a HIP graph, weights in FP8Linear's tiled layout rotated over {copies} copies "
                        f"({copies * per_copy / 2**20:.0f} MiB)",
            "tokens": M,
            "device": dev_name,
        },
        "roofline": {"bound": "hbm", "kernel": "gemm_decode_kernel (gate+up, N=24576 K=4096, M=16)",
                     "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(k_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(f"decode_gate_up_m{M}"), "avg_launch_us": round(k_ms * 1e3, 3),
                     "bytes_per_launch": k_bytes},
        "decode_kernels": per_shape,
    }

    if not args.no_prefill:
        Mp = args.prefill_rows
        log(f"bench: prefill M={Mp}")
        del rot, graphs
        torch.cuda.empty_cache()
        prot, pxs, pcopies, _ = build_set(torch, synthetic, quantize_rows, Mp, synthetic.prefill_case)
        flops = sum(2 * Mp * n_ * k_ for n_, k_ in synthetic.SHAPES.values())

        def pstep(c):
            for name in synthetic.SHAPES:
                wq, sw = prot[c][name]
                fp8.fp8_matmul(pxs[name], wq, sw, tiled=True)

        pgraphs = [b.capture(lambda c=c: pstep(c)) for c in range(pcopies)]
        pms = b.time_graphs(pgraphs, max(args.steps // 8, 20), 3)
        pshape = {}
        for name, (n_, k_) in synthetic.SHAPES.items():
            t = kernel_ms(b, fp8, prot, quantized_operands(torch, fp8, pxs[name]), name, 8)
            pshape[name] = {"us": round(t * 1e3, 2), "TFLOP/s": round(2 * Mp * n_ * k_ / (t * 1e-3) / 1e12, 1)}
        pk = pshape["gate_up"]["us"] * 1e-3
        pk_tf = 2 * Mp * N * K / (pk * 1e-3) / 1e12
        result["prefill"] = {
            "tokens": Mp, "ms_per_step": round(pms, 4), "TFLOP/s": round(flops / (pms * 1e-3) / 1e12, 1),
            "roofline": {"bound": "mfma", "kernel": "gemm_prefill_pp_kernel (gate+up, N=24576 K=4096, M=2048)",
                         "achieved": round(pk_tf, 1), "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pk_tf / FP8_PEAK_TFLOPS, 4), "avg_launch_us": round(pk * 1e3, 2),
                         "traffic": measured_traffic(f"prefill_gate_up_m{Mp}"),
                         "flops_per_launch": 2 * Mp * N * K},
            "kernels": pshape,
        }
        log(f"bench: prefill step {pms:.3f} ms, kernels {pshape}")

    if not args.no_workloads:
        result["workloads"] = workloads(torch, b, fp8, synthetic, quantize_rows)

    if not args.no_cpu_baseline:
        log("bench: cpu baseline")
        result["cpu_baseline"] = cpu_baseline(synthetic, M, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
