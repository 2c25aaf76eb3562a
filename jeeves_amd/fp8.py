"""Drop-in for ``inference/fp8.py``: the FP8 linear layer on MI355X.

Same public names and behaviour as the reference module -- ``fp8_matmul``,
``FP8Linear`` (``load_codes``, ``load_weight``, ``concatenated``,
``forward``), ``load_view``, ``warm``, ``split_for``, ``TILE_COUNTERS`` and
the module constants -- with the Triton kernels replaced by the gfx950 HIP
kernels of ``libjeeves_fp8.so``, called through its C ABI:

* activations are quantized per token to e4m3fn with ``quantize_rows``
  semantics (``inference/fp8_weights.py:16-19``) instead of being converted
  to fp16 with a power-of-two row scale (``inference/fp8.py:46-58``);
* the GEMM multiplies e4m3 by e4m3 on the FP8 MFMA units and applies
  ``acc * sx[m] * sw[n]`` (+ bias, + optional LoRA) in its epilogue;
* 1-16 tokens run the HBM-bound split-K decode kernel; 17-128 tokens the
  batch-decode kernel on weights of up to one round of workgroups at
  K = 4096 / 12288 (whole k ranges of weights in registers, the batch's token
  tiles split across workgroups), else deep-ring 64x64 / 64x128 prefill tiles
  (gate+up, the lm_head, down past 32 tokens); larger batches the LDS-tiled
  prefill kernels. ``jv_fp8_launch_shape`` reports the plan for a shape.

Everything is enqueued on ``torch.cuda.current_stream()`` without host
synchronisation; outputs and workspaces come from torch's caching allocator
(or the graph pool under capture).
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib
from .device import sm_count
from .fp8_weights import FP8, quantize_rows

# Decode batches (the role of SPLIT_K_MAX_ROWS, inference/fp8.py:20): up to
# four 16-token MFMA column tiles; the quantizer of h reads the SwiGLU
# epilogue's maxima at these sizes, and warm() covers them.
DECODE_MAX_ROWS = 64
# Longest row the single-pass quantizer (and so the packed code layout) covers.
QUANT_MAX_PACKED_COLS = 16384
BLOCK_K = 128
TILE_COUNTER_SLOTS = 1 << 16
# One row count per kernel variant: 1-4 decode token tiles, then prefill
# batches that select the 256x256, 256x128, 128x128, 64x128 and 64x64 tiles on
# large and small N (inference/fp8.py:32 plays the same role for Triton's JIT).
WARM_ROWS = (1, 16, 17, 32, 33, 48, 49, 64, 65, 256, 300, 2048)
LORA_RANKS = (16,)

TILE_COUNTERS: dict[tuple[torch.device, int], torch.Tensor] = {}


def split_for(N: int, K: int, sms: int) -> int:
    """K splits across workgroups of the decode kernel for an (N, K) weight on a
    device with ``sms`` compute units (``inference/fp8.py:105-109``'s role)."""
    return _lib.lib().jv_fp8_split_for(1, N, K, sms)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _stream_counters(device: torch.device) -> torch.Tensor:
    # Launches on different streams can overlap and must not share tile
    # counters (inference/fp8.py:126), so they are kept per (device, stream).
    key = (device, _stream(device))
    counters = TILE_COUNTERS.get(key)
    if counters is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("run an fp8 GEMM on this stream before capturing a CUDA graph on it, so that the stream's tile "
                               "counters exist outside the graph")
        counters = TILE_COUNTERS[key] = torch.zeros(TILE_COUNTER_SLOTS, dtype=torch.int32, device=device)
    return counters


def _tile_counters(device: torch.device, M: int, N: int, K: int) -> torch.Tensor | None:
    need = _lib.lib().jv_fp8_counters_needed(M, N, K, sm_count(device))
    if need <= 0:
        return None
    counters = _stream_counters(device)
    if need > counters.numel():
        raise ValueError(f"{need} tiles exceed the {counters.numel()} tile counters")
    return counters


def _rows_aligned(t: torch.Tensor, elem: int) -> bool:
    return t.stride(-1) == 1 and (t.stride(0) * elem) % 16 == 0 and t.data_ptr() % 16 == 0


def _check_weight(K: int, weight: torch.Tensor) -> None:
    if K == 0 or K % BLOCK_K or weight.dim() != 2 or weight.shape[1] != K:
        raise ValueError(f"the fp8 GEMM needs in_features divisible by {BLOCK_K} and equal to the weight's, got {K} for a weight "
                         f"of shape {tuple(weight.shape)}")


def _check_operands(dev: torch.device, N: int, weight: torch.Tensor, scale: torch.Tensor,
                    bias: torch.Tensor | None = None, *others: torch.Tensor | None) -> None:
    """Every operand on the activations' HIP device (a host or foreign-device
    pointer in a kernel argument is a GPU memory fault, not an error; the
    reference's Triton launcher rejects such tensors with a ValueError too),
    one-byte weight codes, and one scale (and bias) per output channel."""
    if dev.type != "cuda":
        raise ValueError(f"the fp8 GEMM runs on a HIP device; the activations are on {dev}")
    if weight.element_size() != 1:
        raise ValueError(f"weight codes must be float8_e4m3fn (or uint8), got {weight.dtype}")
    if scale.numel() != N:
        raise ValueError(f"scale needs one value per output channel ({N}), got {scale.numel()}")
    if bias is not None and bias.numel() != N:
        raise ValueError(f"bias needs one value per output channel ({N}), got {bias.numel()}")
    for t in (weight, scale, bias, *others):
        if t is not None and t.device != dev:
            raise ValueError(f"the fp8 GEMM's operands must all be on {dev}, got one on {t.device}")


def _weight_operand(weight: torch.Tensor, tiled: bool) -> tuple[torch.Tensor, int]:
    """Weight bytes and the C ABI's ldw: the row stride, or 0 for the tiled
    layout (``tile_weight``)."""
    w = weight.view(torch.uint8)
    if tiled:
        if weight.shape[0] % 16 or not w.is_contiguous():
            raise ValueError(f"tiled weights are a contiguous [N, K] buffer with N divisible by 16, got {tuple(weight.shape)}")
        return w, 0
    if not _rows_aligned(w, 1):
        w = w.contiguous()
    return w, w.stride(0)


def tileable(out_features: int, in_features: int) -> bool:
    """Shapes the tiled weight layout covers (whole 16-row tiles, 128-deep steps)."""
    return out_features % 16 == 0 and in_features % BLOCK_K == 0 and in_features > 0


def tile_weight(codes: torch.Tensor) -> torch.Tensor:
    """Row-major e4m3 codes [N, K] -> the same bytes in the tiled fragment
    layout (C ABI ``jv_fp8_tile_weight``; ``ldw = 0``), same shape and dtype.
    For 16-row tile t and 128-deep step s the 2 KB fragment holds two 1 KB
    halves (h = (k % 32) / 16) of 64 lanes x 16 bytes, lane = n % 16 +
    16 * ((k % 128) / 32): the order a decode wave loads, 1 KB contiguous per
    instruction. A layout change only (the reference's Metal path tiles its
    codes the same way for its kernel, ``inference/fp8_metal.py:23-24``)."""
    N, K = codes.shape
    if not tileable(N, K):
        raise ValueError(f"tiling needs N divisible by 16 and K by {BLOCK_K}, got {N} x {K}")
    src = codes.view(torch.uint8)
    if codes.device.type != "cuda":
        out = src.reshape(N // 16, 16, K // 128, 4, 2, 16).permute(0, 2, 4, 3, 1, 5).contiguous().view(N, K)
        return out.view(codes.dtype)
    if not _rows_aligned(src, 1):
        src = src.contiguous()
    out = torch.empty(N, K, dtype=torch.uint8, device=codes.device)
    with torch.cuda.device(codes.device):
        _lib.check(_lib.lib().jv_fp8_tile_weight(src.data_ptr(), src.stride(0), N, K, out.data_ptr(), _stream(codes.device)))
    return out.view(codes.dtype)


def untile_weight(tiled: torch.Tensor) -> torch.Tensor:
    """Inverse of ``tile_weight``: row-major codes [N, K]."""
    N, K = tiled.shape
    if not tileable(N, K):
        raise ValueError(f"untiling needs N divisible by 16 and K by {BLOCK_K}, got {N} x {K}")
    src = tiled.view(torch.uint8).contiguous()
    if tiled.device.type != "cuda":
        out = src.view(N // 16, K // 128, 2, 4, 16, 16).permute(0, 4, 1, 3, 2, 5).contiguous().view(N, K)
        return out.view(tiled.dtype)
    out = torch.empty(N, K, dtype=torch.uint8, device=tiled.device)
    with torch.cuda.device(tiled.device):
        _lib.check(_lib.lib().jv_fp8_untile_weight(src.data_ptr(), N, K, out.data_ptr(), K, _stream(tiled.device)))
    return out.view(tiled.dtype)


def _tile_into(codes: torch.Tensor, out: torch.Tensor) -> None:
    """``tile_weight`` written into an existing buffer (same device and size)."""
    N, K = codes.shape
    src = codes.view(torch.uint8)
    if codes.device.type != "cuda":
        out.copy_(tile_weight(codes).view(torch.uint8))
        return
    if not _rows_aligned(src, 1):
        src = src.contiguous()
    with torch.cuda.device(codes.device):
        _lib.check(_lib.lib().jv_fp8_tile_weight(src.data_ptr(), src.stride(0), N, K, out.data_ptr(), _stream(codes.device)))


def _check_lora(lora, K: int, N: int):
    if lora is None:
        return None, None, 0, 0.0
    a, b, scaling = lora
    r = a.shape[0]
    if r not in LORA_RANKS or a.shape != (r, K) or b.shape != (N, r):
        raise ValueError(f"LoRA factors must be A [r,{K}] and B [{N},r] with r in {LORA_RANKS}, got {tuple(a.shape)} and "
                         f"{tuple(b.shape)}")
    return a.to(torch.bfloat16).contiguous(), b.to(torch.bfloat16).contiguous(), r, float(scaling)


def fp8_matmul(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, *, bias: torch.Tensor | None = None,
               lora: tuple[torch.Tensor, torch.Tensor, float] | None = None, tiled: bool = False) -> torch.Tensor:
    """``y = bf16(quant(x) @ weight^T * scale)`` (``inference/fp8.py:112-148``).

    x: bf16 [M,K] with unit column stride (any 16-byte aligned row stride);
    weight: float8_e4m3fn [N,K]; scale: float32 [N]. Returns a new bf16 [M,N]
    on x's device; inputs are never written. ``bias`` (bf16 [N]) and ``lora``
    (``(A [r,K], B [N,r], scaling)``) are folded into the same epilogue.
    ``tiled``: ``weight`` holds the codes in the ``tile_weight`` layout.
    """
    M, K = x.shape
    N = weight.shape[0]
    _check_weight(K, weight)
    a, b, rank, scaling = _check_lora(lora, K, N)
    dev = x.device
    _check_operands(dev, N, weight, scale, bias, a, b)
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    if not _rows_aligned(x, 2):
        x = x.contiguous()
    w, ldw = _weight_operand(weight, tiled)
    y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    if M == 0:
        return y
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    scale = scale.to(torch.float32).contiguous()
    L = _lib.lib()
    with torch.cuda.device(dev):
        counters = _tile_counters(dev, M, N, K)
        ws_bytes = L.jv_fp8_linear_workspace_bytes(M, N, K, rank)
        if ws_bytes < 0:
            _lib.check(_lib.JV_ERR_HIP)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        _lib.check(L.jv_fp8_linear(x.data_ptr(), x.stride(0), w.data_ptr(), ldw, scale.data_ptr(),
                                   bias.data_ptr() if bias is not None else None, a.data_ptr() if rank else None,
                                   b.data_ptr() if rank else None, rank, scaling, y.data_ptr(), N, M, N, K, ws.data_ptr(),
                                   ws_bytes, _lib.counters_ptr(counters), counters.numel() if counters is not None else 0,
                                   _stream(dev)))
    return y


def fp8_matmul_w8a16(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, *,
                     bias: torch.Tensor | None = None, tiled: bool = False) -> torch.Tensor:
    """W8A16 parity mode: the reference's own arithmetic,
    ``((x.float() @ weight.float().t()) * scale).to(bf16)`` (``model/metal_test.py:213``,
    ``inference/fp8.py:62-99``), then ``+ bias`` in bf16 (``inference/fp8.py:183-184``).

    The bf16 activations are not quantized; the e4m3 weights are widened to
    bf16 (exactly) inside the kernel. Same arguments and errors as
    ``fp8_matmul`` without LoRA.
    """
    M, K = x.shape
    N = weight.shape[0]
    _check_weight(K, weight)
    dev = x.device
    _check_operands(dev, N, weight, scale, bias)
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    if not _rows_aligned(x, 2):
        x = x.contiguous()
    w, ldw = _weight_operand(weight, tiled)
    y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    if M == 0:
        return y
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    scale = scale.to(torch.float32).contiguous()
    L = _lib.lib()
    with torch.cuda.device(dev):
        ws_bytes = L.jv_w8a16_workspace_bytes(M, N, K)
        if ws_bytes < 0:
            _lib.check(_lib.JV_ERR_HIP)
        # a workspace means a K split (decode or prefill kernel), which counts
        # its tiles in; the library checks that they fit the counters
        counters = _stream_counters(dev) if ws_bytes > 0 else None
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        _lib.check(L.jv_w8a16_linear(x.data_ptr(), x.stride(0), w.data_ptr(), ldw, scale.data_ptr(),
                                     bias.data_ptr() if bias is not None else None, y.data_ptr(), N, M, N, K,
                                     ws.data_ptr(), ws_bytes, _lib.counters_ptr(counters),
                                     counters.numel() if counters is not None else 0, _stream(dev)))
    return y


def packed_codes_bytes(rows: int, cols: int) -> int:
    """Bytes of ``rows x cols`` activation codes in the GEMMs' packed fragment
    order (cols a multiple of 128; rows padded to a multiple of 16)."""
    n = _lib.lib().jv_fp8_packed_codes_bytes(rows, cols)
    if n < 0:
        raise ValueError(f"the packed layout takes a multiple of {BLOCK_K} columns, got {rows} x {cols}")
    return n


def fp8_matmul_quantized(xq: torch.Tensor, x_scale: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, *,
                         bias: torch.Tensor | None = None, lora_t: torch.Tensor | None = None,
                         lora_b: torch.Tensor | None = None, lora_scaling: float = 0.0,
                         packed_rows: int | None = None, tiled: bool = False) -> torch.Tensor:
    """The GEMM alone on activations already quantized per token (codes
    float8_e4m3fn/uint8 [M,K] and scales float32 [M]), e.g. by
    ``swiglu_quantize``. ``lora_t`` is ``x A^T`` (float32 [M,r]).
    ``packed_rows=M``: ``xq`` is a flat uint8 buffer of M token rows in the
    packed fragment order (``swiglu_quantize(..., packed=True)``). ``tiled``:
    ``weight`` is in the ``tile_weight`` layout."""
    N = weight.shape[0]
    if packed_rows is not None:
        M, K = packed_rows, weight.shape[1]
        if xq.dim() != 1 or xq.numel() < packed_codes_bytes(M, K):
            raise ValueError(f"packed codes for {M} x {K} need {packed_codes_bytes(M, K)} bytes")
    else:
        M, K = xq.shape
    _check_weight(K, weight)
    rank = 0 if lora_t is None else lora_t.shape[1]
    if rank and (rank not in LORA_RANKS or lora_b is None or lora_b.shape != (N, rank) or lora_t.shape != (M, rank)):
        raise ValueError(f"lora_t [M, r] needs lora_b [N, r] with r in {LORA_RANKS}")
    dev = xq.device
    if xq.element_size() != 1:
        raise ValueError(f"activation codes must be float8_e4m3fn (or uint8), got {xq.dtype}")
    if x_scale.numel() != M:
        raise ValueError(f"x_scale needs one value per token row ({M}), got {x_scale.numel()}")
    _check_operands(dev, N, weight, scale, bias, x_scale, lora_t, lora_b)
    xq = xq.view(torch.uint8)
    if packed_rows is None and not _rows_aligned(xq, 1):
        xq = xq.contiguous()
    w, ldw = _weight_operand(weight, tiled)
    y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    if M == 0:
        return y
    bias = bias.to(torch.bfloat16).contiguous() if bias is not None else None
    if rank:
        lora_t = lora_t.to(torch.float32).contiguous()
        lora_b = lora_b.to(torch.bfloat16).contiguous()
    L = _lib.lib()
    with torch.cuda.device(dev):
        counters = _tile_counters(dev, M, N, K)
        ws_bytes = L.jv_fp8_gemm_workspace_bytes(M, N, K)
        if ws_bytes < 0:
            _lib.check(_lib.JV_ERR_HIP)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        _lib.check(L.jv_fp8_gemm(xq.data_ptr(), 0 if packed_rows is not None else xq.stride(0),
                                 x_scale.to(torch.float32).contiguous().data_ptr(), w.data_ptr(),
                                 ldw, scale.to(torch.float32).contiguous().data_ptr(),
                                 bias.data_ptr() if bias is not None else None, lora_t.data_ptr() if rank else None,
                                 lora_b.data_ptr() if rank else None, rank, float(lora_scaling), y.data_ptr(), N, M, N, K,
                                 ws.data_ptr(), ws_bytes, _lib.counters_ptr(counters),
                                 counters.numel() if counters is not None else 0, _stream(dev)))
    return y


def swiglu_quantize(gate: torch.Tensor, up: torch.Tensor, *, lora_a: torch.Tensor | None = None,
                    return_h: bool = False, packed: bool = False) -> tuple[torch.Tensor, ...]:
    """``h = F.silu(gate) * up`` on bf16 (``model/model.py:583``) fused with the
    down projection's per-token quantization. Returns ``(codes, scales)``, plus
    ``t = h A^T`` (float32 [M,r]) when ``lora_a`` is given and ``h`` (bf16) when
    ``return_h``. ``packed``: codes come as a flat uint8 buffer in the GEMMs'
    fragment order, for ``fp8_matmul_quantized(..., packed_rows=M)``."""
    M, I = gate.shape
    if up.shape != gate.shape:
        raise ValueError(f"gate {tuple(gate.shape)} and up {tuple(up.shape)} differ")
    dev = gate.device
    if dev.type != "cuda" or up.device != dev or (lora_a is not None and lora_a.device != dev):
        raise ValueError(f"swiglu_quantize needs gate, up and lora_a on one HIP device, got {dev} and {up.device}")
    gate, up = gate.to(torch.bfloat16), up.to(torch.bfloat16)
    if not _rows_aligned(gate, 2):
        gate = gate.contiguous()
    if not _rows_aligned(up, 2):
        up = up.contiguous()
    codes = torch.empty(packed_codes_bytes(M, I) if packed else (M, I), dtype=torch.uint8, device=dev)
    scales = torch.empty(M, dtype=torch.float32, device=dev)
    h = torch.empty(M, I, dtype=torch.bfloat16, device=dev) if return_h else None
    rank = 0
    t = None
    if lora_a is not None:
        rank = lora_a.shape[0]
        if rank not in LORA_RANKS or lora_a.shape[1] != I:
            raise ValueError(f"lora_a must be [r,{I}] with r in {LORA_RANKS}, got {tuple(lora_a.shape)}")
        lora_a = lora_a.to(torch.bfloat16).contiguous()
        t = torch.empty(M, rank, dtype=torch.float32, device=dev)
    if M:
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().jv_fp8_swiglu_quantize(gate.data_ptr(), gate.stride(0), up.data_ptr(), up.stride(0), M, I,
                                                         codes.data_ptr(), 0 if packed else I, scales.data_ptr(),
                                                         h.data_ptr() if h is not None else None, I,
                                                         lora_a.data_ptr() if rank else None, rank,
                                                         t.data_ptr() if rank else None, _stream(dev)))
    out: tuple[torch.Tensor, ...] = (codes if packed else codes.view(FP8), scales)
    if rank:
        out += (t,)
    if return_h:
        out += (h,)
    return out


def gate_up_swiglu(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, *, bias: torch.Tensor | None = None,
                   lora: tuple[torch.Tensor, torch.Tensor, float] | None = None, tiled: bool = False,
                   amax: bool = False) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """``F.silu(gate(x)) * up(x)`` (``model/model.py:583``) with both
    projections as one FP8 GEMM whose epilogue applies SwiGLU (C ABI
    ``jv_fp8_linear_swiglu``): ``weight`` [2I, K] holds the gate rows, then the
    up rows (the fused gate+up linear), ``scale``/``bias`` [2I], LoRA B
    [2I, r]. Returns h bf16 [M, I], bitwise ``swiglu(fp8_matmul(x, ...))`` of
    the two halves; with ``amax`` also the per-token largest |h| over each
    16 channels (uint16 bf16 magnitude patterns [M, I/16]). h is the
    reference's ``F.silu(gate) * up`` branch on bf16 (silu rounded, then the
    product); its fla branch (``_fla_swiglu``, one rounding) is not matched and
    parity with it is unpinned."""
    M, K = x.shape
    N = weight.shape[0]
    _check_weight(K, weight)
    if N % 32:
        raise ValueError(f"the fused gate+up weight needs 2I rows with I divisible by 16, got {N}")
    I = N // 2
    a, b, rank, scaling = _check_lora(lora, K, N)
    dev = x.device
    _check_operands(dev, N, weight, scale, bias, a, b)
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    if not _rows_aligned(x, 2):
        x = x.contiguous()
    w, ldw = _weight_operand(weight, tiled)
    h = torch.empty(M, I, device=dev, dtype=torch.bfloat16)
    parts = torch.empty(M, I // 16, device=dev, dtype=torch.int16) if amax else None
    if M:
        bias = bias.to(torch.bfloat16).contiguous() if bias is not None else None
        scale = scale.to(torch.float32).contiguous()
        L = _lib.lib()
        with torch.cuda.device(dev):
            counters = _tile_counters(dev, M, N, K)
            ws_bytes = L.jv_fp8_linear_workspace_bytes(M, N, K, rank)
            if ws_bytes < 0:
                _lib.check(_lib.JV_ERR_HIP)
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
            _lib.check(L.jv_fp8_linear_swiglu(x.data_ptr(), x.stride(0), w.data_ptr(), ldw, scale.data_ptr(),
                                              bias.data_ptr() if bias is not None else None, a.data_ptr() if rank else None,
                                              b.data_ptr() if rank else None, rank, scaling, h.data_ptr(), I,
                                              parts.data_ptr() if parts is not None else None, M, I, K, ws.data_ptr(),
                                              ws_bytes, _lib.counters_ptr(counters),
                                              counters.numel() if counters is not None else 0, _stream(dev)))
    return (h, parts) if amax else h


def quantize_swiglu_output(h: torch.Tensor, amax: torch.Tensor | None = None, *, lora_a: torch.Tensor | None = None,
                           packed: bool = True) -> tuple[torch.Tensor, ...]:
    """The down projection's per-token quantization of h (``quantize_rows``
    semantics; C ABI ``jv_fp8_quantize_swiglu_output``). Returns
    ``(codes, scales)``, plus ``t = h A^T`` (float32 [M,r]) with ``lora_a``.
    ``packed``: codes as a flat uint8 buffer in the GEMMs' fragment order (for
    ``fp8_matmul_quantized(..., packed_rows=M)``); ``amax``: the maxima
    ``gate_up_swiglu(..., amax=True)`` returned with this h, or None. Decode
    batches (M <= 128) in the packed layout without LoRA read each row's
    maximum from them, so a row splits over several workgroups; elsewhere
    they are not read (each row's maximum comes from h in the pass that
    encodes it). The result is the same bits either way."""
    M, I = h.shape
    dev = h.device
    if dev.type != "cuda" or h.dtype != torch.bfloat16:
        raise ValueError(f"h must be bf16 on a HIP device, got {h.dtype} on {dev}")
    if not _rows_aligned(h, 2):
        h = h.contiguous()
    codes = torch.empty(packed_codes_bytes(M, I) if packed else (M, I), dtype=torch.uint8, device=dev)
    scales = torch.empty(M, dtype=torch.float32, device=dev)
    rank, t = 0, None
    if lora_a is not None:
        rank = lora_a.shape[0]
        if rank not in LORA_RANKS or lora_a.shape[1] != I:
            raise ValueError(f"lora_a must be [r,{I}] with r in {LORA_RANKS}, got {tuple(lora_a.shape)}")
        lora_a = lora_a.to(torch.bfloat16).contiguous()
        t = torch.empty(M, rank, dtype=torch.float32, device=dev)
    if amax is not None and (amax.shape != (M, I // 16) or amax.element_size() != 2 or not amax.is_contiguous()):
        raise ValueError(f"amax must be a contiguous 16-bit [{M}, {I // 16}] tensor")
    if M:
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().jv_fp8_quantize_swiglu_output(h.data_ptr(), h.stride(0),
                                                                amax.data_ptr() if amax is not None else None, M, I,
                                                                codes.data_ptr(), 0 if packed else I, scales.data_ptr(),
                                                                lora_a.data_ptr() if rank else None, rank,
                                                                t.data_ptr() if rank else None, _stream(dev)))
    out: tuple[torch.Tensor, ...] = (codes if packed else codes.view(FP8), scales)
    return out + (t,) if rank else out


class FP8Linear(nn.Module):
    """``inference/fp8.py:151-185``: buffers ``weight`` (float8_e4m3fn [N,K],
    row-major, as the reference keeps it) and ``scale`` (float32 [N]),
    optional bf16 ``bias``. ``set_lora`` attaches a LoRA adapter
    (``model/lora.py:122-133``) that the GEMM epilogue adds.

    When the shape allows (``tileable``: N % 16 == 0, K % 128 == 0) and
    ``TILED_COPY`` is set, the kernels read a second copy of the codes,
    ``tiled_codes`` (uint8 [N,K] in the ``tile_weight`` layout), the way the
    reference's Metal module keeps ``tiled_codes`` for its kernel
    (``inference/fp8_metal.py:17``): a decode wave then loads one contiguous
    1 KB per instruction. The copy is not part of the state dict; it is
    rebuilt from ``weight`` whenever ``weight`` changed (an in-place write, a
    new tensor, ``load_state_dict``), so ``weight`` stays the one source of
    truth. It doubles the codes' HBM footprint; with ``TILED_COPY = False``
    the kernels read ``weight`` itself (``tiled`` is then False).

    ``activations`` picks the arithmetic: ``"fp8"`` (default) quantizes the
    activations per token and runs the FP8 x FP8 GEMM; ``"bf16"`` is the
    W8A16 parity mode (``fp8_matmul_w8a16``), the reference's own math, for
    checking a model against the reference's outputs (no LoRA in that mode).
    """

    ACTIVATIONS = ("fp8", "bf16")
    TILED_COPY = True

    def __init__(self, in_features: int, out_features: int, bias: bool = False, device: torch.device | str | None = None):
        super().__init__()
        self.register_buffer("weight", torch.empty(out_features, in_features, dtype=FP8, device=device))
        self.register_buffer("scale", torch.empty(out_features, dtype=torch.float32, device=device))
        self.bias = nn.Parameter(torch.empty(out_features, dtype=torch.bfloat16, device=device), requires_grad=False) if bias else None
        self.in_features, self.out_features = in_features, out_features
        self.tiled = self.TILED_COPY and tileable(out_features, in_features)
        self.register_buffer("tiled_codes", torch.empty(out_features, in_features, dtype=torch.uint8, device=device)
                             if self.tiled else None, persistent=False)
        # (address, version) of the weight the tiled copy was made from
        self._tiled_from: tuple[int, int] | None = None
        self.lora: tuple[torch.Tensor, torch.Tensor, float] | None = None
        self.activations = "fp8"
        self.register_load_state_dict_post_hook(FP8Linear._retile_loaded)

    @staticmethod
    def _retile_loaded(module: "FP8Linear", incompatible_keys) -> None:
        if module.weight.device.type == "cuda":
            module.kernel_weight()

    def _weight_key(self) -> tuple[int, int]:
        # Inference tensors (made under torch.inference_mode) keep no version
        # counter: their key is the address alone, and in-place writes to them
        # need retile().
        w = self.weight
        return w.data_ptr(), (-1 if torch.is_inference(w) else w._version)

    def kernel_weight(self) -> tuple[torch.Tensor, bool]:
        """The codes the kernels read and whether they are tiled: the tiled
        copy, rebuilt first if ``weight`` changed since it was made, or
        ``weight`` itself. A change is a new ``weight`` tensor or an in-place
        write that bumps its version counter (``copy_``, ``load_state_dict``);
        writes that bypass the counter (through ``weight.data``, or into an
        inference tensor) must be followed by ``retile()``."""
        if not self.tiled:
            return self.weight, False
        key = self._weight_key()
        if self._tiled_from != key:
            _tile_into(self.weight, self.tiled_codes)
            self._tiled_from = key
        return self.tiled_codes, True

    @torch.no_grad()
    def retile(self) -> None:
        """Rebuild the tiled copy from ``weight`` now (after writes the
        version counter does not see)."""
        if self.tiled:
            self._tiled_from = None
            self.kernel_weight()

    def codes(self) -> torch.Tensor:
        """The e4m3 codes, row-major [N, K] (``weight``)."""
        return self.weight

    def set_activations(self, mode: str) -> None:
        """``"fp8"`` (per-token e4m3 activations) or ``"bf16"`` (W8A16 parity mode)."""
        if mode not in self.ACTIVATIONS:
            raise ValueError(f"activations must be one of {self.ACTIVATIONS}, got {mode!r}")
        if mode == "bf16" and self.lora is not None:
            raise ValueError("the W8A16 parity mode has no LoRA epilogue")
        self.activations = mode

    @torch.no_grad()
    def load_codes(self, codes: torch.Tensor, scale: torch.Tensor) -> None:
        self.weight.copy_(codes)
        self.scale.copy_(scale)
        if self.weight.device.type == "cuda":
            self.kernel_weight()

    @torch.no_grad()
    def load_weight(self, weight: torch.Tensor) -> None:
        self.load_codes(*quantize_rows(weight.to(self.weight.device)))

    def set_lora(self, a: torch.Tensor, b: torch.Tensor, scaling: float) -> None:
        """Attach ``y += scaling * (x A^T) B^T`` (A [r,in], B [out,r], bf16)."""
        _check_lora((a, b, scaling), self.in_features, self.out_features)
        if self.activations == "bf16":
            raise ValueError("the W8A16 parity mode has no LoRA epilogue")
        self.lora = (a.to(torch.bfloat16).contiguous(), b.to(torch.bfloat16).contiguous(), float(scaling))

    @classmethod
    def concatenated(cls, parts: list["FP8Linear"]) -> "FP8Linear":
        """One linear over the parts' output rows (``inference/fp8.py:168-175``);
        the parts' ``weight`` and ``scale`` become views of the merged buffers.
        Tiles are whole 16-row groups, so the parts' tiled copies concatenate
        as they are and become views of the merged copy too; if any part
        cannot tile, the merged module and every part read row-major codes."""
        sizes = [p.out_features for p in parts]
        merged = cls(parts[0].in_features, sum(sizes), device="meta")
        tiled = merged.tiled and all(p.tiled for p in parts)
        copies = [p.kernel_weight()[0] for p in parts] if tiled else None
        merged.weight, merged.scale = torch.cat([p.weight for p in parts]), torch.cat([p.scale for p in parts])
        merged.tiled = tiled
        merged.tiled_codes = torch.cat(copies) if tiled else None
        merged._tiled_from = merged._weight_key() if tiled else None
        tiles = merged.tiled_codes.split(sizes) if tiled else [None] * len(parts)
        for p, weight, scale, t in zip(parts, merged.weight.split(sizes), merged.scale.split(sizes), tiles):
            p.weight, p.scale, p.tiled, p.tiled_codes = weight, scale, tiled, t
            p._tiled_from = p._weight_key() if tiled else None
        return merged

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).to(torch.bfloat16)
        if x2.stride(-1) != 1:
            x2 = x2.contiguous()
        w, tiled = self.kernel_weight()
        if self.activations == "bf16":
            y = fp8_matmul_w8a16(x2, w, self.scale, bias=self.bias, tiled=tiled)
        else:
            y = fp8_matmul(x2, w, self.scale, bias=self.bias, lora=self.lora, tiled=tiled)
        return y.view(*shape[:-1], self.out_features)


class FP8SwiGLU(nn.Module):
    """``SwiGLU`` (``model/model.py:574-584``) over FP8 projections: the gate
    and up projections as one FP8 GEMM (``gate_up``: gate rows first, then up
    rows) whose epilogue applies SwiGLU and writes h, the down projection's
    quantization of h, then the down GEMM. The gate+up output never reaches
    memory; the result is bitwise that of the separate steps.

    h is ``F.silu(gate) * up`` on bf16 tensors (silu rounded to bf16, then the
    product rounded), the reference's own expression where its fused
    ``_fla_swiglu`` is not in use (``model/model.py:583``). fla's kernel rounds
    once; flash-linear-attention is not installed here and no fixture holds its
    outputs, so parity with that branch is unpinned.

    Built with ``parts`` (``from_mlp``/``fuse_swiglus``), the module keeps the
    reference's attribute and state-dict names: ``gate_proj``, ``up_proj`` and
    ``down_proj`` are its submodules (the first two views of the merged
    ``gate_up``, as ``FP8Linear.concatenated`` makes them), and ``gate_up`` is
    held outside the module tree, as the engine's merged projections are
    (``inference/engine.py:154-165``). Build it after the weights are on their
    device: moving the module afterwards would break the views."""

    def __init__(self, gate_up: FP8Linear, down: FP8Linear, parts: tuple[FP8Linear, FP8Linear] | None = None):
        super().__init__()
        if gate_up.out_features != 2 * down.in_features:
            raise ValueError("gate_up must have twice down's in_features outputs")
        if parts is None:
            self.gate_up, self.down = gate_up, down
        else:
            self.gate_proj, self.up_proj, self.down_proj = parts[0], parts[1], down
            object.__setattr__(self, "gate_up", gate_up)
            object.__setattr__(self, "down", down)

    @classmethod
    def from_mlp(cls, mlp: nn.Module) -> "FP8SwiGLU":
        """The fused form of a module shaped like the reference's ``SwiGLU``
        (``gate_proj``, ``up_proj``, ``down_proj`` as ``FP8Linear``s, e.g. after
        ``replace_linears``): gate and up merged with ``FP8Linear.concatenated``
        (gate rows, then up rows), so both become views of the merged codes."""
        gate, up, down = mlp.gate_proj, mlp.up_proj, mlp.down_proj
        if not all(isinstance(m, FP8Linear) for m in (gate, up, down)):
            raise ValueError("gate_proj, up_proj and down_proj must be FP8Linear modules")
        if gate.in_features != up.in_features or gate.out_features != up.out_features or \
                gate.out_features != down.in_features:
            raise ValueError(f"gate {gate.out_features}x{gate.in_features}, up {up.out_features}x{up.in_features} and "
                             f"down {down.out_features}x{down.in_features} do not form a SwiGLU block")
        if gate.lora is not None or up.lora is not None:
            raise ValueError("gate_proj and up_proj carry their own LoRA adapters; the merged gate+up GEMM takes one")
        if (gate.bias is None) != (up.bias is None):
            raise ValueError("gate_proj and up_proj must both have a bias or neither")
        merged = FP8Linear.concatenated([gate, up])
        if gate.bias is not None:
            # One bias buffer as for the codes: the parts' biases become views of it.
            merged.bias = nn.Parameter(torch.cat([gate.bias, up.bias]), requires_grad=False)
            gate.bias, up.bias = (nn.Parameter(b, requires_grad=False) for b in merged.bias.split(gate.out_features))
        merged.activations = gate.activations
        return cls(merged, down, parts=(gate, up))

    def set_activations(self, mode: str) -> None:
        """``FP8Linear.set_activations`` on every projection of the block."""
        for m in {id(m): m for m in (self.gate_up, self.down, *self.children())}.values():
            m.set_activations(mode)

    def fused(self) -> bool:
        """Whether the gate+up GEMM applies SwiGLU in its epilogue (the
        intermediate size a multiple of 16, the hidden size at most 16384)."""
        return self.down.in_features % 16 == 0 and self.gate_up.in_features <= QUANT_MAX_PACKED_COLS

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        M, inter = x2.shape[0], self.down.in_features
        if self.down.activations == "bf16":
            # W8A16 parity mode: h = silu(gate) * up in bf16 feeds the down GEMM as is.
            gu = self.gate_up(x2)
            h = swiglu_quantize(gu[:, :inter], gu[:, inter:], return_h=True)[-1]
            w, tiled = self.down.kernel_weight()
            y = fp8_matmul_w8a16(h, w, self.down.scale, bias=self.down.bias, tiled=tiled)
            return y.view(*shape[:-1], self.down.out_features)
        lora_a = self.down.lora[0] if self.down.lora is not None else None
        # The down GEMM reads its codes fastest in fragment order (both the
        # decode and the prefill kernels); the quantizers write them so for
        # rows up to 16384 channels.
        packed = M > 0 and inter % BLOCK_K == 0 and inter <= QUANT_MAX_PACKED_COLS
        if self.gate_up.activations == "fp8" and self.fused():
            w, tiled = self.gate_up.kernel_weight()
            # Decode batches (up to 128 tokens) quantize h from the
            # epilogue's maxima: 1.4 / 1.1 us less for the quantizer at 96 /
            # 128 tokens against 0.6 / 0.7 more in the GEMM's epilogue.
            amax = packed and lora_a is None and M <= 2 * DECODE_MAX_ROWS
            res = gate_up_swiglu(x2.to(torch.bfloat16), w, self.gate_up.scale, bias=self.gate_up.bias,
                                 lora=self.gate_up.lora, tiled=tiled, amax=amax)
            h, parts = res if amax else (res, None)
            out = quantize_swiglu_output(h, parts, lora_a=lora_a, packed=packed)
        else:
            gu = self.gate_up(x2)
            out = swiglu_quantize(gu[:, :inter], gu[:, inter:], lora_a=lora_a, packed=packed)
        lora_t = out[2] if lora_a is not None else None
        w, tiled = self.down.kernel_weight()
        y = fp8_matmul_quantized(out[0], out[1], w, self.down.scale, bias=self.down.bias, lora_t=lora_t,
                                 lora_b=self.down.lora[1] if lora_a is not None else None,
                                 lora_scaling=self.down.lora[2] if lora_a is not None else 0.0,
                                 packed_rows=M if packed else None, tiled=tiled)
        return y.view(*shape[:-1], self.down.out_features)


def _swiglu_block(m: nn.Module) -> bool:
    return not isinstance(m, FP8SwiGLU) and all(isinstance(getattr(m, name, None), FP8Linear)
                                                for name in ("gate_proj", "up_proj", "down_proj"))


def fuse_swiglus(module: nn.Module) -> int:
    """Swap every SwiGLU block under ``module`` (a child with ``FP8Linear``
    ``gate_proj``, ``up_proj`` and ``down_proj``, the reference's ``SwiGLU``
    after ``replace_linears``, ``model/model.py:574-584``) for
    ``FP8SwiGLU.from_mlp`` of it, in place, the way the engine merges
    projections that read the same input (``inference/engine.py:154-165``).
    Blocks whose gate or up carries its own LoRA adapter stay as they are.
    Returns the number of blocks fused."""
    n = 0
    for name, child in module.named_children():
        if _swiglu_block(child):
            if child.gate_proj.lora is None and child.up_proj.lora is None:
                setattr(module, name, FP8SwiGLU.from_mlp(child))
                n += 1
        else:
            n += fuse_swiglus(child)
    return n


def load_view(model: str, drafter: str, block: int, device: torch.device):
    """``inference/fp8.py:188-191``: the reference's FP8 loader with this
    module's FP8Linear, then ``warm``. Needs the jeeves tree on ``sys.path``
    (the loader, model and drafter are the caller's code)."""
    try:
        from inference.fp8_checkpoint import load_fp8_view
    except ImportError as e:
        raise ImportError("load_view builds the jeeves model with inference.fp8_checkpoint.load_fp8_view; run it from the "
                          "jeeves tree") from e
    view, head, encoder = load_fp8_view(model, drafter, block, device, FP8Linear)
    warm(view)
    return view, head, encoder


@torch.no_grad()
def warm(module: nn.Module) -> int:
    """``inference/fp8.py:194-203``: run every distinct (N, K) at ``WARM_ROWS``
    so each kernel variant has loaded and each stream's tile counters exist
    before graph capture."""
    seen = set()
    for m in module.modules():
        if isinstance(m, FP8Linear) and (m.out_features, m.in_features) not in seen:
            seen.add((m.out_features, m.in_features))
            w = m.weight
            for rows in WARM_ROWS:
                m(torch.zeros(rows, m.in_features, device=w.device, dtype=torch.bfloat16))
    return len(seen)
