"""Drop-in for ``inference/fp8_weights.py``: the FP8 constants, the per-row
quantizer, the quantizability rule and module replacement.

``quantize_rows`` computes the reference's arithmetic
(``inference/fp8_weights.py:16-19``) with the gfx950 quantizer kernel
(``jeeves_amd/csrc/quant.hip``) and returns the same codes and scales bit for
bit. It runs on the HIP device (tensors on the CPU are moved to the current
HIP device for the kernel and the results moved back) and raises when there
is none. The exporter's ``quantize_row_blocks_on_cpu`` keeps the reference's
CPU-in, CPU-out contract: it uses the HIP quantizer when a device is present
and otherwise the library's host quantizer
(``jeeves_amd/csrc/quant_host.hip``, the same bits), so an FP8 checkpoint can
be exported on a machine without a GPU, as the reference's exporter is.
"""

from __future__ import annotations

from typing import Callable, Iterator

import torch
import torch.nn as nn

from . import _lib

FP8 = torch.float8_e4m3fn
FP8_MAX = torch.finfo(FP8).max
# inference/fp8_weights.py:9-10: the scale multiplies by the float32 reciprocal.
FP8_MAX_RECIPROCAL = float(torch.tensor(1 / FP8_MAX, dtype=torch.float32))
SCALE_SUFFIX = "_scale"
QUANTIZE_BLOCK_ROWS = 16384


def _hip_device(t: torch.Tensor) -> torch.device:
    if t.device.type == "cuda":
        return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("quantize_rows runs on the HIP device and none is available")
    return torch.device("cuda", torch.cuda.current_device())


def quantize_rows_host(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """quantize_rows of a CPU tensor on the host CPU, with the library's host
    quantizer (``jv_fp8_quantize_rows_host``): the same codes and scales as the
    HIP quantizer, on torch's intra-op thread count."""
    w = weight.detach()
    if w.dim() != 2:
        raise ValueError(f"quantize_rows takes a 2-D tensor, got shape {tuple(w.shape)}")
    if w.shape[0] and not w.shape[1]:
        raise ValueError("quantize_rows needs at least one column")
    src = w.cpu().float().contiguous()
    rows, cols = src.shape
    codes = torch.empty(rows, cols, dtype=torch.uint8)
    scale = torch.empty(rows, dtype=torch.float32)
    if rows:
        _lib.check(_lib.lib().jv_fp8_quantize_rows_host(src.data_ptr(), cols, rows, cols, codes.data_ptr(), cols,
                                                         scale.data_ptr(), torch.get_num_threads()))
    return codes.view(FP8), scale


def quantize_rows(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row e4m3fn quantization (``inference/fp8_weights.py:16-19``).

    Returns ``(codes float8_e4m3fn [R,C], scale float32 [R])`` on the input's
    device: ``scale = max(amax_row(|w|), 1e-12) * FP8_MAX_RECIPROCAL`` and
    ``codes = e4m3fn(w / scale)``.
    """
    w = weight.detach()
    if w.dim() != 2:
        raise ValueError(f"quantize_rows takes a 2-D tensor, got shape {tuple(w.shape)}")
    home = w.device
    dev = _hip_device(w)
    rows, cols = w.shape
    if rows and not cols:
        # No columns: amax over an empty row is undefined in the reference too.
        raise ValueError("quantize_rows needs at least one column")
    codes = torch.empty(rows, cols, dtype=torch.uint8, device=dev)
    scale = torch.empty(rows, dtype=torch.float32, device=dev)
    if rows and cols:
        with torch.cuda.device(dev):
            stream = torch.cuda.current_stream(dev).cuda_stream
            if w.dtype == torch.bfloat16 and cols % 8 == 0:
                src = w.to(dev)
                if src.stride(-1) != 1 or (src.stride(0) * 2) % 16 or src.data_ptr() % 16:
                    src = src.contiguous()
                _lib.check(_lib.lib().jv_fp8_quantize_rows_bf16(src.data_ptr(), src.stride(0), rows, cols, codes.data_ptr(),
                                                                 cols, scale.data_ptr(), stream))
            else:
                # w.float() as the reference does; zero padding to a multiple of 4
                # columns changes no row maximum and is sliced off the codes.
                padded = (cols + 3) // 4 * 4
                src = torch.zeros(rows, padded, dtype=torch.float32, device=dev)
                src[:, :cols] = w.to(dev).float()
                out = codes if padded == cols else torch.empty(rows, padded, dtype=torch.uint8, device=dev)
                _lib.check(_lib.lib().jv_fp8_quantize_rows_f32(src.data_ptr(), padded, rows, padded, out.data_ptr(), padded,
                                                                scale.data_ptr(), stream))
                if out is not codes:
                    codes.copy_(out[:, :cols])
    codes = codes.view(FP8)
    if home != dev:
        codes, scale = codes.to(home), scale.to(home)
    return codes.contiguous(), scale.contiguous()


def quantize_row_blocks_on_cpu(weight: torch.Tensor) -> Iterator[tuple[slice, torch.Tensor, torch.Tensor]]:
    """``inference/fp8_weights.py:22-26``: quantize in blocks of rows, CPU tensors
    out. Each block goes through the HIP quantizer, or the host quantizer on a
    machine without a HIP device (the reference quantizes these blocks on the
    CPU; both give its bits)."""
    quantize = quantize_rows if torch.cuda.is_available() else quantize_rows_host
    for start in range(0, weight.shape[0], QUANTIZE_BLOCK_ROWS):
        rows = slice(start, start + QUANTIZE_BLOCK_ROWS)
        codes, scale = quantize(weight[rows])
        yield rows, codes.cpu(), scale.cpu()


def quantizable(linear: nn.Linear) -> bool:
    """``inference/fp8_weights.py:29-30``."""
    return linear.in_features % 256 == 0 and linear.out_features >= 1024 and linear.out_features % 16 == 0


def replace_linears(module: nn.Module, make: Callable[[nn.Linear], nn.Module]) -> int:
    """``inference/fp8_weights.py:33-41``: swap every quantizable nn.Linear."""
    n = 0
    for name, child in module.named_children():
        if isinstance(child, nn.Linear) and quantizable(child):
            setattr(module, name, make(child))
            n += 1
        else:
            n += replace_linears(child, make)
    return n
