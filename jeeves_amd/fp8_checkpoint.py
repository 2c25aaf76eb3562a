"""The FP8 checkpoint format of the jeeves ``--precision fp8`` path
(``inference/fp8_checkpoint.py:26-85``), without the model stack.

On disk a quantized linear ``<name>`` is two safetensors entries:
``<name>.weight`` float8_e4m3fn ``[N, K]`` codes and ``<name>.weight_scale``
float32 ``[N]`` (``SCALE_SUFFIX``), exactly what ``quantize_rows`` returns
(``inference/fp8_weights.py:16-19``); every other tensor is stored unchanged.
The loader accepts either that pair or a plain bf16/fp32 ``<name>.weight``,
which it quantizes while loading (``FP8Linear.load_weight``).

The reference builds the module tree from its Qwen3.5 model and maps
checkpoint keys with the model's ``map_checkpoint_key``; here both come from
the caller (``quantized_linears(module)``, ``map_key``), so any module tree
whose linears were swapped by ``replace_linears`` loads the same files.
"""

from __future__ import annotations

from pathlib import Path
from typing import Callable

import torch
import torch.nn as nn
from safetensors import safe_open
from safetensors.torch import save_file

from .fp8_weights import FP8, SCALE_SUFFIX, quantizable, quantize_row_blocks_on_cpu


def quantized_linears(module: nn.Module) -> set[str]:
    """Names of the ``nn.Linear`` modules the FP8 path quantizes
    (``inference/fp8_checkpoint.py:26-27``)."""
    return {name for name, m in module.named_modules() if isinstance(m, nn.Linear) and quantizable(m)}


def quantize_on_cpu(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """CPU weight in, CPU ``(codes, scale)`` out, quantized in row blocks
    (``inference/fp8_checkpoint.py:30-35``; each block runs on the HIP device,
    or on the host quantizer where there is none)."""
    codes = torch.empty(weight.shape, dtype=FP8)
    scale = torch.empty(weight.shape[0], dtype=torch.float32)
    for rows, block_codes, block_scale in quantize_row_blocks_on_cpu(weight):
        codes[rows], scale[rows] = block_codes, block_scale
    return codes, scale


def write_quantized(src: Path | str, dst: Path | str, linears: set[str],
                    quantize: Callable[[torch.Tensor], tuple[torch.Tensor, torch.Tensor]] | None = None) -> dict[str, int]:
    """Rewrite the safetensors file ``src`` as ``dst``: the weight of every
    linear named in ``linears`` becomes its e4m3 codes plus a
    ``<name>.weight_scale`` entry, everything else is kept as is
    (``inference/fp8_checkpoint.py:38-47``). Returns the byte size of each
    written entry."""
    quantize = quantize or quantize_on_cpu
    out: dict[str, torch.Tensor] = {}
    with safe_open(str(src), framework="pt", device="cpu") as fh:
        for key in fh.keys():
            tensor = fh.get_tensor(key)
            owner = key[: -len(".weight")] if key.endswith(".weight") else None
            if owner in linears:
                codes, scale = quantize(tensor)
                out[key], out[key + SCALE_SUFFIX] = codes, scale
            else:
                out[key] = tensor
    save_file(out, str(dst), metadata={"format": "pt"})
    return {key: t.numel() * t.element_size() for key, t in out.items()}


def checked(key: str, tensor: torch.Tensor, shape: tuple[int, ...] | torch.Size) -> torch.Tensor:
    """The tensor, after checking its shape against the model's
    (``inference/fp8_checkpoint.py:50-53``)."""
    if tensor.shape != torch.Size(shape):
        raise ValueError(f"{key}: checkpoint {tuple(tensor.shape)} vs model {tuple(shape)}")
    return tensor


def _load_linear(linear: nn.Module, fh, key: str, scale_keys: set[str]) -> str | None:
    """Fill one FP8 linear from ``key`` (and its scale entry when present);
    returns the scale key it used."""
    weight = checked(key, fh.get_tensor(key), (linear.out_features, linear.in_features))
    scale_key = key + SCALE_SUFFIX
    if scale_key not in scale_keys:
        linear.load_weight(weight)  # bf16/fp32 checkpoint: quantize while loading
        return None
    linear.load_codes(weight, checked(scale_key, fh.get_tensor(scale_key), (linear.out_features,)))
    return scale_key


@torch.no_grad()
def load_tensors(module: nn.Module, files: list[Path], linear_class: type[nn.Module],
                 map_key: Callable[[str], str | None] = lambda key: key) -> tuple[set[str], list[str]]:
    """Load safetensors ``files`` into ``module`` (``inference/fp8_checkpoint.py:56-85``).

    A checkpoint weight that belongs to an FP8 linear (``linear_class``) goes
    through ``load_codes`` when its scale entry is in the same file, else
    through ``load_weight``; any other key is copied into the parameter or
    buffer of that name. ``map_key`` turns a checkpoint key into a module name
    (None: skip the key). Returns (loaded names, keys nothing consumed).
    """
    tensors = dict(module.named_parameters())
    tensors.update(module.named_buffers())
    fp8 = {name: m for name, m in module.named_modules() if isinstance(m, linear_class)}
    loaded: set[str] = set()
    unexpected: list[str] = []
    for path in files:
        with safe_open(str(path), framework="pt", device="cpu") as fh:
            keys = list(fh.keys())
            scale_keys = {k for k in keys if k.endswith(SCALE_SUFFIX)}
            consumed: set[str] = set()
            for key in keys:
                target = None if key in scale_keys else map_key(key)
                if target is None:
                    continue
                owner, _, leaf = target.rpartition(".")
                if leaf == "weight" and owner in fp8:
                    used = _load_linear(fp8[owner], fh, key, scale_keys)
                    if used:
                        consumed.add(used)
                    loaded.update(f"{owner}.{b}" for b, _ in fp8[owner].named_buffers())
                elif target in tensors:
                    tensors[target].copy_(checked(key, fh.get_tensor(key), tensors[target].shape))
                    loaded.add(target)
                else:
                    unexpected.append(key)
            unexpected.extend(sorted(scale_keys - consumed))
    return loaded, unexpected
