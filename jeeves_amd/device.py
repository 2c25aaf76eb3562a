"""Device queries for the FP8 path (``model/triton_kernels.py:18-20``'s role)."""

from __future__ import annotations

from functools import lru_cache

import torch

from . import _lib


@lru_cache
def sm_count(device: torch.device) -> int:
    """Compute units of a HIP device, from the library (hipDeviceGetAttribute)."""
    index = device.index if isinstance(device, torch.device) and device.index is not None else -1
    n = _lib.lib().jv_device_cu_count(index)
    if n <= 0:
        raise RuntimeError(f"cannot query the compute units of {device}")
    return n
