"""MI355X-native FP8 linear-layer path for the jeeves workload.

Public API mirrors the reference's ``inference/fp8.py`` and
``inference/fp8_weights.py`` (see ``jeeves_amd.fp8`` and
``jeeves_amd.fp8_weights``); the kernels are gfx950 HIP code in
``libjeeves_fp8.so`` behind the C ABI of ``include/jeeves_fp8.h``.
"""

from .device import sm_count
from .fp8 import (BLOCK_K, DECODE_MAX_ROWS, TILE_COUNTER_SLOTS, TILE_COUNTERS, WARM_ROWS, FP8Linear, FP8SwiGLU, fp8_matmul,
                  fp8_matmul_quantized, fp8_matmul_w8a16, fuse_swiglus, load_view, packed_codes_bytes, split_for, swiglu_quantize,
                  tile_weight, tileable, untile_weight, warm)
from .fp8_weights import (FP8, FP8_MAX, FP8_MAX_RECIPROCAL, QUANTIZE_BLOCK_ROWS, SCALE_SUFFIX, quantizable, quantize_row_blocks_on_cpu,
                          quantize_rows, replace_linears)

__all__ = [
    "BLOCK_K", "DECODE_MAX_ROWS", "TILE_COUNTER_SLOTS", "TILE_COUNTERS", "WARM_ROWS", "FP8Linear", "FP8SwiGLU", "fp8_matmul",
    "fp8_matmul_quantized", "fp8_matmul_w8a16", "fuse_swiglus", "load_view", "packed_codes_bytes", "split_for", "swiglu_quantize", "tile_weight", "tileable",
    "untile_weight", "warm", "sm_count",
    "FP8", "FP8_MAX", "FP8_MAX_RECIPROCAL", "QUANTIZE_BLOCK_ROWS", "SCALE_SUFFIX", "quantizable", "quantize_row_blocks_on_cpu",
    "quantize_rows", "replace_linears",
]
