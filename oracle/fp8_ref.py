"""Numpy restatement of the reference's FP8 linear-layer arithmetic (CPU oracle).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``; never by the product path.

Data conventions: bf16 tensors travel as ``uint16`` bit patterns, e4m3fn codes
as ``uint8``, scales as ``float32``. Nothing here uses torch, so the oracle is
independent of the library whose casts it restates; torch is used only by the
tests and the golden-fixture script to pin it.

Pinning summary (what checks each function; details in each docstring):

==========================  ===================================================
function                    pinned by
==========================  ===================================================
``e4m3_decode``             all 256 codes vs ``torch.float8_e4m3fn`` decode;
                            OCP spec known answers (max 448, min normal 2^-6,
                            min subnormal 2^-9, NaN only at S.1111.111)
``e4m3_encode``             dense fp32 sweeps (every e4m3 midpoint +-4 ulp,
                            every exponent, random bits) vs torch's cast;
                            round trip decode(encode(v)) == v on all 254
                            finite codes
``quantize_rows``           committed golden fixtures made by torch (the
                            library the reference calls); known answers for the
                            reciprocal constant, the 1e-12 clamp, +-inf and NaN
                            rows; invariant: the row's amax encodes to +-448
``bf16`` rounding           every f32 bit pattern class vs torch's cast; the
                            double->float->bf16 path vs torch
``gemm_exact_f64``          brute-force triple loop on tiny shapes; identity
                            matrix decode of every finite code; exactness
                            argument (below)
``dequant_matmul_f64``      linearity and brute force on tiny shapes
``w8a16_math``              brute force on tiny shapes (float32 sums)
``add_bias_bf16``           torch's bf16 add on dense random and edge pairs
``lora_f64``                closed form evaluated on tiny shapes by loops
``swiglu_bf16``             torch's ``F.silu(gate) * up`` on every bf16 gate
                            value (65536) times random bf16 ups
==========================  ===================================================
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "FP8_MAX", "FP8_MAX_RECIPROCAL", "SCALE_CLAMP_MIN", "SCALE_SUFFIX", "QUANTIZE_BLOCK_ROWS", "BLOCK_K",
    "E4M3_TABLE", "e4m3_encode", "e4m3_decode",
    "bf16_to_f32", "f32_to_bf16", "f64_to_bf16",
    "quantize_rows", "quantize_row_blocks_on_cpu", "quantizable",
    "gemm_exact_f64", "gemm_exact_bf16", "dequant_matmul_f64", "dequant_matmul_f32", "w8a16_math",
    "add_bias_bf16", "lora_f64", "silu_f32", "swiglu_bf16",
    "rel_l2", "bitwise_equal_fraction", "within_metal_bound",
]

# inference/fp8_weights.py:8-13. FP8_MAX is torch.finfo(float8_e4m3fn).max.
FP8_MAX = 448.0
# inference/fp8_weights.py:10: float(torch.tensor(1 / 448, dtype=float32)) = 0x1.24924ap-9.
FP8_MAX_RECIPROCAL = np.float32(1.0 / 448.0)
# inference/fp8_weights.py:18: clamp(min=1e-12) on a float32 tensor compares against fp32(1e-12).
SCALE_CLAMP_MIN = np.float32(1e-12)
SCALE_SUFFIX = "_scale"
QUANTIZE_BLOCK_ROWS = 16384
# inference/fp8.py:26: the GEMM needs K divisible by this.
BLOCK_K = 128


# ---------------------------------------------------------------------------
# OCP FP8 E4M3 ("fn": no infinities, one NaN mantissa per sign), from the OCP
# 8-bit floating point specification v1.0: bias 7, exponent field 0 holds
# subnormals m * 2^-9, field 1..15 holds (1 + m/8) * 2^(e-7), and S.1111.111 is
# NaN, so the largest finite magnitude is 1.75 * 2^8 = 448.
# ---------------------------------------------------------------------------

def _build_table() -> np.ndarray:
    table = np.empty(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        e, m = (code >> 3) & 0xF, code & 0x7
        if e == 15 and m == 7:
            value = np.nan
        elif e == 0:
            value = m * 2.0 ** -9
        else:
            value = (1.0 + m / 8.0) * 2.0 ** (e - 7)
        table[code] = sign * value
    return table


E4M3_TABLE = _build_table()


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """e4m3fn code -> float32 value (exact). Mirrors ``codes.view(float8_e4m3fn).float()``."""
    return E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(values: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn code, round to nearest even, NaN on overflow.

    This is what ``tensor.to(torch.float8_e4m3fn)`` does (the cast at
    ``inference/fp8_weights.py:19``): magnitudes above the midpoint 464
    between 448 and the nonexistent 480 become NaN (0x7F with the sign),
    464 itself ties to the even code 0x7E, +-inf and NaN become NaN, and the
    sign bit is carried for zeros and NaNs.
    """
    f = np.ascontiguousarray(values, dtype=np.float32)
    bits = f.view(np.uint32).astype(np.int64)
    sign = (bits >> 24) & 0x80
    mag_bits = bits & 0x7FFFFFFF
    mag = (mag_bits.astype(np.uint32)).view(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        nan = ~(mag <= np.float32(464.0))
        subnormal = mag < np.float32(2.0 ** -6)
        # Normal range: round the 23-bit mantissa to 3 bits (ties to even) on the
        # combined exponent|mantissa field; a carry bumps the exponent, as it should.
        rounded = (mag_bits + 0x7FFFF + ((mag_bits >> 20) & 1)) >> 20
        normal_code = rounded - ((127 - 7) << 3)
        # Subnormal range: the value is m * 2^-9 with m = rne(|f| * 2^9) in 0..8
        # (8 is the smallest normal, code 0x08). Scaling by 2^9 is exact.
        sub_code = np.rint(mag * np.float32(512.0)).astype(np.int64)
    code = np.where(subnormal, sub_code, normal_code)
    code = np.where(nan, 0x7F, code)
    return (code | sign).astype(np.uint8)


# ---------------------------------------------------------------------------
# bf16 helpers (torch semantics: float -> bf16 rounds to nearest even; double
# -> bf16 goes through float first, c10::BFloat16(float)).
# ---------------------------------------------------------------------------

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(values: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(values, dtype=np.float32)
    b = f.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(np.isnan(f), 0x7FC0, r)
    return r.astype(np.uint16)


def f64_to_bf16(values: np.ndarray) -> np.ndarray:
    """double -> float -> bf16, as ``tensor.double().to(torch.bfloat16)`` rounds."""
    with np.errstate(over="ignore"):
        return f32_to_bf16(np.asarray(values, dtype=np.float64).astype(np.float32))


# ---------------------------------------------------------------------------
# The reference quantizer.
# ---------------------------------------------------------------------------

def quantize_rows(weight: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Restates ``quantize_rows`` (``inference/fp8_weights.py:16-19``).

    1. ``w = weight.float()``
    2. ``scale = max(amax_row(|w|), fp32(1e-12)) * fp32(1/448)`` in float32
       (amax and clamp propagate NaN, as torch's ``amax``/``clamp`` do)
    3. ``codes = e4m3(w / scale)`` with an IEEE float32 division.

    The build applies it to weight rows (one scale per output channel) and to
    token rows of the activations (one scale per token). ``weight`` is a 2-D
    float32 array (bf16 inputs go through ``bf16_to_f32`` first).
    """
    w = np.ascontiguousarray(weight, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError("quantize_rows takes a 2-D array")
    rows, cols = w.shape
    # Rows are independent: large inputs go in blocks of about 1M elements so
    # the encoder's temporaries stay small (same result as one pass).
    block = max(1, (1 << 20) // max(cols, 1))
    if rows > block:
        parts = [quantize_rows(w[r:r + block]) for r in range(0, rows, block)]
        return np.concatenate([c for c, _ in parts]), np.concatenate([s for _, s in parts])
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        amax = np.max(np.abs(w), axis=1) if cols else np.zeros(rows, np.float32)
        scale = (np.maximum(amax, SCALE_CLAMP_MIN) * FP8_MAX_RECIPROCAL).astype(np.float32)
        q = (w / scale[:, None]).astype(np.float32)
    return e4m3_encode(q), scale


def quantize_row_blocks_on_cpu(weight: np.ndarray):
    """Restates ``inference/fp8_weights.py:22-26``: quantize in blocks of rows."""
    for start in range(0, weight.shape[0], QUANTIZE_BLOCK_ROWS):
        rows = slice(start, start + QUANTIZE_BLOCK_ROWS)
        yield (rows, *quantize_rows(weight[rows]))


def quantizable(in_features: int, out_features: int) -> bool:
    """Restates ``inference/fp8_weights.py:29-30``."""
    return in_features % 256 == 0 and out_features >= 1024 and out_features % 16 == 0


# ---------------------------------------------------------------------------
# GEMM oracles.
# ---------------------------------------------------------------------------

def gemm_exact_f64(xq: np.ndarray, sx: np.ndarray, wq: np.ndarray, sw: np.ndarray) -> np.ndarray:
    """``(sum_k xq[m,k] * wq[n,k]) * sx[m] * sw[n]`` with an exact sum.

    Every e4m3 value is a multiple of 2^-9 with magnitude <= 448, so each
    product is a multiple of 2^-18 with magnitude < 2^17.7 and any partial sum
    over K <= 131072 terms is an integer multiple of 2^-18 below 2^35: it fits
    float64's 53-bit significand, so float64 accumulation in any order (BLAS,
    FMA) is exact. This is the "exact" of ``inference/cuda_test.py:87`` on
    quantized activations.
    """
    xv = e4m3_decode(xq).astype(np.float64)
    wv = e4m3_decode(wq).astype(np.float64)
    if xv.shape[1] > 131072:
        raise ValueError("exactness argument holds for K <= 131072")
    acc = xv @ wv.T
    return acc * np.asarray(sx, np.float64)[:, None] * np.asarray(sw, np.float64)[None, :]


def gemm_exact_bf16(xq, sx, wq, sw, bias_bits=None) -> np.ndarray:
    """Exact result rounded once to bf16 (via float, as torch rounds double);
    with a bias, that bf16 output plus the bias as ``FP8Linear.forward`` adds
    it (``add_bias_bf16``)."""
    y = f64_to_bf16(gemm_exact_f64(xq, sx, wq, sw))
    return y if bias_bits is None else add_bias_bf16(y, bias_bits)


def add_bias_bf16(y_bits: np.ndarray, bias_bits: np.ndarray) -> np.ndarray:
    """``y + bias`` on bf16 tensors (``inference/fp8.py:183-184``): the sum of
    the two bf16 values in float32, rounded to bf16 (torch's bf16 add)."""
    return f32_to_bf16(bf16_to_f32(y_bits) + bf16_to_f32(bias_bits)[None, :])


def dequant_matmul_f64(xq, sx, wq, sw) -> np.ndarray:
    """Dequantize-then-matmul in float64: ``(xq*sx) @ (wq*sw)^T``."""
    xd = e4m3_decode(xq).astype(np.float64) * np.asarray(sx, np.float64)[:, None]
    wd = e4m3_decode(wq).astype(np.float64) * np.asarray(sw, np.float64)[:, None]
    return xd @ wd.T


def dequant_matmul_f32(xq, sx, wq, sw) -> np.ndarray:
    """The CPU fallback the build times: dequantize to float32, then sgemm."""
    xd = e4m3_decode(xq) * np.asarray(sx, np.float32)[:, None]
    wd = e4m3_decode(wq) * np.asarray(sw, np.float32)[:, None]
    return xd @ wd.T


def w8a16_math(x_bits: np.ndarray, wq: np.ndarray, sw: np.ndarray) -> np.ndarray:
    """The reference's W8A16 math, ``((x.float() @ w8.float().t()) * scale).to(bf16)``
    (``model/metal_test.py:213``): bf16 activations, float32 sums."""
    x = bf16_to_f32(x_bits)
    return f32_to_bf16((x @ e4m3_decode(wq).T) * np.asarray(sw, np.float32)[None, :])


def lora_f64(x: np.ndarray, a: np.ndarray, b: np.ndarray, scaling: float) -> np.ndarray:
    """LoRA term of ``model/lora.py:122-133``: ``(x @ A^T) @ (B * scaling)^T``."""
    x = np.asarray(x, np.float64)
    return (x @ np.asarray(a, np.float64).T) @ (np.asarray(b, np.float64) * scaling).T


def silu_f32(g: np.ndarray) -> np.ndarray:
    """``g / (1 + exp(-g))`` in float32, as torch evaluates ``F.silu`` on bf16
    (float32 arithmetic; exp(-g) overflows to inf for g < -88.7, giving -0)."""
    g = np.asarray(g, np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        return (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)


def swiglu_bf16(gate_bits: np.ndarray, up_bits: np.ndarray) -> np.ndarray:
    """``F.silu(gate) * up`` on bf16 tensors (``model/model.py:583``): silu in
    float32 rounded to bf16, then the product of the two bf16 values (exact in
    float32) rounded to bf16."""
    s = f32_to_bf16(silu_f32(bf16_to_f32(gate_bits)))
    return f32_to_bf16(bf16_to_f32(s) * bf16_to_f32(up_bits))


# ---------------------------------------------------------------------------
# Acceptance criteria.
# ---------------------------------------------------------------------------

def rel_l2(out: np.ndarray, ref: np.ndarray) -> float:
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(out - ref) / den) if den else float(np.linalg.norm(out))


def bitwise_equal_fraction(out_bits: np.ndarray, exact_bits: np.ndarray) -> float:
    """Share of outputs bitwise equal to the exact-rounded result
    (``inference/cuda_test.py:89``); positions where both are NaN count as equal."""
    a = np.asarray(out_bits, np.uint16)
    b = np.asarray(exact_bits, np.uint16)
    both_nan = np.isnan(bf16_to_f32(a)) & np.isnan(bf16_to_f32(b))
    return float(((a == b) | both_nan).mean()) if a.size else 1.0


def within_metal_bound(out: np.ndarray, exact: np.ndarray, magnitude: np.ndarray) -> bool:
    """``|out - exact| <= |exact| * 2^-8 + magnitude * 2^-20`` (``model/metal_test.py:219-221``)."""
    out = np.asarray(out, np.float64)
    return bool((np.abs(out - exact) <= np.abs(exact) * 2.0 ** -8 + magnitude * 2.0 ** -20).all())
