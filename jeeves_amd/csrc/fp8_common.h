// Shared device helpers for the gfx950 FP8 linear-layer kernels.
//
// Data conventions on the device:
//   bf16     uint16_t bit patterns
//   e4m3fn   uint8_t codes (OCP FP8 E4M3, "fn": no infinities, NaN = S.1111.111)
//   scales   float32
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jv {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// fp32(1/448): the reciprocal that inference/fp8_weights.py:10 multiplies by.
// The division is constant-folded with IEEE rounding, giving 0x3B124925.
constexpr float kFp8MaxReciprocal = 1.0f / 448.0f;
// fp32(1e-12): the clamp of inference/fp8_weights.py:18.
constexpr float kScaleClampMin = 1e-12f;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// float -> bf16, round to nearest even; NaN -> 0x7FC0 (torch's c10::BFloat16).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t b = __float_as_uint(f);
  if (f != f) return 0x7FC0u;
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

// Two floats -> two bf16 (a in the low half), round to nearest even, with
// gfx950's v_cvt_pk_bf16_f32. Equal to f32_to_bf16 on every non-NaN input; a
// NaN stays a NaN (its sign and payload are not canonicalised to 0x7FC0).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2));
}

// silu(g) = g / (1 + exp(-g)) for a bf16 g, in the form the epilogues can
// afford: exp(-g) as the hardware 2^x of -g log2(e) (v_exp_f32), and for
// |g| < 64 the quotient from the hardware reciprocal with Markstein's
// correction (one product, two FMAs; the sign put back for -0), the IEEE
// division beyond. Rounded to bf16 it equals torch's float32 silu rounded to
// bf16 for every one of the 65536 bf16 inputs (checked exhaustively on the
// device by the conformance tests), so it is exact where it is used.
__device__ __forceinline__ float silu_of_bf16(float g) {
  const float d = 1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
  if (__builtin_fabsf(g) < 64.0f) {
    const float r = __builtin_amdgcn_rcpf(d);
    const float q0 = g * r;
    const float e = __builtin_fmaf(-q0, d, g);
    return __builtin_copysignf(__builtin_fmaf(e, r, q0), g);
  }
  return g / d;
}

// SwiGLU on bf16 values (SwiGLU.forward, model/model.py:583, as torch runs it
// on bf16 tensors): silu(g) rounded to bf16, times up (exact in fp32), rounded
// to bf16. This is the reference's F.silu(gate) * up branch; its fla branch
// (_fla_swiglu, taken where flash-linear-attention is installed) rounds only
// the product, and parity with it is unpinned. Every kernel's SwiGLU rounding
// goes through this function or swiglu_pair_f32 below, so a single-rounding
// variant would replace these two alone.
__device__ __forceinline__ uint32_t swiglu_bf16(uint32_t g16, uint32_t u16) {
  const float sb = bf16_to_f32(f32_to_bf16(silu_of_bf16(bf16_to_f32(g16))));
  return f32_to_bf16(sb * bf16_to_f32(u16));
}

// SwiGLU of two channels from their fp32 gate and up values before the GEMM's
// bf16 rounding: h0 in the low half, bitwise
// swiglu_bf16(f32_to_bf16(g0), f32_to_bf16(u0)) (and likewise h1). The
// roundings go two at a time through v_cvt_pk_bf16_f32 (equal to f32_to_bf16
// on every non-NaN; a NaN stays a NaN), and a NaN h is canonicalised to
// 0x7FC0 as f32_to_bf16 gives it.
__device__ __forceinline__ uint32_t swiglu_pair_f32(float g0, float g1, float u0, float u1) {
  const uint32_t gb = pack_bf16x2(g0, g1), ub = pack_bf16x2(u0, u1);
  const float s0 = silu_of_bf16(__uint_as_float(gb << 16)), s1 = silu_of_bf16(__uint_as_float(gb & 0xFFFF0000u));
  const uint32_t sb = pack_bf16x2(s0, s1);
  const float h0 = __uint_as_float(sb << 16) * __uint_as_float(ub << 16);
  const float h1 = __uint_as_float(sb & 0xFFFF0000u) * __uint_as_float(ub & 0xFFFF0000u);
  uint32_t hb = pack_bf16x2(h0, h1);
  if (h0 != h0) hb = (hb & 0xFFFF0000u) | 0x7FC0u;
  if (h1 != h1) hb = (hb & 0x0000FFFFu) | 0x7FC00000u;
  return hb;
}

// ---------------------------------------------------------------------------
// e4m3fn encode, round to nearest even, NaN on overflow (|f| > 464), sign kept.
// Written from the OCP FP8 v1.0 format definition; this is the semantics of
// torch's float -> float8_e4m3fn cast that the reference quantizer uses.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ uint32_t e4m3_encode_sw(float f) {
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  const uint32_t sign = (b >> 24) & 0x80u;
  const uint32_t mb = b & 0x7FFFFFFFu;
  const float mag = __builtin_bit_cast(float, mb);
  uint32_t code;
  if (!(mag <= 464.0f)) {
    code = 0x7Fu;
  } else if (mag < 0.015625f) {
    // Subnormal codes m * 2^-9: m = rne(|f| * 2^9) in 0..8 (8 is the smallest normal).
    code = (uint32_t)__builtin_rintf(mag * 512.0f);
  } else {
    // Round the 23-bit mantissa to 3 bits on the exponent|mantissa field (a carry
    // bumps the exponent), then rebias 127 -> 7.
    code = ((mb + 0x7FFFFu + ((mb >> 20) & 1u)) >> 20) - ((127u - 7u) << 3);
  }
  return code | sign;
}

// gfx950's v_cvt_pk_fp8_f32 (OCP e4m3, round to nearest even). Two floats into
// two bytes of a 32-bit word; `hi` selects the upper 16 bits. The quantizer
// only sends it finite quotients with |q| <= 448 * (1 + 2^-22), where its
// result equals e4m3_encode_sw on every input (checked exhaustively over
// that range by the conformance tests).
template <bool HI>
__device__ __forceinline__ int cvt_pk_fp8(float a, float b, int old) {
  return __builtin_amdgcn_cvt_pk_fp8_f32(a, b, old, HI);
}

// ---------------------------------------------------------------------------
// The quantizer's division x / scale for finite nonzero `scale` with
// r = RN(1/scale): one product and two FMAs (Markstein's correction), with the
// sign of x put back (callers apply copysign). For every pair of a bf16 x and
// a bf16 row maximum it equals the IEEE quotient bit for bit wherever either
// has magnitude >= 2^-11, and its e4m3 code equals the IEEE quotient's code
// for every pair (both checked exhaustively by the tests). Rows whose scale is
// inf or NaN take the plain IEEE division instead.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float quotient(float x, float scale, float r) {
  const float q0 = x * r;
  const float e = __builtin_fmaf(-q0, scale, x);
  return __builtin_fmaf(e, r, q0);
}

// The reference's per-row scale from the row's largest magnitude, given as the
// 15-bit bf16 magnitude pattern. NaN propagates as torch's amax and clamp do.
__device__ __forceinline__ float scale_from_amax_bits(uint32_t amax_bits) {
  const float amax = __uint_as_float(amax_bits << 16);
  if (amax_bits > 0x7F80u) return amax;  // NaN
  return fmaxf(amax, kScaleClampMin) * kFp8MaxReciprocal;
}

// Same for a float32 row maximum (already |.|), NaN-propagating.
__device__ __forceinline__ float scale_from_amax_f32(float amax) {
  if (amax != amax) return amax;
  return fmaxf(amax, kScaleClampMin) * kFp8MaxReciprocal;
}

// Quantize 8 bf16 (one uint4) with a row's scale (r = RN(1/scale)) to 8 codes
// (one uint2). fast: the row's maximum is finite, so the scale is finite and
// positive and the Markstein quotient + hardware converter apply; otherwise
// the exact division and the spec encoder (inf rows -> zeros, NaN).
__device__ __forceinline__ uint2 encode8(uint4 v, float scale, float r, bool fast) {
  float f[8];
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[2 * j] = bf16_to_f32(w[j] & 0xFFFFu);
    f[2 * j + 1] = bf16_to_f32(w[j] >> 16);
  }
  float q[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) q[j] = fast ? __builtin_copysignf(quotient(f[j], scale, r), f[j]) : f[j] / scale;
  uint2 out;
  if (fast) {
    int lo = cvt_pk_fp8<false>(q[0], q[1], 0);
    lo = cvt_pk_fp8<true>(q[2], q[3], lo);
    int hi = cvt_pk_fp8<false>(q[4], q[5], 0);
    hi = cvt_pk_fp8<true>(q[6], q[7], hi);
    out.x = (uint32_t)lo;
    out.y = (uint32_t)hi;
  } else {
    // inf / NaN rows: exact division and the spec encoder (NaN on overflow).
    out.x = e4m3_encode_sw(q[0]) | (e4m3_encode_sw(q[1]) << 8) | (e4m3_encode_sw(q[2]) << 16) |
            (e4m3_encode_sw(q[3]) << 24);
    out.y = e4m3_encode_sw(q[4]) | (e4m3_encode_sw(q[5]) << 8) | (e4m3_encode_sw(q[6]) << 16) |
            (e4m3_encode_sw(q[7]) << 24);
  }
  return out;
}

// ---------------------------------------------------------------------------
// Workgroup barriers without the memory fence __syncthreads() carries: that
// fence makes the compiler drain every outstanding global load first, which
// empties a kernel's load pipeline. Callers order their own memory.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void barrier_no_fence() { asm volatile("s_barrier" ::: "memory"); }

// Barrier ordering LDS only: this wave's LDS reads and writes complete
// (lgkmcnt(0); vmcnt and expcnt left unconstrained), then the barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  barrier_no_fence();
}

// ---------------------------------------------------------------------------
// Wave64 reductions.
// ---------------------------------------------------------------------------
// Maximum over the wave, in every lane, by DPP moves (no LDS round trips,
// which the ds_bpermute of __shfl_xor takes at each of its six steps):
// row_shr 1, 2, 4, 8 leave each 16-lane row's maximum in its lane 15 (a
// shifted-out source keeps `old` = 0, the identity of an unsigned max);
// row_bcast:15 carries row 0's into row 1 and row 2's into row 3,
// row_bcast:31 carries lane 31's into rows 2 and 3, so lane 63 holds the
// wave's maximum, which readlane hands to every lane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false));  // row_shr:1
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false));  // row_shr:2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false));  // row_shr:4
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false));  // row_shr:8
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));  // row_bcast:15
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Maximum over each 16-lane row (DPP row_shr 1, 2, 4, 8), left in the row's
// lane 15; the other lanes hold prefix maxima.
__device__ __forceinline__ uint32_t row16_max_u32_in_lane15(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false));  // row_shr:1
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false));  // row_shr:2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false));  // row_shr:4
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false));  // row_shr:8
  return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Max of two packed 16-bit magnitudes (v_pk_max_u16).
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  u16x2 va = __builtin_bit_cast(u16x2, a);
  u16x2 vb = __builtin_bit_cast(u16x2, b);
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(va, vb));
}

// ---------------------------------------------------------------------------
// MFMA wrappers. Format code 0 selects FP8 E4M3 for both operands; zero scale
// operands select the unscaled v_mfma_f32_{32x32x64,16x16x128}_f8f6f4.
// Each lane supplies 32 consecutive-k bytes of one row of A and of one column
// of B; A and B use the same lane -> k mapping, so the k order inside the
// instruction never changes the product.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x16 mfma_32x32x64_fp8(i32x8 a, i32x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_16x16x128_fp8(i32x8 a, i32x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// 8 e4m3 codes (two dwords) -> 8 bf16 (a 16-byte MFMA operand), in order.
__device__ __forceinline__ bf16x8 e4m3x8_to_bf16(uint32_t lo, uint32_t hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false), b = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);
  const f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false), d = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
  // The bf16 value is the upper half of the exact fp32 value.
  const i32x4 v = {(int)__builtin_amdgcn_perm(__float_as_uint(a.y), __float_as_uint(a.x), 0x07060302),
                   (int)__builtin_amdgcn_perm(__float_as_uint(b.y), __float_as_uint(b.x), 0x07060302),
                   (int)__builtin_amdgcn_perm(__float_as_uint(c.y), __float_as_uint(c.x), 0x07060302),
                   (int)__builtin_amdgcn_perm(__float_as_uint(d.y), __float_as_uint(d.x), 0x07060302)};
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ i32x8 cat8(i32x4 lo, i32x4 hi) {
  return i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

}  // namespace jv
