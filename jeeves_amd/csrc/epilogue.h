// The fused output epilogue shared by the decode and prefill GEMMs:
//
//   v[m,n]   = (acc * sx[m]) * sw[n] + lora_scale * sum_r t[m,r] * B[n,r]
//   y[m,n]   = bf16(v)                          without a bias
//   y[m,n]   = bf16(bf16(v) + bias[n])          with a bias
//
// acc * sx * sw is the scale epilogue of _fp8_matmul (inference/fp8.py:83,87),
// rounded to bf16 as fp8_matmul returns it; the bias is then added to that bf16
// output in bf16, as FP8Linear.forward does (inference/fp8.py:183-184), so a
// biased call is bitwise the unbiased call plus the bias. The LoRA term is
// LoRALinear.forward's (model/lora.py:122-133) with t = x A^T from the
// quantizer in fp32, folded into the same rounding as the GEMM (the reference
// merges LoRA before FP8 export, so it never runs one on an FP8 base).
#pragma once

#include "fp8_common.h"

namespace jv {

struct Epilogue {
  const float* sx;        // [M] per-token scales
  const float* sw;        // [N] per-channel scales
  const uint16_t* bias;   // [N] bf16 or null
  const float* lora_t;    // [M, RANK] fp32 or null
  const uint16_t* lora_b; // [N, RANK] bf16 or null
  float lora_scale;
  uint16_t* y;            // [M, ldy] bf16 (with SwiGLU: h [M, half])
  int64_t ldy;
  // Fused SwiGLU (gate+up GEMMs): the weight's rows are gate [0, half) then up
  // [half, 2 half); the kernels pair gate tile p with up tile p (logical
  // channel order g0..g15 u0..u15 g16..., swiglu_channel) and store
  // h = bf16(bf16(silu(y_gate)) * y_up) of width `half`, plus, when `parts` is
  // set, the largest |h| (bf16 magnitude bits) of each token over each 16
  // channels of h: parts[m * (half / 16) + c / 16].
  int64_t half = 0;
  uint16_t* parts = nullptr;
};

// Physical weight row of logical channel c in the SwiGLU pairing (c / 32 is
// the pair p: 16 gate rows 16p.., then 16 up rows half + 16p..).
__host__ __device__ __forceinline__ int64_t swiglu_channel(int64_t c, int64_t half) {
  const int64_t p = c >> 5, r = c & 31;
  return r < 16 ? p * 16 + r : half + p * 16 + (r - 16);
}
// The same for 16-row tiles: logical tile lt -> physical tile.
__host__ __device__ __forceinline__ int64_t swiglu_tile(int64_t lt, int64_t half) {
  return (lt & 1) ? (half >> 4) + (lt >> 1) : (lt >> 1);
}

// The value the caller rounds to bf16 once more: v itself, or bf16(v) + bias.
// biasn: the bias of the channel, already loaded (used only when ep.bias is set).
__device__ __forceinline__ float with_bias(const Epilogue& ep, float v, float biasn) {
  return ep.bias ? bf16_to_f32(f32_to_bf16(v)) + biasn : v;
}

template <int RANK>
__device__ __forceinline__ float epilogue_value(const Epilogue& ep, float acc, int m, int n, float sxm, float swn,
                                                float biasn) {
  float v = (acc * sxm) * swn;
  if constexpr (RANK > 0) {
    const float* t = ep.lora_t + (int64_t)m * RANK;
    const uint16_t* b = ep.lora_b + (int64_t)n * RANK;
    float l = 0.0f;
#pragma unroll
    for (int r = 0; r < RANK; ++r) l = __builtin_fmaf(t[r], bf16_to_f32(b[r]), l);
    v += l * ep.lora_scale;
  }
  return with_bias(ep, v, biasn);
}

}  // namespace jv
