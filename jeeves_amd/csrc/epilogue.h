// The fused output epilogue shared by the decode and prefill GEMMs:
//
//   y[m,n] = bf16( (acc * sx[m]) * sw[n] + bias[n] + lora_scale * sum_r t[m,r] * B[n,r] )
//
// acc * sx * sw is the scale epilogue of _fp8_matmul (inference/fp8.py:83,87);
// the bias is FP8Linear.forward's (inference/fp8.py:183-184); the LoRA term is
// LoRALinear.forward's (model/lora.py:122-133) with t = x A^T computed by the
// quantizer. The sum is rounded to bf16 once.
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
  uint16_t* y;            // [M, ldy] bf16
  int64_t ldy;
};

// biasn: the bias of channel n, already loaded (used only when ep.bias is set).
template <int RANK>
__device__ __forceinline__ float epilogue_value(const Epilogue& ep, float acc, int m, int n, float sxm, float swn,
                                                float biasn) {
  float v = (acc * sxm) * swn;
  if (ep.bias) v += biasn;
  if constexpr (RANK > 0) {
    const float* t = ep.lora_t + (int64_t)m * RANK;
    const uint16_t* b = ep.lora_b + (int64_t)n * RANK;
    float l = 0.0f;
#pragma unroll
    for (int r = 0; r < RANK; ++r) l = __builtin_fmaf(t[r], bf16_to_f32(b[r]), l);
    v += l * ep.lora_scale;
  }
  return v;
}

// Same with the bias read here.
template <int RANK>
__device__ __forceinline__ float epilogue_value(const Epilogue& ep, float acc, int m, int n, float sxm, float swn) {
  return epilogue_value<RANK>(ep, acc, m, n, sxm, swn, ep.bias ? bf16_to_f32(ep.bias[n]) : 0.0f);
}
}  // namespace jv
