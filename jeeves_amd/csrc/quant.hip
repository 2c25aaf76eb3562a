// Per-row e4m3fn quantizer on gfx950: the arithmetic of quantize_rows
// (inference/fp8_weights.py:16-19) applied to token rows of the activations
// (and to weight rows at load time).
//
//   scale[m] = max(amax_k |x[m,k]|, 1e-12) * fp32(1/448)
//   code[m,k] = e4m3fn_rne(x[m,k] / scale[m])        (IEEE fp32 quotient)
//
// One 256-thread workgroup per row. Each thread owns 8-element chunks
// c = tid + i*256 and keeps them in registers between the amax pass and the
// encode pass, so HBM sees each input byte once. The row maximum is taken on
// the 15-bit bf16 magnitude patterns with packed 16-bit integer max, which is
// exact and propagates NaN (NaN patterns sort above inf).
//
// Variants:
//   * SWIGLU: the row is h = bf16(bf16(silu(gate)) * up) (model/model.py:583),
//     built on the fly from the gate and up halves of a fused projection.
//   * RANK > 0: also emits the LoRA down-projection t[m,r] = sum_k x[m,k] A[r,k]
//     (model/lora.py:128-131) in fp32 from the same registers.
#include "fp8_common.h"
#include "kernels.h"

namespace jv {

constexpr int kQuantThreads = 256;

// silu in fp32 rounded to bf16, times up, rounded to bf16.
__device__ __forceinline__ uint32_t swiglu_bf16(uint32_t g16, uint32_t u16) {
  const float g = bf16_to_f32(g16);
  const float s = g / (1.0f + expf(-g));
  const float sb = bf16_to_f32(f32_to_bf16(s));
  return f32_to_bf16(sb * bf16_to_f32(u16));
}

__device__ __forceinline__ uint32_t swiglu_pair(uint32_t g2, uint32_t u2) {
  return swiglu_bf16(g2 & 0xFFFFu, u2 & 0xFFFFu) | (swiglu_bf16(g2 >> 16, u2 >> 16) << 16);
}

template <int RANK>
__device__ __forceinline__ void lora_accumulate(float (&t)[RANK > 0 ? RANK : 1], uint4 v, const uint16_t* __restrict__ a,
                                                int64_t K, int c) {
  if constexpr (RANK > 0) {
    float f[8];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[2 * j] = bf16_to_f32(w[j] & 0xFFFFu);
      f[2 * j + 1] = bf16_to_f32(w[j] >> 16);
    }
#pragma unroll
    for (int r = 0; r < RANK; ++r) {
      const uint4 av = *reinterpret_cast<const uint4*>(a + r * K + (int64_t)c * 8);
      const uint32_t aw[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        t[r] = __builtin_fmaf(f[2 * j], bf16_to_f32(aw[j] & 0xFFFFu), t[r]);
        t[r] = __builtin_fmaf(f[2 * j + 1], bf16_to_f32(aw[j] >> 16), t[r]);
      }
    }
  }
}

// Block-wide max of a per-thread 15-bit magnitude.
__device__ __forceinline__ uint32_t block_max(uint32_t v, uint32_t* red) {
  v = wave_max_u32(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  v = max(max(red[0], red[1]), max(red[2], red[3]));
  return v;
}

// NC: chunks of 8 elements per thread kept in registers (K <= NC * 2048).
// PACKED: codes go to the packed decode layout (packed_x_offset); the grid
// then also covers the padding rows M..16*ceil(M/16)-1, which get zero codes.
template <int NC, bool SWIGLU, int RANK, bool PACKED>
__global__ __launch_bounds__(kQuantThreads) void quant_rows_bf16_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ up, int64_t ldu, int K, int M,
    uint8_t* __restrict__ codes, int64_t ldc, float* __restrict__ scales, uint16_t* __restrict__ h_out, int64_t ldh,
    const uint16_t* __restrict__ lora_a, float* __restrict__ lora_t) {
  __shared__ uint32_t red[4];
  __shared__ float tred[4][RANK > 0 ? RANK : 1];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nchunks = K >> 3;
  if (PACKED && row >= M) {
    for (int c = tid; c < nchunks; c += kQuantThreads)
      *reinterpret_cast<uint2*>(codes + packed_x_offset((int)row, c * 8, K >> 7)) = uint2{0u, 0u};
    return;
  }
  const uint16_t* xr = x + row * ldx;
  uint4 v[NC];
  uint32_t am = 0;
  float t[RANK > 0 ? RANK : 1];
#pragma unroll
  for (int r = 0; r < (RANK > 0 ? RANK : 1); ++r) t[r] = 0.0f;

#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = tid + i * kQuantThreads;
    if (c < nchunks) {
      if constexpr (SWIGLU) {
        const uint4 g = *reinterpret_cast<const uint4*>(xr + (int64_t)c * 8);
        const uint4 u = *reinterpret_cast<const uint4*>(up + row * ldu + (int64_t)c * 8);
        v[i] = uint4{swiglu_pair(g.x, u.x), swiglu_pair(g.y, u.y), swiglu_pair(g.z, u.z), swiglu_pair(g.w, u.w)};
        if (h_out) *reinterpret_cast<uint4*>(h_out + row * ldh + (int64_t)c * 8) = v[i];
      } else {
        v[i] = *reinterpret_cast<const uint4*>(xr + (int64_t)c * 8);
      }
      am = pk_max_u16(am, v[i].x & 0x7FFF7FFFu);
      am = pk_max_u16(am, v[i].y & 0x7FFF7FFFu);
      am = pk_max_u16(am, v[i].z & 0x7FFF7FFFu);
      am = pk_max_u16(am, v[i].w & 0x7FFF7FFFu);
      lora_accumulate<RANK>(t, v[i], lora_a, K, c);
    } else {
      v[i] = uint4{0, 0, 0, 0};
    }
  }
  am = max(am & 0xFFFFu, am >> 16);
  const uint32_t amax_bits = block_max(am, red);
  const float scale = scale_from_amax_bits(amax_bits);
  if (tid == 0) scales[row] = scale;
  const bool fast = amax_bits < 0x7F80u;  // finite row: scale finite and > 0
  const float r = 1.0f / scale;
  uint8_t* cr = codes + (PACKED ? 0 : row * ldc);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = tid + i * kQuantThreads;
    if (c < nchunks) {
      const int64_t off = PACKED ? packed_x_offset((int)row, c * 8, K >> 7) : (int64_t)c * 8;
      *reinterpret_cast<uint2*>(cr + off) = encode8(v[i], scale, r, fast);
    }
  }
  if constexpr (RANK > 0) {
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int q = 0; q < RANK; ++q) {
      const float s = wave_sum_f32(t[q]);
      if (lane == 0) tred[wave][q] = s;
    }
    __syncthreads();
    if (tid < RANK) lora_t[row * RANK + tid] = (tred[0][tid] + tred[1][tid]) + (tred[2][tid] + tred[3][tid]);
  }
}

// Rows longer than the register cache: two passes over the row (the second
// mostly from L2). Plain bf16 rows only.
__global__ __launch_bounds__(kQuantThreads) void quant_rows_bf16_long_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                             int K, uint8_t* __restrict__ codes, int64_t ldc,
                                                                             float* __restrict__ scales) {
  __shared__ uint32_t red[4];
  const int64_t row = blockIdx.x;
  const int nchunks = K >> 3;
  const uint16_t* xr = x + row * ldx;
  uint32_t am = 0;
  for (int c = threadIdx.x; c < nchunks; c += kQuantThreads) {
    const uint4 v = *reinterpret_cast<const uint4*>(xr + (int64_t)c * 8);
    am = pk_max_u16(am, v.x & 0x7FFF7FFFu);
    am = pk_max_u16(am, v.y & 0x7FFF7FFFu);
    am = pk_max_u16(am, v.z & 0x7FFF7FFFu);
    am = pk_max_u16(am, v.w & 0x7FFF7FFFu);
  }
  am = max(am & 0xFFFFu, am >> 16);
  const uint32_t amax_bits = block_max(am, red);
  const float scale = scale_from_amax_bits(amax_bits);
  if (threadIdx.x == 0) scales[row] = scale;
  const bool fast = amax_bits < 0x7F80u;
  const float r = 1.0f / scale;
  for (int c = threadIdx.x; c < nchunks; c += kQuantThreads) {
    const uint4 v = *reinterpret_cast<const uint4*>(xr + (int64_t)c * 8);
    *reinterpret_cast<uint2*>(codes + row * ldc + (int64_t)c * 8) = encode8(v, scale, r, fast);
  }
}

// float32 rows (weights handed over in fp32): plain IEEE division and the
// spec encoder, since the bf16 exhaustive argument for the fast quotient does
// not cover fp32 inputs.
__global__ __launch_bounds__(kQuantThreads) void quant_rows_f32_kernel(const float* __restrict__ x, int64_t ldx, int K,
                                                                       uint8_t* __restrict__ codes, int64_t ldc,
                                                                       float* __restrict__ scales) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * ldx;
  float am = 0.0f;
  bool nan = false;
  for (int k = threadIdx.x * 4; k < K; k += kQuantThreads * 4) {
    const float4 v = *reinterpret_cast<const float4*>(xr + k);
    const float a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      nan |= a[j] != a[j];
      am = fmaxf(am, fabsf(a[j]));
    }
  }
  if (nan) am = __uint_as_float(0x7FC00000u);
  // NaN-propagating block max: NaN's bit pattern sorts above every magnitude.
  uint32_t bits = wave_max_u32(__float_as_uint(am));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = __uint_as_float(bits);
  __syncthreads();
  bits = max(max(__float_as_uint(red[0]), __float_as_uint(red[1])), max(__float_as_uint(red[2]), __float_as_uint(red[3])));
  const float scale = scale_from_amax_f32(__uint_as_float(bits));
  if (threadIdx.x == 0) scales[row] = scale;
  for (int k = threadIdx.x * 4; k < K; k += kQuantThreads * 4) {
    const float4 v = *reinterpret_cast<const float4*>(xr + k);
    const uint32_t c = e4m3_encode_sw(v.x / scale) | (e4m3_encode_sw(v.y / scale) << 8) |
                       (e4m3_encode_sw(v.z / scale) << 16) | (e4m3_encode_sw(v.w / scale) << 24);
    *reinterpret_cast<uint32_t*>(codes + row * ldc + k) = c;
  }
}

template <bool SWIGLU, int RANK, bool PACKED = false>
static hipError_t launch_rows(int NC, const uint16_t* x, int64_t ldx, const uint16_t* up, int64_t ldu, int64_t M, int K,
                              uint8_t* codes, int64_t ldc, float* scales, uint16_t* h_out, int64_t ldh,
                              const uint16_t* lora_a, float* lora_t, hipStream_t stream) {
  const dim3 grid((unsigned)(PACKED ? (M + 15) / 16 * 16 : M)), block(kQuantThreads);
#define JV_QUANT_CASE(n)                                                                                              \
  case n:                                                                                                             \
    quant_rows_bf16_kernel<n, SWIGLU, RANK, PACKED>                                                                  \
        <<<grid, block, 0, stream>>>(x, ldx, up, ldu, K, (int)M, codes, ldc, scales, h_out, ldh, lora_a, lora_t);   \
    break;
  switch (NC) {
    JV_QUANT_CASE(1)
    JV_QUANT_CASE(2)
    JV_QUANT_CASE(3)
    JV_QUANT_CASE(4)
    JV_QUANT_CASE(6)
    JV_QUANT_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef JV_QUANT_CASE
  return hipGetLastError();
}

// Register-cache depth for a row of K elements, or 0 when the row needs the
// two-pass kernel.
int quant_chunks(int K) {
  const int nc = (K + 8 * kQuantThreads - 1) / (8 * kQuantThreads);
  if (nc <= 4) return nc < 1 ? 1 : nc;
  if (nc <= 6) return 6;
  if (nc <= 8) return 8;
  return 0;
}

hipError_t quant_rows_bf16(const uint16_t* x, int64_t ldx, int64_t M, int K, uint8_t* codes, int64_t ldc, float* scales,
                           const uint16_t* lora_a, int rank, float* lora_t, bool packed, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  const int nc = quant_chunks(K);
  if (packed) {
    if (nc == 0 || M > kDecodeMaxRows || (K & 127)) return hipErrorInvalidValue;
    if (rank == 16)
      return launch_rows<false, 16, true>(nc, x, ldx, nullptr, 0, M, K, codes, 0, scales, nullptr, 0, lora_a, lora_t, stream);
    if (rank == 0)
      return launch_rows<false, 0, true>(nc, x, ldx, nullptr, 0, M, K, codes, 0, scales, nullptr, 0, nullptr, nullptr, stream);
    return hipErrorInvalidValue;
  }
  if (rank == 0) {
    if (nc == 0) {
      quant_rows_bf16_long_kernel<<<dim3((unsigned)M), dim3(kQuantThreads), 0, stream>>>(x, ldx, K, codes, ldc, scales);
      return hipGetLastError();
    }
    return launch_rows<false, 0>(nc, x, ldx, nullptr, 0, M, K, codes, ldc, scales, nullptr, 0, nullptr, nullptr, stream);
  }
  if (rank == 16 && nc != 0)
    return launch_rows<false, 16>(nc, x, ldx, nullptr, 0, M, K, codes, ldc, scales, nullptr, 0, lora_a, lora_t, stream);
  return hipErrorInvalidValue;
}

hipError_t quant_swiglu_bf16(const uint16_t* gate, int64_t ldg, const uint16_t* up, int64_t ldu, int64_t M, int K,
                             uint8_t* codes, int64_t ldc, float* scales, uint16_t* h_out, int64_t ldh,
                             const uint16_t* lora_a, int rank, float* lora_t, bool packed, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  const int nc = quant_chunks(K);
  if (nc == 0) return hipErrorInvalidValue;
  if (packed) {
    if (M > kDecodeMaxRows || (K & 127)) return hipErrorInvalidValue;
    if (rank == 0)
      return launch_rows<true, 0, true>(nc, gate, ldg, up, ldu, M, K, codes, 0, scales, h_out, ldh, nullptr, nullptr, stream);
    if (rank == 16)
      return launch_rows<true, 16, true>(nc, gate, ldg, up, ldu, M, K, codes, 0, scales, h_out, ldh, lora_a, lora_t, stream);
    return hipErrorInvalidValue;
  }
  if (rank == 0)
    return launch_rows<true, 0>(nc, gate, ldg, up, ldu, M, K, codes, ldc, scales, h_out, ldh, nullptr, nullptr, stream);
  if (rank == 16)
    return launch_rows<true, 16>(nc, gate, ldg, up, ldu, M, K, codes, ldc, scales, h_out, ldh, lora_a, lora_t, stream);
  return hipErrorInvalidValue;
}

hipError_t quant_rows_f32(const float* x, int64_t ldx, int64_t M, int K, uint8_t* codes, int64_t ldc, float* scales,
                          hipStream_t stream) {
  if (M == 0) return hipSuccess;
  quant_rows_f32_kernel<<<dim3((unsigned)M), dim3(kQuantThreads), 0, stream>>>(x, ldx, K, codes, ldc, scales);
  return hipGetLastError();
}

}  // namespace jv
