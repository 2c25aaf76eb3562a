// The per-row e4m3fn quantizer as a device function (the body of the
// quantizer kernels in quant.hip): quantize_rows (inference/fp8_weights.py:16-19) on one
// token row,
//
//   scale[m] = max(amax_k |x[m,k]|, 1e-12) * fp32(1/448)
//   code[m,k] = e4m3fn_rne(x[m,k] / scale[m])        (IEEE fp32 quotient)
//
// by one workgroup of THREADS threads. Each thread owns 8-element chunks
// c = tid + i*THREADS and keeps them in registers between the amax pass and
// the encode pass, so memory sees each input byte once. The row maximum is
// taken on the 15-bit bf16 magnitude patterns with packed 16-bit integer
// max, which is exact and propagates NaN (NaN patterns sort above inf).
//
// Variants:
//   * SWIGLU: the row is h = bf16(bf16(silu(gate)) * up) (model/model.py:583),
//     built on the fly from the gate and up halves of a fused projection.
//   * RANK > 0: also emits the LoRA down-projection t[m,r] = sum_k x[m,k] A[r,k]
//     (model/lora.py:128-131) in fp32 from the same registers.
//   * PACKED: codes go to the packed decode layout (packed_x_offset); rows
//     M..16*ceil(M/16)-1 are padding and get zero codes.
#pragma once

#include "fp8_common.h"
#include "kernels.h"

namespace jv {

__device__ __forceinline__ uint32_t swiglu_pair(uint32_t g2, uint32_t u2) {
  return swiglu_bf16(g2 & 0xFFFFu, u2 & 0xFFFFu) | (swiglu_bf16(g2 >> 16, u2 >> 16) << 16);
}

// t[r] += sum over the chunk's 8 elements of x * A[r] for ranks r0 .. r0+RB-1,
// from A's 16-byte chunks av[] of those ranks.
template <int RANK, int RB>
__device__ __forceinline__ void lora_accumulate(float (&t)[RANK > 0 ? RANK : 1], uint4 v, const uint4 (&av)[RB], int r0) {
  if constexpr (RANK > 0) {
    float f[8];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[2 * j] = bf16_to_f32(w[j] & 0xFFFFu);
      f[2 * j + 1] = bf16_to_f32(w[j] >> 16);
    }
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const uint32_t aw[4] = {av[b].x, av[b].y, av[b].z, av[b].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        t[r0 + b] = __builtin_fmaf(f[2 * j], bf16_to_f32(aw[j] & 0xFFFFu), t[r0 + b]);
        t[r0 + b] = __builtin_fmaf(f[2 * j + 1], bf16_to_f32(aw[j] >> 16), t[r0 + b]);
      }
    }
  }
}

// LDS the quantizer needs: one word per wave for the row maximum and, with
// LoRA, RANK partial sums per wave.
template <int THREADS, int RANK>
constexpr int quant_row_lds_bytes() {
  return (THREADS / 64) * 4 * (1 + RANK);
}

template <int THREADS, int NC, bool SWIGLU, int RANK, bool PACKED>
__device__ __forceinline__ void quant_row(int row, const uint16_t* __restrict__ x, int64_t ldx,
                                          const uint16_t* __restrict__ up, int64_t ldu, int K, int M,
                                          uint8_t* __restrict__ codes, int64_t ldc, float* __restrict__ scales,
                                          uint16_t* __restrict__ h_out, int64_t ldh, const uint16_t* __restrict__ lora_a,
                                          float* __restrict__ lora_t, uint32_t* lds, bool active = true) {
  constexpr int NW = THREADS / 64;
  const int tid = threadIdx.x;
  const int nchunks = K >> 3;
  // A padding row of a packed tile (row >= M) runs the same path on the last
  // real row and stores zero codes, no scale; an inactive workgroup (past the
  // last tile) stores nothing. With no branch ahead of the loads, the kernel's
  // argument loads go out together (one scalar round trip before the first
  // row load instead of two).
  const bool real = active && (!PACKED || row < M);
  const int src = PACKED ? min(row, M - 1) : row;
  const uint16_t* xr = x + (int64_t)src * ldx;
  uint4 v[NC];
  uint32_t am = 0;
  float t[RANK > 0 ? RANK : 1];
#pragma unroll
  for (int r = 0; r < (RANK > 0 ? RANK : 1); ++r) t[r] = 0.0f;

  // Every chunk's loads are issued before any is used (the index clamped to
  // the row, so they are unconditional): loads guarded one by one would each
  // wait for the previous chunk's data.
  uint4 u[SWIGLU ? NC : 1];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int64_t c = min(tid + i * THREADS, nchunks - 1);
    v[i] = *reinterpret_cast<const uint4*>(xr + c * 8);
    if constexpr (SWIGLU) u[i] = *reinterpret_cast<const uint4*>(up + (int64_t)src * ldu + c * 8);
  }
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = tid + i * THREADS;
    if constexpr (SWIGLU)
      v[i] = uint4{swiglu_pair(v[i].x, u[i].x), swiglu_pair(v[i].y, u[i].y), swiglu_pair(v[i].z, u[i].z),
                   swiglu_pair(v[i].w, u[i].w)};
    if (c < nchunks) {
      if (SWIGLU && h_out && real) *reinterpret_cast<uint4*>(h_out + (int64_t)row * ldh + (int64_t)c * 8) = v[i];
    } else {
      v[i] = uint4{0, 0, 0, 0};
    }
    am = pk_max_u16(am, v[i].x & 0x7FFF7FFFu);
    am = pk_max_u16(am, v[i].y & 0x7FFF7FFFu);
    am = pk_max_u16(am, v[i].z & 0x7FFF7FFFu);
    am = pk_max_u16(am, v[i].w & 0x7FFF7FFFu);
  }
  if constexpr (RANK > 0) {
    // A's chunks are loaded 8 ranks at a time, the next batch while this
    // batch's FMAs run (scheduling barriers keep them apart: left to itself
    // the compiler keeps only ~5 of them in flight, one L2 round trip per few
    // ranks). Batches of 16 ranks cost occupancy (2-3 waves per SIMD), which
    // 2048-row launches need: 28 -> 34 us there.
    constexpr int RB = RANK > 8 ? 8 : RANK, NB = RANK / RB, G = NC * NB;
    uint4 ab[2][RB];
    auto load_a = [&](int g, uint4 (&dst)[RB]) {
      const int c = min(tid + (g / NB) * THREADS, nchunks - 1), r0 = (g % NB) * RB;
#pragma unroll
      for (int b = 0; b < RB; ++b)
        dst[b] = *reinterpret_cast<const uint4*>(lora_a + (r0 + b) * (int64_t)K + (int64_t)c * 8);
    };
    load_a(0, ab[0]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (g + 1 < G) load_a(g + 1, ab[(g + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      const int i = g / NB;
      if (tid + i * THREADS < nchunks) lora_accumulate<RANK, RB>(t, v[i], ab[g & 1], (g % NB) * RB);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  am = max(am & 0xFFFFu, am >> 16);
  // Workgroup maximum: wave maxima through LDS.
  am = wave_max_u32(am);
  const int lane = tid & 63, wave = tid >> 6;
  if (lane == 0) lds[wave] = am;
  __syncthreads();
  uint32_t amax_bits = lds[0];
#pragma unroll
  for (int wv = 1; wv < NW; ++wv) amax_bits = max(amax_bits, lds[wv]);
  const float scale = scale_from_amax_bits(amax_bits);
  if (tid == 0 && real) scales[row] = scale;
  const bool fast = amax_bits < 0x7F80u;  // finite row: scale finite and > 0
  const float r = 1.0f / scale;
  uint8_t* cr = codes + (PACKED ? 0 : (int64_t)row * ldc);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = tid + i * THREADS;
    if (c < nchunks) {
      const int64_t off = PACKED ? packed_x_offset(row, c * 8, K >> 7) : (int64_t)c * 8;
      if (active) *reinterpret_cast<uint2*>(cr + off) = real ? encode8(v[i], scale, r, fast) : uint2{0u, 0u};
    }
  }
  if constexpr (RANK > 0) {
    float* tred = reinterpret_cast<float*>(lds + NW);
#pragma unroll
    for (int q = 0; q < RANK; ++q) {
      const float s = wave_sum_f32(t[q]);
      if (lane == 0) tred[wave * RANK + q] = s;
    }
    __syncthreads();
    if (tid < RANK && real) {
      float sum = tred[tid];
#pragma unroll
      for (int wv = 1; wv < NW; ++wv) sum += tred[wv * RANK + tid];
      lora_t[(int64_t)row * RANK + tid] = sum;
    }
  }
}

}  // namespace jv
