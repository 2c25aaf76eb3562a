// Per-row e4m3fn quantizer kernels on gfx950 (quantize_rows,
// inference/fp8_weights.py:16-19, on token rows of the activations and on
// weight rows at load time): one workgroup per row running quant_row
// (quant_row.h) with one or two 8-element chunks per thread -- 512 threads
// up to K = 4096, 1024 above (the encode is on each thread's critical path:
// measured 4.9 us with 256 threads vs 3.3 us with 1024 at K = 12288, 16
// rows) -- a two-pass kernel for rows longer than 16384, and an fp32-row
// kernel for weights handed over in fp32.
#include "quant_row.h"

namespace jv {

// Threads of the two-pass and fp32 kernels.
constexpr int kQuantThreads = 256;

// Block-wide max of a per-thread 15-bit magnitude.
__device__ __forceinline__ uint32_t block_max(uint32_t v, uint32_t* red) {
  v = wave_max_u32(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  v = red[0];
  for (int i = 1; i < kQuantThreads / 64; ++i) v = max(v, red[i]);
  return v;
}

// Packed codes of more than one 16-token tile: the 16 rows of a tile are
// quantized on one XCD (the hardware hands consecutive workgroups to the 8
// XCDs in turn), so the 16-byte pieces they write into each fragment meet in
// one L2 and reach memory as whole lines. Workgroup b serves row 16 t + j % 16
// of tile t = b % 8 + 8 (j / 16), j = b / 8; -1 past the last tile.
__device__ __forceinline__ int packed_tile_row(int b, int tiles) {
  const int j = b >> 3;
  const int t = (b & 7) + 8 * (j >> 4);
  return t < tiles ? t * 16 + (j & 15) : -1;
}

// NC chunks of 8 elements per thread kept in registers (K <= NC * 8 * THREADS).
// XCD_ROWS: workgroups map to rows through packed_tile_row.
template <int THREADS, int NC, bool SWIGLU, int RANK, bool PACKED, bool XCD_ROWS = false>
__global__ __launch_bounds__(THREADS) void quant_rows_bf16_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ up, int64_t ldu, int K, int M,
    uint8_t* __restrict__ codes, int64_t ldc, float* __restrict__ scales, uint16_t* __restrict__ h_out, int64_t ldh,
    const uint16_t* __restrict__ lora_a, float* __restrict__ lora_t) {
  __shared__ uint32_t lds[quant_row_lds_bytes<THREADS, RANK>() / 4];
  const int prow = XCD_ROWS ? packed_tile_row((int)blockIdx.x, (M + 15) >> 4) : (int)blockIdx.x;
  quant_row<THREADS, NC, SWIGLU, RANK, PACKED>(max(prow, 0), x, ldx, up, ldu, K, M, codes, ldc, scales, h_out, ldh, lora_a,
                                               lora_t, lds, prow >= 0);
}

// Packed codes of h for decode batches from the per-16-channel maxima the
// SwiGLU epilogue stored (parts [M, K/16], bf16 magnitude patterns): with
// each row's maximum known up front, a row splits over K/512 one-wave
// workgroups, one 8-element chunk per lane, instead of one workgroup holding
// the whole row, and the maximum needs no LDS round trip (M = 16, K = 12288,
// back-to-back in a graph: 2.2 us against 3.0 for the one-pass quantizer;
// 128-, 256- and 512-thread workgroups 2.3-2.6 us). Grid (K/512, 16 * tiles);
// a padding row (row >= M) stores zero codes. The maximum over the maxima
// equals the per-element maximum of quant_row, so scales and codes are the
// same bits. Needs K % 128 == 0 and K <= 16384 (at most 256 8-byte quads of
// maxima, four per lane).
__global__ __launch_bounds__(64) void quant_h_maxima_kernel(const uint16_t* __restrict__ h, int64_t ldh,
                                                            const uint16_t* __restrict__ parts, int K, int M,
                                                            uint8_t* __restrict__ codes, float* __restrict__ scales) {
  const int lane = threadIdx.x, row = blockIdx.y;
  const bool real = row < M;
  const int src = min(row, M - 1);
  const int nchunks = K >> 3, nquads = K >> 6;  // quads: 4 maxima, 8 bytes
  const int c = (int)blockIdx.x * 64 + lane;
  // Every load is unconditional (indices clamped; a repeated quad does not
  // change the maximum), so they go out together.
  const uint4 v = *reinterpret_cast<const uint4*>(h + (int64_t)src * ldh + (int64_t)min(c, nchunks - 1) * 8);
  const uint16_t* pr = parts + (int64_t)src * (K >> 4);
  uint32_t am = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint2 p = *reinterpret_cast<const uint2*>(pr + (int64_t)min(lane + 64 * i, nquads - 1) * 4);
    am = pk_max_u16(am, pk_max_u16(p.x, p.y));
  }
  const uint32_t amax_bits = wave_max_u32(max(am & 0xFFFFu, am >> 16));
  const float scale = scale_from_amax_bits(amax_bits);
  if (blockIdx.x == 0 && lane == 0 && real) scales[row] = scale;
  const bool fast = amax_bits < 0x7F80u;
  const float r = 1.0f / scale;
  if (c < nchunks)
    *reinterpret_cast<uint2*>(codes + packed_x_offset(row, c * 8, K >> 7)) =
        real ? encode8(v, scale, r, fast) : uint2{0u, 0u};
}

// Rows longer than the register cache: two passes over the row (the second
// mostly from L2). Plain bf16 rows only.
__global__ __launch_bounds__(kQuantThreads) void quant_rows_bf16_long_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                             int K, uint8_t* __restrict__ codes, int64_t ldc,
                                                                             float* __restrict__ scales) {
  __shared__ uint32_t red[kQuantThreads / 64];
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
  __shared__ float red[kQuantThreads / 64];
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
  bits = __float_as_uint(red[0]);
  for (int i = 1; i < kQuantThreads / 64; ++i) bits = max(bits, __float_as_uint(red[i]));
  const float scale = scale_from_amax_f32(__uint_as_float(bits));
  if (threadIdx.x == 0) scales[row] = scale;
  for (int k = threadIdx.x * 4; k < K; k += kQuantThreads * 4) {
    const float4 v = *reinterpret_cast<const float4*>(xr + k);
    const uint32_t c = e4m3_encode_sw(v.x / scale) | (e4m3_encode_sw(v.y / scale) << 8) |
                       (e4m3_encode_sw(v.z / scale) << 16) | (e4m3_encode_sw(v.w / scale) << 24);
    *reinterpret_cast<uint32_t*>(codes + row * ldc + k) = c;
  }
}

// Register-path shape for rows of K elements: 1 = 512 threads x 1 chunk
// (K <= 4096), 2 = 1024 x 1 (K <= 8192), 3 = 1024 x 2 (K <= 16384); 0 when
// the row needs the two-pass kernel. These minimise one row's latency (the
// encode is on each thread's critical path), which is what decode batches
// see.
int quant_chunks(int K) {
  if (K <= 4096) return 1;
  if (K <= 8192) return 2;
  if (K <= 16384) return 3;
  return 0;
}

// Shape for batches of more than kDecodeMaxRows rows, where throughput
// counts: 256 threads x NC chunks (NC = 1, 2, 4, 6, 8 for K up to 2048, 4096,
// 8192, 12288, 16384): more rows resident per CU and NC loads in flight per
// thread.
static int quant_wide_shape(int K) {
  if (K <= 2048) return 4;
  if (K <= 4096) return 5;
  if (K <= 8192) return 6;
  if (K <= 12288) return 7;
  return 8;
}

template <bool SWIGLU, int RANK, bool PACKED, bool XCD_ROWS>
static hipError_t launch_rows_grid(int shape, const uint16_t* x, int64_t ldx, const uint16_t* up, int64_t ldu, int64_t M,
                                   int K, uint8_t* codes, int64_t ldc, float* scales, uint16_t* h_out, int64_t ldh,
                                   const uint16_t* lora_a, float* lora_t, hipStream_t stream) {
  const int64_t tiles = (M + 15) / 16;
  const dim3 grid((unsigned)(XCD_ROWS ? (tiles + 7) / 8 * 128 : PACKED ? tiles * 16 : M));
  switch (shape) {
    case 1:
      quant_rows_bf16_kernel<512, 1, SWIGLU, RANK, PACKED, XCD_ROWS>
          <<<grid, dim3(512), 0, stream>>>(x, ldx, up, ldu, K, (int)M, codes, ldc, scales, h_out, ldh, lora_a, lora_t);
      break;
    case 2:
      quant_rows_bf16_kernel<1024, 1, SWIGLU, RANK, PACKED, XCD_ROWS>
          <<<grid, dim3(1024), 0, stream>>>(x, ldx, up, ldu, K, (int)M, codes, ldc, scales, h_out, ldh, lora_a, lora_t);
      break;
    case 3:
      quant_rows_bf16_kernel<1024, 2, SWIGLU, RANK, PACKED, XCD_ROWS>
          <<<grid, dim3(1024), 0, stream>>>(x, ldx, up, ldu, K, (int)M, codes, ldc, scales, h_out, ldh, lora_a, lora_t);
      break;
#define JV_QUANT_WIDE(SHAPE, NC)                                                                                         \
    case SHAPE:                                                                                                         \
      quant_rows_bf16_kernel<256, NC, SWIGLU, RANK, PACKED, XCD_ROWS>                                                   \
          <<<grid, dim3(256), 0, stream>>>(x, ldx, up, ldu, K, (int)M, codes, ldc, scales, h_out, ldh, lora_a, lora_t); \
      break;
      JV_QUANT_WIDE(4, 1)
      JV_QUANT_WIDE(5, 2)
      JV_QUANT_WIDE(6, 4)
      JV_QUANT_WIDE(7, 6)
      JV_QUANT_WIDE(8, 8)
#undef JV_QUANT_WIDE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Packed codes of prefill batches (more than kDecodeMaxRows rows) group each
// tile's rows on one XCD; decode batches keep one workgroup per row.
template <bool SWIGLU, int RANK, bool PACKED = false>
static hipError_t launch_rows(int shape, const uint16_t* x, int64_t ldx, const uint16_t* up, int64_t ldu, int64_t M, int K,
                              uint8_t* codes, int64_t ldc, float* scales, uint16_t* h_out, int64_t ldh,
                              const uint16_t* lora_a, float* lora_t, hipStream_t stream) {
  // Above kDecodeMaxRows rows the wide shapes, except rows of up to 4096
  // elements in batches of up to 128 tokens, which keep one 8-element chunk
  // per thread (512 threads; graphs of back-to-back launches, M = 128,
  // K = 4096: 2.36 vs 2.69 us); not with LoRA, so t keeps its summation order.
  if (M > kDecodeMaxRows && !(RANK == 0 && M <= 2 * kDecodeMaxRows && K <= 4096)) shape = quant_wide_shape(K);
  // Long batches of long rows (h of the down projection in prefill): 1024
  // threads x 2 chunks, more bytes in flight per row (graphs of back-to-back
  // launches, K = 12288: 241 vs 269 us at M = 30801, 65.2 vs 67.4 at 8192;
  // at 2048 the 256-thread shape stays ahead, 15.3 vs 15.5). Without LoRA, so
  // t keeps its summation order.
  if (RANK == 0 && K > 8192 && M >= 4096) shape = 3;
  if (PACKED && M > kDecodeMaxRows)
    return launch_rows_grid<SWIGLU, RANK, PACKED, true>(shape, x, ldx, up, ldu, M, K, codes, ldc, scales, h_out, ldh, lora_a,
                                                        lora_t, stream);
  return launch_rows_grid<SWIGLU, RANK, PACKED, false>(shape, x, ldx, up, ldu, M, K, codes, ldc, scales, h_out, ldh, lora_a,
                                                       lora_t, stream);
}

hipError_t quant_rows_bf16(const uint16_t* x, int64_t ldx, int64_t M, int K, uint8_t* codes, int64_t ldc, float* scales,
                           const uint16_t* lora_a, int rank, float* lora_t, bool packed, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  const int nc = quant_chunks(K);
  if (packed) {
    if (nc == 0 || (K & 127)) return hipErrorInvalidValue;
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

hipError_t quant_h_from_maxima(const uint16_t* h, int64_t ldh, const uint16_t* parts, int64_t M, int K, uint8_t* codes,
                               float* scales, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  if (M > 2 * kDecodeMaxRows || K <= 0 || K > 16384 || (K & 127)) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(K / 512 + (K % 512 != 0)), (unsigned)((M + 15) / 16 * 16));
  quant_h_maxima_kernel<<<grid, dim3(64), 0, stream>>>(h, ldh, parts, K, (int)M, codes, scales);
  return hipGetLastError();
}

hipError_t quant_swiglu_bf16(const uint16_t* gate, int64_t ldg, const uint16_t* up, int64_t ldu, int64_t M, int K,
                             uint8_t* codes, int64_t ldc, float* scales, uint16_t* h_out, int64_t ldh,
                             const uint16_t* lora_a, int rank, float* lora_t, bool packed, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  const int nc = quant_chunks(K);
  if (nc == 0) return hipErrorInvalidValue;
  if (packed) {
    if (K & 127) return hipErrorInvalidValue;
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
