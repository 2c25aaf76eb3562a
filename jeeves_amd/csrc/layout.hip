// Weight layout conversion for the tiled fragment order (tiled_w_offset):
// one thread per 16-byte unit, row-major side read or written with 16-byte
// vector accesses. Load-time only.
#include "kernels.h"

namespace jv {

template <bool TO_TILED>
__global__ __launch_bounds__(256) void retile_kernel(const uint8_t* __restrict__ src, int64_t lds_, uint8_t* __restrict__ dst,
                                                     int N, int K) {
  // 16-byte units in 32 bits (the launchers reject 2^32 units or more).
  const uint32_t units = (uint32_t)N * (uint32_t)(K >> 4);
  const uint32_t u = blockIdx.x * 256u + threadIdx.x;
  if (u >= units) return;
  const uint32_t per_row = (uint32_t)(K >> 4);
  const int n = (int)(u / per_row), k = (int)(u % per_row) * 16;
  const int64_t tiled = tiled_w_offset(n, k, K >> 7);
  const int64_t plain = (int64_t)n * lds_ + k;
  if (TO_TILED)
    *reinterpret_cast<uint4*>(dst + tiled) = *reinterpret_cast<const uint4*>(src + plain);
  else
    *reinterpret_cast<uint4*>(dst + plain) = *reinterpret_cast<const uint4*>(src + tiled);
}

hipError_t tile_weight(const uint8_t* codes, int64_t ldc, int N, int K, uint8_t* tiled, hipStream_t stream) {
  const int64_t units = (int64_t)N * (K >> 4);
  if (units == 0) return hipSuccess;
  if (units >= (int64_t(1) << 32)) return hipErrorInvalidValue;
  retile_kernel<true><<<dim3((unsigned)((units + 255) / 256)), dim3(256), 0, stream>>>(codes, ldc, tiled, N, K);
  return hipGetLastError();
}

hipError_t untile_weight(const uint8_t* tiled, int N, int K, uint8_t* codes, int64_t ldc, hipStream_t stream) {
  const int64_t units = (int64_t)N * (K >> 4);
  if (units == 0) return hipSuccess;
  if (units >= (int64_t(1) << 32)) return hipErrorInvalidValue;
  retile_kernel<false><<<dim3((unsigned)((units + 255) / 256)), dim3(256), 0, stream>>>(tiled, ldc, codes, N, K);
  return hipGetLastError();
}

}  // namespace jv
