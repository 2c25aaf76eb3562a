// Per-row e4m3 quantization on the host CPU, for exporters that run where no
// GPU is present: the reference quantizes checkpoint weights on the CPU
// (inference/fp8_weights.py:16-26, export_fp8.py:32-38). Same arithmetic as
// the device quantizer, bit for bit:
//   amax  = max |w| over the row (NaN if the row holds a NaN),
//   scale = max(amax, 1e-12) * fp32(1/448)      (NaN stays NaN),
//   code  = e4m3fn(w / scale), IEEE fp32 quotient, round to nearest even,
//           NaN (0x7F | sign) beyond 464.
// Rows are split over `threads` host threads; each thread owns whole rows, so
// the result does not depend on the thread count.
#include <stdint.h>

#include <cmath>
#include <thread>
#include <vector>

#include "fp8_common.h"
#include "jeeves_fp8.h"

namespace {

float host_row_scale(const float* w, int64_t cols) {
  float amax = 0.0f;
  bool nan = false;
  for (int64_t c = 0; c < cols; ++c) {
    const float a = std::fabs(w[c]);
    nan |= a != a;
    amax = a > amax ? a : amax;
  }
  if (nan) return std::nanf("");
  return (amax > jv::kScaleClampMin ? amax : jv::kScaleClampMin) * jv::kFp8MaxReciprocal;
}

void host_rows(const float* w, int64_t ldw, int64_t r0, int64_t r1, int64_t cols, uint8_t* codes, int64_t ldc,
               float* scales) {
  for (int64_t r = r0; r < r1; ++r) {
    const float* row = w + r * ldw;
    const float s = host_row_scale(row, cols);
    uint8_t* out = codes + r * ldc;
    for (int64_t c = 0; c < cols; ++c) out[c] = (uint8_t)jv::e4m3_encode_sw(row[c] / s);
    scales[r] = s;
  }
}

}  // namespace

extern "C" int jv_fp8_quantize_rows_host(const float* w, int64_t ldw, int64_t rows, int64_t cols, void* codes,
                                         int64_t ldc, float* scales, int threads) {
  if (rows < 0 || cols <= 0 || ldw < cols || ldc < cols || threads < 0) return JV_ERR_VALUE;
  if (rows == 0) return JV_OK;
  if (!w || !codes || !scales) return JV_ERR_VALUE;
  int n = threads ? threads : (int)std::thread::hardware_concurrency();
  if (n < 1) n = 1;
  if ((int64_t)n > rows) n = (int)rows;
  uint8_t* out = static_cast<uint8_t*>(codes);
  if (n == 1) {
    host_rows(w, ldw, 0, rows, cols, out, ldc, scales);
    return JV_OK;
  }
  std::vector<std::thread> pool;
  pool.reserve(n);
  for (int t = 0; t < n; ++t) {
    const int64_t r0 = rows * t / n, r1 = rows * (t + 1) / n;
    pool.emplace_back(host_rows, w, ldw, r0, r1, cols, out, ldc, scales);
  }
  for (auto& th : pool) th.join();
  return JV_OK;
}
