// Command-line driver of the host quantizer (jv_fp8_quantize_rows_host) for
// the sanitizer test: reads rows x ldw float32 values from a file, quantizes
// the first `cols` of each row on `threads` host threads into rows x ldc codes
// (plus rows scales) and writes codes then scales to the output file. Buffers
// are allocated at their exact sizes so AddressSanitizer sees any access past
// them.
//   host_quant_driver IN OUT ROWS COLS LDW LDC THREADS
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

extern "C" int jv_fp8_quantize_rows_host(const float* w, int64_t ldw, int64_t rows, int64_t cols, void* codes,
                                         int64_t ldc, float* scales, int threads);

int main(int argc, char** argv) {
  if (argc != 8) {
    fprintf(stderr, "usage: %s IN OUT ROWS COLS LDW LDC THREADS\n", argv[0]);
    return 2;
  }
  const int64_t rows = atoll(argv[3]), cols = atoll(argv[4]), ldw = atoll(argv[5]), ldc = atoll(argv[6]);
  const int threads = atoi(argv[7]);
  std::vector<float> w((size_t)(rows * ldw));
  FILE* in = fopen(argv[1], "rb");
  if (!in || fread(w.data(), sizeof(float), w.size(), in) != w.size()) return 3;
  fclose(in);
  // Code padding keeps a sentinel the test checks: nothing past `cols` is written.
  std::vector<uint8_t> codes((size_t)(rows * ldc), 0xAB);
  std::vector<float> scales((size_t)rows);
  const int rc = jv_fp8_quantize_rows_host(w.data(), ldw, rows, cols, codes.data(), ldc, scales.data(), threads);
  if (rc) return 10 + rc;
  FILE* out = fopen(argv[2], "wb");
  if (!out || fwrite(codes.data(), 1, codes.size(), out) != codes.size() ||
      fwrite(scales.data(), sizeof(float), scales.size(), out) != scales.size())
    return 4;
  fclose(out);
  return 0;
}
