// Internal launchers shared by the C-ABI (capi.hip). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "epilogue.h"

namespace jv {

// Decode regime: M <= kDecodeMaxRows tokens.
constexpr int kDecodeMaxRows = 64;
constexpr int kDecodeWaves = 4;
constexpr int kDecodeUnroll = 4;

struct PrefillTile {
  int bm, bn;
};

int quant_chunks(int K);
hipError_t quant_rows_bf16(const uint16_t* x, int64_t ldx, int64_t M, int K, uint8_t* codes, int64_t ldc, float* scales,
                           const uint16_t* lora_a, int rank, float* lora_t, hipStream_t stream);
hipError_t quant_swiglu_bf16(const uint16_t* gate, int64_t ldg, const uint16_t* up, int64_t ldu, int64_t M, int K,
                             uint8_t* codes, int64_t ldc, float* scales, uint16_t* h_out, int64_t ldh,
                             const uint16_t* lora_a, int rank, float* lora_t, hipStream_t stream);
hipError_t quant_rows_f32(const float* x, int64_t ldx, int64_t M, int K, uint8_t* codes, int64_t ldc, float* scales,
                          hipStream_t stream);

int decode_splits(int64_t N, int64_t K, int cu_count);
hipError_t gemm_decode(const uint8_t* xq, int64_t ldxq, const uint8_t* w, int64_t ldw, int M, int N, int K, int splits,
                       float* partial, int* counters, const Epilogue& ep, int rank, hipStream_t stream);

PrefillTile prefill_tile(int64_t M, int64_t N, int cu_count);
hipError_t gemm_prefill(const uint8_t* xq, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                        const Epilogue& ep, int rank, PrefillTile tile, hipStream_t stream);

}  // namespace jv
