// C ABI of libjeeves_fp8.so (declared in include/jeeves_fp8.h): argument
// validation, regime dispatch (decode, batch-decode, prefill), workspace carving, and
// per-thread error messages. Launches only; no allocation, no host sync.
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "../../include/jeeves_fp8.h"
#include "kernels.h"

namespace {

thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return JV_OK;
  return fail(JV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];

int cu_count_of(int device) {
  if (device < 0 && hipGetDevice(&device) != hipSuccess) return -1;
  if (device >= kMaxDevices) return -1;
  int v = g_cu_count[device].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n <= 0) return -1;
  g_cu_count[device].store(n, std::memory_order_relaxed);
  return n;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

int check_gemm_shape(int64_t M, int64_t N, int64_t K) {
  if (K <= 0 || K % JV_FP8_BLOCK_K)
    return fail(JV_ERR_VALUE, "the fp8 GEMM needs in_features divisible by %d, got %lld", JV_FP8_BLOCK_K, (long long)K);
  if (M < 0 || N <= 0) return fail(JV_ERR_VALUE, "bad GEMM sizes M=%lld N=%lld", (long long)M, (long long)N);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return fail(JV_ERR_VALUE, "GEMM sizes exceed int32");
  return JV_OK;
}

// Bytes of the decode kernel's split-K partials for these sizes (0 when no
// split).
int64_t split_partial_bytes(int64_t M, int64_t N, int64_t K, int cus) {
  const int s = jv::decode_plan(M, N, K, cus).splits;
  return s > 1 ? round_up((int64_t)s * M * N * 4, 256) : 0;
}

// The same for the fp8 GEMM's kernel choice: decode split-K partials, or the
// prefill tiles' split-K partial tiles.
int64_t partial_bytes(int64_t M, int64_t N, int64_t K, int cus) {
  if (jv::batch_plan(M, N, K, cus, false, nullptr)) return 0;
  if (jv::fp8_decode_kernel_for(M, N, K, cus)) return split_partial_bytes(M, N, K, cus);
  return round_up(jv::prefill_partial_bytes(jv::prefill_tile(M, N, K, cus), M, N), 256);
}

// Activation codes for jv_fp8_linear: the packed fragment order whenever the
// single-pass quantizer covers the row (K <= 16384), row-major above.
bool packed_codes(int64_t K) { return jv::quant_chunks((int)K) != 0; }
int64_t codes_bytes(int64_t M, int64_t K) { return packed_codes(K) ? jv::packed_x_bytes(M, K) : M * K; }

// swiglu_half > 0: the fused SwiGLU epilogue (N = 2 swiglu_half weight rows,
// gate then up; y is h [M, swiglu_half]; h_amax the optional maxima).
int run_gemm(const uint8_t* xq, int64_t ldxq, bool packed_x, const float* sx, const uint8_t* w, int64_t ldw, const float* sw,
             const uint16_t* bias, const float* lora_t, const uint16_t* lora_b, int64_t rank, float lora_scaling, uint16_t* y,
             int64_t ldy, int64_t M, int64_t N, int64_t K, uint8_t* partial_ws, int64_t partial_ws_bytes,
             int32_t* counters, int64_t n_counters, hipStream_t stream, int64_t swiglu_half = 0,
             uint16_t* h_amax = nullptr) {
  const int cus = cu_count_of(-1);
  if (cus <= 0) return fail(JV_ERR_HIP, "cannot query the device's compute units");
  if ((uint64_t)M * (uint64_t)ldxq >= (1ull << 32) || (uint64_t)jv::packed_x_bytes(M, K) >= (1ull << 32))
    return fail(JV_ERR_VALUE, "operands above 4 GiB are not supported");
  jv::Epilogue ep{sx, sw, bias, lora_t, lora_b, lora_scaling, y, ldy, swiglu_half, h_amax};
  jv::BatchPlan batch;
  if (jv::batch_plan(M, N, K, cus, swiglu_half != 0, &batch))
    return hip_status(jv::gemm_batch(xq, ldxq, packed_x, w, ldw, (int)M, (int)N, (int)K, batch, ep, (int)rank, stream),
                      "fp8 batch GEMM launch");
  if (jv::fp8_decode_kernel_for(M, N, K, cus)) {
    const jv::DecodePlan plan = jv::decode_plan(M, N, K, cus, swiglu_half != 0);
    const int splits = plan.splits;
    float* partial = nullptr;
    if (splits > 1) {
      const int64_t tiles = plan.groups;
      if (!counters || tiles > n_counters)
        return fail(JV_ERR_VALUE, "%lld tiles exceed the %lld tile counters", (long long)tiles, (long long)n_counters);
      const int64_t need = (int64_t)splits * M * N * 4;
      if (!partial_ws || partial_ws_bytes < need)
        return fail(JV_ERR_VALUE, "workspace too small for split-K partials: %lld < %lld bytes", (long long)partial_ws_bytes,
                    (long long)need);
      partial = reinterpret_cast<float*>(partial_ws);
    }
    return hip_status(jv::gemm_decode(xq, ldxq, packed_x, w, ldw, (int)M, (int)N, (int)K, plan, partial, counters, ep, (int)rank,
                                      stream),
                      "fp8 decode GEMM launch");
  }
  // The fused SwiGLU GEMM takes the plan of the plain GEMM of the same weight
  // (a K split included), so its gate and up values are bitwise those.
  const jv::PrefillTile tile = jv::prefill_tile(M, N, K, cus);
  float* partials = nullptr;
  if (tile.splits > 1) {
    const int64_t tiles = jv::prefill_counters(tile, M, N);
    if (!counters || tiles > n_counters)
      return fail(JV_ERR_VALUE, "%lld tiles exceed the %lld tile counters", (long long)tiles, (long long)n_counters);
    const int64_t need = jv::prefill_partial_bytes(tile, M, N);
    if (!partial_ws || partial_ws_bytes < need)
      return fail(JV_ERR_VALUE, "workspace too small for split-K partials: %lld < %lld bytes", (long long)partial_ws_bytes,
                  (long long)need);
    partials = reinterpret_cast<float*>(partial_ws);
  }
  return hip_status(jv::gemm_prefill(xq, packed_x ? 0 : ldxq, w, ldw, (int)M, (int)N, (int)K, ep, (int)rank, tile, partials,
                                     counters, stream),
                    "fp8 prefill GEMM launch");
}

// ldw = 0 selects the tiled weight layout (tiled_w_offset), which needs
// whole 16-row tiles; a row-major ldw must cover a row.
int check_weight(int64_t N, int64_t K, int64_t ldw, const void* w) {
  if (!aligned16(w)) return fail(JV_ERR_VALUE, "weight codes must be 16-byte aligned");
  if (ldw == 0) {
    if (N % 16) return fail(JV_ERR_VALUE, "tiled weights need out_features divisible by 16, got %lld", (long long)N);
    if ((uint64_t)N * (uint64_t)K >= (1ull << 32)) return fail(JV_ERR_VALUE, "operands above 4 GiB are not supported");
    return JV_OK;
  }
  if (ldw % 16 || ldw < K) return fail(JV_ERR_VALUE, "weight row stride %lld must be a multiple of 16 and >= K", (long long)ldw);
  if ((uint64_t)N * (uint64_t)ldw >= (1ull << 32)) return fail(JV_ERR_VALUE, "operands above 4 GiB are not supported");
  return JV_OK;
}

int check_lora(int64_t rank, const void* a_or_t, const void* b) {
  if (rank == 0) return JV_OK;
  if (rank != 16) return fail(JV_ERR_VALUE, "LoRA rank %lld is not supported (16 is)", (long long)rank);
  if (!a_or_t || !b) return fail(JV_ERR_VALUE, "LoRA rank %lld given without its matrices", (long long)rank);
  return JV_OK;
}

// ---------------------------------------------------------------------------
// Scratch of the no-allocation entry point (jv_fp8_linear_noalloc): one
// file-scope device array per GPU the library runs on, held until the process
// ends -- the tile counters first, then jv_fp8_linear's workspace. In host code
// `scratch` is only a stand-in for the symbol; its device address comes from
// hipGetSymbolAddress, once per device with that device current, and only that
// address is handed to kernels.
constexpr int64_t kNoAllocCounterSlots = 4096;
constexpr int64_t kNoAllocCounterBytes = kNoAllocCounterSlots * 4;
constexpr int64_t kNoAllocWorkspaceBytes = JV_FP8_NOALLOC_SCRATCH_BYTES - kNoAllocCounterBytes;
static_assert(kNoAllocCounterBytes % 256 == 0, "workspace alignment");
static __device__ __align__(256) uint8_t scratch[JV_FP8_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
std::atomic<uint8_t*> g_scratch[kMaxDevices];

// The calling thread's current device's scratch address. The tile counters at
// its start are zero without a clear: a __device__ array without initializer
// is zero-filled when the code object is loaded onto the device (static
// storage), and every kernel that counts in leaves its counters at zero. So the
// first call puts nothing on `stream` beyond its own launches, and may itself
// be captured into a graph.
int scratch_of_current_device(uint8_t** out) {
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices)
    return fail(JV_ERR_HIP, "cannot query the current HIP device");
  uint8_t* p = g_scratch[device].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[device].load(std::memory_order_relaxed);
    if (!p) {
      if (int rc = hip_status(hipGetSymbolAddress(reinterpret_cast<void**>(&p), HIP_SYMBOL(scratch)),
                              "no-allocation scratch address"))
        return rc;
      g_scratch[device].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return JV_OK;
}

}  // namespace

extern "C" {

const char* jv_fp8_last_error(void) { return g_last_error; }

int jv_device_cu_count(int device) { return cu_count_of(device); }

int jv_fp8_quantize_rows_bf16(const void* x, int64_t ldx, int64_t rows, int64_t cols, void* codes, int64_t ldc,
                              float* scales, void* stream) {
  if (rows < 0 || cols <= 0 || cols % 8 || cols > INT32_MAX || rows > INT32_MAX)
    return fail(JV_ERR_VALUE, "quantize_rows needs a positive column count divisible by 8, got %lld", (long long)cols);
  if (rows == 0) return JV_OK;
  const bool packed = ldc == 0;
  if (packed && (cols % JV_FP8_BLOCK_K || jv::quant_chunks((int)cols) == 0))
    return fail(JV_ERR_VALUE, "the packed layout needs a column count divisible by %d up to 16384", JV_FP8_BLOCK_K);
  if (!aligned16(x) || (ldx * 2) % 16 || !aligned16(codes) || ldc % 16)
    return fail(JV_ERR_VALUE, "quantize_rows needs 16-byte aligned rows");
  return hip_status(jv::quant_rows_bf16((const uint16_t*)x, ldx, rows, (int)cols, (uint8_t*)codes, ldc, scales, nullptr, 0,
                                        nullptr, packed, (hipStream_t)stream),
                    "quantize_rows launch");
}

int64_t jv_fp8_packed_codes_bytes(int64_t rows, int64_t cols) {
  if (rows < 0 || rows > INT32_MAX || cols <= 0 || cols > INT32_MAX || cols % JV_FP8_BLOCK_K) return -1;
  return jv::packed_x_bytes(rows, cols);
}

int jv_fp8_quantize_rows_f32(const float* x, int64_t ldx, int64_t rows, int64_t cols, void* codes, int64_t ldc,
                             float* scales, void* stream) {
  if (rows < 0 || cols <= 0 || cols % 4 || cols > INT32_MAX || rows > INT32_MAX)
    return fail(JV_ERR_VALUE, "quantize_rows needs a positive column count divisible by 4, got %lld", (long long)cols);
  if (rows == 0) return JV_OK;
  if (!aligned16(x) || (ldx * 4) % 16 || (reinterpret_cast<uintptr_t>(codes) & 3) || ldc % 4)
    return fail(JV_ERR_VALUE, "quantize_rows needs 16-byte aligned rows");
  return hip_status(jv::quant_rows_f32(x, ldx, rows, (int)cols, (uint8_t*)codes, ldc, scales, (hipStream_t)stream),
                    "quantize_rows launch");
}

int64_t jv_fp8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  const int cus = cu_count_of(-1);
  if (cus <= 0) return -1;
  return partial_bytes(M, N, K, cus);
}

int64_t jv_fp8_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t lora_rank) {
  const int cus = cu_count_of(-1);
  if (cus <= 0) return -1;
  return round_up(codes_bytes(M, K), 256) + round_up(M * 4, 256) + round_up(M * lora_rank * 4, 256) + partial_bytes(M, N, K, cus);
}

int jv_fp8_gemm(const void* xq, int64_t ldxq, const float* x_scale, const void* w, int64_t ldw, const float* w_scale,
                const void* bias, const float* lora_t, const void* lora_b, int64_t lora_rank, float lora_scaling, void* y,
                int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                int32_t* tile_counters, int64_t n_counters, void* stream) {
  if (int rc = check_gemm_shape(M, N, K)) return rc;
  if (int rc = check_lora(lora_rank, lora_t, lora_b)) return rc;
  if (M == 0) return JV_OK;
  const bool packed = ldxq == 0;
  if (!aligned16(xq) || ldxq % 16) return fail(JV_ERR_VALUE, "the fp8 GEMM needs 16-byte aligned operand rows");
  if (int rc = check_weight(N, K, ldw, w)) return rc;
  return run_gemm((const uint8_t*)xq, ldxq, packed, x_scale, (const uint8_t*)w, ldw, w_scale, (const uint16_t*)bias, lora_t,
                  (const uint16_t*)lora_b, lora_rank, lora_scaling, (uint16_t*)y, ldy, M, N, K, (uint8_t*)workspace,
                  workspace_bytes, tile_counters, n_counters, (hipStream_t)stream);
}

int jv_fp8_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* w_scale, const void* bias,
                  const void* lora_a, const void* lora_b, int64_t lora_rank, float lora_scaling, void* y, int64_t ldy,
                  int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, int32_t* tile_counters,
                  int64_t n_counters, void* stream) {
  if (int rc = check_gemm_shape(M, N, K)) return rc;
  if (int rc = check_lora(lora_rank, lora_a, lora_b)) return rc;
  if (M == 0) return JV_OK;
  if (!aligned16(x) || (ldx * 2) % 16) return fail(JV_ERR_VALUE, "the fp8 GEMM needs 16-byte aligned operand rows");
  if (int rc = check_weight(N, K, ldw, w)) return rc;
  if (lora_rank && jv::quant_chunks((int)K) == 0)
    return fail(JV_ERR_VALUE, "LoRA needs in_features <= 16384, got %lld", (long long)K);
  const int64_t need = jv_fp8_linear_workspace_bytes(M, N, K, lora_rank);
  if (need < 0) return fail(JV_ERR_HIP, "cannot query the device's compute units");
  if (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(JV_ERR_VALUE, "workspace needs %lld bytes, 256-byte aligned", (long long)need);
  uint8_t* ws = (uint8_t*)workspace;
  uint8_t* codes = ws;
  const bool packed = packed_codes(K);
  ws += round_up(codes_bytes(M, K), 256);
  float* sx = (float*)ws;
  ws += round_up(M * 4, 256);
  float* lora_t = lora_rank ? (float*)ws : nullptr;
  ws += round_up(M * lora_rank * 4, 256);
  const int64_t rest = workspace_bytes - (ws - (uint8_t*)workspace);
  hipStream_t s = (hipStream_t)stream;
  if (int rc = hip_status(jv::quant_rows_bf16((const uint16_t*)x, ldx, M, (int)K, codes, K, sx, (const uint16_t*)lora_a,
                                              (int)lora_rank, lora_t, packed, s),
                          "activation quantization launch"))
    return rc;
  return run_gemm(codes, packed ? 0 : K, packed, sx, (const uint8_t*)w, ldw, w_scale, (const uint16_t*)bias, lora_t, (const uint16_t*)lora_b,
                  lora_rank, lora_scaling, (uint16_t*)y, ldy, M, N, K, ws, rest, tile_counters, n_counters, s);
}

int64_t jv_w8a16_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  const int cus = cu_count_of(-1);
  if (cus <= 0) return -1;
  if (jv::w8a16_batch_plan(M, N, K, cus, nullptr)) return 0;
  if (jv::w8a16_decode_kernel_for(M, N, cus)) return split_partial_bytes(M, N, K, cus);
  return round_up(jv::w8a16_prefill_partial_bytes(M, N, K, cus), 256);
}

int jv_w8a16_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* w_scale, const void* bias,
                    void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                    int32_t* tile_counters, int64_t n_counters, void* stream) {
  if (int rc = check_gemm_shape(M, N, K)) return rc;
  if (M == 0) return JV_OK;
  if (!aligned16(x) || (ldx * 2) % 16) return fail(JV_ERR_VALUE, "the W8A16 GEMM needs 16-byte aligned operand rows");
  if (int rc = check_weight(N, K, ldw, w)) return rc;
  if ((uint64_t)M * (uint64_t)ldx * 2 >= (1ull << 32)) return fail(JV_ERR_VALUE, "operands above 4 GiB are not supported");
  const int cus = cu_count_of(-1);
  if (cus <= 0) return fail(JV_ERR_HIP, "cannot query the device's compute units");
  hipStream_t s = (hipStream_t)stream;
  jv::BatchPlan batch;
  if (jv::w8a16_batch_plan(M, N, K, cus, &batch))
    return hip_status(jv::w8a16_batch((const uint16_t*)x, ldx, (const uint8_t*)w, ldw, (int)M, (int)N, (int)K, batch, w_scale,
                                      (const uint16_t*)bias, (uint16_t*)y, ldy, s),
                      "W8A16 batch GEMM launch");
  if (!jv::w8a16_decode_kernel_for(M, N, cus)) {
    const int splits = jv::w8a16_prefill_splits(M, N, K, cus);
    float* partials = nullptr;
    if (splits > 1) {
      const int64_t tiles = jv::w8a16_prefill_counters(M, N, K, cus);
      if (!tile_counters || tiles > n_counters)
        return fail(JV_ERR_VALUE, "%lld tiles exceed the %lld tile counters", (long long)tiles, (long long)n_counters);
      const int64_t need = jv::w8a16_prefill_partial_bytes(M, N, K, cus);
      if (!workspace || workspace_bytes < need)
        return fail(JV_ERR_VALUE, "workspace too small for split-K partials: %lld < %lld bytes", (long long)workspace_bytes,
                    (long long)need);
      partials = reinterpret_cast<float*>(workspace);
    }
    return hip_status(jv::w8a16_prefill((const uint16_t*)x, ldx, (const uint8_t*)w, ldw, (int)M, (int)N, (int)K, w_scale,
                                        (const uint16_t*)bias, (uint16_t*)y, ldy, splits, partials, tile_counters, cus, s),
                      "W8A16 prefill GEMM launch");
  }
  const jv::DecodePlan plan = jv::decode_plan(M, N, K, cus);
  float* partial = nullptr;
  if (plan.splits > 1) {
    if (!tile_counters || plan.groups > n_counters)
      return fail(JV_ERR_VALUE, "%lld tiles exceed the %lld tile counters", (long long)plan.groups, (long long)n_counters);
    const int64_t need = (int64_t)plan.splits * M * N * 4;
    if (!workspace || workspace_bytes < need)
      return fail(JV_ERR_VALUE, "workspace too small for split-K partials: %lld < %lld bytes", (long long)workspace_bytes,
                  (long long)need);
    partial = reinterpret_cast<float*>(workspace);
  }
  return hip_status(jv::w8a16_decode((const uint16_t*)x, ldx, (const uint8_t*)w, ldw, (int)M, (int)N, (int)K, plan, partial,
                                     tile_counters, w_scale, (const uint16_t*)bias, (uint16_t*)y, ldy, s),
                    "W8A16 decode GEMM launch");
}

int jv_fp8_swiglu_quantize(const void* gate, int64_t ldg, const void* up, int64_t ldu, int64_t M, int64_t I, void* codes,
                           int64_t ldc, float* scales, void* h_out, int64_t ldh, const void* lora_a, int64_t lora_rank,
                           float* lora_t, void* stream) {
  if (M < 0 || I <= 0 || I % 8 || jv::quant_chunks((int)(I > INT32_MAX ? 0 : I)) == 0 || I > INT32_MAX)
    return fail(JV_ERR_VALUE, "swiglu_quantize needs 0 < I <= 16384 divisible by 8, got %lld", (long long)I);
  if (int rc = check_lora(lora_rank, lora_a, lora_t)) return rc;
  if (M == 0) return JV_OK;
  const bool packed = ldc == 0;
  if (packed && I % JV_FP8_BLOCK_K)
    return fail(JV_ERR_VALUE, "the packed layout needs I divisible by %d", JV_FP8_BLOCK_K);
  if (!aligned16(gate) || (ldg * 2) % 16 || !aligned16(up) || (ldu * 2) % 16 || !aligned16(codes) || ldc % 16 ||
      (h_out && (!aligned16(h_out) || (ldh * 2) % 16)))
    return fail(JV_ERR_VALUE, "swiglu_quantize needs 16-byte aligned rows");
  return hip_status(jv::quant_swiglu_bf16((const uint16_t*)gate, ldg, (const uint16_t*)up, ldu, M, (int)I, (uint8_t*)codes,
                                          ldc, scales, (uint16_t*)h_out, ldh, (const uint16_t*)lora_a, (int)lora_rank,
                                          lora_t, packed, (hipStream_t)stream),
                    "swiglu_quantize launch");
}

int jv_fp8_tile_weight(const void* codes, int64_t ldc, int64_t N, int64_t K, void* tiled, void* stream) {
  if (N < 0 || N % 16 || K <= 0 || K % JV_FP8_BLOCK_K || N > INT32_MAX || K > INT32_MAX)
    return fail(JV_ERR_VALUE, "tiling needs N divisible by 16 and K by %d, got N=%lld K=%lld", JV_FP8_BLOCK_K, (long long)N,
                (long long)K);
  if (!aligned16(codes) || !aligned16(tiled) || ldc % 16 || ldc < K)
    return fail(JV_ERR_VALUE, "tiling needs 16-byte aligned rows");
  if (codes == tiled) return fail(JV_ERR_VALUE, "tiling cannot run in place");
  return hip_status(jv::tile_weight((const uint8_t*)codes, ldc, (int)N, (int)K, (uint8_t*)tiled, (hipStream_t)stream),
                    "weight tiling launch");
}

int jv_fp8_untile_weight(const void* tiled, int64_t N, int64_t K, void* codes, int64_t ldc, void* stream) {
  if (N < 0 || N % 16 || K <= 0 || K % JV_FP8_BLOCK_K || N > INT32_MAX || K > INT32_MAX)
    return fail(JV_ERR_VALUE, "untiling needs N divisible by 16 and K by %d, got N=%lld K=%lld", JV_FP8_BLOCK_K, (long long)N,
                (long long)K);
  if (!aligned16(codes) || !aligned16(tiled) || ldc % 16 || ldc < K)
    return fail(JV_ERR_VALUE, "untiling needs 16-byte aligned rows");
  if (codes == tiled) return fail(JV_ERR_VALUE, "untiling cannot run in place");
  return hip_status(jv::untile_weight((const uint8_t*)tiled, (int)N, (int)K, (uint8_t*)codes, ldc, (hipStream_t)stream),
                    "weight untiling launch");
}

int jv_fp8_split_for(int64_t M, int64_t N, int64_t K, int cu_count) {
  if (K <= 0 || N <= 0 || M <= 0 || cu_count <= 0) return 1;
  if (jv::batch_plan(M, N, K, cu_count, false, nullptr)) return 1;
  if (!jv::fp8_decode_kernel_for(M, N, K, cu_count)) return jv::prefill_tile(M, N, K, cu_count).splits;
  return jv::decode_plan(M, N, K, cu_count).splits;
}

int64_t jv_fp8_counters_needed(int64_t M, int64_t N, int64_t K, int cu_count) {
  if (K <= 0 || N <= 0 || M <= 0 || cu_count <= 0) return 0;
  if (jv::batch_plan(M, N, K, cu_count, false, nullptr)) return 0;
  if (!jv::fp8_decode_kernel_for(M, N, K, cu_count)) return jv::prefill_counters(jv::prefill_tile(M, N, K, cu_count), M, N);
  const jv::DecodePlan p = jv::decode_plan(M, N, K, cu_count);
  return p.splits > 1 ? p.groups : 0;
}

int jv_fp8_launch_shape(int64_t M, int64_t N, int64_t K, int cu_count, int32_t* shape) {
  if (!shape) return fail(JV_ERR_VALUE, "shape needs 4 slots");
  if (int rc = check_gemm_shape(M, N, K)) return rc;
  if (M <= 0 || cu_count <= 0) return fail(JV_ERR_VALUE, "launch shape needs M > 0 and a CU count");
  jv::BatchPlan b;
  if (jv::batch_plan(M, N, K, cu_count, false, &b)) {
    shape[0] = 3;
    shape[1] = b.groups * b.msplit;
    shape[2] = 64 * b.waves;
    shape[3] = 1;
    return JV_OK;
  }
  if (jv::fp8_decode_kernel_for(M, N, K, cu_count)) {
    const jv::DecodePlan p = jv::decode_plan(M, N, K, cu_count);
    shape[0] = 0;
    shape[1] = p.groups * p.splits;
    shape[2] = 64 * p.waves;
    shape[3] = p.splits;
    return JV_OK;
  }
  const jv::PrefillTile t = jv::prefill_tile(M, N, K, cu_count);
  const int64_t tiles = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
  shape[0] = t.pingpong ? 2 : 1;
  shape[1] = (int32_t)(tiles * t.splits);
  shape[2] = t.pingpong ? 512 : 64 * t.wgm * t.wgn;
  shape[3] = t.splits;
  return JV_OK;
}

int jv_fp8_linear_noalloc(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* w_scale, const void* bias,
                          const void* lora_a, const void* lora_b, int64_t lora_rank, float lora_scaling, void* y,
                          int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream) {
  if (int rc = check_gemm_shape(M, N, K)) return rc;
  if (int rc = check_lora(lora_rank, lora_a, lora_b)) return rc;
  if (M == 0) return JV_OK;
  const int64_t need = jv_fp8_linear_workspace_bytes(M, N, K, lora_rank);
  if (need < 0) return fail(JV_ERR_HIP, "cannot query the device's compute units");
  if (need > kNoAllocWorkspaceBytes)
    return fail(JV_ERR_VALUE,
                "jv_fp8_linear_noalloc: M=%lld N=%lld K=%lld needs %lld bytes of scratch, more than its %lld; call "
                "jv_fp8_linear with a workspace instead",
                (long long)M, (long long)N, (long long)K, (long long)need, (long long)kNoAllocWorkspaceBytes);
  uint8_t* base = nullptr;
  if (int rc = scratch_of_current_device(&base)) return rc;
  return jv_fp8_linear(x, ldx, w, ldw, w_scale, bias, lora_a, lora_b, lora_rank, lora_scaling, y, ldy, M, N, K,
                       base + kNoAllocCounterBytes, kNoAllocWorkspaceBytes, reinterpret_cast<int32_t*>(base),
                       kNoAllocCounterSlots, stream);
}

int jv_fp8_linear_swiglu(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* w_scale, const void* bias,
                         const void* lora_a, const void* lora_b, int64_t lora_rank, float lora_scaling, void* h,
                         int64_t ldh, uint16_t* h_amax, int64_t M, int64_t I, int64_t K, void* workspace,
                         int64_t workspace_bytes, int32_t* tile_counters, int64_t n_counters, void* stream) {
  if (I <= 0 || I % 16 || 2 * I > INT32_MAX)
    return fail(JV_ERR_VALUE, "the fused SwiGLU needs an intermediate size divisible by 16, got %lld", (long long)I);
  if (int rc = check_gemm_shape(M, 2 * I, K)) return rc;
  if (int rc = check_lora(lora_rank, lora_a, lora_b)) return rc;
  if (!packed_codes(K)) return fail(JV_ERR_VALUE, "the fused SwiGLU needs in_features <= 16384, got %lld", (long long)K);
  if (M == 0) return JV_OK;
  if (!aligned16(x) || (ldx * 2) % 16) return fail(JV_ERR_VALUE, "the fp8 GEMM needs 16-byte aligned operand rows");
  if (!h || ldh < I) return fail(JV_ERR_VALUE, "h needs a row stride of at least %lld", (long long)I);
  if (!aligned16(h) || (ldh * 2) % 16) return fail(JV_ERR_VALUE, "h needs 16-byte aligned rows");
  if (h_amax && (reinterpret_cast<uintptr_t>(h_amax) & 1))
    return fail(JV_ERR_VALUE, "h_amax must be 2-byte aligned (uint16 maxima)");
  if (int rc = check_weight(2 * I, K, ldw, w)) return rc;
  const int cus = cu_count_of(-1);
  if (cus <= 0) return fail(JV_ERR_HIP, "cannot query the device's compute units");
  const int64_t pbytes = partial_bytes(M, 2 * I, K, cus);
  const int64_t need =
      round_up(codes_bytes(M, K), 256) + round_up(M * 4, 256) + round_up(M * lora_rank * 4, 256) + pbytes;
  if (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(JV_ERR_VALUE, "workspace needs %lld bytes, 256-byte aligned", (long long)need);
  uint8_t* ws = (uint8_t*)workspace;
  uint8_t* codes = ws;
  ws += round_up(codes_bytes(M, K), 256);
  float* sx = (float*)ws;
  ws += round_up(M * 4, 256);
  float* lora_t = lora_rank ? (float*)ws : nullptr;
  ws += round_up(M * lora_rank * 4, 256);
  hipStream_t s = (hipStream_t)stream;
  if (int rc = hip_status(jv::quant_rows_bf16((const uint16_t*)x, ldx, M, (int)K, codes, K, sx, (const uint16_t*)lora_a,
                                              (int)lora_rank, lora_t, true, s),
                          "activation quantization launch"))
    return rc;
  return run_gemm(codes, 0, true, sx, (const uint8_t*)w, ldw, w_scale, (const uint16_t*)bias, lora_t,
                  (const uint16_t*)lora_b, lora_rank, lora_scaling, (uint16_t*)h, ldh, M, 2 * I, K, pbytes ? ws : nullptr,
                  pbytes, tile_counters, n_counters, s, I, h_amax);
}

int jv_fp8_quantize_swiglu_output(const void* h, int64_t ldh, const uint16_t* h_amax, int64_t M, int64_t I, void* codes,
                                  int64_t ldc, float* scales, const void* lora_a, int64_t lora_rank, float* lora_t,
                                  void* stream) {
  if (M < 0 || I <= 0 || I % 16 || jv::quant_chunks((int)(I > INT32_MAX ? 0 : I)) == 0 || M > INT32_MAX)
    return fail(JV_ERR_VALUE, "quantizing h needs 0 < I <= 16384 divisible by 16, got %lld", (long long)I);
  if (int rc = check_lora(lora_rank, lora_a, lora_t)) return rc;
  if (M == 0) return JV_OK;
  const bool packed = ldc == 0;
  if (packed && I % JV_FP8_BLOCK_K) return fail(JV_ERR_VALUE, "the packed layout needs I divisible by %d", JV_FP8_BLOCK_K);
  if (!aligned16(h) || (ldh * 2) % 16 || !aligned16(codes) || ldc % 16)
    return fail(JV_ERR_VALUE, "quantizing h needs 16-byte aligned rows");
  // Decode batches (up to 128 tokens) split each row over workgroups when its
  // maximum comes from h_amax; elsewhere the maximum is taken from h in the
  // pass that encodes it.
  if (h_amax && packed && lora_rank == 0 && M <= 2 * jv::kDecodeMaxRows && (reinterpret_cast<uintptr_t>(h_amax) & 7) == 0)
    return hip_status(jv::quant_h_from_maxima((const uint16_t*)h, ldh, h_amax, M, (int)I, (uint8_t*)codes, scales,
                                              (hipStream_t)stream),
                      "quantization of h launch");
  return hip_status(jv::quant_rows_bf16((const uint16_t*)h, ldh, M, (int)I, (uint8_t*)codes, ldc, scales,
                                        (const uint16_t*)lora_a, (int)lora_rank, lora_t, packed, (hipStream_t)stream),
                    "quantization of h launch");
}

}  // extern "C"
