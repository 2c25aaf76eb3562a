// Conformance probes for the GPU tests (built into tests/libjeeves_fp8_testhooks.so,
// never shipped with the product library). They call the same device
// functions as the product kernels (fp8_common.h):
//   * th_encode: e4m3 encode of given floats by the hardware converter and by
//     the spec encoder;
//   * th_encode_sweep: every fp32 bit pattern in a range through both encoders,
//     counting disagreements inside and outside the quantizer's domain;
//   * th_quotient_sweep: every (bf16 x, bf16 row maximum) pair through the
//     quantizer's fast quotient + hardware encode vs IEEE division + spec encode;
//   * th_mfma32 / th_mfma16: one FP8 MFMA on lane-supplied operands, to check
//     the output lane layout the GEMM epilogues assume;
//   * th_silu_sweep: the epilogues' silu on every bf16 input;
//   * th_gemm_form: a plain FP8 GEMM, one wave per output tile, through one of
//     gfx950's FP8 MFMA forms (the two f8f6f4 forms the product kernels use and
//     the older 32x32x16 / 16x16x32 fp8_fp8 forms), to compare their
//     accumulation with the exact product.
#include <stdint.h>

#include "fp8_common.h"

using namespace jv;

namespace {

__global__ void encode_kernel(const float* in, uint8_t* hw, uint8_t* sw, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float f = in[i];
  hw[i] = (uint8_t)(cvt_pk_fp8<false>(f, 0.0f, 0) & 0xFF);
  sw[i] = (uint8_t)e4m3_encode_sw(f);
}

__device__ __forceinline__ bool is_nan_code(uint32_t c) { return (c & 0x7F) == 0x7F; }

// counts[0]: disagreements with |f| <= 449 (the quantizer's domain), counts[1]: elsewhere
// (NaN codes compared by position only), counts[2]: number of domain inputs seen.
__global__ void encode_sweep_kernel(uint32_t start, uint32_t n, unsigned long long* counts, uint32_t* first_bad) {
  __shared__ unsigned long long s[3];
  if (threadIdx.x < 3) s[threadIdx.x] = 0;
  __syncthreads();
  unsigned long long c0 = 0, c1 = 0, c2 = 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const uint32_t bits = start + i;
    const float f = __uint_as_float(bits);
    const uint32_t hw = (uint32_t)cvt_pk_fp8<false>(f, 0.0f, 0) & 0xFF;
    const uint32_t sw = e4m3_encode_sw(f);
    const bool same = hw == sw || (is_nan_code(hw) && is_nan_code(sw));
    const bool domain = fabsf(f) <= 449.0f;
    c2 += domain;
    if (!same) {
      if (domain) {
        ++c0;
        atomicMin(first_bad, bits);
      } else {
        ++c1;
      }
    }
  }
  atomicAdd(&s[0], c0);
  atomicAdd(&s[1], c1);
  atomicAdd(&s[2], c2);
  __syncthreads();
  if (threadIdx.x < 3) atomicAdd(&counts[threadIdx.x], s[threadIdx.x]);
}

// One block per row-maximum pattern a (bf16 magnitude 0 .. 0x7F7F); threads walk
// every bf16 x with |x| <= a. counts[0]: quotient bit disagreements (finite-code
// quotients only), counts[1]: code disagreements, counts[2]: pairs checked.
__global__ void quotient_sweep_kernel(uint32_t a_begin, unsigned long long* counts, uint32_t* first_bad) {
  __shared__ unsigned long long s[3];
  if (threadIdx.x < 3) s[threadIdx.x] = 0;
  __syncthreads();
  const uint32_t amax_bits = a_begin + blockIdx.x;
  const float scale = scale_from_amax_bits(amax_bits);
  const float r = 1.0f / scale;
  unsigned long long c0 = 0, c1 = 0, c2 = 0;
  for (uint32_t xb = threadIdx.x; xb < 65536u; xb += blockDim.x) {
    if ((xb & 0x7FFFu) > amax_bits) continue;
    const float x = bf16_to_f32(xb);
    const float exact = x / scale;
    const float fast = __builtin_copysignf(quotient(x, scale, r), x);
    const uint32_t code_exact = e4m3_encode_sw(exact);
    const uint32_t code_fast = (uint32_t)cvt_pk_fp8<false>(fast, 0.0f, 0) & 0xFF;
    ++c2;
    if (__float_as_uint(exact) != __float_as_uint(fast)) ++c0;
    if (code_exact != code_fast) {
      ++c1;
      atomicMin(first_bad, (amax_bits << 16) | xb);
    }
  }
  atomicAdd(&s[0], c0);
  atomicAdd(&s[1], c1);
  atomicAdd(&s[2], c2);
  __syncthreads();
  if (threadIdx.x < 3) atomicAdd(&counts[threadIdx.x], s[threadIdx.x]);
}

__global__ void mfma32_kernel(const i32x8* a, const i32x8* b, f32x16* d) {
  const int l = threadIdx.x;
  f32x16 acc;
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  d[l] = mfma_32x32x64_fp8(a[l], b[l], acc);
}

__global__ void mfma32_acc_kernel(const i32x8* a, const i32x8* b, const f32x16* c, f32x16* d) {
  const int l = threadIdx.x;
  d[l] = mfma_32x32x64_fp8(a[l], b[l], c[l]);
}

__global__ void mfma16_kernel(const i32x8* a, const i32x8* b, f32x4* d) {
  const int l = threadIdx.x;
  d[l] = mfma_16x16x128_fp8(a[l], b[l], f32x4{0.f, 0.f, 0.f, 0.f});
}

// swiglu_bf16(g, 1.0) = bf16(silu(g)) for every bf16 pattern g (one thread each).
__global__ void silu_sweep_kernel(uint16_t* out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < 65536) out[i] = (uint16_t)swiglu_bf16((uint32_t)i, 0x3F80u);
}

// Form 0: 32x32x64 f8f6f4, 1: 16x16x128 f8f6f4, 2: 32x32x16 fp8_fp8,
// 3: 16x16x32 fp8_fp8. Weights are the A operand (channels = output rows),
// tokens the B operand; lane l loads row l % T of each at k byte
// (l / T) * BYTES of the instruction's k range. y = bf16((acc * sx[m]) * sw[n]),
// or, with sx null, the fp32 sums themselves (y then holds floats).
template <int FORM>
__global__ void gemm_form_kernel(const uint8_t* w, const float* sw, const uint8_t* x, const float* sx, uint16_t* y, int N,
                                 int K) {
  constexpr int T = (FORM == 0 || FORM == 2) ? 32 : 16;
  constexpr int BYTES = FORM < 2 ? 32 : 8;
  constexpr int KI = BYTES * (64 / T);
  constexpr int REGS = T * T / 64;
  typedef float facc __attribute__((ext_vector_type(REGS)));
  const int l = threadIdx.x;
  const int n0 = blockIdx.x * T, m0 = blockIdx.y * T;
  const uint8_t* wr = w + (int64_t)(n0 + l % T) * K + (l / T) * BYTES;
  const uint8_t* xr = x + (int64_t)(m0 + l % T) * K + (l / T) * BYTES;
  facc acc;
  for (int r = 0; r < REGS; ++r) acc[r] = 0.0f;
  for (int k = 0; k < K; k += KI) {
    if constexpr (FORM == 0) {
      acc = mfma_32x32x64_fp8(*reinterpret_cast<const i32x8*>(wr + k), *reinterpret_cast<const i32x8*>(xr + k), acc);
    } else if constexpr (FORM == 1) {
      acc = mfma_16x16x128_fp8(*reinterpret_cast<const i32x8*>(wr + k), *reinterpret_cast<const i32x8*>(xr + k), acc);
    } else if constexpr (FORM == 2) {
      acc = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(*reinterpret_cast<const long*>(wr + k),
                                                       *reinterpret_cast<const long*>(xr + k), acc, 0, 0, 0);
    } else {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(*reinterpret_cast<const long*>(wr + k),
                                                       *reinterpret_cast<const long*>(xr + k), acc, 0, 0, 0);
    }
  }
  for (int r = 0; r < REGS; ++r) {
    const int n = n0 + (T == 32 ? 8 * (r / 4) + 4 * (l / 32) + r % 4 : 4 * (l / 16) + r);
    const int m = m0 + l % T;
    if (sx)
      y[(int64_t)m * N + n] = (uint16_t)f32_to_bf16((acc[r] * sx[m]) * sw[n]);
    else
      reinterpret_cast<float*>(y)[(int64_t)m * N + n] = acc[r];
  }
}

}  // namespace

extern "C" {

// M and N multiples of the form's tile (32 or 16), K of its k range (64, 128,
// 16 or 32 bytes); 1 when they are not. With sx null, y receives M x N fp32
// sums (sw unused).
int th_gemm_form(int form, const uint8_t* w, const float* sw, const uint8_t* x, const float* sx, uint16_t* y, int M,
                 int N, int K, void* stream) {
  if (form < 0 || form > 3 || M <= 0 || N <= 0 || K <= 0) return 1;
  const int T = (form == 0 || form == 2) ? 32 : 16;
  const int KI = (form < 2 ? 32 : 8) * (64 / T);
  if (M % T || N % T || K % KI) return 1;
  const dim3 grid((unsigned)(N / T), (unsigned)(M / T)), block(64);
  hipStream_t s = (hipStream_t)stream;
  if (form == 0) gemm_form_kernel<0><<<grid, block, 0, s>>>(w, sw, x, sx, y, N, K);
  else if (form == 1) gemm_form_kernel<1><<<grid, block, 0, s>>>(w, sw, x, sx, y, N, K);
  else if (form == 2) gemm_form_kernel<2><<<grid, block, 0, s>>>(w, sw, x, sx, y, N, K);
  else gemm_form_kernel<3><<<grid, block, 0, s>>>(w, sw, x, sx, y, N, K);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}


int th_silu_sweep(uint16_t* out, void* stream) {
  silu_sweep_kernel<<<dim3(256), dim3(256), 0, (hipStream_t)stream>>>(out);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int th_encode(const float* in, uint8_t* hw, uint8_t* sw, int64_t n, void* stream) {
  if (n <= 0) return 0;
  encode_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(in, hw, sw, n);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int th_encode_sweep(uint32_t start, uint32_t n, unsigned long long* counts, uint32_t* first_bad, void* stream) {
  encode_sweep_kernel<<<dim3(4096), dim3(256), 0, (hipStream_t)stream>>>(start, n, counts, first_bad);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int th_quotient_sweep(uint32_t a_begin, uint32_t a_count, unsigned long long* counts, uint32_t* first_bad, void* stream) {
  if (a_begin + a_count > 0x7F80u) return 1;
  quotient_sweep_kernel<<<dim3(a_count), dim3(256), 0, (hipStream_t)stream>>>(a_begin, counts, first_bad);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int th_mfma32(const void* a, const void* b, float* d, void* stream) {
  mfma32_kernel<<<dim3(1), dim3(64), 0, (hipStream_t)stream>>>((const i32x8*)a, (const i32x8*)b, (f32x16*)d);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int th_mfma32_acc(const void* a, const void* b, const float* c, float* d, void* stream) {
  mfma32_acc_kernel<<<dim3(1), dim3(64), 0, (hipStream_t)stream>>>((const i32x8*)a, (const i32x8*)b, (const f32x16*)c,
                                                                   (f32x16*)d);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int th_mfma16(const void* a, const void* b, float* d, void* stream) {
  mfma16_kernel<<<dim3(1), dim3(64), 0, (hipStream_t)stream>>>((const i32x8*)a, (const i32x8*)b, (f32x4*)d);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

}  // extern "C"
