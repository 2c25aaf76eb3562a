// Small-M FP8 x FP8 GEMM (decode: M <= 64 tokens), HBM-bound on the weights.
//
// Counterpart of _fp8_matmul's split-K regime (inference/fp8.py:62-99,
// :118-123), redesigned for CDNA4:
//   * weights are the MFMA "A" side (16 output channels x 128 k per
//     v_mfma_f32_16x16x128_f8f6f4) and tokens the "B" side, up to 4 token
//     tiles of 16 (swap-AB, as inference/fp8.py:69 does);
//   * each lane streams 32 contiguous bytes of one weight row per 128-k step
//     straight from HBM into the MFMA operand registers (no LDS round trip),
//     UNROLL steps in flight per wave;
//   * a workgroup owns 16 weight rows; its WAVES waves split the workgroup's
//     k range and are summed through LDS in wave order; when there are fewer
//     16-row tiles than CUs, workgroups also split K (grid.y) and the last
//     workgroup to finish a tile sums the fp32 partials in split order, then
//     resets the tile's counter -- one launch, deterministic, capture-safe.
#include "epilogue.h"
#include "kernels.h"

namespace jv {

template <int MT, int WAVES, int UNROLL, int RANK>
__global__ __launch_bounds__(64 * WAVES) void gemm_decode_kernel(const uint8_t* __restrict__ xq, int64_t ldxq,
                                                                 const uint8_t* __restrict__ w, int64_t ldw, int M, int N,
                                                                 int K, int splits, float* __restrict__ partial,
                                                                 int* __restrict__ counters, Epilogue ep) {
  __shared__ f32x4 red[WAVES][MT][64];
  __shared__ int is_last;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tile = blockIdx.x;
  const int split = blockIdx.y;
  const int n0 = tile * 16;

  const int ksteps = K >> 7;
  const int slices = splits * WAVES;
  const int slice = split * WAVES + wave;
  const int s_begin = (int)((int64_t)ksteps * slice / slices);
  const int s_end = (int)((int64_t)ksteps * (slice + 1) / slices);

  const int li = lane & 15;
  const int lk = (lane >> 4) * 32;
  const uint8_t* wp = w + (int64_t)min(n0 + li, N - 1) * ldw + lk;
  const uint8_t* xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xp[mt] = xq + (int64_t)min(mt * 16 + li, M - 1) * ldxq + lk;

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  int s = s_begin;
  for (; s + UNROLL <= s_end; s += UNROLL) {
    i32x4 wa[UNROLL][2];
    i32x4 xa[UNROLL][MT][2];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int64_t off = (int64_t)(s + u) * 128;
      wa[u][0] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(wp + off));
      wa[u][1] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(wp + off + 16));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        xa[u][mt][0] = *reinterpret_cast<const i32x4*>(xp[mt] + off);
        xa[u][mt][1] = *reinterpret_cast<const i32x4*>(xp[mt] + off + 16);
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const i32x8 a = cat8(wa[u][0], wa[u][1]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma_16x16x128_fp8(a, cat8(xa[u][mt][0], xa[u][mt][1]), acc[mt]);
    }
  }
  for (; s < s_end; ++s) {
    const int64_t off = (int64_t)s * 128;
    const i32x8 a = cat8(__builtin_nontemporal_load(reinterpret_cast<const i32x4*>(wp + off)),
                         __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(wp + off + 16)));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      acc[mt] = mfma_16x16x128_fp8(a,
                                   cat8(*reinterpret_cast<const i32x4*>(xp[mt] + off),
                                        *reinterpret_cast<const i32x4*>(xp[mt] + off + 16)),
                                   acc[mt]);
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt) red[wave][mt][lane] = acc[mt];
  __syncthreads();

  // Output (m_local, n_local) of token tile mt lives in lane m_local + 16*(n_local/4),
  // register n_local % 4 (16x16 MFMA layout: row = 4*(lane/16) + reg, col = lane % 16,
  // with rows = weight channels and cols = tokens). Threads walk n fastest so
  // consecutive threads store consecutive channels of one token.
  const float* redf = reinterpret_cast<const float*>(&red[0][0][0]);
  constexpr int kOut = MT * 256;
  if (splits == 1) {
    for (int idx = threadIdx.x; idx < kOut; idx += 64 * WAVES) {
      const int mt = idx >> 8, e = idx & 255, ml = e >> 4, nl = e & 15;
      const int src = ((mt * 64) + ml + 16 * (nl >> 2)) * 4 + (nl & 3);
      float sum = 0.0f;
#pragma unroll
      for (int wv = 0; wv < WAVES; ++wv) sum += redf[wv * MT * 256 + src];
      const int m = mt * 16 + ml, n = n0 + nl;
      if (m < M && n < N) ep.y[(int64_t)m * ep.ldy + n] = (uint16_t)f32_to_bf16(epilogue_value<RANK>(ep, sum, m, n, ep.sx[m], ep.sw[n]));
    }
    return;
  }

  for (int idx = threadIdx.x; idx < kOut; idx += 64 * WAVES) {
    const int mt = idx >> 8, e = idx & 255, ml = e >> 4, nl = e & 15;
    const int src = ((mt * 64) + ml + 16 * (nl >> 2)) * 4 + (nl & 3);
    float sum = 0.0f;
#pragma unroll
    for (int wv = 0; wv < WAVES; ++wv) sum += redf[wv * MT * 256 + src];
    const int m = mt * 16 + ml, n = n0 + nl;
    if (m < M && n < N) partial[((int64_t)split * M + m) * N + n] = sum;
  }
  // Publish the partial (release at agent scope), then count this split in.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(counters + tile, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == splits - 1;
  }
  __syncthreads();
  if (!is_last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  for (int idx = threadIdx.x; idx < kOut; idx += 64 * WAVES) {
    const int mt = idx >> 8, e = idx & 255, ml = e >> 4, nl = e & 15;
    const int m = mt * 16 + ml, n = n0 + nl;
    if (m < M && n < N) {
      float sum = 0.0f;
      for (int sp = 0; sp < splits; ++sp) sum += partial[((int64_t)sp * M + m) * N + n];
      ep.y[(int64_t)m * ep.ldy + n] = (uint16_t)f32_to_bf16(epilogue_value<RANK>(ep, sum, m, n, ep.sx[m], ep.sw[n]));
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int decode_splits(int64_t N, int64_t K, int cu_count) {
  const int64_t tiles = (N + 15) / 16;
  const int64_t ksteps = K / 128;
  if (tiles >= cu_count) return 1;
  int64_t s = (cu_count + tiles - 1) / tiles;
  const int64_t max_s = ksteps / kDecodeWaves;
  if (s > max_s) s = max_s;
  if (s > 16) s = 16;
  return s < 1 ? 1 : (int)s;
}

template <int MT, int RANK>
static void launch_decode_mt(const uint8_t* xq, int64_t ldxq, const uint8_t* w, int64_t ldw, int M, int N, int K,
                             int splits, float* partial, int* counters, const Epilogue& ep, hipStream_t stream) {
  const dim3 grid((unsigned)((N + 15) / 16), (unsigned)splits), block(64 * kDecodeWaves);
  gemm_decode_kernel<MT, kDecodeWaves, kDecodeUnroll, RANK>
      <<<grid, block, 0, stream>>>(xq, ldxq, w, ldw, M, N, K, splits, partial, counters, ep);
}

hipError_t gemm_decode(const uint8_t* xq, int64_t ldxq, const uint8_t* w, int64_t ldw, int M, int N, int K, int splits,
                       float* partial, int* counters, const Epilogue& ep, int rank, hipStream_t stream) {
  const int mt = (M + 15) / 16;
  if (mt < 1 || mt > 4 || (rank != 0 && rank != 16)) return hipErrorInvalidValue;
#define JV_DECODE_CASE(MT_)                                                                          \
  if (mt == MT_) {                                                                                   \
    if (rank == 16)                                                                                  \
      launch_decode_mt<MT_, 16>(xq, ldxq, w, ldw, M, N, K, splits, partial, counters, ep, stream);   \
    else                                                                                             \
      launch_decode_mt<MT_, 0>(xq, ldxq, w, ldw, M, N, K, splits, partial, counters, ep, stream);    \
  }
  JV_DECODE_CASE(1)
  JV_DECODE_CASE(2)
  JV_DECODE_CASE(3)
  JV_DECODE_CASE(4)
#undef JV_DECODE_CASE
  return hipGetLastError();
}

}  // namespace jv
