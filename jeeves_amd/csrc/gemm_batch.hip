// Batch-decode FP8 x FP8 GEMM: 17-128 tokens on weights whose 16-row tiles
// fill at most one round of workgroups (the 9B model's q/o, k/v, merged
// q/k/v and 8192-wide projections on K = 4096, and down on K = 12288 up to
// 32 tokens). Counterpart of _fp8_matmul's split-K regime
// (inference/fp8.py:62-99, :118-123), like the decode kernel (swap-AB:
// weights are the A side of v_mfma_f32_16x16x128_f8f6f4, tokens the B side),
// laid out for what limits 17-128 token batches on CDNA4:
//   * each wave owns a fixed k range of `steps` 128-deep steps (W waves cover
//     the row exactly) and issues ALL of its weight fragments for that range
//     at once, in step order, into registers: one burst per wave, nothing to
//     refill, so the weight stream is never throttled by the activation
//     registers (the decode kernel's bursts shrink to 2 steps at 4 token
//     tiles for that reason);
//   * activation fragments stream two steps ahead of the MFMAs through a
//     small register ring;
//   * workgroups split the batch's token tiles (msplit parts of mt tiles) as
//     well as N, so a narrow weight still occupies the CUs without a K split
//     across workgroups: workgroups that share a weight group sit 8 apart in
//     launch order, which the dispatcher places on the same XCD, so the
//     second read of a weight tile is an L2 hit;
//   * waves are summed through LDS in wave order, every output's k order
//     fixed by (W, steps) alone: the results equal, bit for bit, the decode
//     kernel's with the same waves per row and no K split, whatever the token
//     count, tile shape, token split or operand layouts.
// Weights row-major (ldw > 0) or tiled (ldw = 0); activation codes row-major
// (ldxq > 0) or packed (packed_x_offset). Fused SwiGLU epilogue as the decode
// kernel's (a gate/up tile pair per wave).
#include <type_traits>

#include "epilogue.h"
#include "kernels.h"

namespace jv {

template <int I, int N, typename F>
__device__ __forceinline__ void each_step(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    each_step<I + 1, N>(f);
  }
}

template <int MT, int RT, int W, int NS, bool PACKX, bool PACKW, bool SW>
__global__ __launch_bounds__(64 * W) void gemm_batch_kernel(const uint8_t* __restrict__ xq, int64_t ldxq,
                                                            const uint8_t* __restrict__ w, int64_t ldw, int M, int N, int K,
                                                            int groups, int msplit, int rank, Epilogue ep) {
  static_assert(!SW || RT == 2, "SwiGLU pairs each gate tile with its up tile");
  constexpr int D = 2;  // activation steps loaded ahead of the MFMAs
  constexpr int WSTEP = PACKW ? 2048 : 128, XSTEP = PACKX ? 2048 : 128;
  constexpr int WHALF = PACKW ? 1024 : 16, XHALF = PACKX ? 1024 : 16;
  __shared__ f32x4 red[W][RT * MT][64];
  const int lane = threadIdx.x & 63;
  // Wave-uniform in a scalar register (see the decode kernel: the k range
  // guards must be scalar branches).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Workgroup -> (weight group, token part): whole blocks of 8 groups take
  // 8 msplit consecutive workgroups, group = b % 8 within the block, so the
  // parts of a group are 8 apart; the last groups % 8 groups follow.
  const uint32_t b = blockIdx.x, ms = (uint32_t)msplit, whole = (uint32_t)groups & ~7u;
  int group, mpart;
  if (b < whole * ms) {
    group = (int)((b / (8 * ms)) * 8 + (b & 7));
    mpart = (int)((b >> 3) % ms);
  } else {
    const uint32_t r = (uint32_t)groups - whole, i = b - whole * ms;
    group = (int)(whole + i % r);
    mpart = (int)(i / r);
  }
  const int ksteps = K >> 7;
  const int s_begin = wave * NS;
  const int n0 = group * 16 * RT;
  const int mt0 = mpart * MT;
  const int li = lane & 15, lk = (lane >> 4) * 32;
  const int ntiles = (N + 15) >> 4;

  const uint8_t* wp[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int lt = min(group * RT + rt, ntiles - 1);
    const int64_t pt = SW ? swiglu_tile(lt, ep.half) : lt;
    wp[rt] = PACKW ? w + (pt * ksteps + s_begin) * 2048 + lane * 16
                   : w + (SW ? pt * 16 + li : (int64_t)min(n0 + rt * 16 + li, N - 1)) * ldw + lk + s_begin * 128;
  }
  const uint8_t* xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xp[mt] = PACKX ? xq + ((int64_t)(mt0 + mt) * ksteps + s_begin) * 2048 + lane * 16
                   : xq + (int64_t)min((mt0 + mt) * 16 + li, M - 1) * ldxq + lk + s_begin * 128;

  // Each thread's outputs (idx = threadIdx.x + j * 64 W, channel fastest),
  // their scales and bias loaded ahead of the weights, as in the decode kernel.
  constexpr int kOut = (SW ? RT / 2 : RT) * MT * 256, kThreads = 64 * W, kPer = (kOut + kThreads - 1) / kThreads;
  float pre_sx[kPer], pre_sw[kPer], pre_b[kPer], pre_sw2[SW ? kPer : 1], pre_b2[SW ? kPer : 1];
  {
    const uint16_t* bsrc = ep.bias ? ep.bias : reinterpret_cast<const uint16_t*>(ep.sw);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int idx = min((int)threadIdx.x + j * kThreads, kOut - 1);
      const int t = idx >> 8, e = idx & 255;
      const int m = min((mt0 + t % MT) * 16 + (e >> 4), M - 1);
      pre_sx[j] = ep.sx[m];
      if constexpr (SW) {
        const int64_t hc = (int64_t)(group * (RT / 2) + t / MT) * 16 + (e & 15);
        pre_sw[j] = ep.sw[hc];
        pre_b[j] = bf16_to_f32(bsrc[hc]);
        pre_sw2[j] = ep.sw[ep.half + hc];
        pre_b2[j] = bf16_to_f32(bsrc[ep.half + hc]);
      } else {
        const int n = min(n0 + (t / MT) * 16 + (e & 15), N - 1);
        pre_sw[j] = ep.sw[n];
        pre_b[j] = bf16_to_f32(bsrc[n]);
      }
    }
  }

  i32x4 xa[D][MT][2];
  auto load_x = [&](int u, i32x4 (&dst)[MT][2]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      dst[mt][0] = *reinterpret_cast<const i32x4*>(xp[mt] + u * XSTEP);
      dst[mt][1] = *reinterpret_cast<const i32x4*>(xp[mt] + u * XSTEP + XHALF);
    }
  };
  each_step<0, (D < NS ? D : NS)>([&](auto uc) { load_x(decltype(uc)::value, xa[decltype(uc)::value]); });
  __builtin_amdgcn_sched_barrier(0);
  // The whole k range of weights, in step order (a scheduling barrier after
  // each step keeps that order, so the first steps' fragments arrive first and
  // each step's MFMAs wait only for the loads issued before its own).
  i32x4 wa[NS][RT][2];
  each_step<0, NS>([&](auto uc) {
    constexpr int u = decltype(uc)::value;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      wa[u][rt][0] = *reinterpret_cast<const i32x4*>(wp[rt] + u * WSTEP);
      wa[u][rt][1] = *reinterpret_cast<const i32x4*>(wp[rt] + u * WSTEP + WHALF);
    }
    __builtin_amdgcn_sched_barrier(0);
  });
  f32x4 acc[RT][MT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[rt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  each_step<0, NS>([&](auto uc) {
    constexpr int u = decltype(uc)::value;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const i32x8 bx = cat8(xa[u % D][mt][0], xa[u % D][mt][1]);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) acc[rt][mt] = mfma_16x16x128_fp8(cat8(wa[u][rt][0], wa[u][rt][1]), bx, acc[rt][mt]);
    }
    if constexpr (u + D < NS) {
      __builtin_amdgcn_sched_barrier(0);
      load_x(u + D, xa[u % D]);
      __builtin_amdgcn_sched_barrier(0);
    }
  });

#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[wave][rt * MT + mt][lane] = acc[rt][mt];
  __syncthreads();

  // Output (m_local, n_local) of tile (rt, mt): lane m_local + 16 (n_local / 4),
  // register n_local % 4 (rows of the 16x16 result are weight channels).
  const float* redf = reinterpret_cast<const float*>(&red[0][0][0]);
  auto value = [&](float sum, int m, int n, float sxm, float swn, float bn) {
    return rank == 16 ? epilogue_value<16>(ep, sum, m, n, sxm, swn, bn) : epilogue_value<0>(ep, sum, m, n, sxm, swn, bn);
  };
  if constexpr (SW) {
    // h = bf16(bf16(silu(y_gate)) * y_up) and the per-16-channel maxima of
    // |h|; every break and DPP row maximum is uniform across a wave (kOut and
    // kThreads are multiples of 64).
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int idx = (int)threadIdx.x + j * kThreads;
      if (kOut % kThreads != 0 && idx >= kOut) break;
      const int t = idx >> 8, q = t / MT, mt = t % MT, e = idx & 255, ml = e >> 4, nl = e & 15;
      const int off = ml + 16 * (nl >> 2);
      const int src_g = (((2 * q) * MT + mt) * 64 + off) * 4 + (nl & 3);
      const int src_u = (((2 * q + 1) * MT + mt) * 64 + off) * 4 + (nl & 3);
      float sum_g = 0.0f, sum_u = 0.0f;
#pragma unroll
      for (int wv = 0; wv < W; ++wv) {
        sum_g += redf[wv * RT * MT * 256 + src_g];
        sum_u += redf[wv * RT * MT * 256 + src_u];
      }
      const int m = (mt0 + mt) * 16 + ml;
      const int64_t hc = (int64_t)(group * (RT / 2) + q) * 16 + nl;
      uint32_t hv = 0;
      if (m < M) {
        const uint32_t yg = f32_to_bf16(value(sum_g, m, (int)hc, pre_sx[j], pre_sw[j], pre_b[j]));
        const uint32_t yu = f32_to_bf16(value(sum_u, m, (int)(ep.half + hc), pre_sx[j], pre_sw2[j], pre_b2[j]));
        hv = swiglu_bf16(yg, yu);
        ep.y[(int64_t)m * ep.ldy + hc] = (uint16_t)hv;
      }
      if (ep.parts) {
        const uint32_t mx = row16_max_u32_in_lane15(hv & 0x7FFFu);
        if (nl == 15 && m < M) ep.parts[(int64_t)m * (ep.half >> 4) + (hc >> 4)] = (uint16_t)mx;
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int idx = (int)threadIdx.x + j * kThreads;
    if (kOut % kThreads != 0 && idx >= kOut) break;
    const int t = idx >> 8, rt = t / MT, mt = t % MT, e = idx & 255, ml = e >> 4, nl = e & 15;
    const int src = (t * 64 + ml + 16 * (nl >> 2)) * 4 + (nl & 3);
    float sum = 0.0f;
#pragma unroll
    for (int wv = 0; wv < W; ++wv) sum += redf[wv * RT * MT * 256 + src];
    const int m = (mt0 + mt) * 16 + ml, n = n0 + rt * 16 + nl;
    if (m < M && n < N) ep.y[(int64_t)m * ep.ldy + n] = (uint16_t)f32_to_bf16(value(sum, m, n, pre_sx[j], pre_sw[j], pre_b[j]));
  }
}

template <int MT, int RT, int W, int NS, bool SW>
static void launch_batch(const uint8_t* xq, int64_t ldxq, bool packed_x, const uint8_t* w, int64_t ldw, int M, int N,
                         int K, const BatchPlan& p, const Epilogue& ep, int rank, hipStream_t stream) {
  const dim3 grid((unsigned)(p.groups * p.msplit)), block(64 * W);
#define JV_BATCH_LAUNCH(PX, PW)                                                                             \
  gemm_batch_kernel<MT, RT, W, NS, PX, PW, SW>                                                             \
      <<<grid, block, 0, stream>>>(xq, ldxq, w, ldw, M, N, K, p.groups, p.msplit, rank, ep)
  if constexpr (SW) {
    if (ldw == 0) JV_BATCH_LAUNCH(true, true);
    else JV_BATCH_LAUNCH(true, false);
  } else {
    if (packed_x && ldw == 0) JV_BATCH_LAUNCH(true, true);
    else if (packed_x) JV_BATCH_LAUNCH(true, false);
    else if (ldw == 0) JV_BATCH_LAUNCH(false, true);
    else JV_BATCH_LAUNCH(false, false);
  }
#undef JV_BATCH_LAUNCH
}

hipError_t gemm_batch(const uint8_t* xq, int64_t ldxq, bool packed_x, const uint8_t* w, int64_t ldw, int M, int N, int K,
                      const BatchPlan& p, const Epilogue& ep, int rank, hipStream_t stream) {
  const bool sw = ep.half != 0;
  if (M < 1 || (rank != 0 && rank != 16) || K / 128 != p.waves * p.steps || p.msplit < 1 || p.groups < 1 ||
      (int64_t)p.mt * p.msplit != (M + 15) / 16 || p.mt > batch_max_mt(p.waves, p.rt) ||
      (int64_t)p.groups * p.rt * 16 < N)
    return hipErrorInvalidValue;
  if (sw && (!packed_x || p.rt != 2 || 2 * ep.half != N || ep.half % 16)) return hipErrorInvalidValue;
#define JV_BATCH_CASE(MT_, RT_, W_, NS_)                                                                    \
  if (p.mt == MT_ && p.rt == RT_ && p.waves == W_ && p.steps == NS_) {                                   \
    if (sw) {                                                                                             \
      if constexpr (RT_ == 2) launch_batch<MT_, RT_, W_, NS_, true>(xq, ldxq, packed_x, w, ldw, M, N, K, p, ep, rank, stream); \
    } else {                                                                                              \
      launch_batch<MT_, RT_, W_, NS_, false>(xq, ldxq, packed_x, w, ldw, M, N, K, p, ep, rank, stream);   \
    }                                                                                                     \
    return hipGetLastError();                                                                             \
  }
  // K = 4096: 4 waves x 8 steps, up to 4 token tiles per workgroup.
  JV_BATCH_CASE(1, 1, 4, 8) JV_BATCH_CASE(2, 1, 4, 8) JV_BATCH_CASE(3, 1, 4, 8) JV_BATCH_CASE(4, 1, 4, 8)
  JV_BATCH_CASE(1, 2, 4, 8) JV_BATCH_CASE(2, 2, 4, 8) JV_BATCH_CASE(3, 2, 4, 8) JV_BATCH_CASE(4, 2, 4, 8)
  // K = 12288: 8 waves x 12 steps (the registers of 12 steps bound the tiles).
  JV_BATCH_CASE(1, 1, 8, 12) JV_BATCH_CASE(2, 1, 8, 12) JV_BATCH_CASE(1, 2, 8, 12)
#undef JV_BATCH_CASE
  return hipErrorInvalidValue;
}

}  // namespace jv
