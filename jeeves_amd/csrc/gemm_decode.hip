// Small-M FP8 x FP8 GEMM (decode: M <= 64 tokens), HBM-bound on the weights.
// Weights come row-major (ldw > 0) or in the tiled fragment layout (ldw = 0,
// tiled_w_offset), which turns each wave's weight load into one contiguous
// 1 KB (measured 2-29 % faster over the 9B projection shapes).
//
// Counterpart of _fp8_matmul's split-K regime (inference/fp8.py:62-99,
// :118-123), redesigned for CDNA4:
//   * weights are the MFMA "A" side (16 output channels x 128 k per
//     v_mfma_f32_16x16x128_f8f6f4) and tokens the "B" side, up to 4 token
//     tiles of 16 (swap-AB, as inference/fp8.py:69 does);
//   * each lane streams 32 bytes of one weight row per 128-k step straight
//     from HBM into MFMA operand registers (no LDS round trip), UNROLL steps
//     in flight per wave; a wave owns RT 16-row tiles so each activation
//     fragment it loads feeds RT MFMAs. Plain (cached) loads: on MI355X they
//     stream these matrices 5-10 % faster than non-temporal ones, and a whole
//     wave's k range in one burst beats a deeper rolling pipeline (measured
//     over the 9B projection shapes at M = 1..16);
//   * activation codes come either row-major [M,K] or, from the fused
//     quantizer, pre-packed in MFMA B-fragment order (packed_x_offset), so a
//     wave's activation load is one contiguous 1 KB per instruction;
//   * the WAVES waves of a workgroup split the workgroup's k range and are
//     summed through LDS in wave order; for very small N, workgroups also
//     split K (grid.y): partials go to memory with device-coherent stores, and
//     the last workgroup of a tile (device-scope counter) sums them in split
//     order and resets the counter -- one launch, deterministic, no cache
//     flushes, capture-safe.
#include <type_traits>

#include "epilogue.h"
#include "kernels.h"

namespace jv {

// Upper bound of decode_plan's K splits (the plan caps them at 16).
constexpr int kMaxDecodeSplits = 16;

// SW: fused SwiGLU (gate+up weights, Epilogue::half): the wave's tiles come in
// (gate p, up p) pairs, and the epilogue stores h (no split-K).
// SPLIT: workgroups split K (grid.y = splits > 1). Without it each wave's k
// range is its share of the whole row with the compile-time divisor WAVES;
// with the split count a run-time value the same kernel took 1 us longer
// at M = 16 on gate+up (19.7 vs 18.7 us), even at one split.
template <int MT, int RT, int WAVES, int UNROLL, bool PACKX, int RANK, bool PACKW, bool SW = false, bool SPLIT = false>
__global__ __launch_bounds__(64 * WAVES) void gemm_decode_kernel(const uint8_t* __restrict__ xq, int64_t ldxq,
                                                                 const uint8_t* __restrict__ w, int64_t ldw, int M, int N,
                                                                 int K, int splits, float* __restrict__ partial,
                                                                 int* __restrict__ counters, Epilogue ep) {
  static_assert(!SW || RT % 2 == 0, "SwiGLU pairs each gate tile with its up tile");
  static_assert(!(SW && SPLIT), "the SwiGLU epilogue keeps whole k ranges");
  __shared__ f32x4 red[WAVES][RT * MT][64];
  __shared__ int is_last;
  const int lane = threadIdx.x & 63;
  // Wave-uniform in a scalar register, so the k range [s_begin, s_end) and the
  // tail guards below are scalar branches. Computed in a vector register the
  // guards become EXEC-masked regions, and gfx950 writes an MFMA's result
  // even with EXEC = 0: a guarded-off tail step's MFMA then adds whatever its
  // unloaded operand registers hold (address bits, found with the assembly
  // scan in the kernel-resource tests).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = blockIdx.x;
  const int split = SPLIT ? (int)blockIdx.y : 0;
  const int n0 = group * 16 * RT;

  const int ksteps = K >> 7;
  int s_begin, s_end;
  if constexpr (SPLIT) {
    const int slice = split * WAVES + wave;
    s_begin = slice_begin<WAVES>(ksteps, slice, splits);
    s_end = slice_begin<WAVES>(ksteps, slice + 1, splits);
  } else {
    s_begin = ksteps * wave / WAVES;
    s_end = ksteps * (wave + 1) / WAVES;
  }

  const int li = lane & 15;
  const int lk = (lane >> 4) * 32;
  // Weights: row-major rows (lane -> row n0 + 16 rt + l%16, 32 bytes at k =
  // 32 (l/16)), or the tiled layout (lane -> 16 contiguous bytes of each
  // 1 KB half of the tile's 2 KB step fragment).
  // With SwiGLU, logical tile group*RT + rt is gate tile p (rt even) or up
  // tile p (rt odd) of pair p = group*RT/2 + rt/2.
  const uint8_t* wp[RT];
  const int ntiles = (N + 15) >> 4;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int lt = min(group * RT + rt, ntiles - 1);
    const int64_t pt = SW ? swiglu_tile(lt, ep.half) : lt;
    wp[rt] = PACKW ? w + pt * ksteps * 2048 + lane * 16
                   : w + (SW ? pt * 16 + li : (int64_t)min(n0 + rt * 16 + li, N - 1)) * ldw + lk;
  }
  const uint8_t* xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xp[mt] = PACKX ? xq + (int64_t)mt * ksteps * 2048 + lane * 16 : xq + (int64_t)min(mt * 16 + li, M - 1) * ldxq + lk;

  // Each thread's outputs (idx = threadIdx.x + j * 64 WAVES; channel fastest)
  // and their scales and bias, loaded before the weight stream so the
  // epilogue does not wait for another memory round trip. Indices are clamped
  // so the loads are unconditional; a missing bias reads the scales instead.
  // With SwiGLU each output is one h channel hc = 16 p + nl, from gate row hc
  // and up row half + hc (their scales and biases in the *2 arrays).
  constexpr int kOut = (SW ? RT / 2 : RT) * MT * 256, kThreads = 64 * WAVES, kPer = (kOut + kThreads - 1) / kThreads;
  float pre_sx[kPer], pre_sw[kPer], pre_b[kPer], pre_sw2[SW ? kPer : 1], pre_b2[SW ? kPer : 1];
  {
    const uint16_t* bsrc = ep.bias ? ep.bias : reinterpret_cast<const uint16_t*>(ep.sw);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int idx = min((int)threadIdx.x + j * kThreads, kOut - 1);
      const int t = idx >> 8, e = idx & 255;
      const int m = min((t % MT) * 16 + (e >> 4), M - 1);
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

  f32x4 acc[RT][MT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[rt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One burst of up to UNROLL k steps: all its loads are issued, then the
  // MFMAs consume them. A full burst is straight-line code, so each step's
  // MFMAs wait only for that step's data; the last, partial burst guards each
  // step with a scalar branch (s and s_end are wave-uniform).
  // The burst's addresses are one base per operand plus constant offsets
  // (u steps of 2 KB packed or 128 B row-major), which the loads take as
  // immediates instead of a 64-bit add per step (0.5 us of the 1 us above).
  auto burst = [&](int s, auto full) {
    constexpr bool FULL = decltype(full)::value;
    constexpr int WSTEP = PACKW ? 2048 : 128, XSTEP = PACKX ? 2048 : 128;
    i32x4 wa[UNROLL][RT][2];
    i32x4 xa[UNROLL][MT][2];
    const uint8_t* wb[RT];
    const uint8_t* xb[MT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) wb[rt] = wp[rt] + (int64_t)s * WSTEP;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xb[mt] = xp[mt] + (int64_t)s * XSTEP;
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (!FULL && s + u >= s_end) break;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        wa[u][rt][0] = *reinterpret_cast<const i32x4*>(wb[rt] + u * WSTEP);
        wa[u][rt][1] = *reinterpret_cast<const i32x4*>(wb[rt] + u * WSTEP + (PACKW ? 1024 : 16));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        xa[u][mt][0] = *reinterpret_cast<const i32x4*>(xb[mt] + u * XSTEP);
        xa[u][mt][1] = *reinterpret_cast<const i32x4*>(xb[mt] + u * XSTEP + (PACKX ? 1024 : 16));
      }
    }
    if constexpr (FULL) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (!FULL && s + u >= s_end) break;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const i32x8 b = cat8(xa[u][mt][0], xa[u][mt][1]);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[rt][mt] = mfma_16x16x128_fp8(cat8(wa[u][rt][0], wa[u][rt][1]), b, acc[rt][mt]);
      }
    }
  };
  int s = s_begin;
  for (; s + UNROLL <= s_end; s += UNROLL) burst(s, std::true_type{});
  if (s < s_end) burst(s, std::false_type{});

#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[wave][rt * MT + mt][lane] = acc[rt][mt];
  __syncthreads();

  // Output (m_local, n_local) of tile (rt, mt) lives in lane m_local + 16*(n_local/4),
  // register n_local % 4 (16x16 MFMA layout: row = 4*(lane/16) + reg, col = lane % 16,
  // with rows = weight channels and cols = tokens). Threads walk n fastest so
  // consecutive threads store consecutive channels of one token.
  const float* redf = reinterpret_cast<const float*>(&red[0][0][0]);
  if constexpr (SW) {
    // h[m, hc] = bf16(bf16(silu(y_gate)) * y_up), y = the bf16 outputs the
    // unfused GEMM would store; thread groups of 16 (one token, 16 channels)
    // also take the largest |h| for the row's quantizer. Every break and
    // DPP row maximum below is uniform across a wave (kOut and kThreads are multiples
    // of 64).
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
      for (int wv = 0; wv < WAVES; ++wv) {
        sum_g += redf[wv * RT * MT * 256 + src_g];
        sum_u += redf[wv * RT * MT * 256 + src_u];
      }
      const int m = mt * 16 + ml;
      const int64_t hc = (int64_t)(group * (RT / 2) + q) * 16 + nl;
      uint32_t hv = 0;
      if (m < M) {
        const uint32_t yg = f32_to_bf16(epilogue_value<RANK>(ep, sum_g, m, (int)hc, pre_sx[j], pre_sw[j], pre_b[j]));
        const uint32_t yu =
            f32_to_bf16(epilogue_value<RANK>(ep, sum_u, m, (int)(ep.half + hc), pre_sx[j], pre_sw2[j], pre_b2[j]));
        hv = swiglu_bf16(yg, yu);
        ep.y[(int64_t)m * ep.ldy + hc] = (uint16_t)hv;
      }
      if (ep.parts) {
        // The 16 channels nl = 0..15 of token m are one 16-lane DPP row.
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
    for (int wv = 0; wv < WAVES; ++wv) sum += redf[wv * RT * MT * 256 + src];
    const int m = mt * 16 + ml, n = n0 + rt * 16 + nl;
    if (m < M && n < N) {
      if (!SPLIT || splits == 1)
        ep.y[(int64_t)m * ep.ldy + n] =
            (uint16_t)f32_to_bf16(epilogue_value<RANK>(ep, sum, m, n, pre_sx[j], pre_sw[j], pre_b[j]));
      else  // device-coherent store: visible to the reducing workgroup without a cache flush
        __hip_atomic_store(partial + ((int64_t)split * M + m) * N + n, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if constexpr (!SPLIT) return;
  if (splits == 1) return;

  // The workgroup that sees count splits-1 sums every split's partials in
  // split order and resets the counter.
  // Ordering without cache-wide fences: the partials were written with
  // device-scope atomic stores, which gfx950 performs at the device-coherent
  // level past each XCD's L2; every thread waits for its stores to complete
  // (s_waitcnt 0) before the barrier that precedes thread 0's device-scope
  // count, and the reducing workgroup issues its device-scope loads only after
  // its own count returned. An agent-scope release/acquire pair instead writes
  // back and invalidates the whole L2 of the XCD in every finishing
  // workgroup: 44 vs 6.8 us for two splits at M = 32, N = K = 4096.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    is_last = __hip_atomic_fetch_add(counters + group, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
  __syncthreads();
  if (!is_last) return;
  // Every split's partial of an output is loaded before any is added (all in
  // flight together), then they are added in split order.
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int idx = (int)threadIdx.x + j * kThreads;
    if (kOut % kThreads != 0 && idx >= kOut) break;
    const int t = idx >> 8, rt = t / MT, mt = t % MT, e = idx & 255, ml = e >> 4, nl = e & 15;
    const int m = mt * 16 + ml, n = n0 + rt * 16 + nl;
    if (m < M && n < N) {
      float part[kMaxDecodeSplits];
#pragma unroll
      for (int sp = 0; sp < kMaxDecodeSplits; ++sp)
        if (sp < splits)
          part[sp] = __hip_atomic_load(partial + ((int64_t)sp * M + m) * N + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      float sum = 0.0f;
#pragma unroll
      for (int sp = 0; sp < kMaxDecodeSplits; ++sp)
        if (sp < splits) sum += part[sp];
      ep.y[(int64_t)m * ep.ldy + n] =
          (uint16_t)f32_to_bf16(epilogue_value<RANK>(ep, sum, m, n, pre_sx[j], pre_sw[j], pre_b[j]));
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(counters + group, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// k steps per burst for MT token tiles, RT weight tiles and W waves: bounded so
// the burst's operands fit the registers without spilling.
constexpr int decode_unroll(int mt, int rt, int w) { return rt + mt > 4 ? 2 : ((w == 8 || rt + mt > 3) ? 4 : 8); }

DecodePlan decode_plan(int64_t M, int64_t N, int64_t K, int cu_count, bool swiglu) {
  DecodePlan p;
  const int64_t tiles = (N + 15) / 16;
  const int64_t mt = (M + 15) / 16;
  // A fused SwiGLU wave owns one gate tile and its up tile.
  p.rt = swiglu || tiles >= 4 * (int64_t)cu_count ? 2 : 1;
  // Four waves take 8 k steps each in one burst up to K = 4096; longer rows
  // use eight waves in bursts of 4. More token tiles shorten the burst to
  // bound the registers it holds.
  p.waves = K / 128 > 32 ? 8 : 4;
  // Weights of one to two rounds of 16-row tiles (the merged q/k/v,
  // 6144 x 4096) take two tiles per wave, so every tile pair runs in one
  // round: 7.9 -> 7.5 us at 1-16 tokens, 9.7 -> 8.9 at 32, 13.8 -> 11.0 at 64.
  if (!swiglu && tiles > cu_count && tiles <= 2 * (int64_t)cu_count && K / 128 >= 16) p.rt = 2;
  // Two tiles per wave stream best as eight waves of four k steps rather than
  // four waves of eight (gate+up 19.2 -> 18.5 us at M = 1, 20.0 -> 19.7 at
  // 16), the SwiGLU epilogue's gate/up pairs too (decode layer step at M = 16
  // 60.8 -> 60.6 us in same-box A/B runs).
  if (p.rt == 2 && K / 128 >= 16) p.waves = 8;
  p.unroll = decode_unroll((int)mt, p.rt, p.waves);
  const int64_t groups = (tiles + p.rt - 1) / p.rt;
  p.groups = (int)groups;
  // Splitting K across workgroups only pays when the tiles cannot occupy an
  // eighth of the CUs: below that the launch is latency-bound either way.
  p.splits = 1;
  if (!swiglu && groups * 8 < cu_count) {
    int64_t s = (cu_count + groups - 1) / groups;
    const int64_t max_s = (K / 128) / p.waves;
    if (s > max_s) s = max_s;
    if (s > kMaxDecodeSplits) s = kMaxDecodeSplits;
    p.splits = s < 1 ? 1 : (int)s;
  }
  return p;
}

template <int MT, int RT, int W, int U, bool PACKX, int RANK, bool SW, bool SPLIT>
static void launch_decode_split(const uint8_t* xq, int64_t ldxq, const uint8_t* w, int64_t ldw, int M, int N, int K,
                                const DecodePlan& p, float* partial, int* counters, const Epilogue& ep,
                                hipStream_t stream) {
  const dim3 grid((unsigned)p.groups, (unsigned)p.splits), block(64 * W);
  if (ldw == 0)
    gemm_decode_kernel<MT, RT, W, U, PACKX, RANK, true, SW, SPLIT>
        <<<grid, block, 0, stream>>>(xq, ldxq, w, ldw, M, N, K, p.splits, partial, counters, ep);
  else
    gemm_decode_kernel<MT, RT, W, U, PACKX, RANK, false, SW, SPLIT>
        <<<grid, block, 0, stream>>>(xq, ldxq, w, ldw, M, N, K, p.splits, partial, counters, ep);
}

// K splits come only with one tile per wave (decode_plan splits narrow
// weights, whose tiles take one wave each), so only those shapes have
// split instances.
template <int MT, int RT, int W, int U, bool PACKX, int RANK, bool SW>
static void launch_decode(const uint8_t* xq, int64_t ldxq, const uint8_t* w, int64_t ldw, int M, int N, int K,
                          const DecodePlan& p, float* partial, int* counters, const Epilogue& ep, hipStream_t stream) {
  if constexpr (RT == 1 && !SW) {
    if (p.splits > 1) {
      launch_decode_split<MT, RT, W, U, PACKX, RANK, SW, true>(xq, ldxq, w, ldw, M, N, K, p, partial, counters, ep, stream);
      return;
    }
  }
  launch_decode_split<MT, RT, W, U, PACKX, RANK, SW, false>(xq, ldxq, w, ldw, M, N, K, p, partial, counters, ep, stream);
}

template <int MT, int RT, bool PACKX, int RANK, bool SW>
static void launch_decode_wu(const uint8_t* xq, int64_t ldxq, const uint8_t* w, int64_t ldw, int M, int N, int K,
                             const DecodePlan& p, float* partial, int* counters, const Epilogue& ep, hipStream_t stream) {
  constexpr int U4 = decode_unroll(MT, RT, 4), U8 = decode_unroll(MT, RT, 8);
  if (p.waves == 8)
    launch_decode<MT, RT, 8, U8, PACKX, RANK, SW>(xq, ldxq, w, ldw, M, N, K, p, partial, counters, ep, stream);
  else
    launch_decode<MT, RT, 4, U4, PACKX, RANK, SW>(xq, ldxq, w, ldw, M, N, K, p, partial, counters, ep, stream);
}

template <int MT, bool PACKX, int RANK, bool SW>
static void launch_decode_rt(const uint8_t* xq, int64_t ldxq, const uint8_t* w, int64_t ldw, int M, int N, int K,
                             const DecodePlan& p, float* partial, int* counters, const Epilogue& ep, hipStream_t stream) {
  if constexpr (SW) {
    launch_decode_wu<MT, 2, PACKX, RANK, true>(xq, ldxq, w, ldw, M, N, K, p, partial, counters, ep, stream);
  } else {
    if (p.rt == 2)
      launch_decode_wu<MT, 2, PACKX, RANK, false>(xq, ldxq, w, ldw, M, N, K, p, partial, counters, ep, stream);
    else
      launch_decode_wu<MT, 1, PACKX, RANK, false>(xq, ldxq, w, ldw, M, N, K, p, partial, counters, ep, stream);
  }
}

template <bool PACKX, int RANK, bool SW = false>
static hipError_t launch_decode_mt(const uint8_t* xq, int64_t ldxq, const uint8_t* w, int64_t ldw, int M, int N, int K,
                                   const DecodePlan& p, float* partial, int* counters, const Epilogue& ep,
                                   hipStream_t stream) {
  switch ((M + 15) / 16) {
    case 1: launch_decode_rt<1, PACKX, RANK, SW>(xq, ldxq, w, ldw, M, N, K, p, partial, counters, ep, stream); break;
    case 2: launch_decode_rt<2, PACKX, RANK, SW>(xq, ldxq, w, ldw, M, N, K, p, partial, counters, ep, stream); break;
    case 3: launch_decode_rt<3, PACKX, RANK, SW>(xq, ldxq, w, ldw, M, N, K, p, partial, counters, ep, stream); break;
    case 4: launch_decode_rt<4, PACKX, RANK, SW>(xq, ldxq, w, ldw, M, N, K, p, partial, counters, ep, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t gemm_decode(const uint8_t* xq, int64_t ldxq, bool packed_x, const uint8_t* w, int64_t ldw, int M, int N, int K,
                       const DecodePlan& plan, float* partial, int* counters, const Epilogue& ep, int rank,
                       hipStream_t stream) {
  if (M < 1 || M > kDecodeMaxRows || (rank != 0 && rank != 16) || (plan.rt != 1 && plan.rt != 2) || plan.splits < 1 ||
      plan.splits > kMaxDecodeSplits || (plan.splits > 1 && plan.rt != 1))
    return hipErrorInvalidValue;
  if (ep.half) {
    // Fused SwiGLU: packed activation codes only (jv_fp8_linear_swiglu packs them), one gate/up pair per wave.
    if (!packed_x || plan.rt != 2 || plan.splits != 1 || 2 * ep.half != N || ep.half % 16) return hipErrorInvalidValue;
    return rank == 16 ? launch_decode_mt<true, 16, true>(xq, ldxq, w, ldw, M, N, K, plan, partial, counters, ep, stream)
                      : launch_decode_mt<true, 0, true>(xq, ldxq, w, ldw, M, N, K, plan, partial, counters, ep, stream);
  }
  if (packed_x)
    return rank == 16 ? launch_decode_mt<true, 16>(xq, ldxq, w, ldw, M, N, K, plan, partial, counters, ep, stream)
                      : launch_decode_mt<true, 0>(xq, ldxq, w, ldw, M, N, K, plan, partial, counters, ep, stream);
  return rank == 16 ? launch_decode_mt<false, 16>(xq, ldxq, w, ldw, M, N, K, plan, partial, counters, ep, stream)
                    : launch_decode_mt<false, 0>(xq, ldxq, w, ldw, M, N, K, plan, partial, counters, ep, stream);
}

}  // namespace jv
