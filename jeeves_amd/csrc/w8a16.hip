// W8A16 parity mode: the arithmetic the reference's FP8Linear actually runs
// (inference/fp8.py:62-99, :112-148, stated as ((x.float() @ w8.float().t()) *
// scale).to(bf16) in model/metal_test.py:213): bf16 activations times e4m3
// weights, fp32 sums, times the channel scale, rounded to bf16; a bias is
// added afterwards in bf16 (inference/fp8.py:183-184).
//
// On gfx950 the e4m3 weight bytes become bf16 in registers with
// v_cvt_pk_f32_fp8 (exact: every e4m3 value is a bf16 value) and feed bf16
// MFMAs with the activations as they are -- no activation quantization, no
// fp16 detour. Decode (M <= 64) mirrors the FP8 decode kernel: weights are
// the A side of v_mfma_f32_16x16x32_bf16, each wave streams its k range in
// bursts straight from HBM, waves meet in LDS, narrow N splits K across
// workgroups with the same deterministic last-workgroup reduction.
#include <type_traits>

#include "epilogue.h"
#include "kernels.h"

namespace jv {

// y = bf16(acc * sw), then bf16(y + bias) when there is a bias: the two
// roundings of the reference's GEMM output and its separate bias add.
// biasn is the bias of the channel, already loaded (read only when has_bias).
__device__ __forceinline__ uint16_t w8a16_out(float acc, float swn, bool has_bias, float biasn) {
  uint32_t v = f32_to_bf16(acc * swn);
  if (has_bias) v = f32_to_bf16(bf16_to_f32(v) + biasn);
  return (uint16_t)v;
}

// Weights: lane l holds k bytes [32j, 32j+32) of row l%16 for j = l/16 of each
// 128-k step; the four 16x16x32 MFMAs q of a step use k = 32j + 8q + [0, 8)
// on both operands. SPLIT: workgroups split K (grid.y = splits > 1); without
// it the wave's k range takes the compile-time divisor W, as in
// gemm_decode_kernel.
template <int MT, int RT, int W, int U, bool PACKW, bool SPLIT>
__global__ __launch_bounds__(64 * W) void w8a16_decode_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                              const uint8_t* __restrict__ w, int64_t ldw, int M, int N,
                                                              int K, int splits, float* __restrict__ partial,
                                                              int* __restrict__ counters, const float* __restrict__ sw,
                                                              const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                              int64_t ldy) {
  __shared__ f32x4 red[W][RT * MT][64];
  __shared__ int is_last;
  const int lane = threadIdx.x & 63;
  // Wave-uniform (scalar register): the burst guards below are scalar
  // branches, never EXEC-masked regions, whose MFMAs gfx950 would still
  // execute with EXEC = 0 (see gemm_decode_kernel).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = blockIdx.x, split = SPLIT ? (int)blockIdx.y : 0;
  const int n0 = group * 16 * RT;

  const int ksteps = K >> 7;
  int s_begin, s_end;
  if constexpr (SPLIT) {
    const int slice = split * W + wave;
    s_begin = slice_begin<W>(ksteps, slice, splits);
    s_end = slice_begin<W>(ksteps, slice + 1, splits);
  } else {
    s_begin = ksteps * wave / W;
    s_end = ksteps * (wave + 1) / W;
  }

  const int li = lane & 15, j32 = (lane >> 4) * 32;
  // Row-major weight rows, or the tiled fragment layout (ldw = 0): the same
  // 32 bytes per lane and step, as two 16-byte halves 1 KB apart.
  const uint8_t* wp[RT];
  const int ntiles = (N + 15) >> 4;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
    wp[rt] = PACKW ? w + (int64_t)min(group * RT + rt, ntiles - 1) * ksteps * 2048 + lane * 16
                   : w + (int64_t)min(n0 + rt * 16 + li, N - 1) * ldw + j32;
  const uint16_t* xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xp[mt] = x + (int64_t)min(mt * 16 + li, M - 1) * ldx + j32;

  // Each thread's output channels (idx = threadIdx.x + j * 64 W; channel
  // fastest) and their scales and bias, loaded before the weight stream so the
  // epilogue does not wait for another memory round trip; clamped indices keep
  // the loads unconditional, and a missing bias reads the scales instead.
  constexpr int kOut = RT * MT * 256, kThreads = 64 * W, kPer = (kOut + kThreads - 1) / kThreads;
  float pre_sw[kPer], pre_b[kPer];
  {
    const uint16_t* bsrc = bias ? bias : reinterpret_cast<const uint16_t*>(sw);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int idx = min((int)threadIdx.x + j * kThreads, kOut - 1);
      const int n = min(n0 + ((idx >> 8) / MT) * 16 + (idx & 15), N - 1);
      pre_sw[j] = sw[n];
      pre_b[j] = bf16_to_f32(bsrc[n]);
    }
  }
  const bool has_bias = bias != nullptr;

  f32x4 acc[RT][MT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[rt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One base address per operand and burst, constant offsets per step.
  constexpr int WSTEP = PACKW ? 2048 : 128;
  for (int s = s_begin; s < s_end; s += U) {
    i32x4 wa[U][RT][2];
    i32x4 xa[U][MT][4];
    const uint8_t* wb[RT];
    const uint16_t* xb[MT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) wb[rt] = wp[rt] + (int64_t)s * WSTEP;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xb[mt] = xp[mt] + (int64_t)s * 128;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s + u >= s_end) break;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        wa[u][rt][0] = *reinterpret_cast<const i32x4*>(wb[rt] + u * WSTEP);
        wa[u][rt][1] = *reinterpret_cast<const i32x4*>(wb[rt] + u * WSTEP + (PACKW ? 1024 : 16));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int q = 0; q < 4; ++q) xa[u][mt][q] = *reinterpret_cast<const i32x4*>(xb[mt] + u * 128 + 8 * q);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s + u >= s_end) break;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const i32x4 w0 = wa[u][rt][0], w1 = wa[u][rt][1];
        const bf16x8 a[4] = {e4m3x8_to_bf16(w0.x, w0.y), e4m3x8_to_bf16(w0.z, w0.w), e4m3x8_to_bf16(w1.x, w1.y),
                             e4m3x8_to_bf16(w1.z, w1.w)};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            acc[rt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[q], __builtin_bit_cast(bf16x8, xa[u][mt][q]),
                                                                  acc[rt][mt], 0, 0, 0);
      }
    }
  }

#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[wave][rt * MT + mt][lane] = acc[rt][mt];
  __syncthreads();

  // Output (token ml, channel nl) of tile (rt, mt) sits in lane ml + 16*(nl/4),
  // register nl % 4 (16x16 layout: row = 4*(lane/16) + reg is the channel).
  const float* redf = reinterpret_cast<const float*>(&red[0][0][0]);
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int idx = (int)threadIdx.x + j * kThreads;
    if (kOut % kThreads != 0 && idx >= kOut) break;
    const int t = idx >> 8, rt = t / MT, mt = t % MT, e = idx & 255, ml = e >> 4, nl = e & 15;
    const int src = (t * 64 + ml + 16 * (nl >> 2)) * 4 + (nl & 3);
    float sum = 0.0f;
#pragma unroll
    for (int wv = 0; wv < W; ++wv) sum += redf[wv * RT * MT * 256 + src];
    const int m = mt * 16 + ml, n = n0 + rt * 16 + nl;
    if (m < M && n < N) {
      if (!SPLIT || splits == 1)
        y[(int64_t)m * ldy + n] = w8a16_out(sum, pre_sw[j], has_bias, pre_b[j]);
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
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int idx = (int)threadIdx.x + j * kThreads;
    if (kOut % kThreads != 0 && idx >= kOut) break;
    const int t = idx >> 8, rt = t / MT, mt = t % MT, e = idx & 255, ml = e >> 4, nl = e & 15;
    const int m = mt * 16 + ml, n = n0 + rt * 16 + nl;
    if (m < M && n < N) {
      // every split's partial in flight together, then added in split order
      float part[16];
#pragma unroll
      for (int sp = 0; sp < 16; ++sp)
        if (sp < splits)
          part[sp] = __hip_atomic_load(partial + ((int64_t)sp * M + m) * N + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      float sum = 0.0f;
#pragma unroll
      for (int sp = 0; sp < 16; ++sp)
        if (sp < splits) sum += part[sp];
      y[(int64_t)m * ldy + n] = w8a16_out(sum, pre_sw[j], has_bias, pre_b[j]);
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(counters + group, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Batch-decode form (17-128 tokens, w8a16_batch_plan): the FP8 batch-decode
// kernel's structure (gemm_batch.hip) with this mode's operands -- each wave
// issues its whole k range of e4m3 weight fragments at once, in step order,
// the bf16 activation fragments stream two steps ahead, and workgroups split
// the batch's token tiles (msplit parts per weight group, 8 workgroups apart
// so the parts share an XCD's L2). Every output's k order is the decode
// kernel's at the same waves per row (each wave's steps in order, the four
// 32-deep MFMAs of a step in order, waves summed in order), so the two agree
// bit for bit. Activations are the larger operand here (2 bytes per element
// against 1): splitting the token tiles is what cuts each workgroup's reads.
template <int I, int N, typename F>
__device__ __forceinline__ void w8a16_each_step(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    w8a16_each_step<I + 1, N>(f);
  }
}

template <int MT, int RT, int W, int NS, bool PACKW>
__global__ __launch_bounds__(64 * W) void w8a16_batch_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                             const uint8_t* __restrict__ w, int64_t ldw, int M, int N,
                                                             int K, int groups, int msplit, const float* __restrict__ sw,
                                                             const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                             int64_t ldy) {
  constexpr int D = 2;  // activation steps loaded ahead of the MFMAs
  constexpr int WSTEP = PACKW ? 2048 : 128, WHALF = PACKW ? 1024 : 16;
  __shared__ f32x4 red[W][RT * MT][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
  const int n0 = group * 16 * RT, mt0 = mpart * MT;
  const int li = lane & 15, j32 = (lane >> 4) * 32;
  const int ntiles = (N + 15) >> 4;
  const uint8_t* wp[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
    wp[rt] = PACKW ? w + ((int64_t)min(group * RT + rt, ntiles - 1) * ksteps + s_begin) * 2048 + lane * 16
                   : w + (int64_t)min(n0 + rt * 16 + li, N - 1) * ldw + j32 + s_begin * 128;
  const uint16_t* xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xp[mt] = x + (int64_t)min((mt0 + mt) * 16 + li, M - 1) * ldx + j32 + s_begin * 128;

  constexpr int kOut = RT * MT * 256, kThreads = 64 * W, kPer = (kOut + kThreads - 1) / kThreads;
  float pre_sw[kPer], pre_b[kPer];
  {
    const uint16_t* bsrc = bias ? bias : reinterpret_cast<const uint16_t*>(sw);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int idx = min((int)threadIdx.x + j * kThreads, kOut - 1);
      const int n = min(n0 + ((idx >> 8) / MT) * 16 + (idx & 15), N - 1);
      pre_sw[j] = sw[n];
      pre_b[j] = bf16_to_f32(bsrc[n]);
    }
  }
  const bool has_bias = bias != nullptr;

  i32x4 xa[D][MT][4];
  auto load_x = [&](int u, i32x4 (&dst)[MT][4]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q) dst[mt][q] = *reinterpret_cast<const i32x4*>(xp[mt] + u * 128 + 8 * q);
  };
  w8a16_each_step<0, (D < NS ? D : NS)>([&](auto uc) { load_x(decltype(uc)::value, xa[decltype(uc)::value]); });
  __builtin_amdgcn_sched_barrier(0);
  i32x4 wa[NS][RT][2];
  w8a16_each_step<0, NS>([&](auto uc) {
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
  w8a16_each_step<0, NS>([&](auto uc) {
    constexpr int u = decltype(uc)::value;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const i32x4 w0 = wa[u][rt][0], w1 = wa[u][rt][1];
      const bf16x8 a[4] = {e4m3x8_to_bf16(w0.x, w0.y), e4m3x8_to_bf16(w0.z, w0.w), e4m3x8_to_bf16(w1.x, w1.y),
                           e4m3x8_to_bf16(w1.z, w1.w)};
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc[rt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[q], __builtin_bit_cast(bf16x8, xa[u % D][mt][q]),
                                                                acc[rt][mt], 0, 0, 0);
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
  const float* redf = reinterpret_cast<const float*>(&red[0][0][0]);
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
    if (m < M && n < N) y[(int64_t)m * ldy + n] = w8a16_out(sum, pre_sw[j], has_bias, pre_b[j]);
  }
}

hipError_t w8a16_batch(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                       const BatchPlan& p, const float* sw, const uint16_t* bias, uint16_t* y, int64_t ldy,
                       hipStream_t stream) {
  if (M < 1 || K / 128 != p.waves * p.steps || p.msplit < 1 || p.groups < 1 ||
      (int64_t)p.mt * p.msplit != (M + 15) / 16 || p.mt > w8a16_batch_max_mt(p.waves, p.rt) ||
      (int64_t)p.groups * p.rt * 16 < N)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)(p.groups * p.msplit));
#define JV_W8A16_BATCH_CASE(MT_, RT_, W_, NS_)                                                                      \
  if (p.mt == MT_ && p.rt == RT_ && p.waves == W_ && p.steps == NS_) {                                           \
    if (ldw == 0)                                                                                                 \
      w8a16_batch_kernel<MT_, RT_, W_, NS_, true><<<grid, dim3(64 * W_), 0, stream>>>(x, ldx, w, ldw, M, N, K,     \
                                                                                      p.groups, p.msplit, sw, bias, \
                                                                                      y, ldy);                       \
    else                                                                                                          \
      w8a16_batch_kernel<MT_, RT_, W_, NS_, false><<<grid, dim3(64 * W_), 0, stream>>>(x, ldx, w, ldw, M, N, K,    \
                                                                                       p.groups, p.msplit, sw,      \
                                                                                       bias, y, ldy);               \
    return hipGetLastError();                                                                                     \
  }
  JV_W8A16_BATCH_CASE(1, 1, 4, 8) JV_W8A16_BATCH_CASE(2, 1, 4, 8) JV_W8A16_BATCH_CASE(1, 2, 4, 8)
  JV_W8A16_BATCH_CASE(2, 2, 4, 8) JV_W8A16_BATCH_CASE(1, 1, 8, 12)
#undef JV_W8A16_BATCH_CASE
  return hipErrorInvalidValue;
}

// Bursts of U steps: the operands of a burst (RT weight tiles, MT token tiles
// of 32 bf16 per step) stay within the register budget without spilling.
constexpr int w8a16_unroll(int mt, int rt) { return rt + 2 * mt <= 4 ? 4 : 2; }

template <int MT, int RT, int W>
static void launch_w8a16_decode(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                                const DecodePlan& p, float* partial, int* counters, const float* sw, const uint16_t* bias,
                                uint16_t* y, int64_t ldy, hipStream_t stream) {
  constexpr int U = w8a16_unroll(MT, RT);
  const dim3 grid((unsigned)p.groups, (unsigned)p.splits), block(64 * W);
#define JV_W8A16_LAUNCH(PW, SP)                                                                                \
  w8a16_decode_kernel<MT, RT, W, U, PW, SP><<<grid, block, 0, stream>>>(x, ldx, w, ldw, M, N, K, p.splits, partial, \
                                                                        counters, sw, bias, y, ldy)
  // K splits come only with one tile per wave (as in launch_decode).
  if constexpr (RT == 1) {
    if (p.splits > 1) {
      if (ldw == 0) JV_W8A16_LAUNCH(true, true);
      else JV_W8A16_LAUNCH(false, true);
      return;
    }
  }
  if (ldw == 0) JV_W8A16_LAUNCH(true, false);
  else JV_W8A16_LAUNCH(false, false);
#undef JV_W8A16_LAUNCH
}

template <int MT>
static void launch_w8a16_decode_mt(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                                   const DecodePlan& p, float* partial, int* counters, const float* sw,
                                   const uint16_t* bias, uint16_t* y, int64_t ldy, hipStream_t stream) {
  if (p.rt == 2) {
    if (p.waves == 8)
      launch_w8a16_decode<MT, 2, 8>(x, ldx, w, ldw, M, N, K, p, partial, counters, sw, bias, y, ldy, stream);
    else
      launch_w8a16_decode<MT, 2, 4>(x, ldx, w, ldw, M, N, K, p, partial, counters, sw, bias, y, ldy, stream);
  } else {
    if (p.waves == 8)
      launch_w8a16_decode<MT, 1, 8>(x, ldx, w, ldw, M, N, K, p, partial, counters, sw, bias, y, ldy, stream);
    else
      launch_w8a16_decode<MT, 1, 4>(x, ldx, w, ldw, M, N, K, p, partial, counters, sw, bias, y, ldy, stream);
  }
}

hipError_t w8a16_decode(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                        const DecodePlan& p, float* partial, int* counters, const float* sw, const uint16_t* bias,
                        uint16_t* y, int64_t ldy, hipStream_t stream) {
  if (M < 1 || M > kDecodeMaxRows || (K & 127) || p.splits < 1 || p.splits > 16 || (p.splits > 1 && p.rt != 1))
    return hipErrorInvalidValue;
  switch ((M + 15) / 16) {
    case 1: launch_w8a16_decode_mt<1>(x, ldx, w, ldw, M, N, K, p, partial, counters, sw, bias, y, ldy, stream); break;
    case 2: launch_w8a16_decode_mt<2>(x, ldx, w, ldw, M, N, K, p, partial, counters, sw, bias, y, ldy, stream); break;
    case 3: launch_w8a16_decode_mt<3>(x, ldx, w, ldw, M, N, K, p, partial, counters, sw, bias, y, ldy, stream); break;
    case 4: launch_w8a16_decode_mt<4>(x, ldx, w, ldw, M, N, K, p, partial, counters, sw, bias, y, ldy, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace jv
