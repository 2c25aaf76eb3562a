// Prefill FP8 x FP8 GEMM (M > 64 tokens), MFMA-bound.
//
// Counterpart of _fp8_matmul's tall-tile regime (inference/fp8.py:62-99,
// :118-119), redesigned for CDNA4 instead of translated:
//   * both operands are K-contiguous e4m3 (activation codes [M,K] from the
//     quantizer, weight codes [N,K]) and feed v_mfma_f32_32x32x64_f8f6f4
//     directly: no fp8 -> fp16 conversion in the main loop;
//   * a BM (tokens) x BN (channels) output tile per workgroup of WGM x WGN
//     waves; each wave owns a (BM/WGM) x (BN/WGN) sub-tile of 32x32 MFMA
//     blocks with fp32 accumulators. With 8 waves two waves share each SIMD,
//     so one wave's LDS reads overlap the other's MFMAs;
//   * weights are the MFMA A operand and tokens the B operand, so each lane
//     ends with 4 consecutive channels of one token per register quad and the
//     epilogue stores 8 bytes per lane;
//   * K advances 128 bytes per stage; each stage's A and B rows are copied
//     global -> LDS with global_load_lds_dwordx4 (no VGPR staging), double
//     buffered so the next stage's copy overlaps this stage's MFMAs;
//   * LDS rows are 128 B with the 16-byte chunk index XOR-swizzled by (row & 7),
//     so the 8 lanes of each ds_read_b128 phase hit 8 distinct bank groups;
//   * workgroups are renumbered so that each XCD (the hardware hands
//     consecutive workgroups to the 8 XCDs in turn) works on a contiguous
//     range of tiles: a weight tile is fetched into one XCD's L2, not eight;
//   * fused epilogue acc * sx[m] * sw[n] (+ bias, + LoRA) -> bf16.
#include "epilogue.h"
#include "kernels.h"

namespace jv {

constexpr int kXcds = 8;

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmem_below() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Main-loop barrier: each wave waits for its global -> LDS copies with
// wait_vmem_below before it, and has consumed its earlier LDS reads (their
// MFMAs issued) before reaching it.
__device__ __forceinline__ void barrier_only() { barrier_no_fence(); }

// Copy 16 bytes per lane from global to LDS: lane i's bytes land at dst + 16 * i.
__device__ __forceinline__ void load_lds16(const uint8_t* src, uint8_t* dst_wave_base) {
  typedef __attribute__((address_space(3))) void lds_void;
  typedef __attribute__((address_space(1))) void global_void;
  __builtin_amdgcn_global_load_lds((global_void*)(src), (lds_void*)(dst_wave_base), 16, 0, 0);
}

__device__ __forceinline__ i32x4 lds_read16(const uint8_t* p) { return *reinterpret_cast<const i32x4*>(p); }

// LDS tile rows are BK bytes = BK/16 chunks of 16 B. gfx950 serves a
// ds_read_b128 16 lanes at a time from 64 four-byte banks (256 B), so the 16
// rows a fragment read touches at one logical chunk must fall in 16 distinct
// 16-byte bank groups. Row r's bank groups start at (r * BK/16) mod 16, which
// repeats every P = 256/BK rows; XOR-ing the chunk index with (r / P) mod
// (BK/16) separates the rows that share a start.
template <int BK>
__device__ __forceinline__ int swizzle(int row) {
  constexpr int CH = BK / 16, P = 256 / BK;
  return (row / P) % CH;
}

// Workgroup -> output tile. Workgroup ids are first regrouped so that XCD x
// (ids x, x+8, x+16, ...) receives one contiguous range of logical tiles;
// logical tiles then run in groups of `group_m` M-tiles that walk N together.
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int group_m, int& tile_m, int& tile_n) {
  const int total = tiles_m * tiles_n;
  const int base = total / kXcds, rem = total % kXcds;
  const int xcd = pid % kXcds, local = pid / kXcds;
  const int q = (xcd < rem ? xcd * (base + 1) : rem * (base + 1) + (xcd - rem) * base) + local;
  const int per_group = group_m * tiles_n;
  const int first_m = (q / per_group) * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int r = q % per_group;
  tile_m = first_m + r % gsize;
  tile_n = r / gsize;
}

// Byte offset of stage kt's copy for one 16-byte unit of a tiled weight row,
// relative to stage 0 (BK-deep stages; tiled_w_offset): a 64-deep stage is
// half of a 128-deep step fragment, 512 bytes into it for odd kt.
template <int BK>
__device__ __forceinline__ int64_t tiled_stage_offset(int kt) {
  return BK == 128 ? (int64_t)kt * 2048 : (int64_t)(kt >> 1) * 2048 + (kt & 1) * 512;
}

// LoRA operands of one wave's prefill tile (rank 16), loaded once at the
// start of the epilogue: for block column j the B rows of channels
// nb_j + l%32 (ranks 8h .. 8h+7, h = l/32: 8 bf16), for block row i the t
// rows of tokens mb_i + l%32 (the same 8 ranks, fp32). Loads are clamped to
// the last row; clamped outputs are never stored.
template <int TN, int TM>
struct LoraOperands {
  i32x4 b[TN];
  float4 t[TM][2];
};

template <int TN, int TM>
__device__ __forceinline__ void load_lora(LoraOperands<TN, TM>& o, const Epilogue& ep, int nb, int mb, int M, int N,
                                          int lane) {
  const int h = lane >> 5;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int c = min(nb + j * 32 + (lane & 31), N - 1);
    const int64_t n = ep.half ? swiglu_channel(c, ep.half) : c;
    o.b[j] = *reinterpret_cast<const i32x4*>(ep.lora_b + n * 16 + 8 * h);
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = min(mb + i * 32 + (lane & 31), M - 1);
    const float4* t = reinterpret_cast<const float4*>(ep.lora_t + (int64_t)m * 16 + 8 * h);
    o.t[i][0] = t[0];
    o.t[i][1] = t[1];
  }
}

// LoRA term of block (j, i): l[n, m] = sum_r B[n, r] t[m, r] in the fp8
// blocks' accumulator layout, by two v_mfma_f32_32x32x16_bf16: t is split
// into t_hi = bf16(t) and t_lo = bf16(t - t_hi) (about 16 significant bits),
// the products with the bf16 B entries are exact, the sums fp32.
__device__ __forceinline__ f32x16 lora_block(i32x4 b, const float4 (&t)[2]) {
  const float tv[8] = {t[0].x, t[0].y, t[0].z, t[0].w, t[1].x, t[1].y, t[1].z, t[1].w};
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = pack_bf16x2(tv[2 * e], tv[2 * e + 1]);
    lo[e] = pack_bf16x2(tv[2 * e] - bf16_to_f32(hi[e] & 0xFFFFu), tv[2 * e + 1] - bf16_to_f32(hi[e] >> 16));
  }
  const bf16x8 bb = __builtin_bit_cast(bf16x8, b);
  f32x16 l;
#pragma unroll
  for (int r = 0; r < 16; ++r) l[r] = 0.0f;
  l = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bb, __builtin_bit_cast(bf16x8, i32x4{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]}),
                                              l, 0, 0, 0);
  l = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bb, __builtin_bit_cast(bf16x8, i32x4{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]}),
                                              l, 0, 0, 0);
  return l;
}

// XOR swizzle span of an LDS-staged output tile row of W 16-byte chunks: the
// largest power of two up to 32 dividing W, so chunk ^ (row % span) stays in
// the row (W itself for the power-of-two widths).
template <int W>
constexpr int out_swizzle() {
  int s = 1;
  while (s < 32 && W % (2 * s) == 0) s *= 2;
  return s;
}

// Epilogue of both FP8 prefill kernels. 32x32 MFMA output layout: lane l
// holds column l % 32 (a token) and, in register r, row 8*(r/4) + 4*(l/32) +
// r%4 (a channel): each register quad is 4 consecutive channels of one token.
// y = bf16((acc * sx[m]) * sw[n] (+ lora_scale * l[n, m])), then + bias[n] in bf16. The
// finished bf16 tile goes through LDS ([BM tokens][BN channels], 16-byte
// chunk c of row r stored at chunk c ^ (r % out_swizzle)) so that global stores are
// 16 bytes per lane over whole row segments. The caller's operand reads and
// copies into `lds` are complete (this wave's) when it is called.
template <int BM, int BN, int WGM, int WGN, int RANK>
__device__ __forceinline__ void store_tile(uint8_t* lds, const float* scale_lds,
                                           const f32x16 (&acc)[BN / WGN / 32][BM / WGM / 32], const Epilogue& ep, int m0,
                                           int n0, int M, int N, int wm, int wn, int lane) {
  constexpr int NW = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int OUT_CH = BN * 2 / 16;  // 16-byte chunks per output tile row
  constexpr int SWZ = out_swizzle<OUT_CH>();
  static_assert(RANK == 0 || RANK == 16, "LoRA rank");
  LoraOperands<TN, TM> lo;
  if constexpr (RANK > 0) load_lora(lo, ep, n0 + wn * WN, m0 + wm * WM, M, N, lane);
  float sxm[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) sxm[i] = scale_lds[wm * WM + i * 32 + (lane & 31)];
  // Every wave's operand reads are complete before the tile overwrites them.
  lds_barrier();
#pragma unroll
  for (int j = 0; j < TN; ++j) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int ml = wm * WM + i * 32 + (lane & 31);  // token within the tile
      const int m = min(m0 + ml, M - 1);
      f32x16 lora;
      if constexpr (RANK > 0) lora = lora_block(lo.b[j], lo.t[i]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = wn * WN + j * 32 + 8 * q + 4 * (lane >> 5);  // channel within the tile
        const int n = n0 + nl;
        const float4 swq = *reinterpret_cast<const float4*>(scale_lds + BM + nl);
        const float sw4[4] = {swq.x, swq.y, swq.z, swq.w};
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = (acc[j][i][4 * q + e] * sxm[i]) * sw4[e];
          if constexpr (RANK > 0) v[e] += lora[4 * q + e] * ep.lora_scale;
          if (ep.bias) v[e] = with_bias(ep, v[e], bf16_to_f32(ep.bias[min(n + e, N - 1)]));
        }
        const int chunk = (nl >> 3) ^ (ml % SWZ);
        *reinterpret_cast<uint2*>(lds + ml * (BN * 2) + chunk * 16 + (nl & 4) * 2) =
            uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      }
    }
  }
  lds_barrier();
  const bool y_vec = ((ep.ldy | N) & 7) == 0 && (reinterpret_cast<uintptr_t>(ep.y) & 15) == 0;
  constexpr int NT = 64 * NW;
#pragma unroll 4
  for (int c = threadIdx.x; c < BM * OUT_CH; c += NT) {
    const int ml = c / OUT_CH, ch = c % OUT_CH;
    const int m = m0 + ml, n = n0 + ch * 8;
    if (m >= M || n >= N) continue;
    const uint4 v = *reinterpret_cast<const uint4*>(lds + ml * (BN * 2) + (ch ^ (ml % SWZ)) * 16);
    uint16_t* dst = ep.y + (int64_t)m * ep.ldy + n;
    if (y_vec) {
      *reinterpret_cast<uint4*>(dst) = v;
    } else {
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (n + e < N) dst[e] = (uint16_t)(wv[e >> 1] >> (16 * (e & 1)));
    }
  }
}

// Epilogue of both FP8 prefill kernels with the fused SwiGLU (Epilogue::half):
// the tile's logical channels come in 32-channel blocks of 16 gate and the 16
// matching up channels, so in each 32x32 accumulator block a lane's registers
// 0-7 are gate channels and 8-15 the up channels of the same h channels (the
// register quad q + 2 pairs with q). h = bf16(bf16(silu(y_gate)) * y_up) with
// y = the bf16 output the unfused GEMM would store (bias in bf16 after it).
// The h tile (BM tokens x BN/2 channels) goes through LDS as in store_tile;
// with ep.parts set, each token's largest |h| over each 16 h channels goes to
// parts[m * (half / 16) + h_channel / 16].
template <int BM, int BN, int WGM, int WGN, int RANK>
__device__ __forceinline__ void store_tile_sw(uint8_t* lds, const float* scale_lds,
                                              const f32x16 (&acc)[BN / WGN / 32][BM / WGM / 32], const Epilogue& ep,
                                              int m0, int n0, int M, int N, int wm, int wn, int lane) {
  constexpr int NW = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int HBN = BN / 2;               // h channels per tile
  constexpr int OUT_CH = HBN * 2 / 16;      // 16-byte chunks per h tile row
  constexpr int SWZ = out_swizzle<OUT_CH>();
  static_assert(RANK == 0 || RANK == 16, "LoRA rank");
  LoraOperands<TN, TM> lo;
  if constexpr (RANK > 0) load_lora(lo, ep, n0 + wn * WN, m0 + wm * WM, M, N, lane);
  float sxm[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) sxm[i] = scale_lds[wm * WM + i * 32 + (lane & 31)];
  lds_barrier();
  const int64_t hparts = ep.half >> 4;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int cb = wn * WN + j * 32;  // the block's first logical channel in the tile
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int ml = wm * WM + i * 32 + (lane & 31);
      f32x16 lora;
      if constexpr (RANK > 0) lora = lora_block(lo.b[j], lo.t[i]);
      uint32_t mx = 0;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int o = 8 * q + 4 * (lane >> 5);  // gate channel offset in the block; its up channel is o + 16
        const float4 sg = *reinterpret_cast<const float4*>(scale_lds + BM + cb + o);
        const float4 su = *reinterpret_cast<const float4*>(scale_lds + BM + cb + 16 + o);
        const float swg[4] = {sg.x, sg.y, sg.z, sg.w}, swu[4] = {su.x, su.y, su.z, su.w};
        float vg[4], vu[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vg[e] = (acc[j][i][4 * q + e] * sxm[i]) * swg[e];
          vu[e] = (acc[j][i][4 * (q + 2) + e] * sxm[i]) * swu[e];
          if constexpr (RANK > 0) {
            vg[e] += lora[4 * q + e] * ep.lora_scale;
            vu[e] += lora[4 * (q + 2) + e] * ep.lora_scale;
          }
          if (ep.bias) {
            const int c = min(n0 + cb + o + e, N - 1);
            vg[e] = with_bias(ep, vg[e], bf16_to_f32(ep.bias[swiglu_channel(c, ep.half)]));
            vu[e] = with_bias(ep, vu[e], bf16_to_f32(ep.bias[swiglu_channel(c + 16, ep.half)]));
          }
        }
        const uint32_t h01 = swiglu_pair_f32(vg[0], vg[1], vu[0], vu[1]);
        const uint32_t h23 = swiglu_pair_f32(vg[2], vg[3], vu[2], vu[3]);
        if (ep.parts)
          mx = max(max(mx, max(h01 & 0x7FFFu, (h01 >> 16) & 0x7FFFu)), max(h23 & 0x7FFFu, (h23 >> 16) & 0x7FFFu));
        const int hl = cb / 2 + o;  // h channel within the tile
        const int chunk = (hl >> 3) ^ (ml % SWZ);
        *reinterpret_cast<uint2*>(lds + ml * (HBN * 2) + chunk * 16 + (hl & 4) * 2) = uint2{h01, h23};
      }
      if (ep.parts) {
        // blocks past the last h channel (a ragged last tile) have no slot
        mx = max(mx, (uint32_t)__shfl_xor((int)mx, 32, 64));
        if (lane < 32 && m0 + ml < M && (n0 + cb) / 2 < ep.half)
          ep.parts[(int64_t)(m0 + ml) * hparts + (n0 + cb) / 32] = (uint16_t)mx;
      }
    }
  }
  lds_barrier();
  const int64_t h0 = n0 / 2;
  const bool y_vec = ((ep.ldy | ep.half) & 7) == 0 && (reinterpret_cast<uintptr_t>(ep.y) & 15) == 0;
  constexpr int NT = 64 * NW;
#pragma unroll 4
  for (int c = threadIdx.x; c < BM * OUT_CH; c += NT) {
    const int ml = c / OUT_CH, ch = c % OUT_CH;
    const int m = m0 + ml;
    const int64_t hn = h0 + ch * 8;
    if (m >= M || hn >= ep.half) continue;
    const uint4 v = *reinterpret_cast<const uint4*>(lds + ml * (HBN * 2) + (ch ^ (ml % SWZ)) * 16);
    uint16_t* dst = ep.y + (int64_t)m * ep.ldy + hn;
    if (y_vec) {
      *reinterpret_cast<uint4*>(dst) = v;
    } else {
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (hn + e < ep.half) dst[e] = (uint16_t)(wv[e >> 1] >> (16 * (e & 1)));
    }
  }
}

// Split-K (splits > 1): workgroup tile + s * tiles adds up part s of the k
// range (whole BK stages, split as evenly as they divide), writes its fp32
// accumulators to its partial tile and counts in on the tile's counter; the
// workgroup that counts last adds the partials of every split in split order
// (its own from registers) and runs the epilogue, so the sum is the same
// whichever workgroup finishes last, and resets the counter.
// Ordering: the partials are written and read with device-scope atomic
// stores and loads, which on gfx950 write through and read from the
// device-coherent level past each XCD's L2; every wave's stores complete
// (s_waitcnt vmcnt(0)) before the barrier that precedes the device-scope
// count, and the last workgroup issues its loads after its count returned,
// so they read completed partials. No cache-wide writeback or invalidation
// (an agent-scope release/acquire pair) is needed on this path.
constexpr int kMaxPrefillSplits = 8;
// Largest split-K partial workspace a prefill plan uses.
constexpr int64_t kMaxPrefillPartialBytes = 16 << 20;

template <int TN, int TM, int NW>
__device__ __forceinline__ bool split_k_reduce(f32x16 (&acc)[TN][TM], float* __restrict__ partials,
                                               int* __restrict__ counters, int tile, int split, int splits, int wave,
                                               int lane, int* is_last) {
  constexpr int Q = TN * TM * 16;  // floats per lane
  const auto slot = [&](int s) { return partials + (((int64_t)tile * splits + s) * NW + wave) * Q * 64 + lane; };
  float* mine = slot(split);
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        __hip_atomic_store(mine + ((j * TM + i) * 16 + r) * 64, acc[j][i][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    *is_last = __hip_atomic_fetch_add(counters + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
  __syncthreads();
  if (!*is_last) return false;
  // One 32x32 block at a time: every other split's 16 values are loaded at
  // once (all loads in flight together), then added in split order.
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int b = (j * TM + i) * 16;
      float part[kMaxPrefillSplits][16];
#pragma unroll
      for (int s = 0; s < kMaxPrefillSplits; ++s)
        if (s < splits && s != split) {
          const float* p = slot(s);
#pragma unroll
          for (int r = 0; r < 16; ++r)
            part[s][r] = __hip_atomic_load(p + (b + r) * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      f32x16 sum;
#pragma unroll
      for (int s = 0; s < kMaxPrefillSplits; ++s)
        if (s < splits)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float v = s == split ? acc[j][i][r] : part[s][r];
            sum[r] = s == 0 ? v : sum[r] + v;
          }
      acc[j][i] = sum;
    }
  if (threadIdx.x == 0) __hip_atomic_store(counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

template <int BM, int BN, int WGM, int WGN, int BK, int STAGES, int RANK, bool PACKW, bool PACKX, bool SW = false,
          bool SPLITK = false>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_prefill_kernel(const uint8_t* __restrict__ xq, int64_t ldx,
                                                                      const uint8_t* __restrict__ w, int64_t ldw, int M,
                                                                      int N, int K, int tiles_m, int tiles_n, int group_m,
                                                                      Epilogue ep, int splits, float* __restrict__ partials,
                                                                      int* __restrict__ counters) {
  constexpr int NW = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;  // wave sub-tile: tokens x channels
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int CH = BK / 16;                  // 16-byte chunks per LDS row
  constexpr int RPL = 1024 / BK;               // rows per 1 KB wave-load
  constexpr int ROWS = BM + BN;                // stacked LDS rows: tokens, then channels
  constexpr int STAGE = ROWS * BK;
  constexpr int LOADS = ROWS / RPL / NW;       // wave-loads per wave per stage
  constexpr int SUB = BK / 64;                 // 64-deep MFMA steps per stage
  static_assert(BK == 64 || BK == 128, "stage depth");
  static_assert(ROWS % (RPL * NW) == 0 && TM >= 1 && TN >= 1, "tile does not divide among the waves");
  static_assert(STAGES >= 3 && (STAGES - 2) * LOADS < 64, "pipeline depth");
  constexpr int LDS_BYTES = STAGES * STAGE > BM * BN * 2 ? STAGES * STAGE : BM * BN * 2;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
  __shared__ __attribute__((aligned(256))) float scale_lds[BM + BN];  // sx of the tile's tokens, then sw of its channels
  __shared__ int is_last;

  const int tiles = tiles_m * tiles_n;
  const int split = SPLITK ? (int)blockIdx.x / tiles : 0;
  const int tile = (int)blockIdx.x - split * tiles;
  int tile_m, tile_n;
  tile_of(tile, tiles_m, tiles_n, group_m, tile_m, tile_n);
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WGN, wn = wave % WGN;

  // Global -> LDS assignment. Wave-load g (g = i*NW + wave) fills LDS bytes
  // [g*1024, g*1024 + 1024) of a stage: stacked rows RPL*g .. RPL*g + RPL-1.
  // Lane l writes row RPL*g + l/CH at physical chunk l%CH, which holds logical
  // chunk (l%CH) ^ swizzle(row). Rows past M or N re-read the last valid row;
  // their products land in outputs that are never stored.
  // Tiled weights (PACKW) keep their fragment order in LDS too: the weight
  // part of a stage is, per 16-row tile, the stage's share of the tile's
  // 128-deep step fragment -- both 1 KB halves for 128-deep stages, or the
  // 512-byte piece of each half that a 64-deep stage covers -- so each weight
  // wave-load copies contiguous global memory (one 1 KB half, or two 512-byte
  // pieces) into its contiguous 1 KB of LDS. Each wave-load index i holds
  // only token rows or only weight data.
  // Packed activation codes (PACKX, the same fragment order) are copied the
  // same way into the token part of the stage.
  static_assert(BM % (NW * RPL) == 0, "wave-loads straddle the token/weight boundary");
  const int ntiles = (N + 15) >> 4, mtiles = (M + 15) >> 4;
  const uint8_t* src[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int g = i * NW + wave;
    const int r = g * RPL + lane / CH;
    const int chunk = (lane % CH) ^ swizzle<BK>(r);
    if (r < BM && PACKX) {
      const int tt = BK == 128 ? g >> 1 : g;
      const int h = BK == 128 ? g & 1 : lane >> 5;
      const int lp = BK == 128 ? lane : lane & 31;
      const int tile = min((m0 >> 4) + tt, mtiles - 1);
      src[i] = xq + (((int64_t)tile * (K >> 7)) * 2 + h) * 1024 + lp * 16;
    } else if (r < BM) {
      src[i] = xq + (int64_t)min(m0 + r, M - 1) * ldx + chunk * 16;
    } else if (PACKW) {
      const int gw = g - BM / RPL;  // weight wave-load: tile gw (64-deep) or half gw%2 of tile gw/2
      const int tt = BK == 128 ? gw >> 1 : gw;
      const int h = BK == 128 ? gw & 1 : lane >> 5;
      const int lp = BK == 128 ? lane : lane & 31;
      const int lt = min((n0 >> 4) + tt, ntiles - 1);
      const int64_t tile = SW ? swiglu_tile(lt, ep.half) : lt;
      src[i] = w + ((tile * (K >> 7)) * 2 + h) * 1024 + lp * 16;
    } else {
      const int c = min(n0 + r - BM, N - 1);
      src[i] = w + (SW ? swiglu_channel(c, ep.half) : (int64_t)c) * ldw + chunk * 16;
    }
  }

  // This workgroup's stages: [kt0, kt0 + KT) of the K / BK stages, split as
  // floor(kt_all * s / splits) (32-bit: kt_all * splits <= K); without a K
  // split no division at all (the 64-bit division by a register it replaces
  // sat ahead of every workgroup's first load).
  const int kt_all = K / BK;
  int kt0 = 0, KT = kt_all;
  if constexpr (SPLITK) {
    kt0 = (int)((uint32_t)(kt_all * split) / (uint32_t)splits);
    KT = (int)((uint32_t)(kt_all * (split + 1)) / (uint32_t)splits) - kt0;
  }
  auto issue_stage = [&](int kt) {
    uint8_t* base = lds + (kt % STAGES) * STAGE;
    const int ktg = kt0 + kt;
    const int64_t k0 = (int64_t)ktg * BK;
    const int64_t wk = PACKW ? tiled_stage_offset<BK>(ktg) : k0;
    const int64_t xk = PACKX ? tiled_stage_offset<BK>(ktg) : k0;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) load_lds16(src[i] + (i * NW * RPL < BM ? xk : wk), base + (i * NW + wave) * 1024);
  };

  f32x16 acc[TN][TM];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;

  // Fragment addressing: lane l reads row (l % 32) of a 32-row block, logical
  // chunks 4s + 2(l/32) and 4s + 2(l/32) + 1 for 64-deep step s of the stage.
  const int frow = lane & 31;
  const int fhalf = (lane >> 5) * 2;
  int arow[TN], brow[TM];
#pragma unroll
  for (int j = 0; j < TN; ++j) arow[j] = BM + wn * WN + j * 32 + frow;
#pragma unroll
  for (int i = 0; i < TM; ++i) brow[i] = wm * WM + i * 32 + frow;

  // The tile's token and channel scales go to LDS by DMA before the operand
  // stages (vector-memory loads complete in order, so the first stage wait
  // covers them), out of the epilogue's critical path.
  for (int t = wave * 64; t < BM + BN; t += NW * 64) {
    const int r = t + lane;
    const int c = min(n0 + r - BM, N - 1);
    const float* sp = r < BM ? ep.sx + min(m0 + r, M - 1) : ep.sw + (SW ? swiglu_channel(c, ep.half) : (int64_t)c);
    typedef __attribute__((address_space(3))) void lds_void;
    typedef __attribute__((address_space(1))) void global_void;
    __builtin_amdgcn_global_load_lds((global_void*)sp, (lds_void*)(scale_lds + t), 4, 0, 0);
  }

  // Two fragment sets: while the MFMAs of 64-deep step u run on one set, the
  // LDS reads of step u+1 fill the other.
  i32x8 fa[2][TN], fb[2][TM];
  // Tiled weights in LDS: row rr of the tile's channels, 64-deep step s of
  // the stage, k half kh = l/32: lane rr%16 + 16*(2s + kh) of the fragment
  // (128-deep stages: halves 1 KB apart, 2 KB per tile) or lane
  // rr%16 + 16*kh of the stage's piece (64-deep: halves 512 bytes apart, 1 KB
  // per tile). A 16-lane phase reads 256 consecutive bytes.
  constexpr int TSTRIDE = BK == 128 ? 2048 : 1024, HSTRIDE = BK == 128 ? 1024 : 512;
  int aoff[TN], boff[TM];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int rr = wn * WN + j * 32 + frow;
    aoff[j] = BM * BK + (rr >> 4) * TSTRIDE + ((rr & 15) + 16 * (lane >> 5)) * 16;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int rr = wm * WM + i * 32 + frow;
    boff[i] = (rr >> 4) * TSTRIDE + ((rr & 15) + 16 * (lane >> 5)) * 16;
  }
  auto load_frags = [&](int kt, int s, i32x8 (&a)[TN], i32x8 (&b)[TM]) {
    const uint8_t* base = lds + (kt % STAGES) * STAGE;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (PACKW) {
        const uint8_t* p = base + aoff[j] + s * 512;
        a[j] = cat8(lds_read16(p), lds_read16(p + HSTRIDE));
      } else {
        const int r = arow[j], sw = swizzle<BK>(r);
        a[j] = cat8(lds_read16(base + r * BK + ((4 * s + fhalf) ^ sw) * 16),
                    lds_read16(base + r * BK + ((4 * s + fhalf + 1) ^ sw) * 16));
      }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if constexpr (PACKX) {
        const uint8_t* p = base + boff[i] + s * 512;
        b[i] = cat8(lds_read16(p), lds_read16(p + HSTRIDE));
      } else {
        const int r = brow[i], sw = swizzle<BK>(r);
        b[i] = cat8(lds_read16(base + r * BK + ((4 * s + fhalf) ^ sw) * 16),
                    lds_read16(base + r * BK + ((4 * s + fhalf + 1) ^ sw) * 16));
      }
    }
  };

  // Stage kt+1 has landed (for every wave, after the barrier) once at most
  // min(STAGES-3, KT-2-kt) later stages of this wave's copies are in flight.
  auto wait_stage_after = [&](int kt) {
    const int later = min(STAGES - 3, KT - 2 - kt);
    if (STAGES > 3 && later >= STAGES - 3) wait_vmem_below<(STAGES > 3 ? (STAGES - 3) * LOADS : 0)>();
    else if (STAGES > 4 && later == 1) wait_vmem_below<LOADS>();
    else wait_vmem_below<0>();
    barrier_only();
  };

  const int U = KT * SUB;  // 64-deep steps
#pragma unroll
  for (int p = 0; p < STAGES - 1; ++p)
    if (p < KT) issue_stage(p);
  // stage 0 landed: at most min(STAGES-2, KT-1) later stages in flight
  if (STAGES > 3 && KT >= STAGES - 1) wait_vmem_below<(STAGES > 3 ? (STAGES - 2) * LOADS : 0)>();
  else if (KT >= 2) wait_vmem_below<LOADS>();
  else wait_vmem_below<0>();
  barrier_only();
  load_frags(0, 0, fa[0], fb[0]);

  // Buffer reuse: the copy issued after the barrier of stage kt's last step
  // goes to buffer (kt-1) % STAGES, whose fragments every wave consumed (its
  // MFMAs issued) before reaching that barrier; STAGES >= 3 keeps it apart
  // from buffer (kt+1) % STAGES, read right after.
  for (int u = 0; u < U; u += 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int v = u + h;
      if (v < U) {
        const int kt = v / SUB, s = v % SUB;
        int nkt = kt, ns = s + 1;
        if (ns == SUB) {
          ns = 0;
          nkt = kt + 1;
          if (nkt < KT) {
            wait_stage_after(kt);
            if (kt + STAGES - 1 < KT) issue_stage(kt + STAGES - 1);
          }
        }
        // The last step re-reads its own fragments, so the reads are issued on
        // every path and the MFMAs below wait only for the previous step's.
        if (nkt >= KT) {
          nkt = kt;
          ns = s;
        }
        load_frags(nkt, ns, fa[1 - h], fb[1 - h]);
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int i = 0; i < TM; ++i) acc[j][i] = mfma_32x32x64_fp8(fa[h][j], fb[h][i], acc[j][i]);
      }
    }
  }

  if constexpr (SPLITK)
    if (!split_k_reduce<TN, TM, NW>(acc, partials, counters, tile, split, splits, wave, lane, &is_last)) return;
  if constexpr (SW) store_tile_sw<BM, BN, WGM, WGN, RANK>(lds, scale_lds, acc, ep, m0, n0, M, N, wm, wn, lane);
  else store_tile<BM, BN, WGM, WGN, RANK>(lds, scale_lds, acc, ep, m0, n0, M, N, wm, wn, lane);
}

// ---------------------------------------------------------------------------
// Ping-pong form of the prefill GEMM for 64-deep stages and 8 waves (2 x 4).
// The two waves that share a SIMD belong to different groups: group 0 (waves
// 0-3, one per SIMD) and group 1 (waves 4-7). The groups take turns: while one
// group issues the MFMAs of its step from registers, the other reads its next
// step's fragments from LDS and issues its share of the global -> LDS copies;
// every turn ends at a workgroup barrier. So the MFMA pipe of each SIMD has one
// wave feeding it at a time, and the LDS reads never wait behind the MFMAs of
// the same wave (in the lockstep form both waves of a SIMD read, then both
// multiply).
//
// Turns (phases) P = 0 .. 2U-1 for U steps: group 0 computes step P/2 at
// even P and reads step (P+1)/2 at odd P; group 1 computes step (P-1)/2 at odd
// P and reads step P/2 at even P (it idles at P = 0, group 0 at P = 2U-1).
// Stage j's LDS buffer is read by group 0 in phase 2j-1 and by group 1 in
// phase 2j; in the read turn of step m each group copies its share of stage
// m+STAGES-1 into the buffer of stage m-1, which both groups finished reading
// by the end of phase 2m-2. Stage j must have landed (every wave's copies)
// before phase 2j-1, so each wave waits for its own copies of stage j+1 before
// the barrier that ends phase 2j.
// ---------------------------------------------------------------------------
template <int BM, int BN, int STAGES, int RANK, bool PACKW, bool PACKX, bool SW = false>
__global__ __launch_bounds__(512) void gemm_prefill_pp_kernel(const uint8_t* __restrict__ xq, int64_t ldx,
                                                              const uint8_t* __restrict__ w, int64_t ldw, int M, int N,
                                                              int K, int tiles_m, int tiles_n, int group_m, Epilogue ep) {
  constexpr int WGM = 2, WGN = 4, NW = 8, BK = 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int CH = BK / 16, RPL = 1024 / BK;
  constexpr int ROWS = BM + BN, STAGE = ROWS * BK;
  constexpr int LOADS = ROWS / RPL / NW;  // wave-loads per wave per stage
  static_assert(ROWS % (RPL * NW) == 0 && BM % (NW * RPL) == 0 && TM >= 1 && TN >= 1, "tile shape");
  static_assert(STAGES >= 3 && STAGES <= 5 && (STAGES - 1) * LOADS < 64, "pipeline depth");
  constexpr int LDS_BYTES = STAGES * STAGE > BM * BN * 2 ? STAGES * STAGE : BM * BN * 2;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
  __shared__ __attribute__((aligned(256))) float scale_lds[BM + BN];

  int tile_m, tile_n;
  tile_of(blockIdx.x, tiles_m, tiles_n, group_m, tile_m, tile_n);
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int grp = wave >> 2;

  // Copy assignment as in gemm_prefill_kernel (64-deep stages).
  const int ntiles = (N + 15) >> 4, mtiles = (M + 15) >> 4;
  const uint8_t* src[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int g = i * NW + wave;
    const int r = g * RPL + lane / CH;
    const int chunk = (lane % CH) ^ swizzle<BK>(r);
    if (r < BM && PACKX) {
      const int tile = min((m0 >> 4) + g, mtiles - 1);
      src[i] = xq + (((int64_t)tile * (K >> 7)) * 2 + (lane >> 5)) * 1024 + (lane & 31) * 16;
    } else if (r < BM) {
      src[i] = xq + (int64_t)min(m0 + r, M - 1) * ldx + chunk * 16;
    } else if (PACKW) {
      const int lt = min((n0 >> 4) + (g - BM / RPL), ntiles - 1);
      const int64_t tile = SW ? swiglu_tile(lt, ep.half) : lt;
      src[i] = w + ((tile * (K >> 7)) * 2 + (lane >> 5)) * 1024 + (lane & 31) * 16;
    } else {
      const int c = min(n0 + r - BM, N - 1);
      src[i] = w + (SW ? swiglu_channel(c, ep.half) : (int64_t)c) * ldw + chunk * 16;
    }
  }
  auto issue_stage = [&](int kt) {
    uint8_t* base = lds + (kt % STAGES) * STAGE;
    const int64_t k0 = (int64_t)kt * BK;
    const int64_t wk = PACKW ? tiled_stage_offset<BK>(kt) : k0;
    const int64_t xk = PACKX ? tiled_stage_offset<BK>(kt) : k0;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) load_lds16(src[i] + (i * NW * RPL < BM ? xk : wk), base + (i * NW + wave) * 1024);
  };
  // Wait until at most `stages` later stages of this wave's copies are in flight.
  auto wait_copies = [&](int stages) {
    if (stages >= 3) wait_vmem_below<(STAGES > 3 ? 3 * LOADS : 0)>();
    else if (stages == 2) wait_vmem_below<2 * LOADS>();
    else if (stages == 1) wait_vmem_below<LOADS>();
    else wait_vmem_below<0>();
  };

  f32x16 acc[TN][TM];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;

  for (int t = wave * 64; t < BM + BN; t += NW * 64) {
    const int r = t + lane;
    const int c = min(n0 + r - BM, N - 1);
    const float* sp = r < BM ? ep.sx + min(m0 + r, M - 1) : ep.sw + (SW ? swiglu_channel(c, ep.half) : (int64_t)c);
    typedef __attribute__((address_space(3))) void lds_void;
    typedef __attribute__((address_space(1))) void global_void;
    __builtin_amdgcn_global_load_lds((global_void*)sp, (lds_void*)(scale_lds + t), 4, 0, 0);
  }

  const int frow = lane & 31;
  const int fhalf = (lane >> 5) * 2;
  int brow[TM], boff[TM], aoff[TN], arow[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    brow[i] = wm * WM + i * 32 + frow;
    boff[i] = (brow[i] >> 4) * 1024 + ((brow[i] & 15) + 16 * (lane >> 5)) * 16;
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    arow[j] = BM + wn * WN + j * 32 + frow;
    const int rr = wn * WN + j * 32 + frow;
    aoff[j] = BM * BK + (rr >> 4) * 1024 + ((rr & 15) + 16 * (lane >> 5)) * 16;
  }
  i32x8 fa[TN], fb[TM];
  auto load_frags = [&](int kt) {
    const uint8_t* base = lds + (kt % STAGES) * STAGE;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (PACKW) {
        const uint8_t* p = base + aoff[j];
        fa[j] = cat8(lds_read16(p), lds_read16(p + 512));
      } else {
        const int r = arow[j], sw = swizzle<BK>(r);
        fa[j] = cat8(lds_read16(base + r * BK + (fhalf ^ sw) * 16), lds_read16(base + r * BK + ((fhalf + 1) ^ sw) * 16));
      }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if constexpr (PACKX) {
        fb[i] = cat8(lds_read16(base + boff[i]), lds_read16(base + boff[i] + 512));
      } else {
        const int r = brow[i], sw = swizzle<BK>(r);
        fb[i] = cat8(lds_read16(base + r * BK + (fhalf ^ sw) * 16), lds_read16(base + r * BK + ((fhalf + 1) ^ sw) * 16));
      }
    }
  };

  const int U = K / BK;
#pragma unroll
  for (int p = 0; p < STAGES; ++p)
    if (p < U) issue_stage(p);
  wait_copies(min(STAGES - 1, U - 1));  // stage 0 (and the scales) landed
  barrier_only();
  load_frags(0);
  if (grp == 1) {
    // Phase 0 is group 0's first compute turn; group 1 only waits for stage 1
    // and finishes its reads of stage 0 (that buffer is refilled in phase 1).
    if (U > 1) wait_copies(min(STAGES - 2, U - 2));
    __builtin_amdgcn_s_waitcnt(0xC07F);
    barrier_only();
  }
  for (int k = 0; k < U; ++k) {
    // Compute turn of step k, from the fragments read in the previous turn.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i) acc[j][i] = mfma_32x32x64_fp8(fa[j], fb[i], acc[j][i]);
    __builtin_amdgcn_sched_barrier(0);
    if (grp == 0 && k + 1 < U) wait_copies(min(STAGES - 2, U - 2 - k));
    barrier_only();
    // Read turn of step k+1 (group 0 ends with an idle turn that matches
    // group 1's last compute turn).
    if (k + 1 < U) {
      __builtin_amdgcn_sched_barrier(0);
      if (k + STAGES < U) issue_stage(k + STAGES);
      load_frags(k + 1);
      if (grp == 1 && k + 2 < U) wait_copies(min(STAGES - 2, U - 3 - k));
      // This turn's LDS reads are complete before the barrier: the buffer is
      // refilled by the other group's next read turn.
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_sched_barrier(0);
      barrier_only();
    } else if (grp == 0) {
      barrier_only();
    }
  }
  if constexpr (SW) store_tile_sw<BM, BN, WGM, WGN, RANK>(lds, scale_lds, acc, ep, m0, n0, M, N, wm, wn, lane);
  else store_tile<BM, BN, WGM, WGN, RANK>(lds, scale_lds, acc, ep, m0, n0, M, N, wm, wn, lane);
}

// ---------------------------------------------------------------------------
// W8A16 parity mode, M > 64 or 32-64 tokens on wide weights
// (w8a16_decode_kernel_for):
// bf16 activations x e4m3 weights (converted to bf16 in registers, exact),
// v_mfma_f32_32x32x16_bf16, fp32 sums, then
// y = bf16(acc * sw[n]) and y = bf16(y + bias[n]) -- the reference's own
// arithmetic (inference/fp8.py:62-99, :183-184; model/metal_test.py:213).
// Each 64-deep K stage holds BM token rows of 128 B (bf16) and BN weight rows
// of 64 B (e4m3) in LDS, both swizzled for 16-lane ds_read_b128 phases. A
// lane half h of the 32x32 operand layout covers k = 32h + [0, 32) of the
// stage; MFMA q of the stage uses k = 32h + 8q + [0, 8) on both operands.
// ---------------------------------------------------------------------------
template <int BM, int BN, int WGM, int WGN, int STAGES, bool PACKW, bool SPLITK = false>
__global__ __launch_bounds__(64 * WGM * WGN) void w8a16_prefill_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ w, int64_t ldw, int M, int N, int K,
    int tiles_m, int tiles_n, int group_m, const float* __restrict__ sw, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ y, int64_t ldy, int splits, float* __restrict__ partials, int* __restrict__ counters) {
  constexpr int NW = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int XROW = 128, WROW = 64;               // bytes per LDS row: 64 bf16, 64 e4m3
  constexpr int XBYTES = BM * XROW, STAGE = XBYTES + BN * WROW;
  constexpr int XLOADS = XBYTES / 1024 / NW, WLOADS = BN * WROW / 1024 / NW;
  constexpr int OUT_CH = BN * 2 / 16;
  constexpr int LDS_BYTES = STAGES * STAGE > BM * BN * 2 ? STAGES * STAGE : BM * BN * 2;
  static_assert(XBYTES % (1024 * NW) == 0 && (BN * WROW) % (1024 * NW) == 0 && TM >= 1 && TN >= 1, "tile shape");
  static_assert(STAGES >= 2 && (STAGES - 2) * (XLOADS + WLOADS) < 64, "pipeline depth");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
  __shared__ int is_last;

  // With a K split, workgroup tile + s * tiles adds up part s of the k range
  // (whole 64-deep stages) and the last of a tile's workgroups to count in
  // sums the parts in split order and runs the epilogue (split_k_reduce).
  const int tiles = tiles_m * tiles_n;
  const int split = SPLITK ? (int)blockIdx.x / tiles : 0;
  const int tile = (int)blockIdx.x - split * tiles;
  int tile_m, tile_n;
  tile_of(tile, tiles_m, tiles_n, group_m, tile_m, tile_n);
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WGN, wn = wave % WGN;

  // DMA assignment: token wave-load g covers rows 8g..8g+7 (lane -> row l/8,
  // physical chunk l%8 holding logical chunk (l%8) ^ swizzle<128>(row));
  // weight wave-load g covers rows 16g..16g+15 (lane -> row l/4, chunk l%4).
  const uint8_t* xsrc[XLOADS];
  const uint8_t* wsrc[WLOADS];
#pragma unroll
  for (int i = 0; i < XLOADS; ++i) {
    const int r = (i * NW + wave) * 8 + lane / 8;
    xsrc[i] = reinterpret_cast<const uint8_t*>(x + (int64_t)min(m0 + r, M - 1) * ldx) + ((lane % 8) ^ swizzle<128>(r)) * 16;
  }
#pragma unroll
  for (int i = 0; i < WLOADS; ++i) {
    const int r = (i * NW + wave) * 16 + lane / 4;
    const int chunk = (lane % 4) ^ swizzle<64>(r);
    wsrc[i] = PACKW ? w + tiled_w_offset(min(n0 + r, N - 1), chunk * 16, K >> 7)
                    : w + (int64_t)min(n0 + r, N - 1) * ldw + chunk * 16;
  }
  // This workgroup's stages: [kt0, kt0 + KT) of the K / 64 stages.
  const int kt_all = K / 64;
  int kt0 = 0, KT = kt_all;
  if constexpr (SPLITK) {
    kt0 = (int)((uint32_t)(kt_all * split) / (uint32_t)splits);
    KT = (int)((uint32_t)(kt_all * (split + 1)) / (uint32_t)splits) - kt0;
  }
  auto issue_stage = [&](int kt) {
    uint8_t* base = lds + (kt % STAGES) * STAGE;
    const int ktg = kt0 + kt;
    const int64_t wk = PACKW ? tiled_stage_offset<64>(ktg) : (int64_t)ktg * 64;
#pragma unroll
    for (int i = 0; i < XLOADS; ++i) load_lds16(xsrc[i] + (int64_t)ktg * 128, base + (i * NW + wave) * 1024);
#pragma unroll
    for (int i = 0; i < WLOADS; ++i) load_lds16(wsrc[i] + wk, base + XBYTES + (i * NW + wave) * 1024);
  };

  f32x16 acc[TN][TM];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;

  const int frow = lane & 31, h = lane >> 5;
#pragma unroll
  for (int p = 0; p < STAGES - 1; ++p)
    if (p < KT) issue_stage(p);
  for (int kt = 0; kt < KT; ++kt) {
    // stage kt has landed once at most min(STAGES-2, KT-1-kt) later stages are in flight
    const int later = min(STAGES - 2, KT - 1 - kt);
    if (STAGES > 2 && later >= STAGES - 2) wait_vmem_below<(STAGES > 2 ? (STAGES - 2) * (XLOADS + WLOADS) : 0)>();
    else if (STAGES > 3 && later == 1) wait_vmem_below<XLOADS + WLOADS>();
    else wait_vmem_below<0>();
    barrier_only();
    // buffer (kt-1) % STAGES was consumed (its MFMAs issued) before the barrier
    if (kt + STAGES - 1 < KT) issue_stage(kt + STAGES - 1);
    const uint8_t* base = lds + (kt % STAGES) * STAGE;
    i32x4 a_raw[TN][2];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int r = wn * WN + j * 32 + frow;
      const uint8_t* rowp = base + XBYTES + r * WROW;
      a_raw[j][0] = lds_read16(rowp + ((2 * h) ^ swizzle<64>(r)) * 16);
      a_raw[j][1] = lds_read16(rowp + ((2 * h + 1) ^ swizzle<64>(r)) * 16);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bf16x8 b[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WM + i * 32 + frow;
        b[i] = __builtin_bit_cast(bf16x8, lds_read16(base + r * XROW + ((4 * h + q) ^ swizzle<128>(r)) * 16));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const i32x4 raw = a_raw[j][q >> 1];
        const bf16x8 a = (q & 1) ? e4m3x8_to_bf16(raw.z, raw.w) : e4m3x8_to_bf16(raw.x, raw.y);
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b[i], acc[j][i], 0, 0, 0);
      }
    }
  }

  if constexpr (SPLITK)
    if (!split_k_reduce<TN, TM, NW>(acc, partials, counters, tile, split, splits, wave, lane, &is_last)) return;

  // Epilogue through LDS (as the FP8 kernel): lane l holds token l % 32 and, in
  // register r, channel 8*(r/4) + 4*(l/32) + r%4.
  lds_barrier();
  const bool has_bias = bias != nullptr;
  // The thread's channel scales and biases, every load issued before any is
  // used (loaded next to their use, each waited for the one before it).
  float swv[TN][4][4], bv[TN][4][4];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int qd = 0; qd < 4; ++qd)
#pragma unroll
      for (int e = 0; e < 4; ++e) swv[j][qd][e] = sw[min(n0 + wn * WN + j * 32 + 8 * qd + 4 * (lane >> 5) + e, N - 1)];
  if (has_bias) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          bv[j][qd][e] = bf16_to_f32(bias[min(n0 + wn * WN + j * 32 + 8 * qd + 4 * (lane >> 5) + e, N - 1)]);
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const int nl = wn * WN + j * 32 + 8 * qd + 4 * (lane >> 5);
      uint32_t hv[TM][4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float swn = swv[j][qd][e];
        const float bn = has_bias ? bv[j][qd][e] : 0.0f;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          uint32_t v = f32_to_bf16(acc[j][i][4 * qd + e] * swn);
          if (has_bias) v = f32_to_bf16(bf16_to_f32(v) + bn);
          hv[i][e] = v;
        }
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int ml = wm * WM + i * 32 + (lane & 31);
        const int chunk = (nl >> 3) ^ (ml % OUT_CH);
        *reinterpret_cast<uint2*>(lds + ml * (BN * 2) + chunk * 16 + (nl & 4) * 2) =
            uint2{hv[i][0] | (hv[i][1] << 16), hv[i][2] | (hv[i][3] << 16)};
      }
    }
  }
  lds_barrier();
  const bool y_vec = ((ldy | N) & 7) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
  for (int c = threadIdx.x; c < BM * OUT_CH; c += 64 * NW) {
    const int ml = c / OUT_CH, ch = c % OUT_CH;
    const int m = m0 + ml, n = n0 + ch * 8;
    if (m >= M || n >= N) continue;
    const uint4 v = *reinterpret_cast<const uint4*>(lds + ml * (BN * 2) + (ch ^ (ml % OUT_CH)) * 16);
    uint16_t* dst = y + (int64_t)m * ldy + n;
    if (y_vec) {
      *reinterpret_cast<uint4*>(dst) = v;
    } else {
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (n + e < N) dst[e] = (uint16_t)(wv[e >> 1] >> (16 * (e & 1)));
    }
  }
}

template <int BM, int BN, int WGM, int WGN, int STAGES>
static hipError_t launch_w8a16_prefill(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                                       const float* sw, const uint16_t* bias, uint16_t* y, int64_t ldy, int group_m,
                                       hipStream_t stream, int splits = 1, float* partials = nullptr,
                                       int* counters = nullptr) {
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  const dim3 grid((unsigned)(tm * tn * splits)), block(64 * WGM * WGN);
#define JV_W8A16_PREFILL_LAUNCH(PW, SK)                                                                            \
  w8a16_prefill_kernel<BM, BN, WGM, WGN, STAGES, PW, SK><<<grid, block, 0, stream>>>(x, ldx, w, ldw, M, N, K, tm, tn, \
                                                                                      group_m, sw, bias, y, ldy,     \
                                                                                      splits, partials, counters)
  if (splits > 1) {
    // K splits on the 64x64 tiles only
    if constexpr (BM == 64 && BN == 64) {
      if (ldw == 0) JV_W8A16_PREFILL_LAUNCH(true, true);
      else JV_W8A16_PREFILL_LAUNCH(false, true);
    } else {
      return hipErrorInvalidValue;
    }
  } else if (ldw == 0) {
    JV_W8A16_PREFILL_LAUNCH(true, false);
  } else {
    JV_W8A16_PREFILL_LAUNCH(false, false);
  }
#undef JV_W8A16_PREFILL_LAUNCH
  return hipGetLastError();
}

hipError_t w8a16_prefill(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                         const float* sw, const uint16_t* bias, uint16_t* y, int64_t ldy, int splits, float* partials,
                         int* counters, int cu_count, hipStream_t stream) {
  if (K % 64) return hipErrorInvalidValue;
  if (splits != w8a16_prefill_splits(M, N, K, cu_count) || (splits > 1 && (!partials || !counters)))
    return hipErrorInvalidValue;
  // 32-64 tokens over a wide weight (w8a16_decode_kernel_for), and wherever
  // 128x128 tiles would not fill one round of CUs (q/o at 96 tokens: 32 of
  // them) except on those wide weights: 64x64 tiles, four stages deep
  // (gate+up at 32 tokens 31.3 us; three stages 34.5, six 34.7: each stage
  // holds only 4 KB of weight), K split as w8a16_prefill_splits says.
  if (w8a16_small_tiles(M, N, cu_count))
    return launch_w8a16_prefill<64, 64, 2, 2, 4>(x, ldx, w, ldw, M, N, K, sw, bias, y, ldy, 8, stream, splits, partials,
                                                 counters);
  // From five eighths of a round of 256x256 tiles on, 256x256 or 256x128
  // tiles, whichever needs less time in whole rounds: a round of 256x256
  // tiles takes 1.65 times one of 256x128 (123 / 73 us full at K = 4096, 101 /
  // 63 alone). Merged q/k/v at M = 2048 106.8 us on 256x256 tiles against
  // 132.4 on 256x128, gate+up at M = 512 110.0 against 133.8, the 10240-wide
  // merge at M = 1024 104.0 against 131.2, q/o and down at M = 4096 120.5 /
  // 350.9 against 148.8 / 414.3; 256x128 where the 256x256 tiles spill into a
  // part-filled round: gate+up at M = 768 202.3 against 216.7, the
  // 10240-wide merge at M = 2048 202.8 against 216.0. Below that 256x128
  // from a round of them, else 128x128 (us, graphs over rotated weights).
  const int64_t cus = cu_count;
  const int64_t t256 = ((int64_t)(M + 255) / 256) * ((N + 255) / 256);
  const int64_t t128 = ((int64_t)(M + 255) / 256) * ((N + 127) / 128);
  if (t256 * 8 >= 5 * cus) {
    const int64_t r256 = (t256 + cus - 1) / cus, r128 = (t128 + cus - 1) / cus;
    if (33 * r256 <= 20 * r128)
      return launch_w8a16_prefill<256, 256, 2, 4, 3>(x, ldx, w, ldw, M, N, K, sw, bias, y, ldy, 4, stream);
    return launch_w8a16_prefill<256, 128, 2, 4, 3>(x, ldx, w, ldw, M, N, K, sw, bias, y, ldy, 4, stream);
  }
  if (t128 >= cus)
    return launch_w8a16_prefill<256, 128, 2, 4, 3>(x, ldx, w, ldw, M, N, K, sw, bias, y, ldy, 4, stream);
  return launch_w8a16_prefill<128, 128, 2, 2, 3>(x, ldx, w, ldw, M, N, K, sw, bias, y, ldy, 8, stream);
}

// ldx = 0: activation codes in the packed fragment order (packed_x_offset);
// ldw = 0: tiled weights (tiled_w_offset).
template <int BM, int BN, int WGM, int WGN, int BK, int STAGES>
static hipError_t launch_prefill(const uint8_t* xq, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                                 const Epilogue& ep, int rank, int group_m, int splits, float* partials, int* counters,
                                 hipStream_t stream) {
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  const dim3 grid((unsigned)(tm * tn * splits)), block(64 * WGM * WGN);
  if (group_m < 1) group_m = 1;
#define JV_PREFILL_LAUNCH(R, PW, PX)                                   \
  gemm_prefill_kernel<BM, BN, WGM, WGN, BK, STAGES, R, PW, PX>         \
      <<<grid, block, 0, stream>>>(xq, ldx, w, ldw, M, N, K, tm, tn, group_m, ep, splits, partials, counters)
#define JV_PREFILL_LAUNCH_X(R, PW)             \
  if (ldx == 0) JV_PREFILL_LAUNCH(R, PW, true); \
  else JV_PREFILL_LAUNCH(R, PW, false);
  {
    if (splits > 1) {
      // split-K: plain or LoRA epilogue (the fused SwiGLU keeps whole k ranges)
#define JV_PREFILL_LAUNCH_SK(R, PW, PX)                                         \
  gemm_prefill_kernel<BM, BN, WGM, WGN, BK, STAGES, R, PW, PX, false, true>     \
      <<<grid, block, 0, stream>>>(xq, ldx, w, ldw, M, N, K, tm, tn, group_m, ep, splits, partials, counters)
#define JV_PREFILL_LAUNCH_SK_X(R, PW)             \
  if (ldx == 0) JV_PREFILL_LAUNCH_SK(R, PW, true); \
  else JV_PREFILL_LAUNCH_SK(R, PW, false);
      if (ep.half) {
        // fused SwiGLU, split K: packed activation codes only; the last
        // workgroup of a tile applies the SwiGLU epilogue to the summed tile
#define JV_PREFILL_LAUNCH_SK_SW(R, PW)                                        \
  gemm_prefill_kernel<BM, BN, WGM, WGN, BK, STAGES, R, PW, true, true, true>  \
      <<<grid, block, 0, stream>>>(xq, ldx, w, ldw, M, N, K, tm, tn, group_m, ep, splits, partials, counters)
        if (ldx != 0) return hipErrorInvalidValue;
        if (rank == 16) {
          if (ldw == 0) JV_PREFILL_LAUNCH_SK_SW(16, true);
          else JV_PREFILL_LAUNCH_SK_SW(16, false);
        } else {
          if (ldw == 0) JV_PREFILL_LAUNCH_SK_SW(0, true);
          else JV_PREFILL_LAUNCH_SK_SW(0, false);
        }
#undef JV_PREFILL_LAUNCH_SK_SW
        return hipGetLastError();
      }
      if (rank == 16) {
        if (ldw == 0) { JV_PREFILL_LAUNCH_SK_X(16, true) }
        else { JV_PREFILL_LAUNCH_SK_X(16, false) }
      } else {
        if (ldw == 0) { JV_PREFILL_LAUNCH_SK_X(0, true) }
        else { JV_PREFILL_LAUNCH_SK_X(0, false) }
      }
#undef JV_PREFILL_LAUNCH_SK_X
#undef JV_PREFILL_LAUNCH_SK
      return hipGetLastError();
    }
  }
  if (splits > 1) return hipErrorInvalidValue;
  if (ep.half) {
    // fused SwiGLU: packed activation codes only
#define JV_PREFILL_LAUNCH_SW(R, PW)                                      \
  gemm_prefill_kernel<BM, BN, WGM, WGN, BK, STAGES, R, PW, true, true>   \
      <<<grid, block, 0, stream>>>(xq, ldx, w, ldw, M, N, K, tm, tn, group_m, ep, splits, partials, counters)
    if (rank == 16) {
      if (ldw == 0) JV_PREFILL_LAUNCH_SW(16, true);
      else JV_PREFILL_LAUNCH_SW(16, false);
    } else {
      if (ldw == 0) JV_PREFILL_LAUNCH_SW(0, true);
      else JV_PREFILL_LAUNCH_SW(0, false);
    }
#undef JV_PREFILL_LAUNCH_SW
  } else if (rank == 16) {
    if (ldw == 0) { JV_PREFILL_LAUNCH_X(16, true) }
    else { JV_PREFILL_LAUNCH_X(16, false) }
  } else {
    if (ldw == 0) { JV_PREFILL_LAUNCH_X(0, true) }
    else { JV_PREFILL_LAUNCH_X(0, false) }
  }
#undef JV_PREFILL_LAUNCH_X
#undef JV_PREFILL_LAUNCH
  return hipGetLastError();
}

template <int BM, int BN, int STAGES>
static hipError_t launch_prefill_pp(const uint8_t* xq, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                                    const Epilogue& ep, int rank, int group_m, hipStream_t stream) {
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  const dim3 grid((unsigned)(tm * tn)), block(512);
  if (group_m < 1) group_m = 1;
#define JV_PREFILL_PP_LAUNCH(R, PW, PX) \
  gemm_prefill_pp_kernel<BM, BN, STAGES, R, PW, PX><<<grid, block, 0, stream>>>(xq, ldx, w, ldw, M, N, K, tm, tn, group_m, ep)
#define JV_PREFILL_PP_LAUNCH_R(R)                          \
  if (ldw == 0) {                                          \
    if (ldx == 0) JV_PREFILL_PP_LAUNCH(R, true, true);     \
    else JV_PREFILL_PP_LAUNCH(R, true, false);             \
  } else {                                                 \
    if (ldx == 0) JV_PREFILL_PP_LAUNCH(R, false, true);    \
    else JV_PREFILL_PP_LAUNCH(R, false, false);            \
  }
#define JV_PREFILL_PP_LAUNCH_SW(R, PW) \
  gemm_prefill_pp_kernel<BM, BN, STAGES, R, PW, true, true><<<grid, block, 0, stream>>>(xq, ldx, w, ldw, M, N, K, tm, tn, group_m, ep)
  if (ep.half) {
    if (rank == 16) {
      if (ldw == 0) JV_PREFILL_PP_LAUNCH_SW(16, true);
      else JV_PREFILL_PP_LAUNCH_SW(16, false);
    } else {
      if (ldw == 0) JV_PREFILL_PP_LAUNCH_SW(0, true);
      else JV_PREFILL_PP_LAUNCH_SW(0, false);
    }
  } else if (rank == 16) {
    JV_PREFILL_PP_LAUNCH_R(16)
  } else {
    JV_PREFILL_PP_LAUNCH_R(0)
  }
#undef JV_PREFILL_PP_LAUNCH_SW
#undef JV_PREFILL_PP_LAUNCH_R
#undef JV_PREFILL_PP_LAUNCH
  return hipGetLastError();
}

// Time model of a prefill launch, fitted (least squares on log time) to
// timings on MI355X (graphs of back-to-back launches over rotated weights):
// the five lockstep tiles at 1-8 K splits, 965 timings over 16 weights (N =
// 1024, 4096, 6144, 8192, 10240, 12288, 24576 at K = 4096, the 9B projections
// and merged widths; 1024-4096 at K = 2048, 8192 and 12288) at M = 160-2048;
// the two ping-pong tiles (no K split), 128 timings over 8 of those weights at
// M = 256-4096.
// Workgroups run in rounds of cu_count * per_cu. Per 4096 of K a workgroup
// takes `light` us in a round with few workgroups and `full` us in a full one
// (HBM, L2 and LDS bandwidth shared), plus `item` us of prologue and
// epilogue; a split launch adds the partial write, the count and the last
// workgroup's loads, growing with the partial tile bytes and the rounds. The
// argmin of the model is within 0.2% of the fastest measured choice summed
// over those shapes; the lockstep tiles alone with 256x256 ping-pong tiles
// from five eighths of a round: 1.5% (merged q/k/v at M = 1536 61.9 -> 43.9
// us, the 12288-wide merge at M = 768 63.1 -> 44.8, gate+up at M = 768 96.3 ->
// 88.4, merged q/k/v at M = 3072 91.4 -> 81.2).
struct TileCost {
  PrefillTile tile;
  int per_cu;         // workgroups per CU (LDS and VGPR occupancy)
  double light, full, item;
};
static const TileCost kTileCosts[] = {
    {{256, 256, 2, 4, 64, 4, 4, true}, 1, 29.60, 42.54, 9.98},
    {{128, 384, 2, 4, 64, 4, 8, true}, 1, 30.21, 37.16, 8.92},
    {{256, 128, 2, 4, 128, 3, 4}, 1, 30.22, 34.48, 3.97},
    {{128, 128, 2, 2, 128, 4, 8}, 1, 15.08, 18.21, 5.58},
    {{64, 128, 2, 4, 128, 5, 8}, 1, 11.69, 12.83, 2.46},
    {{64, 64, 2, 2, 128, 5, 8}, 1, 8.66, 8.33, 2.37},
    {{64, 64, 2, 2, 128, 4, 8}, 2, 8.66, 15.29, 2.45},
};
// A split launch: a fixed cost, a cost per split, and a cost per split of a
// 128x128 fp32 partial per round.
constexpr double kSplitBaseUs = 2.51, kSplitEachUs = 0.16, kSplitPerTileUs = 0.81;

static double tile_time_us(const TileCost& c, int64_t M, int64_t N, int64_t K, int splits, int cu_count) {
  const int64_t tiles = ((M + c.tile.bm - 1) / c.tile.bm) * ((N + c.tile.bn - 1) / c.tile.bn);
  const int64_t items = tiles * splits, slots = (int64_t)cu_count * c.per_cu;
  const int64_t rounds = items / slots, rest = items % slots;
  const double k = (double)K / 4096.0 / splits;
  double t = rounds * (c.full * k + c.item);
  if (rest) t += (c.light + (c.full - c.light) * (double)rest / slots) * k + c.item;
  if (splits > 1) {
    const double round_count = items > slots ? (double)items / slots : 1.0;
    t += kSplitBaseUs + kSplitEachUs * splits + kSplitPerTileUs * splits * (c.tile.bm * c.tile.bn / 16384.0) * round_count;
  }
  return t;
}

// Tiles for 17-128 tokens (the engine's decode batches), measured on the 9B
// projection shapes (graphs over rotated weights; us at M = 32 / 48 / 64 /
// 96 / 128). Deeper copy rings than the prefill tiles: these launches are
// bound by how many bytes each CU keeps in flight, not by the MFMAs.
//  * weights of 1.5 rounds of 64-channel tiles (gate+up) at up to 64 tokens:
//    64x128 tiles of 8 waves, 4 stages (21.2 / 22.2 / 23.1 vs 22.0 / 23.0 /
//    24.1 with 64x64 and 4 stages); above 64 tokens the model below (128x128);
//  * above 64 tokens, weights of 0.625 rounds of 64x128 tiles (N >= 10240 at
//    65-128 tokens): 64x128 tiles of 8 waves, 5 stages (10240-wide 17.0 /
//    17.9 at 96 / 128 vs 18.1 / 19.8 before; 12288-wide 17.7 / 18.6 vs 18.9 /
//    20.5);
//  * everything else: 64x64 tiles of 4 waves, 5 stages (80 KB of LDS, one
//    workgroup per CU), K split so the tiles and splits reach the CUs (at most
//    4 ways): q/o 10.2 / 10.3 at 96 / 128 vs 11.4 / 11.8; merged q/k/v 12.0 /
//    12.2 vs 14.2 / 15.1; down 14.9 / 15.4 / 15.8 / 19.5 / 20.4 vs 15.8 /
//    16.7 / 18.8 / 20.3 / 22.1; k/v 8.4 / 8.5 vs 8.6 / 8.7.
static bool small_batch_tile(int64_t M, int64_t N, int64_t K, int64_t cus, bool split_k, PrefillTile& t) {
  const int64_t mt = (M + 63) / 64, n64 = (N + 63) / 64, t64 = mt * n64, t128 = mt * ((N + 127) / 128);
  if (2 * n64 >= 3 * cus) {
    if (M > kDecodeMaxRows) return false;
    t = PrefillTile{64, 128, 2, 4, 128, 4, 8};
    return true;
  }
  if (M > kDecodeMaxRows && 8 * t128 >= 5 * cus) {
    t = PrefillTile{64, 128, 2, 4, 128, 5, 8};
    return true;
  }
  t = PrefillTile{64, 64, 2, 2, 128, 5, 8};
  if (split_k && 8 * t64 < 5 * cus) {
    // each split keeps at least four 128-deep stages, the partials at most
    // kMaxPrefillPartialBytes (a split's partials are one fp32 64x64 tile per tile)
    int s = (int)(cus / t64);
    s = s < 1 ? 1 : (s > 4 ? 4 : s);
    while (s > 1 && (K / t.bk < 4 * s || t64 * s * 64 * 64 * 4 > kMaxPrefillPartialBytes)) --s;
    t.splits = s;
  }
  return true;
}

PrefillTile prefill_tile(int64_t M, int64_t N, int64_t K, int cu_count, bool split_k) {
  PrefillTile small;
  if (M <= 2 * kDecodeMaxRows && small_batch_tile(M, N, K, cu_count, split_k, small)) return small;
  // From five eighths of a round of 256x256 tiles on, the ping-pong tiles
  // (least L2 -> LDS traffic per flop, the fastest tiles per CU) only: the
  // model's lockstep terms were fitted up to M = 2048. Else every tile.
  const int64_t cus = cu_count;
  const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
  const bool pingpong_only = t256 * 8 >= cus * 5;
  // The tile and K split of least modelled time (ping-pong tiles keep whole
  // k ranges); each split keeps at least four BK-deep stages and the
  // partials at most kMaxPrefillPartialBytes, and a split fills at most one
  // round of workgroups (splits that spill into a second round measured
  // slower than the model puts them: down at M = 320 34.2 us on 128x128
  // tiles with 2 splits against 37.9 on 64x128 with 3).
  PrefillTile best{64, 64, 2, 2, 128, 4, 8};
  double best_us = 1e300;
  for (const TileCost& c : kTileCosts) {
    if (pingpong_only && !c.tile.pingpong) continue;
    const int64_t tiles = ((M + c.tile.bm - 1) / c.tile.bm) * ((N + c.tile.bn - 1) / c.tile.bn);
    for (int s = 1; s <= (split_k && !c.tile.pingpong ? kMaxPrefillSplits : 1); ++s) {
      PrefillTile t = c.tile;
      t.splits = s;
      if (s > 1 && (K / t.bk < 4 * s || prefill_partial_bytes(t, M, N) > kMaxPrefillPartialBytes ||
                    tiles * s > cus * c.per_cu))
        break;
      const double us = tile_time_us(c, M, N, K, s, cu_count);
      if (us < best_us) best_us = us, best = t;
    }
  }
  return best;
}

hipError_t gemm_prefill(const uint8_t* xq, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                        const Epilogue& ep, int rank, PrefillTile t, float* partials, int* counters,
                        hipStream_t stream) {
  if (rank != 0 && rank != 16) return hipErrorInvalidValue;
  if (K % t.bk || K % 128) return hipErrorInvalidValue;
  if (ep.half && (ldx != 0 || 2 * ep.half != N || ep.half % 16)) return hipErrorInvalidValue;
  if (t.splits < 1 || t.splits > kMaxPrefillSplits ||
      (t.splits > 1 && (t.pingpong || !partials || !counters || K / t.bk < t.splits)))
    return hipErrorInvalidValue;
  if (t.pingpong) {
    if (t.wgm != 2 || t.wgn != 4 || t.bk != 64) return hipErrorInvalidValue;
#define JV_PREFILL_PP_CASE(BM_, BN_, ST_) \
  if (t.bm == BM_ && t.bn == BN_ && t.stages == ST_) \
    return launch_prefill_pp<BM_, BN_, ST_>(xq, ldx, w, ldw, M, N, K, ep, rank, t.group_m, stream);
    JV_PREFILL_PP_CASE(256, 256, 4)
    JV_PREFILL_PP_CASE(128, 384, 4)
#undef JV_PREFILL_PP_CASE
    return hipErrorInvalidValue;
  }
#define JV_PREFILL_CASE(BM_, BN_, WGM_, WGN_, BK_, ST_)                                                     \
  if (t.bm == BM_ && t.bn == BN_ && t.wgm == WGM_ && t.wgn == WGN_ && t.bk == BK_ && t.stages == ST_)       \
    return launch_prefill<BM_, BN_, WGM_, WGN_, BK_, ST_>(xq, ldx, w, ldw, M, N, K, ep, rank, t.group_m, t.splits, partials, \
                                                         counters, stream);
  // The lockstep shapes prefill_tile picks.
  JV_PREFILL_CASE(256, 128, 2, 4, 128, 3)
  JV_PREFILL_CASE(128, 128, 2, 2, 128, 4)
  JV_PREFILL_CASE(64, 64, 2, 2, 128, 4)
  JV_PREFILL_CASE(64, 64, 2, 2, 128, 5)
  JV_PREFILL_CASE(64, 128, 2, 4, 128, 4)
  JV_PREFILL_CASE(64, 128, 2, 4, 128, 5)
#undef JV_PREFILL_CASE
  return hipErrorInvalidValue;
}

}  // namespace jv
