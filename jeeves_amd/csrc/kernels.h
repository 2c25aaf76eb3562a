// Internal launchers shared by the C-ABI (capi.hip). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "epilogue.h"

namespace jv {

// Decode regime: M <= kDecodeMaxRows tokens.
constexpr int kDecodeMaxRows = 64;

// The W8A16 parity mode's base rule: its decode kernel takes M <= 16 tokens,
// and up to kDecodeMaxRows tokens unless the weight is wide enough for 1.5
// rounds of 64-channel tiles of the prefill kernel (measured on MI355X:
// gate+up, N = 24576, 23.4 vs 30.4 us at M = 64 on the FP8 kernels, 23.1 vs
// 28.7 at M = 40, 21.6 vs 22.4 at M = 24; the lm_head, N = 248320, 193 vs 236
// us at M = 64 and 179 vs 202 at M = 32). Those prefill tiles stage each
// 16-token tile's codes in LDS once per workgroup, where the decode waves each
// load every code fragment.
inline bool decode_kernel_for(int64_t M, int64_t N, int cu_count) {
  if (M > kDecodeMaxRows) return false;
  return M <= 16 || 2 * ((N + 63) / 64) < 3 * (int64_t)cu_count;
}

// The FP8 GEMM's rule: the decode kernel at 1-16 tokens, and at 17-64 tokens
// except on weights wide enough for 1.5 rounds of 64-channel tiles (gate+up,
// the lm_head) and, from 32 tokens, on weights of at least 0.625 rounds
// (N >= 10240: the 9B model's attention and drafter merged projections) or
// long rows whose 64-channel tiles, split K four ways, fill the CUs (K >=
// 8192: down). There every decode workgroup would re-read all M x K
// activation codes from L2 for its 16 or 32 channels -- the time grows by
// about 1 us per 16 tokens on q/o and 2.6 us on down, whatever the plan --
// while the prefill kernel's 64-token tiles share each code fragment among
// 64 or 128 channels. Measured (graphs over rotated weights, us, decode kernel
// vs 64x64 tiles with a 5-stage ring): down M = 32 / 48 / 64: 15.8 / 16.7 /
// 18.8 vs 14.9 / 15.4 / 15.8; the 12288-wide projection 15.1 / 16.8 / 19.1
// vs 13.3 / 14.0 / 14.1; the 10240-wide 13.1 / 15.8 / 18.4 vs 12.6 / 13.1 /
// 13.3; q/o, k/v, merged q/k/v and the 8192-wide stayed on the decode kernel
// (q M = 64: 8.4 vs 9.4). The batch-decode plan (batch_plan, below) is asked
// first and takes most of those: the decode kernel now runs 17-64 tokens
// only where neither it nor the prefill tiles do (the 10240/12288-wide
// projections at 17-31 tokens, other K).
inline bool fp8_decode_kernel_for(int64_t M, int64_t N, int64_t K, int cu_count) {
  if (M > kDecodeMaxRows) return false;
  if (M <= 16) return true;
  const int64_t t64 = (N + 63) / 64, cus = cu_count;
  if (2 * t64 >= 3 * cus) return false;
  if (M >= 32 && (8 * t64 >= 5 * cus || (K >= 8192 && 4 * t64 >= cus))) return false;
  return true;
}

// The W8A16 prefill tiles stage bf16 token rows, twice the bytes of codes,
// and win on those wide weights from 32 tokens (gate+up 35.8 vs 60.5 us at
// 64 tokens, 34.0 vs 43.7 at 48, a tie at 32, 33.6 vs 28.7 at 17; lm_head
// 285 vs 587 at 64, 256 vs 283 at 32, 250 vs 218 at 17).
// Where this rule and decode_kernel_for differ the weight has thousands of
// 16-row tiles, so the decode plan does not split K there: no workspace and
// no tile counters either way.
inline bool w8a16_decode_kernel_for(int64_t M, int64_t N, int cu_count) {
  return M < 32 || decode_kernel_for(M, N, cu_count);
}

// Batch-decode kernel (gemm_batch.hip) for 17-128 tokens: W waves of `steps`
// 128-deep k steps cover each row exactly, every wave holding its whole k
// range of weights in registers; a workgroup takes rt 16-row weight tiles and
// mt 16-token tiles, and msplit workgroups share each weight group, one part
// of the batch each.
struct BatchPlan {
  int waves, steps;  // waves * steps = K / 128
  int rt, mt;        // weight tiles and token tiles per workgroup
  int msplit;        // token parts: mt * msplit = ceil(M / 16)
  int groups;        // weight groups: ceil(ceil(N / 16) / rt)
};

// Token tiles a batch workgroup can hold beside its weights without spilling.
inline int batch_max_mt(int waves, int rt) { return waves == 4 ? 4 : (rt == 1 ? 2 : 1); }

// The batch plan for these sizes, if the batch kernel takes them. Rows of
// 32 k steps (K = 4096) run as 4 waves x 8, rows of 96 (K = 12288) as
// 8 x 12: the decode kernel's waves per row at those K, so both give each
// output the same k order. The plan takes at most one workgroup per CU and
// at least half the CUs, from weights of 64 tiles up, and minimises the
// bytes a workgroup reads, (rt + mt) x 16 x K, keeping it within 6 tiles and
// 576 KiB; ties take one weight tile per workgroup. Measured on MI355X (graphs over
// rotated weights, us, this plan vs the decode or prefill plan it replaces):
// k/v (1024 x 4096) M = 32 / 64 / 128: 4.2 / 4.2 / 4.7 vs 5.7 / 7.8 / 8.5;
// q/o (4096 x 4096) M = 64 / 128: 6.9 / 8.7 vs 8.3 / 10.4; merged q/k/v
// (6144 x 4096) M = 32 / 64: 7.8 / 9.5 vs 8.8 / 10.4; down (4096 x 12288)
// M = 32: 13.6 vs 14.9. Wider weights, longer token tiles and K = 12288
// past 32 tokens stay on the decode and prefill plans, which share each
// activation fragment among more channels (gate+up M = 64: 27 vs 23 us).
// swiglu: the fused SwiGLU GEMM's plan (a gate/up tile pair per workgroup,
// the plain plan's waves and steps, hence the plain plan's sums).
inline bool batch_plan(int64_t M, int64_t N, int64_t K, int cu_count, bool swiglu, BatchPlan* out) {
  if (M < 17 || M > 128 || N <= 0 || cu_count <= 0) return false;
  BatchPlan p{};
  if (K == 32 * 128) {
    p.waves = 4;
    p.steps = 8;
  } else if (K == 96 * 128) {
    p.waves = 8;
    p.steps = 12;
  } else {
    return false;
  }
  const int64_t tiles = (N + 15) / 16, mtall = (M + 15) / 16, cus = cu_count;
  if (tiles < 64) return false;
  int64_t best = 0;
  for (int rt = 1; rt <= 2; ++rt)
    for (int64_t ms = 1; ms <= mtall; ++ms) {
      if (mtall % ms) continue;
      const int64_t mt = mtall / ms, groups = (tiles + rt - 1) / rt, cost = rt + mt;
      if (mt > batch_max_mt(p.waves, rt) || groups * ms > cus || 2 * groups * ms < cus) continue;
      if (cost > 6 || cost * K > 36864) continue;
      if (best == 0 || cost < best) {
        best = cost;
        p.rt = rt;
        p.mt = (int)mt;
        p.msplit = (int)ms;
        p.groups = (int)groups;
      }
    }
  if (best == 0) return false;
  if (swiglu) {
    // Any tiling of the same waves and steps sums alike: pairs of tiles, the
    // fewest token parts whose tiles fit beside them.
    p.rt = 2;
    p.groups = (int)((tiles + 1) / 2);
    for (p.msplit = 1; mtall % p.msplit || mtall / p.msplit > batch_max_mt(p.waves, 2); ++p.msplit) {
    }
    p.mt = (int)(mtall / p.msplit);
  }
  if (out) *out = p;
  return true;
}

// The W8A16 parity mode's batch-decode plan (w8a16_batch_kernel, w8a16.hip):
// the FP8 plan's waves and steps, with this mode's operand bytes: a workgroup
// reads (rt + 2 mt) x 16 x K (bf16 activations), at most 6 such tiles and
// 576 KiB, and holds at most 2 token tiles beside its weights. It is taken
// only where it splits the batch's token tiles (msplit >= 2): unsplit, the
// W8A16 decode kernel's eight waves keep more in flight (merged q/k/v at 32
// tokens 12.4 vs 13.6 us). One round of workgroups; past 64 tokens, where
// the alternative is the W8A16 prefill tiles, two rounds too. Measured on
// MI355X (us, graphs over rotated weights, this plan vs the W8A16 decode
// kernel or, past 64 tokens, its prefill tiles): k/v M = 32 / 64 / 128: 7.0 /
// 6.9 / 7.7 vs 10.4 / 17.8 / 48.2; q/o M = 32 / 64 / 96 / 128: 8.9 / 12.8 /
// 20.9 / 21.0 vs 10.9 / 18.4 / 48.5 / 48.7. Two rounds below 65 tokens lost
// to the decode kernel (merged q/k/v 12.7 vs 10.2 us at 17, down 29.1 vs 19.8).
inline int w8a16_batch_max_mt(int waves, int rt) { return waves == 4 ? 2 : (rt == 1 ? 1 : 0); }
inline bool w8a16_batch_plan(int64_t M, int64_t N, int64_t K, int cu_count, BatchPlan* out) {
  if (M < 17 || M > 128 || N <= 0 || cu_count <= 0) return false;
  BatchPlan p{};
  if (K == 32 * 128) {
    p.waves = 4;
    p.steps = 8;
  } else if (K == 96 * 128) {
    p.waves = 8;
    p.steps = 12;
  } else {
    return false;
  }
  const int64_t tiles = (N + 15) / 16, mtall = (M + 15) / 16, cus = cu_count;
  if (tiles < 64) return false;
  int64_t best = 0;
  for (int64_t rounds = 1; rounds <= (M > kDecodeMaxRows ? 2 : 1) && best == 0; ++rounds)
    for (int rt = 1; rt <= 2; ++rt)
      for (int64_t ms = 2; ms <= mtall; ++ms) {
        if (mtall % ms) continue;
        const int64_t mt = mtall / ms, groups = (tiles + rt - 1) / rt, cost = rt + 2 * mt, wgs = groups * ms;
        if (mt > w8a16_batch_max_mt(p.waves, rt) || wgs > rounds * cus || 2 * wgs < rounds * cus) continue;
        if (cost > 6 || cost * K > 36864) continue;
        if (best == 0 || cost < best) {
          best = cost;
          p.rt = rt;
          p.mt = (int)mt;
          p.msplit = (int)ms;
          p.groups = (int)groups;
        }
      }
  if (best == 0) return false;
  if (out) *out = p;
  return true;
}

struct DecodePlan {
  int rt;      // 16-row tiles per wave
  int waves;   // waves per workgroup, splitting the workgroup's k range
  int unroll;  // k steps of 128 loaded per burst
  int groups;  // workgroups along N
  int splits;  // workgroups along K
};

// First 128-deep k step of K slice `slice` of splits * W (the decode kernels'
// W waves per split): floor(ksteps * slice / (splits * W)). In 32 bits, since
// ksteps * splits * W <= K for W <= 8 and splits <= 16; without a K split the
// divisor is the compile-time W, a shift. (A 64-bit division by a register
// took ~130 scalar instructions, twice, ahead of every wave's first load.)
template <int W>
__device__ __forceinline__ int slice_begin(int ksteps, int slice, int splits) {
  static_assert(W >= 1 && W <= 8 && (W & (W - 1)) == 0, "1-8 waves, a power of two");
  const uint32_t num = (uint32_t)ksteps * (uint32_t)slice;
  return (int)(splits == 1 ? num / (uint32_t)W : num / ((uint32_t)splits * W));
}

// Prefill launch shape: output tile bm (tokens) x bn (channels), a wgm x wgn
// grid of waves per workgroup, K stages of bk bytes in a ring of `stages` LDS
// buffers, and group_m M-tiles walking N together. pingpong selects the form
// whose two wave groups alternate MFMAs and LDS reads (2 x 4 waves, bk = 64).
struct PrefillTile {
  int bm, bn, wgm, wgn, bk, stages, group_m;
  bool pingpong = false;
  // Lockstep tiles: workgroups per tile, each adding up its own part of the
  // k range (1: no split).
  int splits = 1;
};

// Workspace bytes of a prefill launch with this tile: one fp32 partial tile
// per (tile, split) when K is split, else 0.
inline int64_t prefill_partial_bytes(const PrefillTile& t, int64_t M, int64_t N) {
  if (t.splits < 2) return 0;
  return ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) * t.splits * (int64_t)t.bm * t.bn * 4;
}

// Tile counters a prefill launch with this tile needs (one per output tile
// when K is split).
inline int64_t prefill_counters(const PrefillTile& t, int64_t M, int64_t N) {
  return t.splits < 2 ? 0 : ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
}

// Byte offset of activation code (m, k) in the packed layout: for token tile
// mt = m/16 and 128-k step s, two 1 KB halves, each holding 16 bytes per lane
// in the decode MFMA's B-fragment order (lane = m%16 + 16*((k%128)/32),
// half = (k%32)/16). Rows are padded to a multiple of 16 tokens. The prefill
// kernels copy the same 512-byte runs (half a fragment per 64-deep stage)
// into LDS and read their 32x32x64 fragments from them.
__host__ __device__ inline int64_t packed_x_offset(int m, int k, int ksteps) {
  const int mt = m >> 4, s = k >> 7, kk = k & 127;
  const int lane = (m & 15) + 16 * (kk >> 5), half = (kk >> 4) & 1;
  return ((((int64_t)mt * ksteps + s) * 2 + half) << 10) + lane * 16 + (kk & 15);
}

inline int64_t packed_x_bytes(int64_t M, int64_t K) { return (M + 15) / 16 * 16 * K; }

// Tiled weight layout (ldw = 0 for every GEMM launcher here and at the C
// ABI): the same fragment order for
// weight codes, row n of the weight being row n of a 16-row tile (the MFMA A
// side of the decode kernel), so a decode wave's weight load is one
// contiguous 1 KB per instruction. Needs N % 16 == 0 and K % 128 == 0; the
// buffer holds N * K bytes.
__host__ __device__ inline int64_t tiled_w_offset(int n, int k, int ksteps) { return packed_x_offset(n, k, ksteps); }

// Row-major codes <-> tiled layout (16-byte units; in place is not allowed).
hipError_t tile_weight(const uint8_t* codes, int64_t ldc, int N, int K, uint8_t* tiled, hipStream_t stream);
hipError_t untile_weight(const uint8_t* tiled, int N, int K, uint8_t* codes, int64_t ldc, hipStream_t stream);

int quant_chunks(int K);
// packed: write codes in the packed layout (codes sized packed_x_bytes(M, K),
// ldc ignored; the padding rows get zero codes).
hipError_t quant_rows_bf16(const uint16_t* x, int64_t ldx, int64_t M, int K, uint8_t* codes, int64_t ldc, float* scales,
                           const uint16_t* lora_a, int rank, float* lora_t, bool packed, hipStream_t stream);
hipError_t quant_swiglu_bf16(const uint16_t* gate, int64_t ldg, const uint16_t* up, int64_t ldu, int64_t M, int K,
                             uint8_t* codes, int64_t ldc, float* scales, uint16_t* h_out, int64_t ldh,
                             const uint16_t* lora_a, int rank, float* lora_t, bool packed, hipStream_t stream);
// Packed codes of h for M <= 2 kDecodeMaxRows rows from the SwiGLU epilogue's
// maxima (parts [M, K/16], 8-byte aligned); K % 128 == 0, K <= 16384.
hipError_t quant_h_from_maxima(const uint16_t* h, int64_t ldh, const uint16_t* parts, int64_t M, int K, uint8_t* codes,
                               float* scales, hipStream_t stream);
hipError_t quant_rows_f32(const float* x, int64_t ldx, int64_t M, int K, uint8_t* codes, int64_t ldc, float* scales,
                          hipStream_t stream);

// swiglu: the plan of a fused SwiGLU gate+up GEMM (a gate/up tile pair per
// wave, no split-K).
DecodePlan decode_plan(int64_t M, int64_t N, int64_t K, int cu_count, bool swiglu = false);
hipError_t gemm_decode(const uint8_t* xq, int64_t ldxq, bool packed_x, const uint8_t* w, int64_t ldw, int M, int N, int K,
                       const DecodePlan& plan, float* partial, int* counters, const Epilogue& ep, int rank,
                       hipStream_t stream);

// The batch-decode kernel on a batch_plan plan (no workspace, no counters);
// ldxq = 0 with packed_x: packed codes; ldw = 0: tiled weights; ep.half != 0:
// fused SwiGLU (packed codes, a batch_plan(..., swiglu = true) plan).
hipError_t gemm_batch(const uint8_t* xq, int64_t ldxq, bool packed_x, const uint8_t* w, int64_t ldw, int M, int N, int K,
                      const BatchPlan& p, const Epilogue& ep, int rank, hipStream_t stream);

// split_k = false: plans without K splits only.
PrefillTile prefill_tile(int64_t M, int64_t N, int64_t K, int cu_count, bool split_k = true);
// ldx = 0: packed activation codes (packed_x_offset); ldw = 0: tiled weights.
// ep.half != 0: fused SwiGLU epilogue (packed codes only, N = 2 half; with a
// K split on the lockstep tiles the last workgroup of a tile applies it).
// With tile.splits > 1: partials of prefill_partial_bytes and
// prefill_counters zeroed tile counters (left at zero).
hipError_t gemm_prefill(const uint8_t* xq, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                        const Epilogue& ep, int rank, PrefillTile tile, float* partials, int* counters,
                        hipStream_t stream);

// W8A16 parity mode (bf16 activations x e4m3 weights, the reference's own
// arithmetic): y = bf16(acc * sw[n]), then bf16(y + bias[n]) with a bias.
hipError_t w8a16_decode(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                        const DecodePlan& p, float* partial, int* counters, const float* sw, const uint16_t* bias,
                        uint16_t* y, int64_t ldy, hipStream_t stream);
hipError_t w8a16_batch(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                       const BatchPlan& p, const float* sw, const uint16_t* bias, uint16_t* y, int64_t ldy,
                       hipStream_t stream);
// W8A16 prefill GEMM; `splits` must be w8a16_prefill_splits(M, N, K,
// cu_count), with w8a16_prefill_partial_bytes of partials and
// w8a16_prefill_counters zeroed tile counters when above 1.
hipError_t w8a16_prefill(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                         const float* sw, const uint16_t* bias, uint16_t* y, int64_t ldy, int splits, float* partials,
                         int* counters, int cu_count, hipStream_t stream);

// The W8A16 prefill kernel's 64x64 tiles: 32-64 tokens (wide weights, as
// w8a16_decode_kernel_for sends them there), and wherever 128x128 tiles would
// not fill one round of CUs except on weights of 1.5 rounds of 64-channel
// tiles.
inline bool w8a16_small_tiles(int64_t M, int64_t N, int cu_count) {
  if (M <= kDecodeMaxRows) return true;
  const int64_t t128sq = ((M + 127) / 128) * ((N + 127) / 128);
  return t128sq < cu_count && 2 * ((N + 63) / 64) < 3 * (int64_t)cu_count;
}

// K splits of the 64x64 W8A16 prefill tiles where they fill at most a third
// of the CUs: 3 or 4 splits, each keeping at least eight 64-deep stages (us,
// graphs over rotated weights: k/v at 130 / 192 / 256 / 300 tokens 24.9 /
// 25.0 / 24.9 / 25.0 -> 17.9 / 18.0 / 18.3 / 22.3; two splits of 128 tiles
// measured slower, down at 96 tokens 67.7 -> 83.3, k/v at 512 25.2 -> 30.4).
inline int w8a16_prefill_splits(int64_t M, int64_t N, int64_t K, int cu_count) {
  if (!w8a16_small_tiles(M, N, cu_count) || K % 64) return 1;
  const int64_t tiles = ((M + 63) / 64) * ((N + 63) / 64);
  int64_t s = cu_count / tiles;
  if (s < 3) return 1;
  s = s > 4 ? 4 : s;
  while (s > 1 && K / 64 < 8 * s) --s;
  return (int)s;
}

// fp32 partial tiles and tile counters of a split W8A16 prefill launch.
inline int64_t w8a16_prefill_partial_bytes(int64_t M, int64_t N, int64_t K, int cu_count) {
  const int s = w8a16_prefill_splits(M, N, K, cu_count);
  return s > 1 ? ((M + 63) / 64) * ((N + 63) / 64) * s * 64 * 64 * 4 : 0;
}
inline int64_t w8a16_prefill_counters(int64_t M, int64_t N, int64_t K, int cu_count) {
  return w8a16_prefill_splits(M, N, K, cu_count) > 1 ? ((M + 63) / 64) * ((N + 63) / 64) : 0;
}

}  // namespace jv
