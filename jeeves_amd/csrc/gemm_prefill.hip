// Prefill FP8 x FP8 GEMM (M > 64 tokens), MFMA-bound.
//
// Counterpart of _fp8_matmul's tall-tile regime (inference/fp8.py:62-99,
// :118-119), redesigned for CDNA4 instead of translated:
//   * both operands are K-contiguous e4m3 (activation codes [M,K] from the
//     quantizer, weight codes [N,K]) and feed v_mfma_f32_32x32x64_f8f6f4
//     directly: no fp8 -> fp16 conversion in the main loop;
//   * a BM x BN output tile per 256-thread workgroup (2 x 2 waves, each wave a
//     (BM/2) x (BN/2) tile of 32x32 MFMA blocks, fp32 accumulators);
//   * K advances 128 bytes per stage; each stage's A and B rows are copied
//     global -> LDS with global_load_lds_dwordx4 (no VGPR staging), double
//     buffered so the next stage's copy overlaps this stage's MFMAs;
//   * LDS rows are 128 B with the 16-byte chunk index XOR-swizzled by (row & 7),
//     so the 8 lanes of each ds_read_b128 phase hit 8 distinct bank groups;
//   * fused epilogue acc * sx[m] * sw[n] (+ bias, + LoRA) -> bf16.
#include "epilogue.h"
#include "kernels.h"

namespace jv {

constexpr int kBK = 128;

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Copy 16 bytes per lane from global to LDS: lane i's bytes land at dst + 16 * i.
__device__ __forceinline__ void load_lds16(const uint8_t* src, uint8_t* dst_wave_base) {
  typedef __attribute__((address_space(3))) void lds_void;
  typedef __attribute__((address_space(1))) void global_void;
  __builtin_amdgcn_global_load_lds((global_void*)(src), (lds_void*)(dst_wave_base), 16, 0, 0);
}

__device__ __forceinline__ i32x4 lds_read16(const uint8_t* p) { return *reinterpret_cast<const i32x4*>(p); }

template <int BM, int BN, int RANK>
__global__ __launch_bounds__(256) void gemm_prefill_kernel(const uint8_t* __restrict__ xq, int64_t ldx,
                                                           const uint8_t* __restrict__ w, int64_t ldw, int M, int N, int K,
                                                           int tiles_m, int tiles_n, Epilogue ep) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int STAGE = (BM + BN) * kBK;
  constexpr int LOADS = (BM + BN) / 32;  // 1 KB wave-loads per wave per stage
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * STAGE];

  // Tile order: groups of 8 M-tiles walk N together, so concurrently resident
  // workgroups share A rows and B rows in L2.
  const int pid = blockIdx.x;
  constexpr int GROUP = 8;
  const int per_group = GROUP * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * GROUP;
  const int gsize = min(tiles_m - first_m, GROUP);
  const int tile_m = first_m + (pid % per_group) % gsize;
  const int tile_n = (pid % per_group) / gsize;
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Global -> LDS assignment. Wave-load g (g = i*4 + wave) fills LDS bytes
  // [g*1024, g*1024 + 1024) of a stage: rows 8g .. 8g+7 of the stacked
  // (A rows, then B rows) tile. Lane l writes row 8g + l/8, physical chunk
  // l%8, which holds logical chunk (l%8) ^ (row & 7) = (l%8) ^ (l/8).
  const int lrow = lane >> 3;
  const int lchunk = (lane & 7) ^ lrow;
  uint32_t src_off[LOADS];
  bool src_is_a[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int r = (i * 4 + wave) * 8 + lrow;
    if (r < BM) {
      src_is_a[i] = true;
      src_off[i] = (uint32_t)((int64_t)min(m0 + r, M - 1) * ldx) + lchunk * 16;
    } else {
      src_is_a[i] = false;
      src_off[i] = (uint32_t)((int64_t)min(n0 + r - BM, N - 1) * ldw) + lchunk * 16;
    }
  }

  auto issue_stage = [&](int kt, int buf) {
    uint8_t* base = lds + buf * STAGE;
    const int64_t k0 = (int64_t)kt * kBK;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const uint8_t* src = (src_is_a[i] ? xq : w) + src_off[i] + k0;
      load_lds16(src, base + (i * 4 + wave) * 1024);
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Fragment addressing: lane l reads row (l % 32) of a 32-row block, logical
  // chunks 4s + 2(l/32) and 4s + 2(l/32) + 1 for k-step s of the stage.
  const int frow = lane & 31;
  const int fhalf = (lane >> 5) * 2;

  const int KT = K / kBK;
  issue_stage(0, 0);
  for (int kt = 0; kt < KT; ++kt) {
    wait_vmem();
    __syncthreads();
    if (kt + 1 < KT) issue_stage(kt + 1, (kt + 1) & 1);
    const uint8_t* base = lds + (kt & 1) * STAGE;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      i32x8 a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WM + i * 32 + frow;
        const int c0 = (4 * s + fhalf) ^ (r & 7), c1 = (4 * s + fhalf + 1) ^ (r & 7);
        a[i] = cat8(lds_read16(base + r * kBK + c0 * 16), lds_read16(base + r * kBK + c1 * 16));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = BM + wn * WN + j * 32 + frow;
        const int c0 = (4 * s + fhalf) ^ (r & 7), c1 = (4 * s + fhalf + 1) ^ (r & 7);
        b[j] = cat8(lds_read16(base + r * kBK + c0 * 16), lds_read16(base + r * kBK + c1 * 16));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma_32x32x64_fp8(a[i], b[j], acc[i][j]);
    }
  }

  // Epilogue. 32x32 MFMA output layout: lane l holds column l % 32 and, in
  // register r, row 8*(r/4) + 4*(l/32) + r%4. Rows are tokens, columns channels.
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wn * WN + j * 32 + (lane & 31);
    if (n >= N) continue;
    const float swn = ep.sw[n];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < M) ep.y[(int64_t)m * ep.ldy + n] = (uint16_t)f32_to_bf16(epilogue_value<RANK>(ep, acc[i][j][r], m, n, ep.sx[m], swn));
      }
    }
  }
}

template <int BM, int BN>
static hipError_t launch_prefill(const uint8_t* xq, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                                 const Epilogue& ep, int rank, hipStream_t stream) {
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  const dim3 grid((unsigned)(tm * tn)), block(256);
  if (rank == 16)
    gemm_prefill_kernel<BM, BN, 16><<<grid, block, 0, stream>>>(xq, ldx, w, ldw, M, N, K, tm, tn, ep);
  else
    gemm_prefill_kernel<BM, BN, 0><<<grid, block, 0, stream>>>(xq, ldx, w, ldw, M, N, K, tm, tn, ep);
  return hipGetLastError();
}

PrefillTile prefill_tile(int64_t M, int64_t N, int cu_count) {
  // Largest tile that still gives every CU a workgroup; fall back to smaller ones.
  const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
  if (t256 >= cu_count) return PrefillTile{256, 256};
  const int64_t t256x128 = ((M + 255) / 256) * ((N + 127) / 128);
  if (t256x128 >= cu_count) return PrefillTile{256, 128};
  return PrefillTile{128, 128};
}

hipError_t gemm_prefill(const uint8_t* xq, int64_t ldx, const uint8_t* w, int64_t ldw, int M, int N, int K,
                        const Epilogue& ep, int rank, PrefillTile tile, hipStream_t stream) {
  if (rank != 0 && rank != 16) return hipErrorInvalidValue;
  if (tile.bm == 256 && tile.bn == 256) return launch_prefill<256, 256>(xq, ldx, w, ldw, M, N, K, ep, rank, stream);
  if (tile.bm == 256 && tile.bn == 128) return launch_prefill<256, 128>(xq, ldx, w, ldw, M, N, K, ep, rank, stream);
  if (tile.bm == 128 && tile.bn == 128) return launch_prefill<128, 128>(xq, ldx, w, ldw, M, N, K, ep, rank, stream);
  return hipErrorInvalidValue;
}

}  // namespace jv
