// Streaming-read probe: the time a launch of a given shape takes to read a
// buffer from memory and nothing else, the ceiling a weight-streaming decode
// GEMM of the same launch shape can approach. Measurement infrastructure for
// bench.py --read-probe; not part of the product library.
//
// Each wave reads LPW consecutive 1 KB pieces (16 bytes per lane per piece),
// all loads issued before any is used (as the decode GEMM issues a burst),
// and stores one XOR of what it read so the loads cannot be dropped. Wave w
// of workgroup b reads bytes [(b * waves + w) * LPW KB, + LPW KB).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

template <int LPW>
__global__ void read_probe_kernel(const uint8_t* __restrict__ src, uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const uint8_t* p = src + wave * (LPW * 1024) + lane * 16;
  i32x4 v[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) v[i] = *reinterpret_cast<const i32x4*>(p + i * 1024);
  int acc = 0;
#pragma unroll
  for (int i = 0; i < LPW; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  // Folded across the wave, so lane 0's store depends on every lane's loads.
  for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off);
  if (lane == 0) sink[wave] = (uint32_t)acc;
}

template <int LPW>
hipError_t launch(const uint8_t* src, int workgroups, int threads, uint32_t* sink, hipStream_t stream) {
  read_probe_kernel<LPW><<<dim3((unsigned)workgroups), dim3((unsigned)threads), 0, stream>>>(src, sink);
  return hipGetLastError();
}

}  // namespace

extern "C" {

// Reads exactly `bytes` = workgroups * (threads / 64) * loads_per_wave * 1024
// bytes of `src` (anything else is refused with -1 before a launch); `sink`
// holds workgroups * threads / 64 words. loads_per_wave in {4, 8, 16, 24, 32},
// threads a multiple of 64 up to 1024.
int th_read_probe(const void* src, int64_t bytes, int workgroups, int threads, int loads_per_wave, uint32_t* sink,
                  void* stream) {
  if (workgroups <= 0 || threads <= 0 || threads > 1024 || threads % 64) return -1;
  if ((int64_t)workgroups * (threads / 64) * loads_per_wave * 1024 != bytes) return -1;
  if (reinterpret_cast<uintptr_t>(src) & 15) return -1;
  const uint8_t* s = static_cast<const uint8_t*>(src);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (loads_per_wave) {
    case 4: e = launch<4>(s, workgroups, threads, sink, st); break;
    case 8: e = launch<8>(s, workgroups, threads, sink, st); break;
    case 16: e = launch<16>(s, workgroups, threads, sink, st); break;
    case 24: e = launch<24>(s, workgroups, threads, sink, st); break;
    case 32: e = launch<32>(s, workgroups, threads, sink, st); break;
    default: return -1;
  }
  return e == hipSuccess ? 0 : 1;
}

}  // extern "C"
