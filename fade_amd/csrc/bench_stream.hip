// Read-only HBM streaming kernel for bench.py's measured ceiling (not part of
// the product ABI; built as libfade_bench.so next to libfade_hip.so).
//
// Workgroup w reads the w-th contiguous chunk of the buffer with 16-byte
// non-temporal loads, kUnroll of them in flight per thread, and folds them
// into one word that is stored only if it equals a value the data never
// produces (so the loads cannot be optimized away and nothing is written).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kUnroll = 8;

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                               int64_t chunk16, uint32_t* __restrict__ sink) {
  const int64_t lo = static_cast<int64_t>(blockIdx.x) * chunk16;
  const int64_t hi = lo + chunk16 < n16 ? lo + chunk16 : n16;
  u32x4 acc = {0, 0, 0, 0};
  for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads * kUnroll) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = i + static_cast<int64_t>(kThreads) * u;
      v[u] = j < hi ? __builtin_nontemporal_load(&src[j]) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u];
  }
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9E3779B9u) sink[blockIdx.x] = x;
}

}  // namespace

// Reads `bytes` (a multiple of 16, 16-byte aligned) from `src` with `wgs`
// workgroups; `sink` needs `wgs` words.  Returns 0 or -1 (launch error).
extern "C" __attribute__((visibility("default"))) int fade_bench_stream_read(const void* src, int64_t bytes,
                                                                              int32_t wgs, void* sink,
                                                                              void* stream) {
  if (src == nullptr || sink == nullptr || bytes <= 0 || (bytes & 15) || wgs <= 0) return -22;
  const int64_t n16 = bytes / 16;
  const int64_t chunk16 = (n16 + wgs - 1) / wgs;
  hipLaunchKernelGGL(stream_read_kernel, dim3(static_cast<unsigned>(wgs)), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const u32x4*>(src), n16, chunk16,
                     static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
