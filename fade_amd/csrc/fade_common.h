// Shared helpers for the libfade_hip.so kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fade_hip.h"

#define FADE_API extern "C" __attribute__((visibility("default")))

namespace fade {

// Thread-local error text behind fade_hip_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int einval(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
// Checks hipGetLastError() after a launch; returns FADE_OK or FADE_ERUNTIME.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// fp16 helpers on the device.  _Float16 conversions are IEEE round-to-nearest-even.
__device__ __forceinline__ float h2f(uint16_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}
__device__ __forceinline__ uint16_t f2h(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}
// Round an fp32 value through fp16 and back (one fp16 rounding).
__device__ __forceinline__ float round_f16(float x) {
  return static_cast<float>(static_cast<_Float16>(x));
}

// Reduction across `width` consecutive lanes (width a power of two <= 64).
template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
template <int WIDTH>
__device__ __forceinline__ float group_min(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
  return v;
}
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Byte offset of row r of a [B,H,S,*] tensor with element strides.
__device__ __forceinline__ int64_t row_offset(int64_t r, int64_t H, int64_t S, int64_t sb,
                                              int64_t sh, int64_t ss) {
  const int64_t s = r % S;
  const int64_t bh = r / S;
  return (bh / H) * sb + (bh % H) * sh + s * ss;
}

}  // namespace fade
