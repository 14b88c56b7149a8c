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

// bf16 helpers: fp32 -> bf16 rounds to nearest even; NaN becomes the
// canonical quiet NaN 0x7FC0 (torch's c10::BFloat16 conversion).
__device__ __forceinline__ float bf2f(uint16_t bits) { return __uint_as_float(static_cast<uint32_t>(bits) << 16); }
__device__ __forceinline__ uint16_t f2bf(float x) {
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float round_bf16(float x) { return bf2f(f2bf(x)); }
// Two fp32 values -> a bf16 pair (low half = a), each rounded to nearest even
// (v_cvt_pk_bf16_f32; for the kernels' internal operands, not stored results).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}
// 16-bit floats of a kernel instance's dtype: bfloat16 when BF, else fp16.
template <bool BF>
__device__ __forceinline__ float w2f(uint16_t bits) {
  if constexpr (BF) return bf2f(bits);
  else return h2f(bits);
}
template <bool BF>
__device__ __forceinline__ uint16_t f2w(float x) {
  if constexpr (BF) return f2bf(x);
  else return f2h(x);
}

// Float elements of a cache dtype: fp16 as raw uint16_t bits, bf16 as the
// Bf16 tag, fp32 as float.
struct Bf16 {
  uint16_t bits;
};
__device__ __forceinline__ float to_f32(uint16_t h) { return h2f(h); }
__device__ __forceinline__ float to_f32(Bf16 b) { return bf2f(b.bits); }
__device__ __forceinline__ float to_f32(float x) { return x; }
template <typename T>
__device__ __forceinline__ T from_f32(float x);  // round to nearest even
template <>
__device__ __forceinline__ uint16_t from_f32<uint16_t>(float x) { return f2h(x); }
template <>
__device__ __forceinline__ Bf16 from_f32<Bf16>(float x) { return Bf16{f2bf(x)}; }
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
// one rounding of an fp32 value to T and back
template <typename T>
__device__ __forceinline__ float round_to(float x) { return to_f32(from_f32<T>(x)); }

// Reduction across `width` consecutive lanes (width a power of two <= 64).
template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// max(m, |v|) for m >= 0 that keeps NaN, as torch's amax does: on the bit
// patterns of non-negative floats every NaN orders above +inf.
__device__ __forceinline__ float absmax_nan(float m, float v) {
  return __uint_as_float(max(__float_as_uint(m), __float_as_uint(fabsf(v))));
}
// group_max over non-negative values, NaN-propagating like absmax_nan.
template <int WIDTH>
__device__ __forceinline__ float group_max_abs(float v) {
  uint32_t u = __float_as_uint(v);
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) u = max(u, static_cast<uint32_t>(__shfl_xor(static_cast<int>(u), o, 64)));
  return __uint_as_float(u);
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
