// Quantize + bit-pack kernels for the FADE middle tier (gfx950).
//
// Every lane owns 8 consecutive elements of a row (one 16-byte fp16 load),
// so a D=128 row is 16 lanes and a wavefront covers 4 rows per iteration;
// per-row reductions are lane shuffles inside the 16-lane group and the
// packed codes leave as one 4-byte (INT4) or 2-byte (INT2) store per lane.
//
// Arithmetic follows the reference's torch semantics bit for bit
// (fade/quant.py:61-150, fade/rotated_quant.py:106-173):
//   fp16 inputs: each op is evaluated in fp32 and rounded to fp16, and
//     qmax / absmax is reciprocal-then-multiply (two roundings);
//   fp32 (rotated) inputs: each op one fp32 rounding.
// This file is compiled with -ffp-contract=off and IEEE fp32 division.
#include <type_traits>

#include "fade_common.h"

namespace fade {
namespace {

constexpr int kBlock = 256;
// Element arithmetic of the input tensor, as torch rounds it per op: fp16,
// bf16, or fp32 (the rotated path's x_rot, plain fp32 K/V) with the fp32
// scale stored as fp16 (MODE_F32), as fp32 (MODE_F32S) or as bf16
// (MODE_F32B): one rounding of absmax / qmax to the stored type.
enum { MODE_F16 = 0, MODE_F32 = 1, MODE_BF16 = 2, MODE_F32S = 3, MODE_F32B = 4 };
// Storage of the emitted scale: 16-bit (fp16 or bf16 bits) or fp32.
template <int MODE>
struct ScaleOf {
  using T = uint16_t;
};
template <>
struct ScaleOf<MODE_F32S> {
  using T = float;
};

template <int BITS>
struct QRange;
// Bytes one lane (8 codes) occupies in a packed row; 3-bit codes stay raw int8.
template <int BITS>
constexpr int lane_bytes() { return BITS == 3 ? 8 : BITS; }
template <>
struct QRange<4> {
  static constexpr int lo = -8, hi = 7;
};
template <>
struct QRange<3> {
  static constexpr int lo = -4, hi = 3;
};
template <>
struct QRange<2> {
  static constexpr int lo = -2, hi = 1;
};

__device__ __forceinline__ void load8(const uint16_t* p, float* v) {
  const uint4 w = *reinterpret_cast<const uint4*>(p);
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = h2f(static_cast<uint16_t>(u[i] & 0xFFFFu));
    v[2 * i + 1] = h2f(static_cast<uint16_t>(u[i] >> 16));
  }
}
__device__ __forceinline__ void load8(const Bf16* p, float* v) {
  const uint4 w = *reinterpret_cast<const uint4*>(p);
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(u[i] << 16);
    v[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
  }
}
__device__ __forceinline__ void load8(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// inv = qmax / absmax, scale = absmax / qmax in the reference's rounding.
template <int MODE, int QMAX>
__device__ __forceinline__ void sym_params(float absmax, float& inv, typename ScaleOf<MODE>::T& scale_h) {
  if constexpr (MODE == MODE_F16) {
    // clamp(min=1e-8) is a no-op on fp16 (1e-8 rounds to zero).
    const float r = round_f16(1.0f / absmax);
    inv = round_f16(r * static_cast<float>(QMAX));
    scale_h = f2h(absmax / static_cast<float>(QMAX));
  } else if constexpr (MODE == MODE_BF16) {
    // bf16 holds 1e-8: the clamp bites, then every op rounds to bf16
    const float a = round_bf16(absmax != absmax ? absmax : fmaxf(absmax, 1e-8f));
    const float r = round_bf16(1.0f / a);
    inv = round_bf16(r * static_cast<float>(QMAX));
    scale_h = f2bf(a / static_cast<float>(QMAX));
  } else {
    const float a = absmax != absmax ? absmax : fmaxf(absmax, 1e-8f);  // clamp keeps NaN
    const float r = 1.0f / a;
    inv = r * static_cast<float>(QMAX);
    if constexpr (MODE == MODE_F32S)
      scale_h = a / static_cast<float>(QMAX);
    else if constexpr (MODE == MODE_F32B)
      scale_h = f2bf(a / static_cast<float>(QMAX));
    else
      scale_h = f2h(a / static_cast<float>(QMAX));
  }
}

// round-half-even(x * inv), NaN -> 0 (torch CPU int8 cast), clamped.
template <int MODE, int QLO, int QHI>
__device__ __forceinline__ int sym_code(float x, float inv) {
  float p = x * inv;
  if (MODE == MODE_F16) p = round_f16(p);
  if (MODE == MODE_BF16) p = round_bf16(p);
  float q = rintf(p);
  if (q != q) return 0;
  q = fminf(fmaxf(q, static_cast<float>(QLO)), static_cast<float>(QHI));
  return static_cast<int>(q);
}

// Store 8 codes of one lane in the packed layout for BITS.
template <int BITS>
__device__ __forceinline__ void store_codes(uint8_t* dst, const int* c) {
  if (BITS == 4) {
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w |= static_cast<uint32_t>(((c[2 * j] & 0xF) << 4) | (c[2 * j + 1] & 0xF)) << (8 * j);
    *reinterpret_cast<uint32_t*>(dst) = w;
  } else if (BITS == 2) {
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      w |= static_cast<uint32_t>(((c[4 * j] & 3) << 6) | ((c[4 * j + 1] & 3) << 4) |
                                 ((c[4 * j + 2] & 3) << 2) | (c[4 * j + 3] & 3))
           << (8 * j);
    *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(w);
  } else {  // raw int8 (3-bit rotated codes are not packed by the reference)
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lo |= static_cast<uint32_t>(c[j] & 0xFF) << (8 * j);
      hi |= static_cast<uint32_t>(c[4 + j] & 0xFF) << (8 * j);
    }
    *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
  }
}

// ---- packed fp16 INT4 codes (the fp16 reference INT4 quantizers' fast path) ----
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// The largest magnitude of eight fp16 values (four packed pairs, element 2k in
// the low half of pair k) as fp16 bits: non-negative fp16 bit patterns order
// as their values, so an unsigned 16-bit max finds it.  >= 0x7C00: an inf or
// NaN among them.
__device__ __forceinline__ uint32_t maxmag8(const uint4& w) {
  auto mag = [](uint32_t a) { return __builtin_bit_cast(u16x2, a & 0x7FFF7FFFu); };
  const u16x2 t = __builtin_elementwise_max(__builtin_elementwise_max(mag(w.x), mag(w.y)),
                                            __builtin_elementwise_max(mag(w.z), mag(w.w)));
  return t[0] > t[1] ? t[0] : t[1];
}
// Eight fp16 values hold neither inf nor NaN.
__device__ __forceinline__ bool finite8(const uint4& w) { return maxmag8(w) < 0x7C00u; }

__device__ __forceinline__ void f16x8_to_f32(const uint4& w, float* v) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = h2f(static_cast<uint16_t>(u[i] & 0xFFFFu));
    v[2 * i + 1] = h2f(static_cast<uint16_t>(u[i] >> 16));
  }
}

// The INT4 codes of eight fp16 values x times fp16 inverse scales inv (pairs
// laid out alike), packed as store_codes<4> packs them, two elements per
// instruction: p = x * inv rounded once to fp16 (the reference's fp16
// multiply); p + 1536 rounds p half-to-even to an integer held in the sum's
// low mantissa bits (the fp16 ulp at 1536 is 1, and 1536 is even); the clamp
// to [1528, 1543] is the clamp of the code to [-8, 7]; the sum's low 4 bits
// are the code's two's-complement nibble.  Equal to sym_code<MODE_F16, -8, 7>
// for finite x and finite inv > 0 (p is then never NaN; an inf p clamps);
// callers take the scalar path otherwise.
__device__ __forceinline__ uint32_t codes4_f16(const uint4& x, const uint4& inv) {
#pragma clang fp contract(off)
  const h2_t bias = {static_cast<_Float16>(1536.0f), static_cast<_Float16>(1536.0f)};
  const h2_t lo = {static_cast<_Float16>(1528.0f), static_cast<_Float16>(1528.0f)};
  const h2_t hi = {static_cast<_Float16>(1543.0f), static_cast<_Float16>(1543.0f)};
  auto pair = [&](uint32_t a, uint32_t b) {
    const h2_t p = __builtin_bit_cast(h2_t, a) * __builtin_bit_cast(h2_t, b);
    const h2_t c = __builtin_elementwise_min(__builtin_elementwise_max(p + bias, lo), hi);
    return __builtin_bit_cast(uint32_t, c);
  };
  const uint32_t d0 = pair(x.x, inv.x), d1 = pair(x.y, inv.y), d2 = pair(x.z, inv.z), d3 = pair(x.w, inv.w);
  // low byte of every half (the nibble in its low 4 bits), element order
  const uint32_t t = __builtin_amdgcn_perm(d1, d0, 0x06040200u) & 0x0F0F0F0Fu;
  const uint32_t u = __builtin_amdgcn_perm(d3, d2, 0x06040200u) & 0x0F0F0F0Fu;
  // bytes 0 and 2: (nibble 2j << 4) | nibble 2j + 1
  const uint32_t ty = (t << 4) | (t >> 8), uy = (u << 4) | (u >> 8);
  return __builtin_amdgcn_perm(uy, ty, 0x06040200u);
}

// The INT2 codes (clamped to [-2, 1]) of eight fp16 values, as eight int8
// bytes: the same rounding as codes4_f16, clamped to [1534, 1537], whose low
// byte is the code's two's complement.  Same validity as codes4_f16.
__device__ __forceinline__ uint2 codes2_i8_f16(const uint4& x, const uint4& inv) {
#pragma clang fp contract(off)
  const h2_t bias = {static_cast<_Float16>(1536.0f), static_cast<_Float16>(1536.0f)};
  const h2_t lo = {static_cast<_Float16>(1534.0f), static_cast<_Float16>(1534.0f)};
  const h2_t hi = {static_cast<_Float16>(1537.0f), static_cast<_Float16>(1537.0f)};
  auto pair = [&](uint32_t a, uint32_t b) {
    const h2_t p = __builtin_bit_cast(h2_t, a) * __builtin_bit_cast(h2_t, b);
    const h2_t c = __builtin_elementwise_min(__builtin_elementwise_max(p + bias, lo), hi);
    return __builtin_bit_cast(uint32_t, c);
  };
  const uint32_t d0 = pair(x.x, inv.x), d1 = pair(x.y, inv.y), d2 = pair(x.z, inv.z), d3 = pair(x.w, inv.w);
  return make_uint2(__builtin_amdgcn_perm(d1, d0, 0x06040200u), __builtin_amdgcn_perm(d3, d2, 0x06040200u));
}

// Unpack 8 signed codes of one lane.
template <int BITS>
__device__ __forceinline__ void load_codes(const uint8_t* src, int* c) {
  if (BITS == 4) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(src);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int b = (w >> (8 * j)) & 0xFF;
      const int hi = b >> 4, lo = b & 0xF;
      c[2 * j] = hi - ((hi & 8) << 1);
      c[2 * j + 1] = lo - ((lo & 8) << 1);
    }
  } else if (BITS == 2) {
    const uint32_t w = *reinterpret_cast<const uint16_t*>(src);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int b = (w >> (8 * j)) & 0xFF;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int v = (b >> (6 - 2 * k)) & 3;
        c[4 * j + k] = v - ((v & 2) << 1);
      }
    }
  } else {
    const uint2 w = *reinterpret_cast<const uint2*>(src);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c[j] = static_cast<int8_t>((w.x >> (8 * j)) & 0xFF);
      c[4 + j] = static_cast<int8_t>((w.y >> (8 * j)) & 0xFF);
    }
  }
}

// ---------------------------------------------------------------- per token
template <typename InT, int MODE, int BITS, int LPR>
__global__ __launch_bounds__(kBlock) void quant_token_kernel(const InT* __restrict__ x, int D, int64_t rows,
                                                             int64_t H, int64_t S, int64_t sb,
                                                             int64_t sh, int64_t ss, int64_t fs,
                                                             uint8_t* __restrict__ packed,
                                                             typename ScaleOf<MODE>::T* __restrict__ scale) {
  constexpr int RP = kBlock / LPR;
  const int row_bytes = (D / 8) * lane_bytes<BITS>();
  const int c = threadIdx.x % LPR;
  const bool on = c * 8 < D;  // lanes past the row's D / 8 groups of 8 channels idle
  constexpr bool kPk = MODE == MODE_F16 && BITS == 4 && std::is_same<InT, uint16_t>::value;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * RP + threadIdx.x / LPR; r < rows;
       r += static_cast<int64_t>(gridDim.x) * RP) {
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint4 raw = make_uint4(0u, 0u, 0u, 0u);
    const InT* src = x + (fs ? r * fs : row_offset(r, H, S, sb, sh, ss)) + c * 8;
    float a = 0.0f;
    bool fin = false;  // fp16 fast path: this lane's 8 values are finite
    if constexpr (kPk) {
      if (on) raw = *reinterpret_cast<const uint4*>(src);
      const uint32_t mm = maxmag8(raw);
      fin = mm < 0x7C00u;
      if (fin) {
        a = h2f(static_cast<uint16_t>(mm));  // the lane's absmax, exact
      } else {
        f16x8_to_f32(raw, v);
#pragma unroll
        for (int j = 0; j < 8; ++j) a = absmax_nan(a, v[j]);
      }
    } else {
      if (on) load8(src, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) a = absmax_nan(a, v[j]);
    }
    a = group_max_abs<LPR>(a);
    float inv;
    typename ScaleOf<MODE>::T sc;
    sym_params<MODE, QRange<BITS>::hi>(a, inv, sc);
    if constexpr (kPk) {
      if (on && inv > 0.0f && inv < INFINITY && fin) {
        const uint32_t ih = static_cast<uint32_t>(f2h(inv)) * 0x10001u;  // inv is an fp16 value
        *reinterpret_cast<uint32_t*>(packed + r * row_bytes + c * 4) = codes4_f16(raw, make_uint4(ih, ih, ih, ih));
        if (c == 0) scale[r] = sc;
        continue;
      }
      if (fin) f16x8_to_f32(raw, v);  // the scalar path below reads v
    }
    int code[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) code[j] = sym_code<MODE, QRange<BITS>::lo, QRange<BITS>::hi>(v[j], inv);
    if (on) store_codes<BITS>(packed + r * row_bytes + c * lane_bytes<BITS>(), code);
    if (c == 0) scale[r] = sc;
  }
}

// -------------------------------------------------------------- per channel
// Pass 1: column absmax of each S-block -> partial[bh][block][d] (fp32).
template <typename InT, int LPR>
__global__ __launch_bounds__(kBlock) void colmax_kernel(const InT* __restrict__ x, int D, int64_t H,
                                                        int64_t S, int64_t sb, int64_t sh,
                                                        int64_t ss, int64_t rows_per_block,
                                                        float* __restrict__ partial) {
  constexpr int RP = kBlock / LPR;
  constexpr int DP = LPR * 8;  // the instance's channel capacity (>= D)
  const int64_t bh = blockIdx.y;
  const int c = threadIdx.x % LPR, rs = threadIdx.x / LPR;
  const int64_t s0 = static_cast<int64_t>(blockIdx.x) * rows_per_block;
  const int64_t s1 = s0 + rows_per_block < S ? s0 + rows_per_block : S;
  const InT* base = x + (bh / H) * sb + (bh % H) * sh + c * 8;
  float m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t s = s0 + rs; c * 8 < D && s < s1; s += RP) {
    float v[8];
    load8(base + s * ss, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) m[j] = absmax_nan(m[j], v[j]);
  }
  __shared__ float red[RP * DP];
#pragma unroll
  for (int j = 0; j < 8; ++j) red[rs * DP + c * 8 + j] = m[j];
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += kBlock) {
    float mm = 0.0f;
    for (int r = 0; r < RP; ++r) mm = absmax_nan(mm, red[r * DP + d]);
    partial[(bh * gridDim.x + blockIdx.x) * D + d] = mm;
  }
}

// Pass 2: finish the column absmax from nparts partial maxima per (b, h)
// (partial[bh][k][d]; pass 1's S-blocks, or partials another kernel
// gathered), emit the scale, quantize this S-block.
template <typename InT, int MODE, int BITS, int LPR>
__global__ __launch_bounds__(kBlock) void quant_channel_kernel(
    const InT* __restrict__ x, int D, int64_t H, int64_t S, int64_t sb, int64_t sh, int64_t ss,
    int64_t rows_per_block, const float* __restrict__ partial, int nparts, uint8_t* __restrict__ packed,
    typename ScaleOf<MODE>::T* __restrict__ scale) {
  constexpr int RP = kBlock / LPR;
  constexpr int DP = LPR * 8;  // the instance's channel capacity (>= D)
  const int row_bytes = (D / 8) * lane_bytes<BITS>();
  const int64_t bh = blockIdx.y;
  __shared__ float inv_s[DP];
  for (int d = threadIdx.x; d < D; d += kBlock) {
    float a = 0.0f;
    for (int k = 0; k < nparts; ++k) a = absmax_nan(a, partial[(bh * nparts + k) * D + d]);
    float inv;
    typename ScaleOf<MODE>::T sc;
    sym_params<MODE, QRange<BITS>::hi>(a, inv, sc);
    inv_s[d] = inv;
    if (blockIdx.x == 0) scale[bh * D + d] = sc;
  }
  __syncthreads();
  const int c = threadIdx.x % LPR, rs = threadIdx.x / LPR;
  if (c * 8 >= D) return;  // past the row's channels (no barrier follows)
  float iv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) iv[j] = inv_s[c * 8 + j];
  const int64_t s0 = static_cast<int64_t>(blockIdx.x) * rows_per_block;
  const int64_t s1 = s0 + rows_per_block < S ? s0 + rows_per_block : S;
  const InT* base = x + (bh / H) * sb + (bh % H) * sh + c * 8;
  constexpr bool kPk = MODE == MODE_F16 && BITS == 4 && std::is_same<InT, uint16_t>::value;
  if constexpr (kPk) {
    // fp16 inverse scales as packed pairs; any non-finite or zero one sends
    // this lane's rows through the scalar path
    bool inv_ok = true;
    uint32_t ivp[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      inv_ok = inv_ok && iv[2 * j] > 0.0f && iv[2 * j] < INFINITY && iv[2 * j + 1] > 0.0f && iv[2 * j + 1] < INFINITY;
      ivp[j] = static_cast<uint32_t>(f2h(iv[2 * j])) | (static_cast<uint32_t>(f2h(iv[2 * j + 1])) << 16);
    }
    const uint4 invv = make_uint4(ivp[0], ivp[1], ivp[2], ivp[3]);
    for (int64_t s = s0 + rs; s < s1; s += RP) {
      const uint4 raw = *reinterpret_cast<const uint4*>(base + s * ss);
      uint8_t* dst = packed + (bh * S + s) * row_bytes + c * 4;
      if (inv_ok && finite8(raw)) {
        *reinterpret_cast<uint32_t*>(dst) = codes4_f16(raw, invv);
      } else {
        float v[8];
        f16x8_to_f32(raw, v);
        int code[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) code[j] = sym_code<MODE, QRange<BITS>::lo, QRange<BITS>::hi>(v[j], iv[j]);
        store_codes<BITS>(dst, code);
      }
    }
    return;
  }
  for (int64_t s = s0 + rs; s < s1; s += RP) {
    float v[8];
    load8(base + s * ss, v);
    int code[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) code[j] = sym_code<MODE, QRange<BITS>::lo, QRange<BITS>::hi>(v[j], iv[j]);
    store_codes<BITS>(packed + (bh * S + s) * row_bytes + c * lane_bytes<BITS>(), code);
  }
}

// ---------------------------------------------------------- dequant (sym)
// out = code * scale rounded to the output type; scale and out share it:
// fp16 (uint16_t), bf16 (Bf16) or fp32.
__device__ __forceinline__ float scale_ld(uint16_t u) { return h2f(u); }
__device__ __forceinline__ float scale_ld(Bf16 u) { return bf2f(u.bits); }
__device__ __forceinline__ float scale_ld(float u) { return u; }
__device__ __forceinline__ void store8(uint16_t* p, const float* y) {
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = static_cast<uint32_t>(f2h(y[2 * j])) | (static_cast<uint32_t>(f2h(y[2 * j + 1])) << 16);
  *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}
__device__ __forceinline__ void store8(Bf16* p, const float* y) {
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = static_cast<uint32_t>(f2bf(y[2 * j])) | (static_cast<uint32_t>(f2bf(y[2 * j + 1])) << 16);
  *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}
__device__ __forceinline__ void store8(float* p, const float* y) {
  reinterpret_cast<float4*>(p)[0] = make_float4(y[0], y[1], y[2], y[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(y[4], y[5], y[6], y[7]);
}

template <int BITS, int LPR, typename T>
__global__ __launch_bounds__(kBlock) void dequant_sym_kernel(const uint8_t* __restrict__ packed,
                                                             const T* __restrict__ scale, int D, int axis,
                                                             int64_t rows, int64_t S, T* __restrict__ out) {
  constexpr int RP = kBlock / LPR;
  const int row_bytes = (D / 8) * lane_bytes<BITS>();
  const int c = threadIdx.x % LPR;
  if (c * 8 >= D) return;  // past the row's channels
  if constexpr (BITS == 4 && std::is_same<T, uint16_t>::value) {
    // fp16 out: packed fp16 arithmetic, two elements per instruction.  Byte k
    // of the lane's 4 code bytes holds elements 2k (high nibble) and 2k + 1
    // (low nibble); v_perm puts the byte in both halves, a (0, 4) packed
    // shift brings each nibble to bits 4..7 of its half, and (x & 0x00F0) ^
    // 0x5480 is the fp16 72 + code (the nibble as offset binary in the
    // mantissa of 64.0).  72 + code - 72 is exact, and the product with the
    // fp16 scale is rounded once: fp16(float(code) * float(scale)), the
    // reference's dequantization, for every scale (inf and NaN included).
    const h2_t k72 = {static_cast<_Float16>(72.0f), static_cast<_Float16>(72.0f)};
    const u16x2 sh = {0, 4};
    // per-channel scales are read 8 at a time (16 bytes): an unaligned scale
    // tensor takes the scalar loop below
    const bool vec_ok = axis == FADE_AXIS_TOKEN || (reinterpret_cast<uintptr_t>(scale) & 15) == 0;
    for (int64_t r = static_cast<int64_t>(blockIdx.x) * RP + threadIdx.x / LPR; vec_ok && r < rows;
         r += static_cast<int64_t>(gridDim.x) * RP) {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(packed + r * row_bytes + c * 4);
      uint32_t sp[4];
      if (axis == FADE_AXIS_TOKEN) {
        const uint32_t s1 = scale[r];
        sp[0] = sp[1] = sp[2] = sp[3] = s1 | (s1 << 16);
      } else {
        // the (b, h) of row r: a 32-bit division wherever the values fit
        const int64_t bh = ((r | S) >> 31) == 0 ? static_cast<int64_t>(static_cast<uint32_t>(r) / static_cast<uint32_t>(S))
                                                : r / S;
        const uint4 sv = *reinterpret_cast<const uint4*>(scale + bh * D + c * 8);
        sp[0] = sv.x, sp[1] = sv.y, sp[2] = sv.z, sp[3] = sv.w;
      }
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t t = __builtin_amdgcn_perm(w, w, 0x0C000C00u | (k << 16) | k);  // byte k in both halves
        const uint32_t x = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, t) << sh);
        const h2_t v = __builtin_bit_cast(h2_t, (x & 0x00F000F0u) ^ 0x54805480u) - k72;
        o[k] = __builtin_bit_cast(uint32_t, v * __builtin_bit_cast(h2_t, sp[k]));
      }
      *reinterpret_cast<uint4*>(out + r * D + c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
    }
    if (vec_ok) return;
  }
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * RP + threadIdx.x / LPR; r < rows;
       r += static_cast<int64_t>(gridDim.x) * RP) {
    int code[8];
    load_codes<BITS>(packed + r * row_bytes + c * lane_bytes<BITS>(), code);
    float y[8];
    if (axis == FADE_AXIS_TOKEN) {
      const float sc = scale_ld(scale[r]);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = static_cast<float>(code[j]) * sc;
    } else {
      const T* sp = scale + (r / S) * D + c * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = static_cast<float>(code[j]) * scale_ld(sp[j]);
    }
    store8(out + r * D + c * 8, y);
  }
}

// ------------------------------------------------ grouped INT2 (reference)
// One block per (group, b*h); one thread per channel.  Rows >= S are zero.
// T: uint16_t (fp16 bits), Bf16 or float; the scale is stored in the same format
// (MODE = Int2Mode<T>::value).  MODE is a plain int template argument: an
// expression over the unnamed mode enum in the signature would be mangled
// differently by the host and device passes.
template <typename T>
struct Int2Mode {
  static constexpr int value = std::is_same<T, Bf16>::value ? MODE_BF16
                               : std::is_same<T, float>::value ? MODE_F32S : MODE_F16;
};
template <typename T, int MODE>
__global__ void quant_int2_grouped_kernel(const T* __restrict__ x, int64_t H, int64_t S,
                                          int64_t S_pad, int64_t sb, int64_t sh, int64_t ss,
                                          int group, int8_t* __restrict__ codes,
                                          typename ScaleOf<MODE>::T* __restrict__ scale) {
  const int d = threadIdx.x;
  const int D = blockDim.x;
  const int64_t g = blockIdx.x, bh = blockIdx.y;
  const int64_t G = gridDim.x;
  const T* base = x + (bh / H) * sb + (bh % H) * sh + d;
  float a = 0.0f;
  for (int i = 0; i < group; ++i) {
    const int64_t s = g * group + i;
    const float v = s < S ? to_f32(base[s * ss]) : 0.0f;
    a = absmax_nan(a, v);
  }
  float inv;
  typename ScaleOf<MODE>::T sc;
  sym_params<MODE, 1>(a, inv, sc);
  scale[(bh * G + g) * D + d] = sc;
  for (int i = 0; i < group; ++i) {
    const int64_t s = g * group + i;
    const float v = s < S ? to_f32(base[s * ss]) : 0.0f;
    codes[(bh * S_pad + s) * D + d] = static_cast<int8_t>(sym_code<MODE, -2, 1>(v, inv));
  }
}

// One (S-group, (b, h)) per block in a single pass: each lane loads 8
// channels (16 bytes) of up to NR of the group's rows once, the group's column
// absmax is reduced through LDS, and the codes come from the registers.
// Rows past S (the padding up to S_pad) count as zeros, as in the kernel above.
template <typename T, int MODE, int LPR, int NR>
__global__ __launch_bounds__(kBlock) void quant_int2_grouped_rows_kernel(
    const T* __restrict__ x, int D, int64_t H, int64_t S, int64_t S_pad, int64_t sb, int64_t sh, int64_t ss,
    int group, int8_t* __restrict__ codes, typename ScaleOf<MODE>::T* __restrict__ scale) {
  constexpr int RP = kBlock / LPR;
  constexpr int DP = LPR * 8;  // the instance's channel capacity (>= D)
  const int c = threadIdx.x % LPR, rs = threadIdx.x / LPR;
  const bool on = c * 8 < D;
  const int64_t g = blockIdx.x, bh = blockIdx.y, G = gridDim.x;
  const T* base = x + (bh / H) * sb + (bh % H) * sh + (on ? c * 8 : 0);
  // fp16: the rows stay as their fp16 bits (4 registers a row) and the codes
  // come from packed fp16 arithmetic where the values and scales are finite
  constexpr bool kPk = MODE == MODE_F16 && std::is_same<T, uint16_t>::value;
  float v[kPk ? 1 : NR][8];
  uint4 raw[kPk ? NR : 1];
  float m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int r = rs + i * RP;
    const int64_t srow = g * group + r;
    const bool ld = on && r < group && srow < S;
    float t[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if constexpr (kPk) {
      raw[i] = ld ? *reinterpret_cast<const uint4*>(base + srow * ss) : make_uint4(0u, 0u, 0u, 0u);
      f16x8_to_f32(raw[i], t);
    } else {
      if (ld) load8(base + srow * ss, t);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = t[j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) m[j] = absmax_nan(m[j], t[j]);
  }
  __shared__ float red[RP][DP];
  __shared__ float inv_s[DP];
#pragma unroll
  for (int j = 0; j < 8; ++j) red[rs][c * 8 + j] = m[j];
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += kBlock) {
    float a = 0.0f;
    for (int k = 0; k < RP; ++k) a = absmax_nan(a, red[k][d]);
    float inv;
    typename ScaleOf<MODE>::T sc;
    sym_params<MODE, 1>(a, inv, sc);
    inv_s[d] = inv;
    scale[(bh * G + g) * D + d] = sc;
  }
  __syncthreads();
  if (!on) return;
  float iv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) iv[j] = inv_s[c * 8 + j];
  bool inv_ok = true;
  uint32_t ivp[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    inv_ok = inv_ok && iv[2 * j] > 0.0f && iv[2 * j] < INFINITY && iv[2 * j + 1] > 0.0f && iv[2 * j + 1] < INFINITY;
    ivp[j] = static_cast<uint32_t>(f2h(iv[2 * j])) | (static_cast<uint32_t>(f2h(iv[2 * j + 1])) << 16);
  }
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int r = rs + i * RP;
    if (r < group) {
      uint2* dst = reinterpret_cast<uint2*>(codes + (bh * S_pad + g * group + r) * D + c * 8);
      float t[8];
      if constexpr (kPk) {
        if (inv_ok && finite8(raw[i])) {
          *dst = codes2_i8_f16(raw[i], make_uint4(ivp[0], ivp[1], ivp[2], ivp[3]));
          continue;
        }
        f16x8_to_f32(raw[i], t);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = v[i][j];
      }
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo |= static_cast<uint32_t>(sym_code<MODE, -2, 1>(t[j], iv[j]) & 0xFF) << (8 * j);
        hi |= static_cast<uint32_t>(sym_code<MODE, -2, 1>(t[4 + j], iv[4 + j]) & 0xFF) << (8 * j);
      }
      *dst = make_uint2(lo, hi);
    }
  }
}

template <typename T>
__global__ void dequant_int2_grouped_kernel(const int8_t* __restrict__ codes,
                                            const T* __restrict__ scale, int64_t BH,
                                            int64_t S_pad, int64_t D, int64_t group, int64_t S_out,
                                            T* __restrict__ out) {
  const int64_t n = BH * S_out * D;
  const int64_t G = S_pad / group;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t d = i % D;
    const int64_t s = (i / D) % S_out;
    const int64_t bh = i / (D * S_out);
    const float q = static_cast<float>(codes[(bh * S_pad + s) * D + d]);
    out[i] = from_f32<T>(q * to_f32(scale[(bh * G + s / group) * D + d]));
  }
}

// Row-vectorized form of the kernel above: each lane takes 8 channels of a row
// (8 code bytes, 8 scales, 8 outputs); the same products and roundings.
template <typename T, int LPR>
__global__ __launch_bounds__(kBlock) void dequant_int2_grouped_rows_kernel(const int8_t* __restrict__ codes,
                                                                           const T* __restrict__ scale, int D,
                                                                           int64_t S_pad, int64_t group, int64_t S_out,
                                                                           int64_t rows, T* __restrict__ out) {
  constexpr int RP = kBlock / LPR;
  const int c = threadIdx.x % LPR;
  if (c * 8 >= D) return;  // past the row's channels
  const int64_t G = S_pad / group;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * RP + threadIdx.x / LPR; r < rows;
       r += static_cast<int64_t>(gridDim.x) * RP) {
    const int64_t bh = r / S_out, s = r - bh * S_out;
    const uint2 w = *reinterpret_cast<const uint2*>(codes + (bh * S_pad + s) * D + c * 8);
    const T* sp = scale + (bh * G + s / group) * D + c * 8;
    float y[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      y[j] = static_cast<float>(static_cast<int8_t>((w.x >> (8 * j)) & 0xFF)) * to_f32(sp[j]);
      y[4 + j] = static_cast<float>(static_cast<int8_t>((w.y >> (8 * j)) & 0xFF)) * to_f32(sp[4 + j]);
    }
    store8(out + r * D + c * 8, y);
  }
}

// ------------------------------------------------------ asymmetric groups
template <int BITS, int LPG, int LPR>
__global__ __launch_bounds__(kBlock) void quant_asym_kernel(const uint16_t* __restrict__ x, int D,
                                                            int64_t rows, int64_t H, int64_t S,
                                                            int64_t sb, int64_t sh, int64_t ss, int64_t fs,
                                                            uint8_t* __restrict__ packed,
                                                            uint16_t* __restrict__ scale,
                                                            uint16_t* __restrict__ zero) {
  constexpr int RP = kBlock / LPR;
  const int NG = D / (8 * LPG);  // groups per row (D is a multiple of the group)
  const int row_bytes = D * BITS / 8;
  constexpr float QMAXU = static_cast<float>((1 << BITS) - 1);
  const int c = threadIdx.x % LPR;
  const bool on = c * 8 < D;  // whole groups of lanes idle past the row's channels
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * RP + threadIdx.x / LPR; r < rows;
       r += static_cast<int64_t>(gridDim.x) * RP) {
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (on) load8(x + (fs ? r * fs : row_offset(r, H, S, sb, sh, ss)) + c * 8, v);
    float mn = v[0], mx = v[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) {
      mn = fminf(mn, v[j]);
      mx = fmaxf(mx, v[j]);
    }
    mn = group_min<LPG>(mn);
    mx = group_max<LPG>(mx);
    const uint16_t sc = f2h((mx - mn) / QMAXU);
    const float s = h2f(sc);
    // one correctly rounded reciprocal per group, then a rounded product per element
    const float inv = s == 0.0f ? 0.0f : 1.0f / s;
    int code[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float t = rintf((v[j] - mn) * inv);
      code[j] = static_cast<int>(fminf(fmaxf(t, 0.0f), QMAXU));
    }
    if (!on) continue;
    uint8_t* dst = packed + r * row_bytes + c * BITS;
    if (BITS == 4) {
      uint32_t w = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w |= static_cast<uint32_t>((code[2 * j] << 4) | code[2 * j + 1]) << (8 * j);
      *reinterpret_cast<uint32_t*>(dst) = w;
    } else {
      uint32_t w = 0;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        w |= static_cast<uint32_t>((code[4 * j] << 6) | (code[4 * j + 1] << 4) |
                                   (code[4 * j + 2] << 2) | code[4 * j + 3])
             << (8 * j);
      *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(w);
    }
    if (c % LPG == 0) {
      scale[r * NG + c / LPG] = sc;
      zero[r * NG + c / LPG] = f2h(mn);
    }
  }
}

template <int BITS, int LPG, int LPR>
__global__ __launch_bounds__(kBlock) void dequant_asym_kernel(const uint8_t* __restrict__ packed,
                                                              const uint16_t* __restrict__ scale,
                                                              const uint16_t* __restrict__ zero, int D,
                                                              int64_t rows,
                                                              uint16_t* __restrict__ out) {
  constexpr int RP = kBlock / LPR;
  const int NG = D / (8 * LPG);
  const int row_bytes = D * BITS / 8;
  const int c = threadIdx.x % LPR;
  if (c * 8 >= D) return;  // past the row's channels
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * RP + threadIdx.x / LPR; r < rows;
       r += static_cast<int64_t>(gridDim.x) * RP) {
    const float s = h2f(scale[r * NG + c / LPG]);
    const float z = h2f(zero[r * NG + c / LPG]);
    const uint8_t* src = packed + r * row_bytes + c * BITS;
    int code[8];
    if (BITS == 4) {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(src);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        code[2 * j] = (w >> (8 * j + 4)) & 0xF;
        code[2 * j + 1] = (w >> (8 * j)) & 0xF;
      }
    } else {
      const uint32_t w = *reinterpret_cast<const uint16_t*>(src);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int k = 0; k < 4; ++k) code[4 * j + k] = (w >> (8 * j + 6 - 2 * k)) & 3;
    }
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = static_cast<float>(code[2 * j]) * s + z;
      const float b = static_cast<float>(code[2 * j + 1]) * s + z;
      w[j] = static_cast<uint32_t>(f2h(a)) | (static_cast<uint32_t>(f2h(b)) << 16);
    }
    *reinterpret_cast<uint4*>(out + r * D + c * 8) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// ------------------------------------------------------- pack / unpack
template <int BITS>
__global__ void pack_kernel(const int8_t* __restrict__ q, int64_t n8, uint8_t* __restrict__ out) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n8;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const uint2 w = *reinterpret_cast<const uint2*>(q + i * 8);
    int c[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c[j] = static_cast<int8_t>((w.x >> (8 * j)) & 0xFF);
      c[4 + j] = static_cast<int8_t>((w.y >> (8 * j)) & 0xFF);
    }
    store_codes<BITS>(out + i * BITS, c);
  }
}

template <int BITS>
__global__ void unpack_kernel(const uint8_t* __restrict__ packed, int64_t n8, int8_t* __restrict__ q) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n8;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int c[8];
    load_codes<BITS>(packed + i * BITS, c);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lo |= static_cast<uint32_t>(c[j] & 0xFF) << (8 * j);
      hi |= static_cast<uint32_t>(c[4 + j] & 0xFF) << (8 * j);
    }
    *reinterpret_cast<uint2*>(q + i * 8) = make_uint2(lo, hi);
  }
}

// ---------------------------------------------------------------- host side
int check_dims(const char* fn, int64_t B, int64_t H, int64_t S, int64_t D) {
  if (B < 0 || H < 0 || S < 0) return einval("%s: negative size (B=%lld H=%lld S=%lld)", fn, (long long)B, (long long)H, (long long)S);
  if (D < 8 || D > 256 || D % 8 != 0)
    return einval("%s: head_dim must be a multiple of 8 in [8, 256], got %lld", fn, (long long)D);
  return FADE_OK;
}

// At most 16384 blocks (a grid-stride loop covers the rest): measured best on
// MI355X for the full-size quantizers (4096 to 2^20 blocks tried).
int grid_for_rows(int64_t rows, int lpr) {
  const int64_t rp = kBlock / lpr;
  const int64_t g = cdiv(rows, rp);
  return static_cast<int>(g < 16384 ? (g > 0 ? g : 1) : 16384);
}

// Element stride between consecutive rows when the [B, H, S] row index maps
// to one uniform stride (then a row's offset is r * stride); 0 otherwise.
int64_t flat_row_stride(int64_t H, int64_t S, int64_t sb, int64_t sh, int64_t ss) {
  return (sh == S * ss && sb == H * sh) ? ss : 0;
}

// S-blocking of the two-pass per-channel quantizer (shared with the workspace query).
void channel_blocking(int64_t BH, int64_t S, int64_t* nsb, int64_t* rows_per_block) {
  int64_t target = BH > 0 ? 2048 / BH : 1;
  if (target < 1) target = 1;
  int64_t n = cdiv(S, 64);
  if (n > target) n = target;
  if (n < 1) n = 1;
  int64_t rpb = cdiv(S, n);
  if (rpb < 1) rpb = 1;
  *rows_per_block = rpb;
  *nsb = cdiv(S, rpb) > 0 ? cdiv(S, rpb) : 1;
}

// Lanes per row: the power of two that covers D / 8 lanes (8 channels each);
// the lanes past D / 8 idle.
#define FADE_DISPATCH_LPR(D, ...)                                        \
  if ((D) <= 32) { constexpr int LPR = 4; __VA_ARGS__; }                 \
  else if ((D) <= 64) { constexpr int LPR = 8; __VA_ARGS__; }            \
  else if ((D) <= 128) { constexpr int LPR = 16; __VA_ARGS__; }          \
  else { constexpr int LPR = 32; __VA_ARGS__; }

template <typename InT, int MODE, int BITS>
int launch_channel(const char* fn, const InT* x, int64_t B, int64_t H, int64_t S, int64_t D,
                   int64_t sb, int64_t sh, int64_t ss, void* packed, void* scale, void* ws,
                   int64_t ws_bytes, hipStream_t st) {
  const int64_t BH = B * H;
  if (BH == 0) return FADE_OK;
  if (S == 0) return einval("%s: S must be > 0 for a per-channel scale", fn);
  int64_t nsb, rpb;
  channel_blocking(BH, S, &nsb, &rpb);
  const int64_t need = BH * nsb * D * static_cast<int64_t>(sizeof(float));
  if (ws == nullptr || ws_bytes < need)
    return einval("%s: workspace too small (%lld < %lld bytes)", fn, (long long)ws_bytes, (long long)need);
  if (BH > 65535) return einval("%s: B*H=%lld exceeds 65535", fn, (long long)BH);
  dim3 grid(static_cast<unsigned>(nsb), static_cast<unsigned>(BH));
  FADE_DISPATCH_LPR(D, {
    hipLaunchKernelGGL((colmax_kernel<InT, LPR>), grid, dim3(kBlock), 0, st, x, static_cast<int>(D), H, S, sb, sh, ss,
                       rpb, static_cast<float*>(ws));
    hipLaunchKernelGGL((quant_channel_kernel<InT, MODE, BITS, LPR>), grid, dim3(kBlock), 0, st, x,
                       static_cast<int>(D), H, S, sb, sh, ss, rpb, static_cast<const float*>(ws), static_cast<int>(nsb),
                       static_cast<uint8_t*>(packed), static_cast<typename ScaleOf<MODE>::T*>(scale));
  });
  return check_launch(fn);
}

// Pass 2 alone, on column maxima another kernel produced: partial [B*H][nparts][D].
template <typename InT, int MODE, int BITS>
int launch_channel_given(const char* fn, const InT* x, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                         int64_t sh, int64_t ss, const float* partial, int64_t nparts, void* packed, void* scale,
                         hipStream_t st) {
  const int64_t BH = B * H;
  if (BH == 0) return FADE_OK;
  if (S == 0) return einval("%s: S must be > 0 for a per-channel scale", fn);
  if (partial == nullptr || nparts < 1 || nparts > 65535) return einval("%s: need 1..65535 column-max partials", fn);
  if (BH > 65535) return einval("%s: B*H=%lld exceeds 65535", fn, (long long)BH);
  int64_t nsb, rpb;
  channel_blocking(BH, S, &nsb, &rpb);
  dim3 grid(static_cast<unsigned>(nsb), static_cast<unsigned>(BH));
  FADE_DISPATCH_LPR(D, {
    hipLaunchKernelGGL((quant_channel_kernel<InT, MODE, BITS, LPR>), grid, dim3(kBlock), 0, st, x,
                       static_cast<int>(D), H, S, sb, sh, ss, rpb, partial, static_cast<int>(nparts),
                       static_cast<uint8_t*>(packed), static_cast<typename ScaleOf<MODE>::T*>(scale));
  });
  return check_launch(fn);
}

template <typename InT, int MODE, int BITS>
int launch_token(const char* fn, const InT* x, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                 int64_t sh, int64_t ss, void* packed, void* scale, hipStream_t st) {
  const int64_t rows = B * H * S;
  if (rows == 0) return FADE_OK;
  FADE_DISPATCH_LPR(D, {
    hipLaunchKernelGGL((quant_token_kernel<InT, MODE, BITS, LPR>), dim3(grid_for_rows(rows, LPR)),
                       dim3(kBlock), 0, st, x, static_cast<int>(D), rows, H, S, sb, sh, ss, flat_row_stride(H, S, sb, sh, ss),
                       static_cast<uint8_t*>(packed), static_cast<typename ScaleOf<MODE>::T*>(scale));
  });
  return check_launch(fn);
}

bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

}  // namespace
}  // namespace fade

using namespace fade;

FADE_API int fade_pack_codes(const void* q_i8, int64_t n_rows, int64_t D, int32_t bits,
                             void* packed_u8, void* stream) {
  if (bits != 4 && bits != 2) return einval("fade_pack_codes: bits must be 4 or 2, got %d", bits);
  if (D % 8 != 0) return einval("fade_pack_codes: last dim must be a multiple of 8, got %lld", (long long)D);
  const int64_t n8 = n_rows * D / 8;
  if (n8 == 0) return FADE_OK;
  const int grid = static_cast<int>(cdiv(n8, 256) < 16384 ? cdiv(n8, 256) : 16384);
  if (bits == 4)
    hipLaunchKernelGGL(pack_kernel<4>, dim3(grid), dim3(256), 0, as_stream(stream),
                       static_cast<const int8_t*>(q_i8), n8, static_cast<uint8_t*>(packed_u8));
  else
    hipLaunchKernelGGL(pack_kernel<2>, dim3(grid), dim3(256), 0, as_stream(stream),
                       static_cast<const int8_t*>(q_i8), n8, static_cast<uint8_t*>(packed_u8));
  return check_launch("fade_pack_codes");
}

FADE_API int fade_unpack_codes(const void* packed_u8, int64_t n_rows, int64_t D, int32_t bits,
                               void* q_i8, void* stream) {
  if (bits != 4 && bits != 2) return einval("fade_unpack_codes: bits must be 4 or 2, got %d", bits);
  if (D % 8 != 0) return einval("fade_unpack_codes: last dim must be a multiple of 8, got %lld", (long long)D);
  const int64_t n8 = n_rows * D / 8;
  if (n8 == 0) return FADE_OK;
  const int grid = static_cast<int>(cdiv(n8, 256) < 16384 ? cdiv(n8, 256) : 16384);
  if (bits == 4)
    hipLaunchKernelGGL(unpack_kernel<4>, dim3(grid), dim3(256), 0, as_stream(stream),
                       static_cast<const uint8_t*>(packed_u8), n8, static_cast<int8_t*>(q_i8));
  else
    hipLaunchKernelGGL(unpack_kernel<2>, dim3(grid), dim3(256), 0, as_stream(stream),
                       static_cast<const uint8_t*>(packed_u8), n8, static_cast<int8_t*>(q_i8));
  return check_launch("fade_unpack_codes");
}

FADE_API int fade_quant_k_int4_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D,
                                               int64_t* bytes) {
  if (bytes == nullptr) return einval("fade_quant_k_int4_workspace_bytes: null output");
  int64_t nsb, rpb;
  channel_blocking(B * H, S, &nsb, &rpb);
  *bytes = B * H * nsb * D * static_cast<int64_t>(sizeof(float));
  return FADE_OK;
}

FADE_API int fade_quant_k_int4_from_colmax(const void* k_f16, int64_t B, int64_t H, int64_t S, int64_t D,
                                           int64_t sb, int64_t sh, int64_t ss, const float* colmax,
                                           int64_t parts, void* packed_u8, void* scale_f16, void* stream) {
  int rc = check_dims("fade_quant_k_int4_from_colmax", B, H, S, D);
  if (rc) return rc;
  if (!aligned(k_f16, 16) || (sb | sh | ss) % 8 != 0)
    return einval("fade_quant_k_int4_from_colmax: input must be 16-byte aligned with strides a multiple of 8");
  return launch_channel_given<uint16_t, MODE_F16, 4>("fade_quant_k_int4_from_colmax",
                                                     static_cast<const uint16_t*>(k_f16), B, H, S, D, sb, sh, ss,
                                                     colmax, parts, packed_u8, scale_f16, as_stream(stream));
}

FADE_API int fade_quant_k_int4(const void* k_f16, int64_t B, int64_t H, int64_t S, int64_t D,
                               int64_t sb, int64_t sh, int64_t ss, void* packed_u8, void* scale_f16,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_dims("fade_quant_k_int4", B, H, S, D);
  if (rc) return rc;
  if (!aligned(k_f16, 16) || (sb | sh | ss) % 8 != 0)
    return einval("fade_quant_k_int4: input must be 16-byte aligned with strides a multiple of 8");
  return launch_channel<uint16_t, MODE_F16, 4>("fade_quant_k_int4", static_cast<const uint16_t*>(k_f16),
                                               B, H, S, D, sb, sh, ss, packed_u8, scale_f16,
                                               workspace, workspace_bytes, as_stream(stream));
}

FADE_API int fade_quant_v_int4(const void* v_f16, int64_t B, int64_t H, int64_t S, int64_t D,
                               int64_t sb, int64_t sh, int64_t ss, void* packed_u8, void* scale_f16,
                               void* stream) {
  int rc = check_dims("fade_quant_v_int4", B, H, S, D);
  if (rc) return rc;
  if (!aligned(v_f16, 16) || (sb | sh | ss) % 8 != 0)
    return einval("fade_quant_v_int4: input must be 16-byte aligned with strides a multiple of 8");
  return launch_token<uint16_t, MODE_F16, 4>("fade_quant_v_int4", static_cast<const uint16_t*>(v_f16),
                                             B, H, S, D, sb, sh, ss, packed_u8, scale_f16,
                                             as_stream(stream));
}

FADE_API int fade_quant_k_int4_dtype(const void* k, int32_t dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                                     int64_t sb, int64_t sh, int64_t ss, void* packed_u8, void* scale,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  const char* fn = "fade_quant_k_int4_dtype";
  int rc = check_dims(fn, B, H, S, D);
  if (rc) return rc;
  if (!aligned(k, 16) || (sb | sh | ss) % 8 != 0)
    return einval("%s: input must be 16-byte aligned with strides a multiple of 8", fn);
  switch (dtype) {
    case FADE_DTYPE_F16:
      return launch_channel<uint16_t, MODE_F16, 4>(fn, static_cast<const uint16_t*>(k), B, H, S, D, sb, sh, ss,
                                                   packed_u8, scale, workspace, workspace_bytes, as_stream(stream));
    case FADE_DTYPE_BF16:
      return launch_channel<Bf16, MODE_BF16, 4>(fn, static_cast<const Bf16*>(k), B, H, S, D, sb, sh, ss, packed_u8,
                                                scale, workspace, workspace_bytes, as_stream(stream));
    case FADE_DTYPE_F32:
      return launch_channel<float, MODE_F32S, 4>(fn, static_cast<const float*>(k), B, H, S, D, sb, sh, ss,
                                                 packed_u8, scale, workspace, workspace_bytes, as_stream(stream));
    default: return einval("%s: unknown dtype %d", fn, dtype);
  }
}

FADE_API int fade_quant_v_int4_dtype(const void* v, int32_t dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                                     int64_t sb, int64_t sh, int64_t ss, void* packed_u8, void* scale,
                                     void* stream) {
  const char* fn = "fade_quant_v_int4_dtype";
  int rc = check_dims(fn, B, H, S, D);
  if (rc) return rc;
  if (!aligned(v, 16) || (sb | sh | ss) % 8 != 0)
    return einval("%s: input must be 16-byte aligned with strides a multiple of 8", fn);
  switch (dtype) {
    case FADE_DTYPE_F16:
      return launch_token<uint16_t, MODE_F16, 4>(fn, static_cast<const uint16_t*>(v), B, H, S, D, sb, sh, ss,
                                                 packed_u8, scale, as_stream(stream));
    case FADE_DTYPE_BF16:
      return launch_token<Bf16, MODE_BF16, 4>(fn, static_cast<const Bf16*>(v), B, H, S, D, sb, sh, ss, packed_u8,
                                              scale, as_stream(stream));
    case FADE_DTYPE_F32:
      return launch_token<float, MODE_F32S, 4>(fn, static_cast<const float*>(v), B, H, S, D, sb, sh, ss, packed_u8,
                                               scale, as_stream(stream));
    default: return einval("%s: unknown dtype %d", fn, dtype);
  }
}

namespace fade {
namespace {
template <typename T>
int dequant_sym(const char* fn, const void* packed_u8, const void* scale, int32_t bits, int32_t axis, int64_t B,
                int64_t H, int64_t S, int64_t D, void* out, void* stream) {
  int rc = check_dims(fn, B, H, S, D);
  if (rc) return rc;
  if (bits != 4 && bits != 3 && bits != 2) return einval("%s: bits must be 4, 3 or 2, got %d", fn, bits);
  if (axis != FADE_AXIS_CHANNEL && axis != FADE_AXIS_TOKEN) return einval("%s: bad axis %d", fn, axis);
  const int64_t rows = B * H * S;
  if (rows == 0) return FADE_OK;
  const uint8_t* pk = static_cast<const uint8_t*>(packed_u8);
  const T* sc = static_cast<const T*>(scale);
  T* o = static_cast<T*>(out);
  FADE_DISPATCH_LPR(D, {
    const dim3 grid(grid_for_rows(rows, LPR));
    if (bits == 4)
      hipLaunchKernelGGL((dequant_sym_kernel<4, LPR, T>), grid, dim3(kBlock), 0, as_stream(stream), pk, sc,
                         static_cast<int>(D), axis,
                         rows, S, o);
    else if (bits == 3)
      hipLaunchKernelGGL((dequant_sym_kernel<3, LPR, T>), grid, dim3(kBlock), 0, as_stream(stream), pk, sc,
                         static_cast<int>(D), axis,
                         rows, S, o);
    else
      hipLaunchKernelGGL((dequant_sym_kernel<2, LPR, T>), grid, dim3(kBlock), 0, as_stream(stream), pk, sc,
                         static_cast<int>(D), axis,
                         rows, S, o);
  });
  return check_launch(fn);
}
}  // namespace
}  // namespace fade

FADE_API int fade_dequant_sym(const void* packed_u8, const void* scale_f16, int32_t bits,
                              int32_t axis, int64_t B, int64_t H, int64_t S, int64_t D,
                              void* out_f16, void* stream) {
  return dequant_sym<uint16_t>("fade_dequant_sym", packed_u8, scale_f16, bits, axis, B, H, S, D, out_f16, stream);
}

FADE_API int fade_dequant_sym_dtype(const void* packed_u8, const void* scale, int32_t dtype, int32_t bits,
                                    int32_t axis, int64_t B, int64_t H, int64_t S, int64_t D, void* out,
                                    void* stream) {
  const char* fn = "fade_dequant_sym_dtype";
  switch (dtype) {
    case FADE_DTYPE_F16: return dequant_sym<uint16_t>(fn, packed_u8, scale, bits, axis, B, H, S, D, out, stream);
    case FADE_DTYPE_BF16: return dequant_sym<Bf16>(fn, packed_u8, scale, bits, axis, B, H, S, D, out, stream);
    case FADE_DTYPE_F32: return dequant_sym<float>(fn, packed_u8, scale, bits, axis, B, H, S, D, out, stream);
    default: return einval("%s: unknown dtype %d", fn, dtype);
  }
}

namespace fade {
namespace {
template <typename T>
int quant_int2_grouped(const char* fn, const void* x, int64_t B, int64_t H, int64_t S, int64_t S_pad, int64_t D,
                       int64_t sb, int64_t sh, int64_t ss, int64_t group, void* codes_i8, void* scale, void* stream) {
  int rc = check_dims(fn, B, H, S, D);
  if (rc) return rc;
  if (group < 1 || S_pad % group != 0 || S_pad < S)
    return einval("S=%lld must be divisible by group_size=%lld", (long long)S_pad, (long long)group);
  const int64_t BH = B * H, G = S_pad / group;
  if (BH == 0 || G == 0) return FADE_OK;
  if (BH > 65535) return einval("%s: B*H=%lld exceeds 65535", fn, (long long)BH);
  constexpr int MODE = Int2Mode<T>::value;
  // single pass with register-resident rows: 8 channels per lane (D a
  // multiple of 8 up to 256, 16-byte aligned rows, 8-byte aligned codes) and
  // at most 8 rows per lane
  const int lpr = D <= 32 ? 4 : (D <= 64 ? 8 : (D <= 128 ? 16 : 32));
  if (D % 8 == 0 && D <= 256 && group <= 8 * (kBlock / lpr) && aligned(x, 16) && (sb | sh | ss) % 8 == 0 &&
      aligned(codes_i8, 8)) {
    const dim3 grid(static_cast<unsigned>(G), static_cast<unsigned>(BH));
    FADE_DISPATCH_LPR(D, {
      hipLaunchKernelGGL((quant_int2_grouped_rows_kernel<T, MODE, LPR, 8>), grid, dim3(kBlock), 0, as_stream(stream),
                         static_cast<const T*>(x), static_cast<int>(D), H, S, S_pad, sb, sh, ss,
                         static_cast<int>(group), static_cast<int8_t*>(codes_i8),
                         static_cast<typename ScaleOf<MODE>::T*>(scale));
    });
    return check_launch(fn);
  }
  hipLaunchKernelGGL((quant_int2_grouped_kernel<T, MODE>), dim3(static_cast<unsigned>(G), static_cast<unsigned>(BH)),
                     dim3(static_cast<unsigned>(D)), 0, as_stream(stream), static_cast<const T*>(x), H, S, S_pad,
                     sb, sh, ss, static_cast<int>(group), static_cast<int8_t*>(codes_i8),
                     static_cast<typename ScaleOf<MODE>::T*>(scale));
  return check_launch(fn);
}
template <typename T>
int dequant_int2_grouped(const char* fn, const void* codes_i8, const void* scale, int64_t B, int64_t H,
                         int64_t S_pad, int64_t D, int64_t group, int64_t S_out, void* out, void* stream) {
  if (group < 1 || S_pad % group != 0 || S_out > S_pad || S_out < 0)
    return einval("%s: bad sizes (S_pad=%lld group=%lld S_out=%lld)", fn, (long long)S_pad, (long long)group,
                  (long long)S_out);
  const int64_t n = B * H * S_out * D;
  if (n == 0) return FADE_OK;
  if (D % 8 == 0 && D >= 8 && D <= 256 && aligned(codes_i8, 8) && aligned(scale, 16) && aligned(out, 16)) {
    const int64_t rows = B * H * S_out;
    FADE_DISPATCH_LPR(D, {
      hipLaunchKernelGGL((dequant_int2_grouped_rows_kernel<T, LPR>), dim3(grid_for_rows(rows, LPR)), dim3(kBlock), 0,
                         as_stream(stream), static_cast<const int8_t*>(codes_i8), static_cast<const T*>(scale),
                         static_cast<int>(D), S_pad, group, S_out, rows, static_cast<T*>(out));
    });
    return check_launch(fn);
  }
  const int grid = static_cast<int>(cdiv(n, 256) < 16384 ? cdiv(n, 256) : 16384);
  hipLaunchKernelGGL(dequant_int2_grouped_kernel<T>, dim3(grid), dim3(256), 0, as_stream(stream),
                     static_cast<const int8_t*>(codes_i8), static_cast<const T*>(scale), B * H, S_pad, D, group,
                     S_out, static_cast<T*>(out));
  return check_launch(fn);
}
}  // namespace
}  // namespace fade

FADE_API int fade_quant_int2_grouped(const void* x_f16, int64_t B, int64_t H, int64_t S,
                                     int64_t S_pad, int64_t D, int64_t sb, int64_t sh, int64_t ss,
                                     int64_t group, void* codes_i8, void* scale_f16, void* stream) {
  return quant_int2_grouped<uint16_t>("fade_quant_int2_grouped", x_f16, B, H, S, S_pad, D, sb, sh, ss, group,
                                      codes_i8, scale_f16, stream);
}
FADE_API int fade_quant_int2_grouped_dtype(const void* x, int32_t dtype, int64_t B, int64_t H, int64_t S,
                                           int64_t S_pad, int64_t D, int64_t sb, int64_t sh, int64_t ss,
                                           int64_t group, void* codes_i8, void* scale, void* stream) {
  const char* fn = "fade_quant_int2_grouped_dtype";
  switch (dtype) {
    case FADE_DTYPE_F16:
      return quant_int2_grouped<uint16_t>(fn, x, B, H, S, S_pad, D, sb, sh, ss, group, codes_i8, scale, stream);
    case FADE_DTYPE_BF16:
      return quant_int2_grouped<Bf16>(fn, x, B, H, S, S_pad, D, sb, sh, ss, group, codes_i8, scale, stream);
    case FADE_DTYPE_F32:
      return quant_int2_grouped<float>(fn, x, B, H, S, S_pad, D, sb, sh, ss, group, codes_i8, scale, stream);
    default: return einval("%s: unknown dtype %d", fn, dtype);
  }
}
FADE_API int fade_dequant_int2_grouped(const void* codes_i8, const void* scale_f16, int64_t B,
                                       int64_t H, int64_t S_pad, int64_t D, int64_t group,
                                       int64_t S_out, void* out_f16, void* stream) {
  return dequant_int2_grouped<uint16_t>("fade_dequant_int2_grouped", codes_i8, scale_f16, B, H, S_pad, D, group,
                                        S_out, out_f16, stream);
}
FADE_API int fade_dequant_int2_grouped_dtype(const void* codes_i8, const void* scale, int32_t dtype, int64_t B,
                                             int64_t H, int64_t S_pad, int64_t D, int64_t group, int64_t S_out,
                                             void* out, void* stream) {
  const char* fn = "fade_dequant_int2_grouped_dtype";
  switch (dtype) {
    case FADE_DTYPE_F16:
      return dequant_int2_grouped<uint16_t>(fn, codes_i8, scale, B, H, S_pad, D, group, S_out, out, stream);
    case FADE_DTYPE_BF16:
      return dequant_int2_grouped<Bf16>(fn, codes_i8, scale, B, H, S_pad, D, group, S_out, out, stream);
    case FADE_DTYPE_F32:
      return dequant_int2_grouped<float>(fn, codes_i8, scale, B, H, S_pad, D, group, S_out, out, stream);
    default: return einval("%s: unknown dtype %d", fn, dtype);
  }
}

FADE_API int fade_quant_rotated_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D,
                                                int32_t axis, int64_t* bytes) {
  if (bytes == nullptr) return einval("fade_quant_rotated_workspace_bytes: null output");
  if (axis == FADE_AXIS_TOKEN) {
    *bytes = 0;
    return FADE_OK;
  }
  return fade_quant_k_int4_workspace_bytes(B, H, S, D, bytes);
}

namespace fade {
namespace {
template <int MODE>
int quant_rotated(const char* fn, const float* x_rot, int64_t B, int64_t H, int64_t S, int64_t D, int32_t bits,
                  int32_t axis, void* packed, void* scale, void* workspace, int64_t workspace_bytes,
                  hipStream_t st) {
  const int64_t sb = H * S * D, sh = S * D, ss = D;
  if (axis == FADE_AXIS_TOKEN) {
    switch (bits) {
      case 4: return launch_token<float, MODE, 4>(fn, x_rot, B, H, S, D, sb, sh, ss, packed, scale, st);
      case 3: return launch_token<float, MODE, 3>(fn, x_rot, B, H, S, D, sb, sh, ss, packed, scale, st);
      case 2: return launch_token<float, MODE, 2>(fn, x_rot, B, H, S, D, sb, sh, ss, packed, scale, st);
      default: return einval("%s: bits must be 2, 3 or 4, got %d", fn, bits);
    }
  }
  if (axis != FADE_AXIS_CHANNEL) return einval("%s: bad axis %d", fn, axis);
  switch (bits) {
    case 4: return launch_channel<float, MODE, 4>(fn, x_rot, B, H, S, D, sb, sh, ss, packed, scale, workspace, workspace_bytes, st);
    case 3: return launch_channel<float, MODE, 3>(fn, x_rot, B, H, S, D, sb, sh, ss, packed, scale, workspace, workspace_bytes, st);
    case 2: return launch_channel<float, MODE, 2>(fn, x_rot, B, H, S, D, sb, sh, ss, packed, scale, workspace, workspace_bytes, st);
    default: return einval("%s: bits must be 2, 3 or 4, got %d", fn, bits);
  }
}
}  // namespace
}  // namespace fade

FADE_API int fade_quant_rotated(const float* x_rot, int64_t B, int64_t H, int64_t S, int64_t D,
                                int32_t bits, int32_t axis, void* packed, void* scale_f16,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_dims("fade_quant_rotated", B, H, S, D);
  if (rc) return rc;
  if (!aligned(x_rot, 16)) return einval("fade_quant_rotated: input must be 16-byte aligned");
  return quant_rotated<MODE_F32>("fade_quant_rotated", x_rot, B, H, S, D, bits, axis, packed, scale_f16, workspace,
                                 workspace_bytes, as_stream(stream));
}

FADE_API int fade_quant_rotated_dtype(const float* x_rot, int64_t B, int64_t H, int64_t S, int64_t D, int32_t bits,
                                      int32_t axis, void* packed, void* scale, int32_t scale_dtype, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  const char* fn = "fade_quant_rotated_dtype";
  int rc = check_dims(fn, B, H, S, D);
  if (rc) return rc;
  if (!aligned(x_rot, 16)) return einval("%s: input must be 16-byte aligned", fn);
  hipStream_t st = as_stream(stream);
  switch (scale_dtype) {
    case FADE_DTYPE_F16:
      return quant_rotated<MODE_F32>(fn, x_rot, B, H, S, D, bits, axis, packed, scale, workspace, workspace_bytes, st);
    case FADE_DTYPE_BF16:
      return quant_rotated<MODE_F32B>(fn, x_rot, B, H, S, D, bits, axis, packed, scale, workspace, workspace_bytes, st);
    case FADE_DTYPE_F32:
      return quant_rotated<MODE_F32S>(fn, x_rot, B, H, S, D, bits, axis, packed, scale, workspace, workspace_bytes, st);
    default: return einval("%s: unknown scale dtype %d", fn, scale_dtype);
  }
}

#define FADE_DISPATCH_ASYM(bits, group, D, ...)                                        \
  do {                                                                                         \
    if ((bits) != 4 && (bits) != 2) return einval("asym: bits must be 4 or 2, got %d", (bits)); \
    if ((group) != 16 && (group) != 32 && (group) != 64)                                       \
      return einval("asym: group must be 16, 32 or 64, got %d", (group));                     \
    if ((D) % (group) != 0) return einval("asym: D must be divisible by group");              \
    FADE_DISPATCH_LPR(D, {                                                                     \
      if ((bits) == 4) {                                                                       \
        constexpr int BITS = 4;                                                                \
        if ((group) == 16) { constexpr int LPG = 2; __VA_ARGS__; }                             \
        else if ((group) == 32) { constexpr int LPG = 4; __VA_ARGS__; }                        \
        else { constexpr int LPG = 8; __VA_ARGS__; }                                           \
      } else {                                                                                 \
        constexpr int BITS = 2;                                                                \
        if ((group) == 16) { constexpr int LPG = 2; __VA_ARGS__; }                             \
        else if ((group) == 32) { constexpr int LPG = 4; __VA_ARGS__; }                        \
        else { constexpr int LPG = 8; __VA_ARGS__; }                                           \
      }                                                                                        \
    });                                                                                        \
  } while (0)

FADE_API int fade_quant_asym(const void* x_f16, int64_t B, int64_t H, int64_t S, int64_t D,
                             int64_t sb, int64_t sh, int64_t ss, int32_t bits, int32_t group,
                             void* packed_u8, void* scale_f16, void* zero_f16, void* stream) {
  int rc = check_dims("fade_quant_asym", B, H, S, D);
  if (rc) return rc;
  if (!aligned(x_f16, 16) || (sb | sh | ss) % 8 != 0)
    return einval("fade_quant_asym: input must be 16-byte aligned with strides a multiple of 8");
  const int64_t rows = B * H * S;
  if (rows == 0) return FADE_OK;
  FADE_DISPATCH_ASYM(bits, group, D,
                     hipLaunchKernelGGL((quant_asym_kernel<BITS, LPG, LPR>),
                                         dim3(grid_for_rows(rows, LPR)), dim3(kBlock), 0,
                                         as_stream(stream), static_cast<const uint16_t*>(x_f16),
                                         static_cast<int>(D), rows, H, S, sb, sh, ss,
                                         flat_row_stride(H, S, sb, sh, ss),
                                         static_cast<uint8_t*>(packed_u8),
                                         static_cast<uint16_t*>(scale_f16),
                                         static_cast<uint16_t*>(zero_f16)));
  return check_launch("fade_quant_asym");
}

FADE_API int fade_dequant_asym(const void* packed_u8, const void* scale_f16, const void* zero_f16,
                               int32_t bits, int32_t group, int64_t B, int64_t H, int64_t S,
                               int64_t D, void* out_f16, void* stream) {
  int rc = check_dims("fade_dequant_asym", B, H, S, D);
  if (rc) return rc;
  const int64_t rows = B * H * S;
  if (rows == 0) return FADE_OK;
  FADE_DISPATCH_ASYM(bits, group, D,
                     hipLaunchKernelGGL((dequant_asym_kernel<BITS, LPG, LPR>),
                                         dim3(grid_for_rows(rows, LPR)), dim3(kBlock), 0,
                                         as_stream(stream), static_cast<const uint8_t*>(packed_u8),
                                         static_cast<const uint16_t*>(scale_f16),
                                         static_cast<const uint16_t*>(zero_f16), static_cast<int>(D), rows,
                                         static_cast<uint16_t*>(out_f16)));
  return check_launch("fade_dequant_asym");
}
