// Fused rotation + symmetric quantization of the rotated backend
// (fade/rotated_quant.py:106-131,148-173) for fp16 K/V with head_dim 128.
//
// x_rot = x @ R^T runs on f16 matrix cores without leaving the chip.  x is
// fp16, so it is exact as an MFMA operand; R is carried at scale 2^10 as
// R_hi = fp16(2^10 R) and R_lo = fp16(2^10 R - R_hi) (both normal for every
// entry that matters), and both products accumulate into one fp32 register:
// y = x R_hi^T + x R_lo^T = 2^10 x_rot to about 2^-22 relative, the error of
// an fp32 GEMM, not of an fp16 one.  The power-of-two scale is exact in fp32,
// so it is folded into the quantizer rather than divided out: absmax =
// 2^-10 max|y|, and y * (2^-10 inv) is the same fp32 product as x_rot * inv.
// The quantizer follows the reference's fp32 steps as quant.hip's rotated
// path does: inv = fp32(fp32(1 / max(absmax, 1e-8)) * qmax),
// code = clamp(rne(fp32(x_rot * inv))), scale = fp16(absmax / qmax).
//
// MFMA (32x32x16 f16): C^T[out channel][row] = R[out][in] x^T[in][row].
// A = 32 rows of R (hi or lo) from LDS, B = 8 input channels of one x row
// straight from HBM.  Lane l (row n = l % 32, half h = l / 32), register i of
// output tile mt holds x_rot[row n][32 mt + 8 (i / 4) + 4 h + i % 4]: four
// consecutive channels of one row per register quad, so codes pack in
// registers and go out through a small per-wave LDS stage as whole rows.
//
// Per-token scales (V): one pass; each wave takes 32-row tiles in turn.
// Per-channel scales (K): pass 1 writes the column absmax of x_rot per
// S-block, pass 2 finishes it and quantizes its S-block, recomputing x_rot
// (re-reading fp16 x costs less than an fp32 round trip through HBM).
#include "fade_common.h"

namespace fade {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kD = 128;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kRows = 32;     // rows per wave tile
constexpr int kRPitch = 136;  // halves per R row in LDS: 16-byte reads of 8 rows hit distinct banks
constexpr float kRScale = 1024.0f;         // R is carried as 2^10 R
constexpr float kRUnscale = 1.0f / 1024.0f;

template <int BITS>
struct RQ;
template <>
struct RQ<4> {
  static constexpr int lo = -8, hi = 7, row_bytes = 64;
};
template <>
struct RQ<3> {
  static constexpr int lo = -4, hi = 3, row_bytes = 128;  // raw int8, as the reference stores 3-bit
};
template <>
struct RQ<2> {
  static constexpr int lo = -2, hi = 1, row_bytes = 32;
};

// Stage rows padded by 8 bytes: the pitch (10, 18 or 34 dwords) is twice an
// odd number, so one code write of the 32 rows lands on 32 distinct banks,
// and rows stay 8-byte aligned for the flush.
template <int BITS>
struct StagePitch {
  static constexpr int value = RQ<BITS>::row_bytes + 8;
};

struct Geom {
  int64_t H, S, sb, sh, ss, fs;  // fs: uniform row stride of the flattened rows, or 0
};

struct RTile {
  uint16_t hi[kD][kRPitch];
  uint16_t lo[kD][kRPitch];
};

__device__ __forceinline__ int64_t row_off(const Geom& gm, int64_t r) {
  return gm.fs ? r * gm.fs : row_offset(r, gm.H, gm.S, gm.sb, gm.sh, gm.ss);
}

// R (fp32 [128][128], row-major, 16-byte aligned) -> R_hi / R_lo rows in LDS.
__device__ __forceinline__ void load_r(const float* __restrict__ R, RTile& rt) {
  for (int e = threadIdx.x; e < kD * kD / 4; e += kThreads) {
    const float4 v = reinterpret_cast<const float4*>(R)[e];
    const int row = e >> 5, col = (e & 31) * 4;
    const float f[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float fs = f[j] * kRScale;  // exact
      const _Float16 h = static_cast<_Float16>(fs);
      const _Float16 l = static_cast<_Float16>(fs - static_cast<float>(h));
      rt.hi[row][col + j] = __builtin_bit_cast(uint16_t, h);
      rt.lo[row][col + j] = __builtin_bit_cast(uint16_t, l);
    }
  }
}

// Input channels 16 ks + 8 h .. + 7 of the row at element offset `off` (the
// B operands).  Callers pass the last valid row for lanes past the end: a
// duplicated row changes no row's or column's absmax and is never stored.
__device__ __forceinline__ void load_x(const uint16_t* __restrict__ x, int64_t off, int h, f16x8 (&xb)[8]) {
#pragma unroll
  for (int ks = 0; ks < 8; ++ks)
    xb[ks] = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(x + off + 16 * ks + 8 * h));
}

// Output tile mt (channels 32 mt .. + 31) of 2^10 x_rot for the wave's 32 rows.
__device__ __forceinline__ f32x16 rotate_tile(const f16x8 (&xb)[8], const RTile& rt, int mt, int n, int h) {
  f32x16 acc = {};
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const f16x8 ah = *reinterpret_cast<const f16x8*>(&rt.hi[32 * mt + n][16 * ks + 8 * h]);
    const f16x8 al = *reinterpret_cast<const f16x8*>(&rt.lo[32 * mt + n][16 * ks + 8 * h]);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, xb[ks], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, xb[ks], acc, 0, 0, 0);
  }
  return acc;
}

// The same tile for two 32-row x tiles at once: each R fragment read from LDS
// feeds two MFMAs (the per-channel passes, whose registers have room for it;
// LDS reads of R then cost half the MFMA time instead of all of it).
__device__ __forceinline__ void rotate_tile2(const f16x8 (&xa)[8], const f16x8 (&xb)[8], const RTile& rt, int mt,
                                             int n, int h, f32x16& ya, f32x16& yb) {
  ya = f32x16{};
  yb = f32x16{};
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const f16x8 ah = *reinterpret_cast<const f16x8*>(&rt.hi[32 * mt + n][16 * ks + 8 * h]);
    const f16x8 al = *reinterpret_cast<const f16x8*>(&rt.lo[32 * mt + n][16 * ks + 8 * h]);
    ya = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, xa[ks], ya, 0, 0, 0);
    yb = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, xb[ks], yb, 0, 0, 0);
    ya = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, xa[ks], ya, 0, 0, 0);
    yb = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, xb[ks], yb, 0, 0, 0);
  }
}

// From the scaled absmax (2^10 max|x_rot|): the scale, and the inverse scale
// for the scaled values (2^-10 inv).
__device__ __forceinline__ float sym_inv(float absmax_scaled, float qmax, uint16_t* scale_h) {
  const float a = fmaxf(absmax_scaled * kRUnscale, 1e-8f);
  *scale_h = f2h(a / qmax);
  return ((1.0f / a) * qmax) * kRUnscale;
}

// Code of x * inv as the low bits of an fp32: clamp to [lo, hi] (integer
// bounds, so clamping before rounding equals clamping after), then adding
// 1.5 * 2^23 rounds to the nearest integer, ties to even (the add's own RNE
// at ulp 1), leaving 0x4B400000 + code in the bits: code & mask is its
// two's-complement low bits.
constexpr float kMagic = 12582912.0f;

template <int BITS>
__device__ __forceinline__ uint32_t code_bits(float x, float inv) {
  const float y = x * inv;
  const float c = __builtin_amdgcn_fmed3f(y, static_cast<float>(RQ<BITS>::lo), static_cast<float>(RQ<BITS>::hi));
  return __builtin_bit_cast(uint32_t, c + kMagic);
}

__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) { return (a & mask) | (b & ~mask); }

// Four consecutive codes (code bits t0..t3) in the row's byte layout: 4-bit
// two bytes, high nibble = even channel; 2-bit one byte, first code in bits
// 7:6; 3-bit four raw int8 bytes.
template <int BITS>
__device__ __forceinline__ uint32_t pack4(uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  if (BITS == 4) {
    const uint32_t b0 = bfi(0xFu, t1, t0 << 4), b1 = bfi(0xFu, t3, t2 << 4);
    return __builtin_amdgcn_perm(b1, b0, 0x0C0C0400u);
  }
  if (BITS == 2) {
    uint32_t b = bfi(0x3u, t3, t2 << 2);
    b = bfi(0xFu, b, t1 << 4);
    return bfi(0x3Fu, b, t0 << 6);
  }
  const uint32_t lo = __builtin_amdgcn_perm(t1, t0, 0x0C0C0400u), hi = __builtin_amdgcn_perm(t3, t2, 0x0C0C0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// Codes of tile mt into the wave's stage (row n).  inv[i * inv_step] is the
// inverse scale of register i's channel (inv_step 0: one per row).
template <int BITS>
__device__ __forceinline__ void stage_codes(const f32x16& xr, int mt, int n, int h, const float* inv,
                                            int inv_step, uint8_t* stage) {
  constexpr int RB = RQ<BITS>::row_bytes;
  constexpr int PB = RB / 32;  // bytes per four codes
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float* iv = inv + q * 4 * inv_step;
    const uint32_t w = pack4<BITS>(code_bits<BITS>(xr[4 * q + 0], iv[0]), code_bits<BITS>(xr[4 * q + 1], iv[inv_step]),
                                   code_bits<BITS>(xr[4 * q + 2], iv[2 * inv_step]),
                                   code_bits<BITS>(xr[4 * q + 3], iv[3 * inv_step]));
    uint8_t* dst = stage + n * StagePitch<BITS>::value + ((32 * mt + 8 * q + 4 * h) / 4) * PB;
    if (PB == 1) *dst = static_cast<uint8_t>(w);
    else if (PB == 2) *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(w);
    else *reinterpret_cast<uint32_t*>(dst) = w;
  }
}

// The stage's rows row0 .. row0 + 31 (those below `rows`) out to packed rows,
// 8 bytes per lane and step: consecutive lanes write consecutive bytes.
template <int BITS>
__device__ __forceinline__ void flush_stage(const uint8_t* stage, uint8_t* __restrict__ packed, int64_t row0,
                                            int64_t rows, int lane) {
  constexpr int RB = RQ<BITS>::row_bytes;
  constexpr int kChunks = kRows * RB / 8;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int k = lane; k < kChunks; k += 64) {
    const int rr = k / (RB / 8), cc = k % (RB / 8);
    if (row0 + rr < rows)
      *reinterpret_cast<uint2*>(packed + (row0 + rr) * RB + 8 * cc) =
          *reinterpret_cast<const uint2*>(stage + rr * StagePitch<BITS>::value + 8 * cc);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Per-token scales: the waves of the grid take 32-row tiles of the flattened
// [B*H*S] rows in turn; the next tile's x is in flight during this one.
template <int BITS>
__global__ __launch_bounds__(kThreads) void rotq_token_kernel(const uint16_t* __restrict__ x, Geom gm, int64_t rows,
                                                              const float* __restrict__ R,
                                                              uint8_t* __restrict__ packed,
                                                              uint16_t* __restrict__ scale) {
  constexpr float QMAX = static_cast<float>(RQ<BITS>::hi);
  __shared__ __attribute__((aligned(16))) RTile rt;
  __shared__ __attribute__((aligned(16))) uint8_t stage[kWaves][kRows * StagePitch<BITS>::value];
  load_r(R, rt);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 31, h = lane >> 5;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kWaves * kRows;
  int64_t r0 = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * kRows;
  const int64_t last = rows - 1;
  f16x8 xb[8];
  load_x(x, row_off(gm, r0 + n < rows ? r0 + n : last), h, xb);
  for (; r0 < rows; r0 += step) {
    __asm__ volatile("" ::: "memory");  // keep the R fragment reads inside the loop
    f16x8 cur[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) cur[ks] = xb[ks];
    const int64_t nx = r0 + step + n;
    load_x(x, row_off(gm, nx < rows ? nx : last), h, xb);
    f32x16 xr[4];
    float a = 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      xr[mt] = rotate_tile(cur, rt, mt, n, h);
#pragma unroll
      for (int i = 0; i < 16; ++i) a = fmaxf(a, fabsf(xr[mt][i]));
    }
    a = fmaxf(a, __shfl_xor(a, 32, 64));  // row n's absmax
    uint16_t sc;
    const float inv = sym_inv(a, QMAX, &sc);
    if (h == 0 && r0 + n < rows) scale[r0 + n] = sc;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) stage_codes<BITS>(xr[mt], mt, n, h, &inv, 0, &stage[wave][0]);
    flush_stage<BITS>(&stage[wave][0], packed, r0, rows, lane);
  }
}

// Per-channel pass 1: column absmax of 2^10 x_rot over S-block blockIdx.x of (b, h) = blockIdx.y.
__global__ __launch_bounds__(kThreads) void rotq_colmax_kernel(const uint16_t* __restrict__ x, Geom gm,
                                                               int64_t rows_per_block, const float* __restrict__ R,
                                                               float* __restrict__ partial) {
  __shared__ __attribute__((aligned(16))) RTile rt;
  __shared__ float red[kWaves][kD];
  load_r(R, rt);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 31, h = lane >> 5;
  const int64_t bh = blockIdx.y;
  const int64_t s0 = static_cast<int64_t>(blockIdx.x) * rows_per_block;
  const int64_t s1 = s0 + rows_per_block < gm.S ? s0 + rows_per_block : gm.S;
  const uint16_t* base = x + (bh / gm.H) * gm.sb + (bh % gm.H) * gm.sh;
  f32x16 m[4] = {};
  // each wave takes two 32-row tiles per step (rows past the block: its last
  // row again, which changes no column's absmax)
  constexpr int64_t kStep = 2 * kRows * kWaves;
  int64_t t0 = s0 + 2 * kRows * wave;
  auto rowc = [&](int64_t r) { return (r < s1 ? r : s1 - 1) * gm.ss; };
  f16x8 xa[8], xb[8];
  load_x(base, rowc(t0 + n), h, xa);
  load_x(base, rowc(t0 + kRows + n), h, xb);
  for (; t0 < s1; t0 += kStep) {
    __asm__ volatile("" ::: "memory");  // keep the R fragment reads inside the loop
    f16x8 ca[8], cb[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      ca[ks] = xa[ks];
      cb[ks] = xb[ks];
    }
    load_x(base, rowc(t0 + kStep + n), h, xa);
    load_x(base, rowc(t0 + kStep + kRows + n), h, xb);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      f32x16 ya, yb;
      rotate_tile2(ca, cb, rt, mt, n, h, ya, yb);
#pragma unroll
      for (int i = 0; i < 16; ++i) m[mt][i] = fmaxf(m[mt][i], fmaxf(fabsf(ya[i]), fabsf(yb[i])));
    }
  }
  // over the wave's 32 rows (lanes n), then over the waves
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float v = group_max<32>(m[mt][i]);
      if (n == 0) red[wave][32 * mt + 8 * (i / 4) + 4 * h + i % 4] = v;
    }
  __syncthreads();
  for (int d = threadIdx.x; d < kD; d += kThreads) {
    float v = red[0][d];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) v = fmaxf(v, red[w][d]);
    partial[(bh * gridDim.x + blockIdx.x) * kD + d] = v;
  }
}

// Per-channel pass 2: finish the absmax, emit the scales, quantize this S-block.
template <int BITS>
__global__ __launch_bounds__(kThreads) void rotq_channel_kernel(const uint16_t* __restrict__ x, Geom gm,
                                                                int64_t rows_per_block, const float* __restrict__ R,
                                                                const float* __restrict__ partial,
                                                                uint8_t* __restrict__ packed,
                                                                uint16_t* __restrict__ scale) {
  constexpr float QMAX = static_cast<float>(RQ<BITS>::hi);
  constexpr int RB = RQ<BITS>::row_bytes;
  __shared__ __attribute__((aligned(16))) RTile rt;
  __shared__ __attribute__((aligned(16))) uint8_t stage[kWaves][2 * kRows * StagePitch<BITS>::value];
  __shared__ float inv_s[kD];
  load_r(R, rt);
  const int64_t bh = blockIdx.y;
  const int nsb = gridDim.x;
  for (int d = threadIdx.x; d < kD; d += kThreads) {
    float a = 0.0f;
    for (int k = 0; k < nsb; ++k) a = fmaxf(a, partial[(bh * nsb + k) * kD + d]);
    uint16_t sc;
    inv_s[d] = sym_inv(a, QMAX, &sc);
    if (blockIdx.x == 0) scale[bh * kD + d] = sc;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 31, h = lane >> 5;
  const int64_t s0 = static_cast<int64_t>(blockIdx.x) * rows_per_block;
  const int64_t s1 = s0 + rows_per_block < gm.S ? s0 + rows_per_block : gm.S;
  const uint16_t* base = x + (bh / gm.H) * gm.sb + (bh % gm.H) * gm.sh;
  uint8_t* out = packed + bh * gm.S * RB;
  float inv[4][16];  // this lane's channels' inverse scales, fixed for the block
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) inv[mt][i] = inv_s[32 * mt + 8 * (i / 4) + 4 * h + i % 4];
  // two 32-row tiles per step, as in pass 1 (rows past the block are computed
  // from its last row and never stored)
  constexpr int64_t kStep = 2 * kRows * kWaves;
  constexpr int kHalf = kRows * StagePitch<BITS>::value;  // stage bytes of one 32-row tile
  int64_t t0 = s0 + 2 * kRows * wave;
  auto rowc = [&](int64_t r) { return (r < s1 ? r : s1 - 1) * gm.ss; };
  f16x8 xa[8], xb[8];
  load_x(base, rowc(t0 + n), h, xa);
  load_x(base, rowc(t0 + kRows + n), h, xb);
  for (; t0 < s1; t0 += kStep) {
    __asm__ volatile("" ::: "memory");  // keep the R fragment reads inside the loop
    f16x8 ca[8], cb[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      ca[ks] = xa[ks];
      cb[ks] = xb[ks];
    }
    load_x(base, rowc(t0 + kStep + n), h, xa);
    load_x(base, rowc(t0 + kStep + kRows + n), h, xb);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      f32x16 ya, yb;
      rotate_tile2(ca, cb, rt, mt, n, h, ya, yb);
      stage_codes<BITS>(ya, mt, n, h, inv[mt], 1, &stage[wave][0]);
      stage_codes<BITS>(yb, mt, n, h, inv[mt], 1, &stage[wave][kHalf]);
    }
    flush_stage<BITS>(&stage[wave][0], out, t0, s1, lane);
    flush_stage<BITS>(&stage[wave][kHalf], out, t0 + kRows, s1, lane);
  }
}

int num_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// S-blocking of the per-channel passes: about one block per CU in all (a
// block holds most of a CU's LDS), at least 256 rows per block.
void rotq_blocking(int64_t BH, int64_t S, int64_t* nsb, int64_t* rows_per_block) {
  int64_t n = BH > 0 ? cdiv(num_cus(), BH) : 1;
  const int64_t by_rows = cdiv(S, 256);
  if (n > by_rows) n = by_rows;
  if (n < 1) n = 1;
  *rows_per_block = cdiv(cdiv(S, n), kRows) * kRows;
  *nsb = S > 0 ? cdiv(S, *rows_per_block) : 1;
}

int check(const char* fn, int64_t B, int64_t H, int64_t S, int64_t D, int32_t bits, int32_t axis) {
  if (B < 0 || H < 0 || S < 0) return einval("%s: negative dimension", fn);
  if (D != kD) return einval("%s: head_dim must be %d, got %lld", fn, kD, (long long)D);
  if (bits != 2 && bits != 3 && bits != 4) return einval("%s: bits must be 2, 3 or 4, got %d", fn, bits);
  if (axis != FADE_AXIS_TOKEN && axis != FADE_AXIS_CHANNEL) return einval("%s: bad axis %d", fn, axis);
  if (B * H > 65535) return einval("%s: B*H must be at most 65535", fn);
  return FADE_OK;
}

}  // namespace
}  // namespace fade

using namespace fade;

FADE_API int fade_rotate_quant_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D, int32_t axis,
                                               int64_t* bytes) {
  if (bytes == nullptr) return einval("fade_rotate_quant_workspace_bytes: null output");
  const int rc = check("fade_rotate_quant_workspace_bytes", B, H, S, D, 4, axis);
  if (rc) return rc;
  *bytes = 0;
  if (axis == FADE_AXIS_CHANNEL && B * H * S > 0) {
    int64_t nsb, rpb;
    rotq_blocking(B * H, S, &nsb, &rpb);
    *bytes = B * H * nsb * kD * static_cast<int64_t>(sizeof(float));
  }
  return FADE_OK;
}

FADE_API int fade_rotate_quant(const void* x_f16, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                               int64_t sh, int64_t ss, const float* R, int32_t bits, int32_t axis, void* packed,
                               void* scale_f16, void* workspace, int64_t workspace_bytes, void* stream) {
  const char* fn = "fade_rotate_quant";
  int rc = check(fn, B, H, S, D, bits, axis);
  if (rc) return rc;
  const int64_t rows = B * H * S;
  if (rows == 0) return FADE_OK;
  if (x_f16 == nullptr || R == nullptr || packed == nullptr || scale_f16 == nullptr)
    return einval("%s: null pointer", fn);
  if ((reinterpret_cast<uintptr_t>(x_f16) & 15) || (sb % 8) || (sh % 8) || (ss % 8) ||
      (reinterpret_cast<uintptr_t>(packed) & 15) || (reinterpret_cast<uintptr_t>(R) & 15))
    return einval("%s: x (rows), R and packed must be 16-byte aligned", fn);
  const Geom gm{H, S, sb, sh, ss, (sh == S * ss && sb == H * sh) ? ss : 0};
  const uint16_t* x = static_cast<const uint16_t*>(x_f16);
  uint8_t* pk = static_cast<uint8_t*>(packed);
  uint16_t* sc = static_cast<uint16_t*>(scale_f16);
  hipStream_t st = as_stream(stream);
  if (axis == FADE_AXIS_TOKEN) {
    const int64_t want = cdiv(rows, static_cast<int64_t>(kRows) * kWaves);
    const int64_t cap = num_cus();
    const dim3 grid(static_cast<unsigned>(want < cap ? want : cap));
    switch (bits) {
      case 4: hipLaunchKernelGGL(rotq_token_kernel<4>, grid, dim3(kThreads), 0, st, x, gm, rows, R, pk, sc); break;
      case 3: hipLaunchKernelGGL(rotq_token_kernel<3>, grid, dim3(kThreads), 0, st, x, gm, rows, R, pk, sc); break;
      default: hipLaunchKernelGGL(rotq_token_kernel<2>, grid, dim3(kThreads), 0, st, x, gm, rows, R, pk, sc); break;
    }
    return check_launch(fn);
  }
  int64_t nsb, rpb;
  rotq_blocking(B * H, S, &nsb, &rpb);
  const int64_t need = B * H * nsb * kD * static_cast<int64_t>(sizeof(float));
  if (workspace == nullptr || workspace_bytes < need)
    return einval("%s: workspace too small (%lld < %lld bytes)", fn, (long long)workspace_bytes, (long long)need);
  float* partial = static_cast<float*>(workspace);
  const dim3 grid(static_cast<unsigned>(nsb), static_cast<unsigned>(B * H));
  hipLaunchKernelGGL(rotq_colmax_kernel, grid, dim3(kThreads), 0, st, x, gm, rpb, R, partial);
  rc = check_launch(fn);
  if (rc) return rc;
  switch (bits) {
    case 4: hipLaunchKernelGGL(rotq_channel_kernel<4>, grid, dim3(kThreads), 0, st, x, gm, rpb, R, partial, pk, sc); break;
    case 3: hipLaunchKernelGGL(rotq_channel_kernel<3>, grid, dim3(kThreads), 0, st, x, gm, rpb, R, partial, pk, sc); break;
    default: hipLaunchKernelGGL(rotq_channel_kernel<2>, grid, dim3(kThreads), 0, st, x, gm, rpb, R, partial, pk, sc); break;
  }
  return check_launch(fn);
}
