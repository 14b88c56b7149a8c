// Tiered decode attention: one query token per (batch, query head) against
// the cache laid out as  sink (fp16) | middle (packed codes) | recent (fp16),
// without materializing fp16 K/V (the reference dequantizes and torch.cat's
// the whole cache every step: fade/cache.py:683-842).
//
// Work split (flash-decoding): one workgroup per (split of the token range,
// kv head, batch row) serves the whole GQA group of Hq/Hkv query heads, so
// each KV byte is read once.  Each workgroup writes an unnormalized partial
// (m, l, acc[D]) in the log2 domain; decode_combine_kernel merges the splits.
// Head dims: any multiple of 8 up to 256 (the matrix-core kernels take 128 only).
//
// This file holds the portable VALU kernel (any middle format) and the
// combine pass.  decode_mfma.hip holds the matrix-core kernel for the
// packed symmetric formats.
#include <math.h>

#include "decode_common.h"

namespace fade {
namespace decode {
namespace {

constexpr int kTile = 64;
constexpr int kThreads = 256;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// fp32 += a.x * b.x + a.y * b.y over 16-bit pairs of the instance's dtype
// (BF: bfloat16, else fp16), products and sum in fp32.
template <bool BF>
__device__ __forceinline__ float dot2w(uint32_t a, uint32_t b, float c) {
  if constexpr (BF) return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
  else return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

// Eight consecutive fp16 values (channels 8 cg .. 8 cg + 7) of a row, with a
// 16-byte load where the address allows it.
__device__ __forceinline__ uint4 load8h(const uint16_t* src) {
  if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) return *reinterpret_cast<const uint4*>(src);
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = static_cast<uint32_t>(src[2 * j]) | (static_cast<uint32_t>(src[2 * j + 1]) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Eight fp32 values rounded to the instance's 16-bit dtype (nearest even).
template <bool BF>
__device__ __forceinline__ uint4 pack8h(const float* x) {
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = static_cast<uint32_t>(f2w<BF>(x[2 * j])) | (static_cast<uint32_t>(f2w<BF>(x[2 * j + 1])) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// One staging unit (channels 8 cg .. 8 cg + 7 of one token's K or V) as loaded
// from HBM, before dequantization: fp16 tiers: the eight values; packed
// middle tiers: x = codes (first code in the high bits; the reference INT4
// format: the dword as stored, first code in bits 4..7), y = per-token scale
// (low half) and zero (high half) where the format has them; literal INT2 V:
// x, y = the eight int8 codes.
struct RawUnit {
  uint4 w;
};

// Where unit (token t, group cg) lives: seg 0 sink, 1 middle, 2 recent; r = row in the tier.
struct UnitRef {
  int seg;
  int64_t r;
};
__device__ __forceinline__ UnitRef unit_ref(int64_t t, int64_t ns, int64_t nm) {
  if (t < ns) return {0, t};
  if (t < ns + nm) return {1, t - ns};
  return {2, t - ns - nm};
}

// SYM44: the middle tier is the reference INT4 format (FADE_MID_SYM, 4-bit K
// and V), known at compile time.  Rows are p.D channels long.
template <bool IS_V, bool SYM44>
__device__ __forceinline__ RawUnit load_unit(const Params& p, int64_t b, int64_t kvh, UnitRef u, int cg) {
  const int d0 = 8 * cg;
  const int D = p.D;
  RawUnit ru;
  if (u.seg != 1) {
    const Fp16Tier& seg = u.seg == 0 ? p.sink : p.recent;
    const uint16_t* src = IS_V ? seg.v + b * seg.v_sb + kvh * seg.v_sh + u.r * seg.v_ss
                               : seg.k + b * seg.k_sb + kvh * seg.k_sh + u.r * seg.k_ss;
    ru.w = load8h(src + d0);
    return ru;
  }
  const int64_t m = u.r;
  const int64_t bkv = b * p.Hkv + kvh;
  const int64_t row = bkv * p.mid.len + m;
  const int fmt = SYM44 ? FADE_MID_SYM : p.mid.fmt;
  if (fmt == FADE_MID_FP16) {
    const uint8_t* base = IS_V ? p.mid.v_codes : p.mid.k_codes;
    ru.w = load8h(reinterpret_cast<const uint16_t*>(base) + row * D + d0);
    return ru;
  }
  ru.w = make_uint4(0, 0, 0, 0);
  if (IS_V && fmt == FADE_MID_K4V2G) {  // eight int8 codes
    const uint8_t* src = p.mid.v_codes + (bkv * p.mid.v_rows + m) * D + d0;
    if ((reinterpret_cast<uintptr_t>(src) & 7) == 0) {
      const uint2 c8 = *reinterpret_cast<const uint2*>(src);
      ru.w.x = c8.x;
      ru.w.y = c8.y;
    } else {
      for (int j = 0; j < 4; ++j) {
        ru.w.x |= static_cast<uint32_t>(src[j]) << (8 * j);
        ru.w.y |= static_cast<uint32_t>(src[4 + j]) << (8 * j);
      }
    }
    return ru;
  }
  const int bits = SYM44 || fmt == FADE_MID_K4V2G ? 4 : (IS_V ? p.mid.v_bits : p.mid.k_bits);
  const uint8_t* src = (IS_V ? p.mid.v_codes : p.mid.k_codes) + row * (D * bits / 8);
  if (SYM44) {  // the dword as stored (sym4_to_f16 takes it so)
    const uint8_t* c = src + 4 * cg;
    if ((reinterpret_cast<uintptr_t>(c) & 3) == 0)
      ru.w.x = *reinterpret_cast<const uint32_t*>(c);
    else
      ru.w.x = static_cast<uint32_t>(c[0]) | (static_cast<uint32_t>(c[1]) << 8) |
               (static_cast<uint32_t>(c[2]) << 16) | (static_cast<uint32_t>(c[3]) << 24);
  } else if (bits == 4) {
    const uint8_t* c = src + 4 * cg;
    if ((reinterpret_cast<uintptr_t>(c) & 3) == 0)
      ru.w.x = __builtin_bswap32(*reinterpret_cast<const uint32_t*>(c));
    else
      ru.w.x = (static_cast<uint32_t>(c[0]) << 24) | (static_cast<uint32_t>(c[1]) << 16) |
               (static_cast<uint32_t>(c[2]) << 8) | static_cast<uint32_t>(c[3]);
  } else {
    const uint8_t* c = src + 2 * cg;
    if ((reinterpret_cast<uintptr_t>(c) & 1) == 0)
      ru.w.x = static_cast<uint32_t>(__builtin_bswap16(*reinterpret_cast<const uint16_t*>(c))) << 16;
    else
      ru.w.x = (static_cast<uint32_t>(c[0]) << 24) | (static_cast<uint32_t>(c[1]) << 16);
  }
  if (fmt == FADE_MID_ASYM) {
    const int g = p.mid.group;  // >= 16: one group holds the unit's eight channels
    const uint16_t* sc = IS_V ? p.mid.v_scale : p.mid.k_scale;
    const uint16_t* zp = IS_V ? p.mid.v_zero : p.mid.k_zero;
    ru.w.y = static_cast<uint32_t>(sc[row * (D / g) + d0 / g]) | (static_cast<uint32_t>(zp[row * (D / g) + d0 / g]) << 16);
  } else if (IS_V) {
    ru.w.y = p.mid.v_scale[row];
  }
  return ru;
}

// Eight two's-complement nibbles (one dword as stored: byte k holds channel
// 2k in its high and 2k + 1 in its low nibble) -> fp16(c * scale) of the
// eight channels in order, dword k = channels (2k, 2k + 1).  Each nibble goes
// to mantissa bits 4..7 of 64.0 (one code step = 1.0) with its top bit
// flipped, i.e. the fp16 value 72 + c, exact; then - 72 and one packed fp16
// multiply, whose single rounding equals the reference's fp16(code * scale).
// s2: the scales of the four channel pairs (for V one scale twice).
__device__ __forceinline__ uint4 sym4_to_f16(uint32_t w, const uint32_t (&s2)[4]) {
  const uint32_t o0 = ((w << 4) & 0x00F000F0u) ^ 0x54805480u;  // channels (1, 5)
  const uint32_t o1 = (w & 0x00F000F0u) ^ 0x54805480u;         // (0, 4)
  const uint32_t o2 = ((w >> 4) & 0x00F000F0u) ^ 0x54805480u;  // (3, 7)
  const uint32_t o3 = ((w >> 8) & 0x00F000F0u) ^ 0x54805480u;  // (2, 6)
  const uint32_t n[4] = {__builtin_amdgcn_perm(o0, o1, 0x05040100u), __builtin_amdgcn_perm(o2, o3, 0x05040100u),
                         __builtin_amdgcn_perm(o0, o1, 0x07060302u), __builtin_amdgcn_perm(o2, o3, 0x07060302u)};
  const f16x2 m72 = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
  uint32_t x[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    x[k] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, n[k]) + m72) * __builtin_bit_cast(f16x2, s2[k]));
  return make_uint4(x[0], x[1], x[2], x[3]);
}

// A loaded unit dequantized as the reference does (fp16(code * scale),
// fp16(code * scale + zero) for the asymmetric format; bf16(code * scale) in
// a bfloat16 instance): eight values of the instance's dtype.
// ks_s: the row's per-channel K scales (fp32); ks2_s: the same as fp16 pairs.
template <bool IS_V, bool SYM44, bool BF>
__device__ __forceinline__ uint4 convert_unit(const Params& p, int64_t b, int64_t kvh, UnitRef u, int cg,
                                              const RawUnit& ru, const float* ks_s, const uint32_t* ks2_s) {
  const int fmt = SYM44 ? FADE_MID_SYM : p.mid.fmt;
  if (u.seg != 1 || fmt == FADE_MID_FP16) return ru.w;
  const int d0 = 8 * cg;
  const int D = p.D;
  if (SYM44) {
    uint32_t s2[4];
    if (IS_V) {
      const uint32_t sv = ru.w.y & 0xFFFFu;
#pragma unroll
      for (int k = 0; k < 4; ++k) s2[k] = sv | (sv << 16);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) s2[k] = ks2_s[d0 / 2 + k];
    }
    return sym4_to_f16(ru.w.x, s2);
  }
  float x[8];
  if (IS_V && fmt == FADE_MID_K4V2G) {  // literal grouped INT2 V: per-(group, channel) scales
    const int64_t bkv = b * p.Hkv + kvh;
    const int64_t Gr = p.mid.v_rows / p.mid.group;
    const uint4 sc = load8h(p.mid.v_scale + (bkv * Gr + u.r / p.mid.group) * D + d0);
    const uint32_t sw[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int8_t c = static_cast<int8_t>(((j < 4 ? ru.w.x : ru.w.y) >> (8 * (j & 3))) & 0xFF);
      x[j] = static_cast<float>(c) * w2f<BF>(static_cast<uint16_t>(sw[j >> 1] >> (16 * (j & 1))));
    }
    return pack8h<BF>(x);
  }
  const int bits = SYM44 || fmt == FADE_MID_K4V2G ? 4 : (IS_V ? p.mid.v_bits : p.mid.k_bits);
  int c[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (bits == 4)
      c[j] = static_cast<int>((ru.w.x >> (28 - 4 * j)) & 0xF);
    else
      c[j] = static_cast<int>((ru.w.x >> (30 - 2 * j)) & 0x3);
  }
  if (fmt == FADE_MID_ASYM) {
    const float s = h2f(static_cast<uint16_t>(ru.w.y & 0xFFFFu));
    const float z = h2f(static_cast<uint16_t>(ru.w.y >> 16));
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = static_cast<float>(c[j]) * s + z;
    return pack8h<BF>(x);
  }
  // symmetric: two's complement codes
  const int sgn = bits == 4 ? 8 : 2;
#pragma unroll
  for (int j = 0; j < 8; ++j) c[j] -= (c[j] & sgn) << 1;
  if (IS_V) {
    const float s = w2f<BF>(static_cast<uint16_t>(ru.w.y & 0xFFFFu));
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = static_cast<float>(c[j]) * s;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = static_cast<float>(c[j]) * ks_s[d0 + j];
  }
  return pack8h<BF>(x);
}

// Max over the 64 lanes of a wave (all lanes active): DPP exchanges within
// each row of 16 lanes (lane ^ 1, lane ^ 2, rotations by 4 and 8), then the
// four row maxima read as scalars.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_max64(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = fmaxf(v, dpp_f<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp_f<0x128>(v));  // row_ror:8
  const int iv = __builtin_bit_cast(int, v);
  return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16))),
               fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48))));
}

// Portable kernel, head_dim p.D (a multiple of 8 up to the instance's capacity
// DP = 32, 64, 128 or 256; the 8-channel units past p.D stage zeros and emit
// nothing), up to HP query heads per kv head (4 or 8), any middle format.
// Per tile of 64 tokens:
//   stage: all threads dequantize the tile's K and V into LDS (fp16, the
//          reference's rounding), one (token pair, 8-channel group) unit per
//          thread and step, coalesced global loads; K rows as they are, V as
//          dwords of one channel of two consecutive tokens;
//   QK:    thread (token = lane, heads wave and wave + 4) dots the K row with
//          the fp16 query (v_dot2_f32_f16: fp16 pairs, fp32 sums), then the
//          wave's online softmax in the log2 domain; the probabilities are
//          kept in fp16 for PV (as the matrix-core kernels do), the row sums
//          in fp32;
//   PV:    thread (head, 8-channel group, token slice) accumulates P V over its
//          slice of the tile's tokens, one v_dot2_f32_f16 per channel and
//          token pair; the slices are summed once per split.
// The split's partial (m, l, acc) goes to the workspace and
// decode_combine_kernel merges the splits; with one split the kernel writes
// the output directly.  (Merging in the last workgroup to finish, as the
// matrix-core kernel does, measured slower here: these workgroups are short,
// and each then waits for its partial stores and a counter round trip.)
// BF: every 16-bit float of the call is bfloat16 (SYM44, a packed fp16
// dequantization, has no bfloat16 instance).
template <int DP, int HP, bool SYM44, bool BF>
__global__ __launch_bounds__(kThreads) void decode_valu_kernel(Params p) {
  static_assert(!(SYM44 && BF), "the SYM44 fast path dequantizes in fp16");
  constexpr int CG = DP / 8;                // 8-channel units per row (capacity)
  constexpr int KP = DP + 8;                // K row pitch in LDS (halves)
  constexpr int VPP = DP + 4;               // V token-pair row pitch in LDS (dwords)
  constexpr int NU = HP * CG;               // (head, unit) outputs
  constexpr int TQ = kThreads / NU;         // token slices per output
  constexpr int TPS = kTile / TQ;           // tokens per slice
  constexpr int HPW = HP / 4;               // heads per wave in QK
  static_assert(TQ >= 1 && kThreads % NU == 0 && TPS % 2 == 0, "PV decomposition");
  const int split = blockIdx.x;
  const int64_t kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = p.G;
  const int D = p.D;  // the row's channels (<= DP)

  __shared__ __attribute__((aligned(16))) uint32_t q2_s[HP][DP / 2];  // fp16 query pairs (0 past D)
  __shared__ float ks_s[DP];
  __shared__ uint32_t ks2_s[SYM44 ? DP / 2 : 1];
  __shared__ __attribute__((aligned(16))) uint16_t kt[kTile][KP];
  __shared__ __attribute__((aligned(16))) uint32_t vp[kTile / 2][VPP];  // (token 2i, 2i + 1) of one channel
  __shared__ __attribute__((aligned(4))) uint16_t ph_s[HP][kTile];     // fp16 probabilities
  __shared__ float alpha_s[HP];
  __shared__ __attribute__((aligned(16))) float red[TQ > 1 ? TQ : 1][NU][8];

  for (int i = tid; i < HP * DP / 2; i += kThreads) {
    const int h = i / (DP / 2), d = 2 * (i % (DP / 2));
    const uint16_t* qr = p.q + b * p.q_sb + (kvh * G + h) * p.q_sh + d;
    q2_s[h][d / 2] = h < G && d < D ? static_cast<uint32_t>(qr[0]) | (static_cast<uint32_t>(qr[1]) << 16) : 0u;
  }
  if (p.mid.fmt == FADE_MID_SYM || p.mid.fmt == FADE_MID_K4V2G)
    for (int d = tid; d < DP; d += kThreads) ks_s[d] = d < D ? w2f<BF>(p.mid.k_scale[(b * p.Hkv + kvh) * D + d]) : 0.0f;
  if (SYM44)
    for (int d = tid; d < DP / 2; d += kThreads) {
      const uint16_t* ks = p.mid.k_scale + (b * p.Hkv + kvh) * D + 2 * d;
      ks2_s[d] = 2 * d < D ? static_cast<uint32_t>(ks[0]) | (static_cast<uint32_t>(ks[1]) << 16) : 0u;
    }
  if (tid < HP) alpha_s[tid] = 1.0f;

  // the row's tier lengths: the tiers' own, or per row (lens, clamped to the padded tiers)
  int64_t ns = p.sink.len, nm = p.mid.len, nr = p.recent.len;
  if (p.lens != nullptr) {
    auto clampl = [](int64_t x, int64_t cap) { return x < 0 ? 0 : (x > cap ? cap : x); };
    ns = clampl(p.lens[3 * b], p.sink.len);
    nm = clampl(p.lens[3 * b + 1], p.mid.len);
    nr = clampl(p.lens[3 * b + 2], p.recent.len);
  }
  const int64_t total = ns + nm + nr;
  const int64_t t_begin = static_cast<int64_t>(split) * p.tokens_per_split;
  const int64_t t_end = t_begin + p.tokens_per_split < total ? t_begin + p.tokens_per_split : total;

  float m_run[HPW], l_lane[HPW];
#pragma unroll
  for (int i = 0; i < HPW; ++i) {
    m_run[i] = -INFINITY;
    l_lane[i] = 0.0f;
  }
  // PV: output (head ph, unit pc), token slice pq
  const int po = tid % NU, pq = tid / NU;
  const int ph = po / CG, pc = po % CG;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0f;

  // Staging: thread tid owns units tid + kThreads * i (tokens 2 (u / CG) and
  // 2 (u / CG) + 1, group u % CG) of every tile: all loads of the tile are
  // issued, then dequantized into LDS.  (Loading the next tile's units during
  // this tile's compute measured no faster.)
  constexpr int NPU = kTile / 2 * CG;
  constexpr int PPT = (NPU + kThreads - 1) / kThreads;
  RawUnit rk[PPT][2], rv[PPT][2];
  auto load_tile = [&](int64_t ts, int nv) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int uidx = tid + kThreads * i;
      const int rp = uidx / CG, cg = uidx % CG;
#pragma unroll
      for (int e = 0; e < 2; ++e)
        if (uidx < NPU && 2 * rp + e < nv && 8 * cg < D) {
          const UnitRef ur = unit_ref(ts + 2 * rp + e, ns, nm);
          rk[i][e] = load_unit<false, SYM44>(p, b, kvh, ur, cg);
          rv[i][e] = load_unit<true, SYM44>(p, b, kvh, ur, cg);
        }
    }
  };
  auto store_tile = [&](int64_t ts, int nv) {  // tokens past nv as zeros
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int uidx = tid + kThreads * i;
      const int rp = uidx / CG, cg = uidx % CG;
      if (uidx < NPU) {
        uint32_t vw[2][4];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int r = 2 * rp + e;
          uint4 kw = make_uint4(0, 0, 0, 0), v = make_uint4(0, 0, 0, 0);
          if (r < nv && 8 * cg < D) {
            const UnitRef ur = unit_ref(ts + r, ns, nm);
            kw = convert_unit<false, SYM44, BF>(p, b, kvh, ur, cg, rk[i][e], ks_s, ks2_s);
            v = convert_unit<true, SYM44, BF>(p, b, kvh, ur, cg, rv[i][e], ks_s, ks2_s);
          }
          *reinterpret_cast<uint4*>(&kt[r][8 * cg]) = kw;
          vw[e][0] = v.x;
          vw[e][1] = v.y;
          vw[e][2] = v.z;
          vw[e][3] = v.w;
        }
        // channel 2k: the low halves of dword k of both tokens; 2k + 1: the high halves
        uint32_t pr[8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          pr[2 * k] = __builtin_amdgcn_perm(vw[1][k], vw[0][k], 0x05040100u);
          pr[2 * k + 1] = __builtin_amdgcn_perm(vw[1][k], vw[0][k], 0x07060302u);
        }
        *reinterpret_cast<uint4*>(&vp[rp][8 * cg]) = make_uint4(pr[0], pr[1], pr[2], pr[3]);
        *reinterpret_cast<uint4*>(&vp[rp][8 * cg + 4]) = make_uint4(pr[4], pr[5], pr[6], pr[7]);
      }
    }
  };
  auto tile_len = [&](int64_t ts) { return static_cast<int>(t_end - ts < kTile ? t_end - ts : kTile); };
  __syncthreads();  // q_s, ks_s

  for (int64_t ts = t_begin; ts < t_end; ts += kTile) {
    const int nv = tile_len(ts);
    load_tile(ts, nv);
    store_tile(ts, nv);
    __syncthreads();
    // ---- QK and the online softmax: heads wave (+ 4) of token lane ----
    {
      float s[HPW];
#pragma unroll
      for (int i = 0; i < HPW; ++i) s[i] = 0.0f;
#pragma unroll 4
      for (int cg = 0; cg < CG; ++cg) {
        const uint4 kw = *reinterpret_cast<const uint4*>(&kt[lane][8 * cg]);
        const uint32_t k2[4] = {kw.x, kw.y, kw.z, kw.w};
#pragma unroll
        for (int i = 0; i < HPW; ++i) {
          const uint4 qw = *reinterpret_cast<const uint4*>(&q2_s[wave + 4 * i][4 * cg]);
          const uint32_t q2[4] = {qw.x, qw.y, qw.z, qw.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) s[i] = dot2w<BF>(k2[j], q2[j], s[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < HPW; ++i) s[i] *= p.scale_log2;  // log2 domain
#pragma unroll
      for (int i = 0; i < HPW; ++i) {
        const int h = wave + 4 * i;
        if (h < G) {
          const float sc = lane < nv ? s[i] : -INFINITY;
          const float m_new = fmaxf(m_run[i], wave_max64(sc));
          float alpha = 1.0f, pv = 0.0f;
          if (m_new != -INFINITY) {
            alpha = __builtin_amdgcn_exp2f(m_run[i] - m_new);
            pv = __builtin_amdgcn_exp2f(sc - m_new);
          }
          l_lane[i] = l_lane[i] * alpha + pv;
          ph_s[h][lane] = f2w<BF>(pv);
          if (lane == 0) alpha_s[h] = alpha;
          m_run[i] = m_new;
        }
      }
    }
    __syncthreads();
    // ---- PV over this thread's token slice ----
    if (ph < G) {
      const float al = alpha_s[ph];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] *= al;
      // token pairs; past nv the probabilities and V are zeros
      const int r0 = pq * TPS;
      const int nv2 = (nv + 1) & ~1;
      const int r1 = r0 + TPS < nv2 ? r0 + TPS : nv2;
      for (int r = r0; r < r1; r += 2) {
        const uint32_t p2 = *reinterpret_cast<const uint32_t*>(&ph_s[ph][r]);
        const uint4 va = *reinterpret_cast<const uint4*>(&vp[r / 2][8 * pc]);
        const uint4 vb = *reinterpret_cast<const uint4*>(&vp[r / 2][8 * pc + 4]);
        const uint32_t v8[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = dot2w<BF>(v8[j], p2, acc[j]);
      }
    }
    __syncthreads();
  }

  // ---- partial (m, l, acc) of each head, or the output with one split ----
  __shared__ float l_s[HP];
  const int n = p.n_splits;
  const int64_t row0 = b * p.Hq + kvh * G;  // partial rows: query head (b, kvh G + h)
#pragma unroll
  for (int i = 0; i < HPW; ++i) {
    const int h = wave + 4 * i;
    if (h < G) {
      const float l = group_sum<64>(l_lane[i]);
      if (lane == 0) {
        l_s[h] = l;
        if (n > 1) {
          p.ws_ml[2 * ((row0 + h) * n + split)] = m_run[i];
          p.ws_ml[2 * ((row0 + h) * n + split) + 1] = l;
        }
      }
    }
  }
  auto emit = [&](int h, int d, float v) {  // the split's P V sum of (head h, channel d < D)
    if (d >= D) return;
    if (n == 1)
      p.out[b * p.o_sb + (kvh * G + h) * p.o_sh + d] = f2w<BF>(v / l_s[h]);
    else
      p.ws_acc[((row0 + h) * n + split) * D + d] = v;
  };
  if (TQ > 1) {
#pragma unroll
    for (int j = 0; j < 8; ++j) red[TQ > 1 ? pq : 0][po][j] = acc[j];
    __syncthreads();
    for (int o = tid; o < NU * 8; o += kThreads) {
      const int oo = o / 8, j = o % 8, h = oo / CG, cg = oo % CG;
      if (h < G) {
        float sum = 0.0f;
        for (int q = 0; q < TQ; ++q) sum += red[q][oo][j];
        emit(h, 8 * cg + j, sum);
      }
    }
  } else {
    __syncthreads();  // l_s
    if (ph < G) {
#pragma unroll
      for (int j = 0; j < 8; ++j) emit(ph, 8 * pc + j, acc[j]);
    }
  }
}

}  // namespace

// Merge the n_splits partials of each (b, hq) into the fp16 output; one
// thread per channel (blockDim.x = head_dim D).
__global__ __launch_bounds__(256) void decode_combine_kernel(const float* __restrict__ ws_ml,
                                                             const float* __restrict__ ws_acc,
                                                             int n_splits, int64_t Hq,
                                                             uint16_t* __restrict__ out,
                                                             int64_t o_sb, int64_t o_sh, int bf16) {
  const int64_t bh = blockIdx.x;
  const int d = threadIdx.x, D = blockDim.x;
  const float* ml = ws_ml + bh * n_splits * 2;
  float M = -INFINITY;
  for (int s = 0; s < n_splits; ++s) M = fmaxf(M, ml[2 * s]);
  float L = 0.0f, o = 0.0f;
  if (M != -INFINITY) {
    for (int s = 0; s < n_splits; ++s) {
      const float m = ml[2 * s];
      if (m == -INFINITY) continue;
      const float w = exp2f(m - M);
      L += ml[2 * s + 1] * w;
      o += ws_acc[(bh * n_splits + s) * D + d] * w;
    }
  }
  out[(bh / Hq) * o_sb + (bh % Hq) * o_sh + d] = bf16 ? f2bf(o / L) : f2h(o / L);
}

int launch_valu(const Params& p, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(p.n_splits), static_cast<unsigned>(p.Hkv),
                  static_cast<unsigned>(p.B));
  const bool h8 = p.G > 4;
  const bool bf = p.bf16 != 0;
  const bool s44 = !bf && p.mid.fmt == FADE_MID_SYM && p.mid.k_bits == 4 && p.mid.v_bits == 4;
#define FADE_VALU_LAUNCH(DD)                                                                                 \
  if (bf && h8) hipLaunchKernelGGL((decode_valu_kernel<DD, 8, false, true>), grid, dim3(kThreads), 0, st, p);   \
  else if (bf) hipLaunchKernelGGL((decode_valu_kernel<DD, 4, false, true>), grid, dim3(kThreads), 0, st, p);    \
  else if (h8 && s44) hipLaunchKernelGGL((decode_valu_kernel<DD, 8, true, false>), grid, dim3(kThreads), 0, st, p); \
  else if (h8) hipLaunchKernelGGL((decode_valu_kernel<DD, 8, false, false>), grid, dim3(kThreads), 0, st, p);   \
  else if (s44) hipLaunchKernelGGL((decode_valu_kernel<DD, 4, true, false>), grid, dim3(kThreads), 0, st, p);   \
  else hipLaunchKernelGGL((decode_valu_kernel<DD, 4, false, false>), grid, dim3(kThreads), 0, st, p);
  // the smallest instance whose capacity covers the head_dim
  if (p.D < 8 || p.D > 256 || p.D % 8 != 0)
    return einval("fade_tiered_decode_attn: head_dim must be a multiple of 8 in [8, 256], got %d", p.D);
  if (p.D <= 32) { FADE_VALU_LAUNCH(32) }
  else if (p.D <= 64) { FADE_VALU_LAUNCH(64) }
  else if (p.D <= 128) { FADE_VALU_LAUNCH(128) }
  else { FADE_VALU_LAUNCH(256) }
#undef FADE_VALU_LAUNCH
  return check_launch("fade_tiered_decode_attn(valu)");
}

}  // namespace decode
}  // namespace fade
