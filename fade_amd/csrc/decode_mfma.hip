// Matrix-core (MFMA) tiered decode attention for gfx950.
//
// One workgroup = 4 wavefronts serving one (batch row, kv head, split); each
// wavefront walks its own 64-token tiles with its own online-softmax state
// and the four are merged through LDS at the end.  The whole GQA group of
// query heads rides in the 16 rows of every MFMA, so each KV byte is read
// once.  Per 64-token tile:
//
//   QK^T  int8 MFMA 16x16x64.  A = K codes of 16 tokens (a lane's 16-byte
//         load of a packed row becomes 32 offset-binary int8 codes u = c + 8,
//         two k-steps); B = the query, pre-scaled by the per-channel K scale,
//         quantized to 16 bits and split into two int8 digits (hi*256 + lo).
//         score = hi_acc*256 + lo_acc - 8*sum(q_int), exact in int32.
//   PV    f16 MFMA 16x16x32.  A = P * v_scale[token] (fp16); B = V codes
//         staged through LDS and transposed by ds_read_b64_tr_b4 (each lane
//         receives one channel of 16 tokens), turned into fp16 with the
//         0x6400 | nibble trick.
//
// fp16 tiles (sink + recent tokens, or every tile of the fp16 comparator)
// use an f16 MFMA for QK^T and direct fp16 V loads; they accumulate into the
// same fragments.
//
// Fragment bookkeeping (lane = 16*g + n, C fragment row = 4*g + i):
//   QK m-tile j, A row m  <->  token 16*(m/4) + 4*j + (m%4) of the tile
//   score reg i of m-tile j in lane (h=n, g)  <->  token 16*g + 4*j + i
//   PV k-step s, lane (., g), VGPR v  <->  tokens (16g + 8s + v, 16g + 8s + v + 4)
//   O n-tile c, column n  <->  channel 16*c + (n ^ 1)
#include <math.h>

#include "decode_common.h"
#include "lds_dma.h"

namespace fade {
namespace decode {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
typedef __attribute__((address_space(3))) uint8_t lds_u8;

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kTileT = 64;
constexpr float kQMax = 32000.0f;
constexpr float kNegBig = -1.0e30f;  // running-max sentinel (finite: no inf-inf guards)

// Head-dim geometry (DK = 64, 128 or 256).  A stage holds one packed tile: K
// codes (64 rows of DK/2 bytes) | V codes (the same) | V scales (64 dwords).
// Lane group g of a QK^T MFMA covers channels DK/4 g .. + DK/4 - 1 (DK/64
// int8 k-steps of 64, 16 channels of the lane's each); PV has DK/16 column blocks.
template <int DK>
struct Geo {
  static constexpr int kRowB = DK / 2;                 // packed bytes per token
  static constexpr int kUnits = DK / 32;               // 16-byte units per packed row
  static constexpr int kStageK = 0, kStageV = 32 * DK, kStageVS = 64 * DK;
  static constexpr int kStageBytes = 64 * DK + 256;    // the 2-byte DMA writes one dword per lane
  static constexpr int kKS = DK / 64;                  // int8 QK^T k-steps
  static constexpr int kCPL = DK / 4;                  // channels per lane group
  static constexpr int kNC = DK / 16;                  // PV column blocks
  static constexpr int kV16Pitch = DK + 8;             // halfs per staged fp16 V row (16 rows fit the V region)
  static constexpr int kOpsPerStage = 2 * kUnits + 1;  // direct loads per packed tile
};

__device__ __forceinline__ uint4 ldg16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// Direct HBM -> LDS loads (lds_dma.h): 16 bytes land at lds_base + 16*i; a
// 2-byte load lands zero-extended in the dword at lds_base + 4*i.  Issued as
// inline asm so that the only waits on these loads are the explicit per-stage
// s_waitcnt vmcnt of the packed-tile loop (the compiler cannot tell two ring
// stages apart and would wait for both).  Register-destination loads stay
// correct: any wait the compiler emits for them also covers older LDS loads
// and at worst over-waits for newer ones.


// Offset-binary int8 codes (u = c + 8) of one packed dword: lo nibbles
// (odd channels) and hi nibbles (even channels), four bytes each.
__device__ __forceinline__ void nib_to_u8(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t x = w ^ 0x88888888u;
  lo = x & 0x0F0F0F0Fu;
  hi = (x >> 4) & 0x0F0F0F0Fu;
}

// fp16 pairs (nibble v, nibble v+4), v = 0..3, of 8 two's-complement codes c,
// as the values 48 + 2c: the nibble moves to mantissa bits 6..9 of 32.0
// (0x5000, ulp 1/32, so one code step is 2.0) and bit 3 is flipped
// (c + 8 = offset binary).  Two bit ops per pair; the constant 48 per token
// is removed once at the end with an MFMA-accumulated sum of P.
__device__ __forceinline__ void nib8_to_f16(uint32_t w, uint32_t* out) {
  out[0] = ((w << 6) & 0x03C003C0u) ^ 0x52005200u;
  out[1] = ((w << 2) & 0x03C003C0u) ^ 0x52005200u;
  out[2] = ((w >> 2) & 0x03C003C0u) ^ 0x52005200u;
  out[3] = ((w >> 6) & 0x03C003C0u) ^ 0x52005200u;
}

// The same for bfloat16 values 72 + c: the nibble moves to mantissa bits 1..4
// of 64.0 (0x4280, ulp 1/2, one code step = 1.0), bit 3 flipped.
__device__ __forceinline__ void nib8_to_bf16(uint32_t w, uint32_t* out) {
  out[0] = ((w << 1) & 0x001E001Eu) ^ 0x42904290u;
  out[1] = ((w >> 3) & 0x001E001Eu) ^ 0x42904290u;
  out[2] = ((w >> 7) & 0x001E001Eu) ^ 0x42904290u;
  out[3] = ((w >> 11) & 0x001E001Eu) ^ 0x42904290u;
}

// 16-bit operands of the call's dtype (BF: bfloat16, else fp16) as bit patterns.
template <bool BF>
__device__ __forceinline__ f32x4 mfma_k32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
template <bool BF>
__device__ __forceinline__ f32x4 mfma_k16(i32x2 a, i32x2 b, f32x4 c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4, a), __builtin_bit_cast(bf16x4, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
}
template <bool BF>
__device__ __forceinline__ uint32_t pack_w2(float a, float b) {
  if constexpr (BF) return pack_bf16(a, b);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(a))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(b))) << 16);
}

struct FpTok {  // one fp16 token row (K and V pointers)
  const uint16_t* k;
  const uint16_t* v;
};

// Row pointers of virtual fp16 token f: sink, (fp16 middle), recent; ns / nm
// are the row's sink and fp16-middle tokens (the middle rows are mid.len apart).
template <bool MID_F16, int DK>
__device__ __forceinline__ FpTok fp16_token(const Params& p, int64_t b, int64_t kvh, int64_t f, int64_t ns,
                                            int64_t nm) {
  FpTok r;
  if (f < ns) {
    r.k = p.sink.k + b * p.sink.k_sb + kvh * p.sink.k_sh + f * p.sink.k_ss;
    r.v = p.sink.v + b * p.sink.v_sb + kvh * p.sink.v_sh + f * p.sink.v_ss;
    return r;
  }
  f -= ns;
  if (MID_F16) {
    if (f < nm) {
      const int64_t row = (b * p.Hkv + kvh) * p.mid.len + f;
      r.k = reinterpret_cast<const uint16_t*>(p.mid.k_codes) + row * DK;
      r.v = reinterpret_cast<const uint16_t*>(p.mid.v_codes) + row * DK;
      return r;
    }
    f -= nm;
  }
  r.k = p.recent.k + b * p.recent.k_sb + kvh * p.recent.k_sh + f * p.recent.k_ss;
  r.v = p.recent.v + b * p.recent.v_sb + kvh * p.recent.v_sh + f * p.recent.v_ss;
  return r;
}

// BF: q, the tiers, the scales and the output are bfloat16; probabilities and
// V values enter the PV MFMAs as bfloat16.  Packed V codes become 72 + c
// (bfloat16) instead of 48 + 2c (fp16), so the fp16-tier tiles' PV takes P
// once instead of twice and the constant removed is 72 instead of 48.
template <bool MID_F16, int DK, bool BF>
__global__ __launch_bounds__(kThreads) void decode_mfma_kernel(Params p) {
  using GE = Geo<DK>;
  constexpr float kVMul = BF ? 1.0f : 2.0f;   // V value per code step
  constexpr float kVOff = BF ? 72.0f : 48.0f;  // V value offset per token of a packed tile
  constexpr int kStageK = GE::kStageK, kStageV = GE::kStageV, kStageVS = GE::kStageVS, kStageBytes = GE::kStageBytes;
  constexpr int kKS = GE::kKS, kCPL = GE::kCPL, kNC = GE::kNC, kV16Pitch = GE::kV16Pitch;
  const int split = blockIdx.x;
  const int64_t kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, grp = lane >> 4;
  const int G = p.G;
  const int64_t bkv = b * p.Hkv + kvh;
  // this row's sink, middle and recent tokens: the tiers' lengths, or the row's
  // own (per-row lengths, clamped to the padded capacities)
  const int64_t Mc = p.mid.len;                                // middle rows per (row, kv head)
  int64_t ns = p.sink.len, nm = Mc, nr = p.recent.len;
  if (p.lens != nullptr) {
    const int64_t ls = __builtin_amdgcn_readfirstlane(p.lens[3 * b]);
    const int64_t lm = __builtin_amdgcn_readfirstlane(p.lens[3 * b + 1]);
    const int64_t lr = __builtin_amdgcn_readfirstlane(p.lens[3 * b + 2]);
    ns = ls < 0 ? 0 : (ls < p.sink.len ? ls : p.sink.len);
    nm = lm < 0 ? 0 : (lm < Mc ? lm : Mc);
    nr = lr < 0 ? 0 : (lr < p.recent.len ? lr : p.recent.len);
  }
  const int64_t M = MID_F16 ? 0 : nm;                          // packed middle tokens
  const int64_t F = ns + nr + (MID_F16 ? nm : 0);              // fp16 tokens
  const int64_t nF = (F + kTileT - 1) / kTileT;

  // Per-wave ring of two stages; a stage holds one packed tile:
  // K codes (4 KB) | V codes (4 KB) | V scales (64 dwords), swizzled 16-byte units.
  __shared__ __attribute__((aligned(16))) uint8_t ring0[kWaves][kStageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t ring1[kWaves][kStageBytes];
  __shared__ __attribute__((aligned(16))) float alpha_s[kWaves][16];
  __shared__ float red_m[kWaves][16], red_l[kWaves][16];
  __shared__ __attribute__((aligned(16))) uint16_t q16_s[16][DK + 8];

  // ---- query operands (lane = head n16, k-group grp: channels kCPL grp ..) ----
  const bool hvalid = n16 < G;
  uint4 qraw[kCPL / 8];
  {
    const uint16_t* qp = p.q + b * p.q_sb + (kvh * G + (hvalid ? n16 : 0)) * p.q_sh + kCPL * grp;
#pragma unroll
    for (int c = 0; c < kCPL / 8; ++c) qraw[c] = hvalid ? ldg16(qp + 8 * c) : make_uint4(0, 0, 0, 0);
  }
  // fp16 query rows for the fp16 tiles' QK^T (B operand read from LDS when needed)
  if (wave == 0) {
#pragma unroll
    for (int c = 0; c < kCPL / 8; ++c) *reinterpret_cast<uint4*>(&q16_s[n16][kCPL * grp + 8 * c]) = qraw[c];
  }
  i32x4 qd_hi[kKS], qd_lo[kKS];  // int8 digits of q * k_scale for the packed middle
  int corr = 0;
  float qscale = 0.0f;
  if (!MID_F16 && M > 0) {
    float qf[kCPL];
#pragma unroll
    for (int c = 0; c < kCPL / 8; ++c) {
      const uint32_t u[4] = {qraw[c].x, qraw[c].y, qraw[c].z, qraw[c].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qf[8 * c + 2 * e] = w2f<BF>(static_cast<uint16_t>(u[e] & 0xFFFFu));
        qf[8 * c + 2 * e + 1] = w2f<BF>(static_cast<uint16_t>(u[e] >> 16));
      }
    }
    const uint16_t* ksp = p.mid.k_scale + bkv * DK + kCPL * grp;
#pragma unroll
    for (int c = 0; c < kCPL / 8; ++c) {
      const uint4 w = ldg16(ksp + 8 * c);
      const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qf[8 * c + 2 * e] *= w2f<BF>(static_cast<uint16_t>(u[e] & 0xFFFFu));
        qf[8 * c + 2 * e + 1] *= w2f<BF>(static_cast<uint16_t>(u[e] >> 16));
      }
    }
    float mx = 0.0f;
#pragma unroll
    for (int d = 0; d < kCPL; ++d) mx = fmaxf(mx, fabsf(qf[d]));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float inv = mx > 0.0f ? kQMax / mx : 0.0f;
    qscale = mx > 0.0f ? (mx / kQMax) * p.scale_log2 : 0.0f;
    int qi[kCPL];
    int sum = 0;
#pragma unroll
    for (int d = 0; d < kCPL; ++d) {
      qi[d] = static_cast<int>(rintf(qf[d] * inv));
      sum += qi[d];
    }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    corr = 8 * sum;
    // k-step ks, dword js, byte e  <->  channel kCPL*grp + 8*(2ks + js/2) + 2e + (js even ? 1 : 0)
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) {
#pragma unroll
      for (int js = 0; js < 4; ++js) {
        uint32_t whi = 0, wlo = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int dl = 8 * (2 * ks + js / 2) + 2 * e + ((js % 2 == 0) ? 1 : 0);
          const int hi = (qi[dl] + 128) >> 8;
          const int lo = qi[dl] - hi * 256;
          whi |= static_cast<uint32_t>(hi & 0xFF) << (8 * e);
          wlo |= static_cast<uint32_t>(lo & 0xFF) << (8 * e);
        }
        qd_hi[ks][js] = static_cast<int>(whi);
        qd_lo[ks][js] = static_cast<int>(wlo);
      }
    }
  } else {
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) qd_hi[ks] = qd_lo[ks] = i32x4{0, 0, 0, 0};
  }

  // ---- tiles of this split; wave w takes tiles w, w+4, ... ----
  const int64_t tiles_per_split = p.tokens_per_split / kTileT;
  const int64_t t0 = static_cast<int64_t>(split) * tiles_per_split;
  const int64_t nT = nF + (M + kTileT - 1) / kTileT;
  const int64_t t1 = t0 + tiles_per_split < nT ? t0 + tiles_per_split : nT;

  __syncthreads();
  // acc holds kVMul * sum(P V) + kVOff * sum_{packed tiles}(P'), acc48 the kVOff * sum(P') part.
  float m_run = kNegBig, l_lane = 0.0f;
  f32x4 acc[kNC];
#pragma unroll
  for (int c = 0; c < kNC; ++c) acc[c] = f32x4{0, 0, 0, 0};
  f32x4 acc48 = {0, 0, 0, 0};

  uint8_t* my_vtile = ring0[wave];  // fp16 tiles stage V chunks here (before the packed ring starts)

  // Online-softmax update of head n16 with the 64 scores s of one tile; P
  // (times the V scale) leaves as the two PV A operands, plain P in pw.
  // Online-softmax update of head n16 with the 64 scores of one tile.  P
  // times pscale[token] leaves as the two PV A operands (fp16), plain P in pw.
  // Accumulators are rescaled only when some head's running max rises.
  auto softmax_tile = [&](float (&sc)[4][4], const float* pscale, float (&pw)[4][4], u32x4& pa0, u32x4& pa1) {
    float tmax = sc[0][0];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, sc[j][i]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    if (__builtin_amdgcn_ballot_w64(tmax > m_run) != 0) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_lane *= alpha;
      m_run = m_new;
      if (grp == 0) alpha_s[wave][n16] = alpha;
      __builtin_amdgcn_wave_barrier();
      const f32x4 al = *reinterpret_cast<const f32x4*>(&alpha_s[wave][4 * grp]);
#pragma unroll
      for (int c = 0; c < kNC; ++c) acc[c] *= al;
      acc48 *= al;
    }
    float psum = 0.0f;
    uint32_t pa[2][4];  // k-step s, VGPR v = tokens (16g+8s+v, 16g+8s+v+4)
#pragma unroll
    for (int sk = 0; sk < 2; ++sk) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float p0 = __builtin_amdgcn_exp2f(sc[2 * sk][v] - m_run);
        const float p1 = __builtin_amdgcn_exp2f(sc[2 * sk + 1][v] - m_run);
        psum += p0 + p1;
        pw[2 * sk][v] = p0;
        pw[2 * sk + 1][v] = p1;
        pa[sk][v] = pack_w2<BF>(p0 * pscale[8 * sk + v], p1 * pscale[8 * sk + v + 4]);
      }
    }
    l_lane += psum;
    pa0 = u32x4{pa[0][0], pa[0][1], pa[0][2], pa[0][3]};
    pa1 = u32x4{pa[1][0], pa[1][1], pa[1][2], pa[1][3]};
  };

  // -------------------------------------------------------------- fp16 tiles
  const int64_t f_end = t1 < nF ? t1 : nF;
  for (int64_t tau = t0 + wave; tau < f_end; tau += kWaves) {
    float sc[4][4], pw[4][4], vsc[16];
    const int64_t f0 = tau * kTileT;
#pragma unroll 1
    for (int j = 0; j < 4; ++j) {
      const int rloc = 16 * (n16 >> 2) + 4 * j + (n16 & 3);
      const int64_t f = f0 + rloc < F ? f0 + rloc : F - 1;
      const uint16_t* kr = fp16_token<MID_F16, DK>(p, b, kvh, f, ns, nm).k + kCPL * grp;
      f32x4 c4 = {0, 0, 0, 0};
#pragma unroll
      for (int ks = 0; ks < kCPL / 8; ++ks) {
        const u32x4 qb = *reinterpret_cast<const u32x4*>(&q16_s[n16][kCPL * grp + 8 * ks]);
        const uint4 kw = ldg16(kr + 8 * ks);
        c4 = mfma_k32<BF>(u32x4{kw.x, kw.y, kw.z, kw.w}, qb, c4);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t tok = f0 + 16 * grp + 4 * j + i;
        sc[j][i] = tok < F ? c4[i] * p.scale_log2 : -INFINITY;
      }
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) vsc[k] = kVMul;
    u32x4 pa0, pa1;
    softmax_tile(sc, vsc, pw, pa0, pa1);
    // fp16 V in four 16-token chunks through LDS; chunk q = tokens 16g + 4q + i
    uint16_t* vt16 = reinterpret_cast<uint16_t*>(my_vtile);
#pragma unroll 1
    for (int q = 0; q < 4; ++q) {
      __builtin_amdgcn_wave_barrier();
      {
        const int r = lane >> 2;  // staged row: g = r/4, i = r%4
        const int64_t tok = f0 + 16 * (r >> 2) + 4 * q + (r & 3);
        const uint16_t* src = fp16_token<MID_F16, DK>(p, b, kvh, tok < F ? tok : F - 1, ns, nm).v + kCPL * (lane & 3);
#pragma unroll
        for (int c = 0; c < kCPL / 8; ++c)
          *reinterpret_cast<uint4*>(vt16 + r * kV16Pitch + kCPL * (lane & 3) + 8 * c) = ldg16(src + 8 * c);
      }
      __builtin_amdgcn_wave_barrier();
      const i32x2 pa4 = {static_cast<int>(pack_w2<BF>(kVMul * pw[q][0], kVMul * pw[q][1])),
                         static_cast<int>(pack_w2<BF>(kVMul * pw[q][2], kVMul * pw[q][3]))};
#pragma unroll
      for (int c = 0; c < kNC; ++c) {
        const int d = 16 * c + (n16 ^ 1);
        const i32x2 vb = {static_cast<int>(vt16[(4 * grp + 0) * kV16Pitch + d] | (static_cast<uint32_t>(vt16[(4 * grp + 1) * kV16Pitch + d]) << 16)),
                          static_cast<int>(vt16[(4 * grp + 2) * kV16Pitch + d] | (static_cast<uint32_t>(vt16[(4 * grp + 3) * kV16Pitch + d]) << 16))};
        acc[c] = mfma_k16<BF>(pa4, vb, acc[c]);
      }
    }
  }

  // ------------------------------------------ packed INT4 tiles, pipelined
  // Tile codes and scales move HBM -> LDS with direct global_load_lds
  // (16 bytes per lane, no VGPRs), two tiles ahead of the math.
  // 16-byte units are swizzled so the K-operand reads (16 lanes = 16 rows,
  // one chunk) and the tr4 V reads (16 consecutive rows, one 8-byte half)
  // hit 16 different bank groups:
  //   K unit (row r, chunk q) at 4r + (q ^ ((r >> 4) & 3))
  //   V unit (row r, chunk q) at 4r + (q ^ ((r >> 2) & 3))
  // (DK = 64 / 256: U = DK / 32 units per row, unit U r + q, unswizzled)
  int64_t tau = t0 + wave;
  if (tau < nF) tau += ((nF - tau + kWaves - 1) / kWaves) * kWaves;
  if (!MID_F16 && tau < t1) {
    constexpr int kRowB = GE::kRowB;
    const uint8_t* kc = p.mid.k_codes + bkv * Mc * kRowB;
    const uint8_t* vc = p.mid.v_codes + bkv * Mc * kRowB;
    const uint16_t* vsg = p.mid.v_scale + bkv * Mc;
    auto issue = [&](int64_t t, uint32_t st) {
      const int64_t m0 = (t - nF) * kTileT;
      if constexpr (DK == 128) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int r = 16 * k + (lane >> 2);
          const int64_t row = m0 + r < M ? m0 + r : M - 1;
          const int qk = (lane & 3) ^ k;
          lds_dma16(kc + row * 64 + 16 * qk, st + kStageK + 1024 * k);
          const int qv = (lane & 3) ^ ((lane >> 4) & 3);
          lds_dma16(vc + row * 64 + 16 * qv, st + kStageV + 1024 * k);
        }
      } else {
        // load k fills units 64 k + lane: row (64 k + lane) / U, chunk (64 k + lane) % U
        constexpr int U = GE::kUnits;
#pragma unroll
        for (int k = 0; k < U; ++k) {
          const int r = (64 * k + lane) / U, qc = (64 * k + lane) % U;
          const int64_t row = m0 + r < M ? m0 + r : M - 1;
          lds_dma16(kc + row * kRowB + 16 * qc, st + kStageK + 1024 * k);
          lds_dma16(vc + row * kRowB + 16 * qc, st + kStageV + 1024 * k);
        }
      }
      const int64_t vrow = m0 + lane < M ? m0 + lane : M - 1;
      lds_dma2(vsg + vrow, st + kStageVS);
    };
    constexpr int kOpsPerStage = GE::kOpsPerStage;
    // vmcnt operand of s_waitcnt with expcnt / lgkmcnt left unconstrained
    auto wait_vm = [](bool keep_one_stage) {
      if (keep_one_stage) __builtin_amdgcn_s_waitcnt((kOpsPerStage & 15) | (7 << 4) | (15 << 8));
      else __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
    };
    // One packed tile from stage buffer st (a distinct __shared__ array per
    // stage, so the compiler's LDS-DMA waits stay per stage).
    auto compute = [&](int64_t t, const uint8_t* st, lds_u8* st_lds) {
      const int64_t m0 = (t - nF) * kTileT;
      float sc[4][4], pw[4][4], vsc[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int rloc = 16 * (n16 >> 2) + 4 * j + (n16 & 3);
        i32x4 chi = {0, 0, 0, 0}, clo = {0, 0, 0, 0};
        if constexpr (DK == 128) {
          const int unit = 4 * rloc + (grp ^ ((rloc >> 4) & 3));
          const uint4 w = *reinterpret_cast<const uint4*>(st + kStageK + 16 * unit);
          uint32_t lo0, hi0, lo1, hi1, lo2, hi2, lo3, hi3;
          nib_to_u8(w.x, lo0, hi0);
          nib_to_u8(w.y, lo1, hi1);
          nib_to_u8(w.z, lo2, hi2);
          nib_to_u8(w.w, lo3, hi3);
          const i32x4 a0 = {static_cast<int>(lo0), static_cast<int>(hi0), static_cast<int>(lo1), static_cast<int>(hi1)};
          const i32x4 a1 = {static_cast<int>(lo2), static_cast<int>(hi2), static_cast<int>(lo3), static_cast<int>(hi3)};
          chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, qd_hi[0], chi, 0, 0, 0);
          chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, qd_hi[kKS - 1], chi, 0, 0, 0);
          clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, qd_lo[0], clo, 0, 0, 0);
          clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, qd_lo[kKS - 1], clo, 0, 0, 0);
        } else {
          // k-step ks: the lane's channels kCPL grp + 16 ks .. + 15, bytes
          // kCPL/2 grp + 8 ks .. + 7 of the row
#pragma unroll
          for (int ks = 0; ks < kKS; ++ks) {
            const uint2 w = *reinterpret_cast<const uint2*>(st + kStageK + GE::kRowB * rloc + (kCPL / 2) * grp + 8 * ks);
            uint32_t lo0, hi0, lo1, hi1;
            nib_to_u8(w.x, lo0, hi0);
            nib_to_u8(w.y, lo1, hi1);
            const i32x4 a = {static_cast<int>(lo0), static_cast<int>(hi0), static_cast<int>(lo1), static_cast<int>(hi1)};
            chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qd_hi[ks], chi, 0, 0, 0);
            clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qd_lo[ks], clo, 0, 0, 0);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[j][i] = static_cast<float>(chi[i] * 256 + clo[i] - corr) * qscale;
      }
      if (m0 + kTileT > M) {  // partial last tile: mask tokens past the middle tier
        const int valid = static_cast<int>(M - m0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (16 * grp + 4 * j + i >= valid) sc[j][i] = -INFINITY;
      }
      {  // V scale of token k sits in the low half of dword k
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint4 v = *reinterpret_cast<const uint4*>(st + kStageVS + 64 * grp + 16 * c);
          vsc[4 * c + 0] = w2f<BF>(static_cast<uint16_t>(v.x & 0xFFFFu));
          vsc[4 * c + 1] = w2f<BF>(static_cast<uint16_t>(v.y & 0xFFFFu));
          vsc[4 * c + 2] = w2f<BF>(static_cast<uint16_t>(v.z & 0xFFFFu));
          vsc[4 * c + 3] = w2f<BF>(static_cast<uint16_t>(v.w & 0xFFFFu));
        }
      }
      u32x4 pa0, pa1;
      softmax_tile(sc, vsc, pw, pa0, pa1);
      const int vrow = 16 * grp + n16;
#pragma unroll
      for (int c = 0; c < kNC; ++c) {
        const int unit = DK == 128 ? 4 * vrow + ((c >> 1) ^ ((vrow >> 2) & 3)) : GE::kUnits * vrow + (c >> 1);
        const i32x2 x = __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_i32x2*)(st_lds + kStageV + 16 * unit + 8 * (c & 1)));
        uint32_t vb0[4], vb1[4];
        if constexpr (BF) {
          nib8_to_bf16(static_cast<uint32_t>(x[0]), vb0);
          nib8_to_bf16(static_cast<uint32_t>(x[1]), vb1);
        } else {
          nib8_to_f16(static_cast<uint32_t>(x[0]), vb0);
          nib8_to_f16(static_cast<uint32_t>(x[1]), vb1);
        }
        acc[c] = mfma_k32<BF>(pa0, u32x4{vb0[0], vb0[1], vb0[2], vb0[3]}, acc[c]);
        acc[c] = mfma_k32<BF>(pa1, u32x4{vb1[0], vb1[1], vb1[2], vb1[3]}, acc[c]);
      }
      {  // kVOff * sum(P') per head, accumulated exactly like acc
        const uint32_t o2 = pack_w2<BF>(kVOff, kVOff);
        const u32x4 b48 = {o2, o2, o2, o2};
        acc48 = mfma_k32<BF>(pa0, b48, acc48);
        acc48 = mfma_k32<BF>(pa1, b48, acc48);
      }
      // every LDS read of this stage has returned before it is refilled
      __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4));
      __builtin_amdgcn_wave_barrier();
    };
    lds_u8* st0 = (lds_u8*)&ring0[wave][0];
    lds_u8* st1 = (lds_u8*)&ring1[wave][0];
    const uint32_t a0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(st0)));
    const uint32_t a1 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(st1)));
    issue(tau, a0);
    if (tau + kWaves < t1) issue(tau + kWaves, a1);
    while (tau < t1) {
      wait_vm(tau + kWaves < t1);
      __builtin_amdgcn_wave_barrier();
      compute(tau, &ring0[wave][0], st0);
      if (tau + 2 * kWaves < t1) issue(tau + 2 * kWaves, a0);
      tau += kWaves;
      if (tau >= t1) break;
      wait_vm(tau + kWaves < t1);
      __builtin_amdgcn_wave_barrier();
      compute(tau, &ring1[wave][0], st1);
      if (tau + 2 * kWaves < t1) issue(tau + 2 * kWaves, a1);
      tau += kWaves;
    }
  }

  // ---- merge the four wavefronts, write this split's partial ----
  float l_tot = l_lane;
  l_tot += __shfl_xor(l_tot, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (grp == 0) {
    red_m[wave][n16] = m_run;
    red_l[wave][n16] = l_tot;
  }
  __syncthreads();
  float* red_acc = reinterpret_cast<float*>(&ring0[0][0]);  // [wave][h < G][DK] (spans ring0, ring1)
  static_assert(2 * kWaves * kStageBytes >= kWaves * kMaxG * DK * 4, "the wave merge fits the two rings");
  {
    // scale of each of this lane's accumulator rows (heads 4*grp + i)
    float wscale[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * grp + i;
      float Mh = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) Mh = fmaxf(Mh, red_m[w][h]);
      wscale[i] = (1.0f / kVMul) * exp2f(red_m[wave][h] - Mh);
    }
#pragma unroll
    for (int c = 0; c < kNC; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = 4 * grp + i;
        if (h < G) red_acc[(wave * G + h) * DK + 16 * c + (n16 ^ 1)] = (acc[c][i] - acc48[i]) * wscale[i];
      }
  }
  __syncthreads();
  for (int idx = tid; idx < G * DK; idx += kThreads) {
    const int h = idx / DK, d = idx % DK;
    float Mh = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) Mh = fmaxf(Mh, red_m[w][h]);
    float o = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) o += red_acc[(w * G + h) * DK + d];
    const int64_t pidx = (b * p.Hq + kvh * G + h) * p.n_splits + split;
    p.ws_acc[pidx * DK + d] = o;
    if (d == 0) {
      float L = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) L += red_l[w][h] * exp2f(red_m[w][h] - Mh);
      p.ws_ml[2 * pidx] = Mh;
      p.ws_ml[2 * pidx + 1] = L;
    }
  }
}

bool aligned16(const void* x) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0; }

bool fp16_tier_ok(const Fp16Tier& t) {
  if (t.len == 0) return true;
  return aligned16(t.k) && aligned16(t.v) && ((t.k_sb | t.k_sh | t.k_ss | t.v_sb | t.v_sh | t.v_ss) % 8 == 0);
}

}  // namespace

bool mfma_supports(const Params& p) {
  if (p.D != 128 && p.D != 64 && p.D != 256) return false;
  if (!fp16_tier_ok(p.sink) || !fp16_tier_ok(p.recent)) return false;
  if (p.G > kMaxG) return false;
  if (reinterpret_cast<uintptr_t>(p.q) % 16 || p.q_sb % 8 || p.q_sh % 8) return false;
  switch (p.mid.fmt) {
    case FADE_MID_NONE:
      return true;
    case FADE_MID_FP16:
      return aligned16(p.mid.k_codes) && aligned16(p.mid.v_codes);
    case FADE_MID_SYM:
      return p.mid.k_bits == 4 && p.mid.v_bits == 4 && aligned16(p.mid.k_codes) && aligned16(p.mid.v_codes) &&
             aligned16(p.mid.k_scale);
    default:
      return false;
  }
}

int mfma_tile() { return kTileT; }

// Workgroups of one machine-wide wave at the call's head dim: LDS and registers
// allow 3 resident workgroups per CU at head_dim 64, 2 at 128 and 1 at 256
// (measured at B=16, S=8192: 6 splits of 128 (row, kv head) pairs at 64 and 2
// at 256 beat the D=128 choice of 4 by 3.5% and 10%).
int64_t mfma_target_wgs(const Params& p) {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        n > 0)
      cus = n;
    else
      (void)hipGetLastError();
  }
  const int64_t per_cu = p.D == 64 ? 3 : (p.D == 256 ? 1 : 2);
  return static_cast<int64_t>(cus > 0 ? cus : 256) * per_cu;
}

// Token tiles: fp16 tokens first (sink, [fp16 middle], recent), then packed middle tiles.
int64_t mfma_tiles(const Params& p) {
  const bool mid_f16 = p.mid.fmt == FADE_MID_FP16 || p.mid.fmt == FADE_MID_NONE;
  const int64_t M = mid_f16 ? 0 : p.mid.len;
  return cdiv(p.total - M, kTileT) + cdiv(M, kTileT);
}

int launch_mfma(const Params& p, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(p.n_splits), static_cast<unsigned>(p.Hkv), static_cast<unsigned>(p.B));
  const bool f16 = p.mid.fmt == FADE_MID_FP16 || p.mid.fmt == FADE_MID_NONE;
#define FADE_MFMA_LAUNCH(DK)                                                                                         \
  if (p.bf16 && f16) hipLaunchKernelGGL((decode_mfma_kernel<true, DK, true>), grid, dim3(kThreads), 0, st, p);   \
  else if (p.bf16) hipLaunchKernelGGL((decode_mfma_kernel<false, DK, true>), grid, dim3(kThreads), 0, st, p);    \
  else if (f16) hipLaunchKernelGGL((decode_mfma_kernel<true, DK, false>), grid, dim3(kThreads), 0, st, p);       \
  else hipLaunchKernelGGL((decode_mfma_kernel<false, DK, false>), grid, dim3(kThreads), 0, st, p);
  if (p.D == 64) { FADE_MFMA_LAUNCH(64) }
  else if (p.D == 256) { FADE_MFMA_LAUNCH(256) }
  else { FADE_MFMA_LAUNCH(128) }
#undef FADE_MFMA_LAUNCH
  return check_launch("fade_tiered_decode_attn(mfma)");
}

}  // namespace decode
}  // namespace fade
