// Ragged tiered prefill attention on matrix cores (gfx950).
//
// Row b of the batch appends a chunk of Sq tokens to its cache
// [sink | middle | recent]; query j of the chunk attends to the whole cache
// and to chunk tokens 0..j (bottom-right causal, as the model's SDPA over
// the reference's materialized tiers, fade/cache.py:347-379,683-842).
//
// Workgroup = (32-query block, kv head, batch row); wave w serves query head
// kvh*G + w (G <= 4), its 32 query rows as two 16-row M tiles.  The virtual
// key sequence (cache, then chunk) is walked in 64-token tiles.  All 256
// threads fetch a tile (thread = one token x 32 channels), dequantize middle
// codes exactly as the reference does (fp16(code * scale)), and store fp16
// K [token][channel] and V^T [channel][token] in LDS (double-buffered: the
// next tile's global loads fly while the current one is computed).
//
// Per tile and wave:
//   S^T = K Q^T     f16 MFMA 16x16x32, A = K rows (16 keys), B = Q^T (16 rows);
//                   lane (n, g), register i  <->  query row n, key 4g + i
//   online softmax  row n's max/sum: lane-local over 16 keys, then 2 shuffles
//   O += P V        f16 MFMA 16x16x32, A = P straight from the S^T registers
//                   (key blocks paired), B = V^T rows from LDS
// Each K and V fragment read from LDS feeds both M tiles.
#include <math.h>

#include "fade_common.h"

namespace fade {
namespace prefill {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kQB = 32;       // queries per workgroup
constexpr int kKT = 64;       // keys per tile
constexpr int kKPitch = 136;  // halves per K row in LDS (conflict-free 16-byte reads)
constexpr int kVPitch = 72;   // halves per V^T row in LDS
constexpr float kNegBig = -1.0e30f;
constexpr float kTau = 8.0f;  // the running max moves only when a score exceeds it by kTau (log2)

struct Tier {
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sb, k_sh, k_ss, v_sb, v_sh, v_ss;
};

struct PParams {
  int64_t B, Hq, Hkv, Sq;
  int G;
  const uint16_t* q;
  int64_t q_sb, q_sh, q_ss;
  uint16_t* out;
  int64_t o_sb, o_sh, o_ss;
  float scale_log2;
  const int32_t* lens;
  const int32_t* order;
  Tier sink, recent, chunk;
  int has_mid;
  int64_t mid_cap, sink_cap, recent_cap;  // padded tier capacities: per-row lengths are clamped to them
  const uint8_t* kq;
  const uint16_t* ks;
  const uint8_t* vq;
  const uint16_t* vs;
};

__device__ __forceinline__ uint32_t pack2(_Float16 a, _Float16 b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

// Signed nibbles of one packed byte (high nibble = even channel) as fp16.
__device__ __forceinline__ void nib2(uint32_t byte, _Float16& even, _Float16& odd) {
  const int hi = static_cast<int>(static_cast<int8_t>(byte & 0xFFu)) >> 4;
  const int lo = static_cast<int>((byte & 0xFu) << 28) >> 28;
  even = static_cast<_Float16>(hi);
  odd = static_cast<_Float16>(lo);
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_kernel(PParams p) {
  const int qb = blockIdx.x;
  const int64_t kvh = blockIdx.y;
  int64_t b = blockIdx.z;
  if (p.order) {
    const int o = __builtin_amdgcn_readfirstlane(p.order[blockIdx.z]);
    b = o < 0 ? 0 : (o >= p.B ? p.B - 1 : o);
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, g = lane >> 4;
  const int G = p.G;
  const int64_t bkv = b * p.Hkv + kvh;
  // per-row tier lengths, clamped to the padded capacities (no read past a tier)
  auto clampi = [](int x, int64_t cap) { return x < 0 ? 0 : (x > cap ? static_cast<int>(cap) : x); };
  const int ns = clampi(__builtin_amdgcn_readfirstlane(p.lens[3 * b + 0]), p.sink_cap);
  const int nm = clampi(__builtin_amdgcn_readfirstlane(p.lens[3 * b + 1]), p.mid_cap);
  const int nr = clampi(__builtin_amdgcn_readfirstlane(p.lens[3 * b + 2]), p.recent_cap);
  const int L = ns + nm + nr;  // cache tokens of this row
  const int Sq = static_cast<int>(p.Sq);
  const int j0 = qb * kQB;
  const int jn = Sq - j0 < kQB ? Sq - j0 : kQB;  // queries of this block
  const int t_end = L + j0 + jn;                 // keys any query of the block can see
  const int n_tiles = (t_end + kKT - 1) / kKT;

  __shared__ __attribute__((aligned(16))) uint16_t kt[2][kKT][kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t vt[2][kD][kVPitch];

  // ---- tile fetch: thread = token r of the tile, channels 32*cp .. 32*cp+31 ----
  const int r = tid >> 2, cp = tid & 3;
  uint32_t ksc[16];  // fp16 K scales of this thread's channels (middle tier)
  if (p.has_mid) {
    const uint4* s4 = reinterpret_cast<const uint4*>(p.ks + bkv * kD + 32 * cp);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 w = s4[i];
      ksc[4 * i + 0] = w.x;
      ksc[4 * i + 1] = w.y;
      ksc[4 * i + 2] = w.z;
      ksc[4 * i + 3] = w.w;
    }
  }
  // sink / recent / chunk row pointers of this (b, kv head)
  const uint16_t* sk = p.sink.k + b * p.sink.k_sb + kvh * p.sink.k_sh;
  const uint16_t* sv = p.sink.v + b * p.sink.v_sb + kvh * p.sink.v_sh;
  const uint16_t* rk = p.recent.k + b * p.recent.k_sb + kvh * p.recent.k_sh;
  const uint16_t* rv = p.recent.v + b * p.recent.v_sb + kvh * p.recent.v_sh;
  const uint16_t* ck = p.chunk.k + b * p.chunk.k_sb + kvh * p.chunk.k_sh;
  const uint16_t* cv = p.chunk.v + b * p.chunk.v_sb + kvh * p.chunk.v_sh;
  const int64_t sk_ss = p.sink.k_ss, sv_ss = p.sink.v_ss, rk_ss = p.recent.k_ss, rv_ss = p.recent.v_ss;
  const int64_t ck_ss = p.chunk.k_ss, cv_ss = p.chunk.v_ss;
  const uint8_t* kq = p.kq + bkv * p.mid_cap * 64;
  const uint8_t* vq = p.vq + bkv * p.mid_cap * 64;
  const uint16_t* vsr = p.vs + bkv * p.mid_cap;

  uint4 fk[4], fv[4];  // fetched K / V (fp16 rows: 64 bytes; middle codes: 16 bytes in fk[0] / fv[0])
  int fkind = 0;       // 0 none, 1 fp16 row, 2 middle codes
  uint16_t fvs = 0;    // V scale of a middle token
  auto fetch = [&](int t) {
    const int v = t * kKT + r;
    fkind = 0;
    const uint16_t* kp = nullptr;
    const uint16_t* vp = nullptr;
    if (v < ns) {
      kp = sk + v * sk_ss;
      vp = sv + v * sv_ss;
    } else if (v < ns + nm) {
      const int m = v - ns;
      fk[0] = *reinterpret_cast<const uint4*>(kq + static_cast<int64_t>(m) * 64 + 16 * cp);
      fv[0] = *reinterpret_cast<const uint4*>(vq + static_cast<int64_t>(m) * 64 + 16 * cp);
      fvs = vsr[m];
      fkind = 2;
    } else if (v < L) {
      kp = rk + (v - ns - nm) * rk_ss;
      vp = rv + (v - ns - nm) * rv_ss;
    } else if (v < L + Sq) {
      kp = ck + (v - L) * ck_ss;
      vp = cv + (v - L) * cv_ss;
    }
    if (kp != nullptr) {
      const uint4* k4 = reinterpret_cast<const uint4*>(kp + 32 * cp);
      const uint4* v4 = reinterpret_cast<const uint4*>(vp + 32 * cp);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        fk[i] = k4[i];
        fv[i] = v4[i];
      }
      fkind = 1;
    }
  };
  auto store = [&](int buf) {
    uint32_t kw[16], vw[16];
    if (fkind == 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kw[4 * i + 0] = fk[i].x; kw[4 * i + 1] = fk[i].y; kw[4 * i + 2] = fk[i].z; kw[4 * i + 3] = fk[i].w;
        vw[4 * i + 0] = fv[i].x; vw[4 * i + 1] = fv[i].y; vw[4 * i + 2] = fv[i].z; vw[4 * i + 3] = fv[i].w;
      }
    } else if (fkind == 2) {
      // fp16(code * scale): the reference's dequantization (fade/quant.py:124-127)
      const _Float16 vscale = __builtin_bit_cast(_Float16, fvs);
      const uint32_t kb4[4] = {fk[0].x, fk[0].y, fk[0].z, fk[0].w};
      const uint32_t vb4[4] = {fv[0].x, fv[0].y, fv[0].z, fv[0].w};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t kbyte = (kb4[i >> 2] >> (8 * (i & 3))) & 0xFFu;
        const uint32_t vbyte = (vb4[i >> 2] >> (8 * (i & 3))) & 0xFFu;
        _Float16 ke, ko, ve, vo;
        nib2(kbyte, ke, ko);
        nib2(vbyte, ve, vo);
        const uint32_t s2 = ksc[i];
        const _Float16 se = __builtin_bit_cast(_Float16, static_cast<uint16_t>(s2 & 0xFFFFu));
        const _Float16 so = __builtin_bit_cast(_Float16, static_cast<uint16_t>(s2 >> 16));
        kw[i] = pack2(ke * se, ko * so);
        vw[i] = pack2(ve * vscale, vo * vscale);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) kw[i] = vw[i] = 0u;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<u32x4*>(&kt[buf][r][32 * cp + 8 * i]) = u32x4{kw[4 * i], kw[4 * i + 1], kw[4 * i + 2], kw[4 * i + 3]};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      vt[buf][32 * cp + 2 * i][r] = static_cast<uint16_t>(vw[i] & 0xFFFFu);
      vt[buf][32 * cp + 2 * i + 1][r] = static_cast<uint16_t>(vw[i] >> 16);
    }
  };

  // ---- query fragments: rows j0 + 16*mt + n16, B operand of S^T = K Q^T ----
  const bool active = wave < G;
  const int64_t h = kvh * G + (active ? wave : 0);
  f16x8 qf[2][4];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int j = j0 + 16 * mt + n16;
    const uint16_t* qr = p.q + b * p.q_sb + h * p.q_sh + static_cast<int64_t>(j < Sq ? j : Sq - 1) * p.q_ss;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const uint4 w = (active && j < Sq) ? *reinterpret_cast<const uint4*>(qr + 32 * ks + 8 * g) : make_uint4(0, 0, 0, 0);
      qf[mt][ks] = __builtin_bit_cast(f16x8, w);
    }
  }

  f32x4 acc[2][8];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[mt][c] = f32x4{0, 0, 0, 0};
  float m_run[2] = {kNegBig, kNegBig}, l_run[2] = {0.0f, 0.0f};
  const float sl2 = p.scale_log2;

  auto compute = [&](int t, int buf) {
    // S^T for both M tiles; each K fragment feeds both
    f32x4 s[2][4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) s[mt][kb] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16x8 a = *reinterpret_cast<const f16x8*>(&kt[buf][16 * kb + n16][32 * ks + 8 * g]);
        s[0][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[0][ks], s[0][kb], 0, 0, 0);
        s[1][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[1][ks], s[1][kb], 0, 0, 0);
      }
    f16x8 pa[2][2];  // PV A operands: [M tile][key-block pair]
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int jq = j0 + 16 * mt + n16;  // this lane's query (column n16)
      const int lim = L + jq;             // last visible key
      float x[4][4];
      float lmax = kNegBig;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int v = t * kKT + 16 * kb + 4 * g + i;
          x[kb][i] = v <= lim ? s[mt][kb][i] * sl2 : -INFINITY;
          lmax = fmaxf(lmax, x[kb][i]);
        }
      lmax = fmaxf(lmax, __shfl_xor(lmax, 16, 64));
      lmax = fmaxf(lmax, __shfl_xor(lmax, 32, 64));
      if (__builtin_amdgcn_ballot_w64(lmax - m_run[mt] > kTau) != 0) {
        const float m_new = fmaxf(m_run[mt], lmax);
        const float alpha = __builtin_amdgcn_exp2f(m_run[mt] - m_new);
        m_run[mt] = m_new;
        l_run[mt] *= alpha;
        // accumulator row 4g + i lives in lanes whose column n16 is that row
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float ai = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
          for (int c = 0; c < 8; ++c) acc[mt][c][i] *= ai;
        }
      }
      float ps = 0.0f;
      _Float16 ph[4][4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pv = __builtin_amdgcn_exp2f(x[kb][i] - m_run[mt]);
          ps += pv;
          ph[kb][i] = static_cast<_Float16>(pv);
        }
      l_run[mt] += ps;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
        pa[mt][pp] = f16x8{ph[2 * pp][0], ph[2 * pp][1], ph[2 * pp][2], ph[2 * pp][3],
                           ph[2 * pp + 1][0], ph[2 * pp + 1][1], ph[2 * pp + 1][2], ph[2 * pp + 1][3]};
    }
    // O += P V; each V fragment feeds both M tiles
#pragma unroll
    for (int pp = 0; pp < 2; ++pp)
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const u32x2 lo = *reinterpret_cast<const u32x2*>(&vt[buf][16 * c + n16][16 * (2 * pp) + 4 * g]);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(&vt[buf][16 * c + n16][16 * (2 * pp + 1) + 4 * g]);
        const f16x8 bv = __builtin_bit_cast(f16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
        acc[0][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[0][pp], bv, acc[0][c], 0, 0, 0);
        acc[1][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[1][pp], bv, acc[1][c], 0, 0, 0);
      }
  };

  fetch(0);
  store(0);
  __syncthreads();
  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < n_tiles) fetch(t + 1);
    if (active) compute(t, buf);
    if (t + 1 < n_tiles) store(buf ^ 1);
    __syncthreads();
  }

  if (!active) return;
  // ---- normalize and store: accumulator lane (channel n16, g), register i <-> row 4g + i ----
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    float l = l_run[mt];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float li = __shfl(l, 4 * g + i, 64);
      const int j = j0 + 16 * mt + 4 * g + i;
      if (j < Sq) {
        uint16_t* orow = p.out + b * p.o_sb + h * p.o_sh + static_cast<int64_t>(j) * p.o_ss;
        const float inv = 1.0f / li;
#pragma unroll
        for (int c = 0; c < 8; ++c) orow[16 * c + n16] = f2h(acc[mt][c][i] * inv);
      }
    }
  }
}

bool aligned16(const void* x) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0; }

bool tier_ok(const fade_fp16_tier& t) {
  if (t.len == 0) return true;
  return t.k && t.v && aligned16(t.k) && aligned16(t.v) && ((t.k_sb | t.k_sh | t.k_ss | t.v_sb | t.v_sh | t.v_ss) % 8 == 0);
}

Tier tier_of(const fade_fp16_tier& t) {
  Tier r{};
  r.k = static_cast<const uint16_t*>(t.k);
  r.v = static_cast<const uint16_t*>(t.v);
  r.k_sb = t.k_sb; r.k_sh = t.k_sh; r.k_ss = t.k_ss;
  r.v_sb = t.v_sb; r.v_sh = t.v_sh; r.v_ss = t.v_ss;
  return r;
}

}  // namespace
}  // namespace prefill
}  // namespace fade

using namespace fade;
using namespace fade::prefill;

FADE_API int fade_tiered_prefill_attn(const fade_prefill_args* a, void* stream) {
  if (a == nullptr) return einval("fade_tiered_prefill_attn: null args");
  if (a->D != kD) return einval("fade_tiered_prefill_attn: head_dim must be %d, got %lld", kD, (long long)a->D);
  if (a->B <= 0 || a->Hq <= 0 || a->Hkv <= 0 || a->Sq <= 0)
    return einval("fade_tiered_prefill_attn: B, Hq, Hkv and Sq must be positive");
  if (a->Hq % a->Hkv != 0 || a->Hq / a->Hkv > 4)
    return einval("fade_tiered_prefill_attn: needs Hq %% Hkv == 0 and Hq/Hkv <= 4 (got %lld/%lld)",
                  (long long)a->Hq, (long long)a->Hkv);
  if (a->B > 65535 || a->Hkv > 65535 || a->Sq > (1 << 24)) return einval("fade_tiered_prefill_attn: shape too large");
  if (a->q == nullptr || a->out == nullptr || a->lens == nullptr)
    return einval("fade_tiered_prefill_attn: null q, out or lens");
  if (!aligned16(a->q) || (a->q_sb | a->q_sh | a->q_ss) % 8)
    return einval("fade_tiered_prefill_attn: q rows must be 16-byte aligned");
  if (a->chunk.len != a->Sq) return einval("fade_tiered_prefill_attn: chunk tier must hold Sq tokens");
  if (!tier_ok(a->sink) || !tier_ok(a->recent) || !tier_ok(a->chunk))
    return einval("fade_tiered_prefill_attn: fp16 tiers need 16-byte aligned rows");
  const fade_mid_tier& m = a->mid;
  const bool has_mid = m.len > 0 && m.fmt != FADE_MID_NONE;
  if (has_mid) {
    if (m.fmt != FADE_MID_SYM || m.k_bits != 4 || m.v_bits != 4)
      return einval("fade_tiered_prefill_attn: the middle tier must be FADE_MID_SYM 4-bit");
    if (!m.k_codes || !m.v_codes || !m.k_scale || !m.v_scale || !aligned16(m.k_codes) || !aligned16(m.v_codes) ||
        (reinterpret_cast<uintptr_t>(m.k_scale) & 15))
      return einval("fade_tiered_prefill_attn: middle tier pointers missing or misaligned");
  }
  PParams p{};
  p.B = a->B;
  p.Hq = a->Hq;
  p.Hkv = a->Hkv;
  p.Sq = a->Sq;
  p.G = static_cast<int>(a->Hq / a->Hkv);
  p.q = static_cast<const uint16_t*>(a->q);
  p.q_sb = a->q_sb; p.q_sh = a->q_sh; p.q_ss = a->q_ss;
  p.out = static_cast<uint16_t*>(a->out);
  p.o_sb = a->o_sb; p.o_sh = a->o_sh; p.o_ss = a->o_ss;
  p.scale_log2 = a->sm_scale * 1.4426950408889634f;
  p.lens = a->lens;
  p.order = a->order;
  p.sink = tier_of(a->sink);
  p.recent = tier_of(a->recent);
  p.chunk = tier_of(a->chunk);
  p.has_mid = has_mid ? 1 : 0;
  p.mid_cap = has_mid ? m.len : 0;
  p.sink_cap = a->sink.len;
  p.recent_cap = a->recent.len;
  p.kq = static_cast<const uint8_t*>(m.k_codes);
  p.ks = static_cast<const uint16_t*>(m.k_scale);
  p.vq = static_cast<const uint8_t*>(m.v_codes);
  p.vs = static_cast<const uint16_t*>(m.v_scale);
  const dim3 grid(static_cast<unsigned>(cdiv(a->Sq, kQB)), static_cast<unsigned>(a->Hkv), static_cast<unsigned>(a->B));
  hipLaunchKernelGGL(prefill_kernel, grid, dim3(kThreads), 0, as_stream(stream), p);
  return check_launch("fade_tiered_prefill_attn");
}
