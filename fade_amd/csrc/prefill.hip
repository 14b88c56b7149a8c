// Ragged tiered prefill attention on matrix cores (gfx950).
//
// Row b of the batch appends a chunk of Sq tokens to its cache
// [sink | middle | recent]; query j of the chunk attends to the whole cache
// and to chunk tokens 0..j (bottom-right causal, as the model's SDPA over
// the reference's materialized tiers, fade/cache.py:347-379,683-842).
//
// Workgroup = (32-query block, kv head, batch row); wave w serves query head
// kvh*G + w (G <= 4), its 32 query rows as two 16-row M tiles.  The row's key
// sequence is walked in 64-token tiles that never straddle a tier (sink,
// middle, recent, then the chunk).  All 256 threads fetch a tile (thread =
// one token x 32 channels) into double-buffered LDS (the next tile's global
// loads fly while the current one is computed): fp16 K and V rows as they
// are, through registers; middle-tier codes and V scales by direct
// global -> LDS loads into a staging area (each thread's load lands the bytes
// that thread converts, so no barrier is needed and no register is held
// across the compute), then dequantized exactly as the reference does,
// fp16(code * scale), with three packed operations per pair of codes (72 + c
// by one bit operation, - 72, * scale).  K and V rows keep channels in the
// order the code conversion produces (1 5 0 4 3 7 2 6 within every 8
// channels); the query and the output use the same order.
//
// Per tile and wave:
//   S^T = K Q^T     f16 MFMA 16x16x32, A = K rows (16 keys), B = Q^T (16 rows);
//                   lane (n, g), register i  <->  query row n, key 4g + i
//   online softmax  row n's max/sum: lane-local over 16 keys, then 2 shuffles
//   O += P V        f16 MFMA 16x16x32, A = P straight from the S^T registers
//                   (key blocks paired), B = V rows via ds_read_b64_tr_b16
// Each K and V fragment read from LDS feeds both M tiles.
#include <math.h>

#include "fade_common.h"
#include "lds_dma.h"

namespace fade {
namespace prefill {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kQB = 32;       // queries per workgroup
constexpr int kKT = 64;       // keys per tile
constexpr int kKPitch = 136;  // halves per K row in LDS (16-byte reads of 16 rows: distinct banks)
constexpr int kVPitch = 144;  // halves per V row in LDS (tr16 reads of 4 rows x 4 chunks: distinct banks)
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

// Eight two's-complement nibbles (one dword of packed codes, high nibble =
// even channel) -> four fp16 pairs of value 72 + c: the nibble goes to
// mantissa bits 4..7 of 64.0 (one code step = 1.0) with its top bit flipped.
// The pairs come out as channels (1,5), (0,4), (3,7), (2,6) of the dword:
// K and V rows are stored in LDS in that order within every 8-channel group.
__device__ __forceinline__ void nib_to_f16(uint32_t w, uint32_t (&o)[4]) {
  o[0] = ((w << 4) & 0x00F000F0u) ^ 0x54805480u;
  o[1] = (w & 0x00F000F0u) ^ 0x54805480u;
  o[2] = ((w >> 4) & 0x00F000F0u) ^ 0x54805480u;
  o[3] = ((w >> 8) & 0x00F000F0u) ^ 0x54805480u;
}
// Eight fp16 channels (natural order, dwords = channel pairs) -> the stored order.
__device__ __forceinline__ u32x4 to_stored(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3) {
  return u32x4{__builtin_amdgcn_perm(d2, d0, 0x07060302u), __builtin_amdgcn_perm(d2, d0, 0x05040100u),
               __builtin_amdgcn_perm(d3, d1, 0x07060302u), __builtin_amdgcn_perm(d3, d1, 0x05040100u)};
}
// Channel of stored half h within an 8-channel group.
// (1 5 0 4 3 7 2 6, one nibble per h)
__device__ __forceinline__ int stored_channel(int h) { return (0x62734051 >> (4 * h)) & 0xF; }

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
  const int Sq = static_cast<int>(p.Sq);
  const int j0 = qb * kQB;
  const int jn = Sq - j0 < kQB ? Sq - j0 : kQB;  // queries of this block
  const int cv = j0 + jn;                        // chunk keys any query of the block can see
  // Key tiles never straddle a tier: sink, middle, recent, chunk tiles in turn.
  const int nts = (ns + kKT - 1) / kKT, ntm = (nm + kKT - 1) / kKT, ntr = (nr + kKT - 1) / kKT;
  const int n_tiles = nts + ntm + ntr + (cv + kKT - 1) / kKT;
  struct TileRef {
    int seg, base, cnt;  // segment (0 sink, 1 middle, 2 recent, 3 chunk), first key, keys
  };
  auto tile_of = [&](int t) {
    TileRef r;
    int len;
    if (t < nts) {
      r.seg = 0; r.base = kKT * t; len = ns;
    } else if (t < nts + ntm) {
      r.seg = 1; r.base = kKT * (t - nts); len = nm;
    } else if (t < nts + ntm + ntr) {
      r.seg = 2; r.base = kKT * (t - nts - ntm); len = nr;
    } else {
      r.seg = 3; r.base = kKT * (t - nts - ntm - ntr); len = cv;
    }
    r.cnt = len - r.base < kKT ? len - r.base : kKT;
    return r;
  };

  __shared__ __attribute__((aligned(16))) uint16_t kt[2][kKT][kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t vt[2][kKT][kVPitch];
  // middle-tile staging: thread tid's 16 bytes of K / V codes at 16 tid, its
  // token's V scale in dword tid (a 2-byte direct load fills one dword per lane)
  __shared__ __attribute__((aligned(16))) uint8_t stg_k[kThreads * 16];
  __shared__ __attribute__((aligned(16))) uint8_t stg_v[kThreads * 16];
  __shared__ __attribute__((aligned(16))) uint32_t stg_s[kThreads];

  // ---- tile fetch: thread = token r of the tile, channels 32*cp .. 32*cp+31 ----
  const int r = tid >> 2, cp = tid & 3;
  const uint16_t* sk = p.sink.k + b * p.sink.k_sb + kvh * p.sink.k_sh;
  const uint16_t* sv = p.sink.v + b * p.sink.v_sb + kvh * p.sink.v_sh;
  const uint16_t* rk = p.recent.k + b * p.recent.k_sb + kvh * p.recent.k_sh;
  const uint16_t* rv = p.recent.v + b * p.recent.v_sb + kvh * p.recent.v_sh;
  const uint16_t* ck = p.chunk.k + b * p.chunk.k_sb + kvh * p.chunk.k_sh;
  const uint16_t* cvp = p.chunk.v + b * p.chunk.v_sb + kvh * p.chunk.v_sh;
  const int64_t sk_ss = p.sink.k_ss, sv_ss = p.sink.v_ss, rk_ss = p.recent.k_ss, rv_ss = p.recent.v_ss;
  const int64_t ck_ss = p.chunk.k_ss, cv_ss = p.chunk.v_ss;
  const uint8_t* kq = p.kq + bkv * p.mid_cap * 64;
  const uint8_t* vq = p.vq + bkv * p.mid_cap * 64;
  const uint16_t* vsr = p.vs + bkv * p.mid_cap;

  // K scales of this thread's 32 channels as fp16 pairs, in the stored order
  uint32_t ksc[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint4 w = make_uint4(0, 0, 0, 0);
    if (p.has_mid) w = *reinterpret_cast<const uint4*>(p.ks + bkv * kD + 32 * cp + 8 * i);
    const u32x4 st = to_stored(w.x, w.y, w.z, w.w);
#pragma unroll
    for (int e = 0; e < 4; ++e) ksc[4 * i + e] = st[e];
  }
  int fok = 0;  // this thread's staged middle row is a real token of the tile
  // staging slots of this wave's lanes (a direct load writes lane l's bytes at base + l * size)
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  const uint32_t stk = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8*)&stg_k[16 * 64 * wave])));
  const uint32_t stv = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8*)&stg_v[16 * 64 * wave])));
  const uint32_t sts = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8*)&stg_s[64 * wave])));
  // Middle tile: codes and V scale to the staging area.  Nothing waits for
  // these loads before store_mid(), so they fly during the current tile's compute.
  auto fetch_mid = [&](const TileRef& tr) {
    const bool ok = r < tr.cnt;
    fok = ok;
    const int key = tr.base + (ok ? r : tr.cnt - 1);  // rows past the tile: a valid row, zeroed in store_mid()
    lds_dma16(kq + static_cast<int64_t>(key) * 64 + 16 * cp, stk);
    lds_dma16(vq + static_cast<int64_t>(key) * 64 + 16 * cp, stv);
    lds_dma2(vsr + key, sts);
  };
  // staged codes -> fp16(code * scale) rows of K and V in LDS buffer buf
  auto store_mid = [&](int buf) {
    // the staging loads are the only vector-memory operations in flight here
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    uint4 kraw = *reinterpret_cast<const uint4*>(&stg_k[16 * tid]);
    uint4 vraw = *reinterpret_cast<const uint4*>(&stg_v[16 * tid]);
    uint32_t vsb = stg_s[tid] & 0xFFFFu;
    if (!fok) {
      kraw = vraw = make_uint4(0, 0, 0, 0);
      vsb = 0;
    }
    // codes -> fp16 72 + c -> c -> fp16(c * scale), already in the stored channel order
    const uint32_t kw[4] = {kraw.x, kraw.y, kraw.z, kraw.w};
    const uint32_t vw[4] = {vraw.x, vraw.y, vraw.z, vraw.w};
    const f16x2 m72 = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
    const f16x2 vs2 = __builtin_bit_cast(f16x2, vsb * 0x00010001u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t o[4];
      u32x4 kd, vd;
      nib_to_f16(kw[i], o);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        kd[e] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, o[e]) + m72) *
                                                 __builtin_bit_cast(f16x2, ksc[4 * i + e]));
      nib_to_f16(vw[i], o);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        vd[e] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, o[e]) + m72) * vs2);
      *reinterpret_cast<u32x4*>(&kt[buf][r][32 * cp + 8 * i]) = kd;
      *reinterpret_cast<u32x4*>(&vt[buf][r][32 * cp + 8 * i]) = vd;
    }
  };
  // fp16 tile (sink, recent or chunk: a few per row): loaded and stored at once
  auto load_store_f16 = [&](const TileRef& tr, int buf) {
    uint4 fk[4], fv[4];
    const int key = tr.base + r;
    if (r < tr.cnt) {
      const uint16_t* kp = tr.seg == 0 ? sk + key * sk_ss : (tr.seg == 2 ? rk + key * rk_ss : ck + key * ck_ss);
      const uint16_t* vp = tr.seg == 0 ? sv + key * sv_ss : (tr.seg == 2 ? rv + key * rv_ss : cvp + key * cv_ss);
      const uint4* k4 = reinterpret_cast<const uint4*>(kp + 32 * cp);
      const uint4* v4 = reinterpret_cast<const uint4*>(vp + 32 * cp);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        fk[i] = k4[i];
        fv[i] = v4[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) fk[i] = fv[i] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<u32x4*>(&kt[buf][r][32 * cp + 8 * i]) = to_stored(fk[i].x, fk[i].y, fk[i].z, fk[i].w);
      *reinterpret_cast<u32x4*>(&vt[buf][r][32 * cp + 8 * i]) = to_stored(fv[i].x, fv[i].y, fv[i].z, fv[i].w);
    }
  };
  // Tile t into LDS buffer buf: fp16 tiles complete here; a middle tile only
  // starts (returns true) and completes in store_mid().
  auto begin_tile = [&](int t, int buf) {
    const TileRef tr = tile_of(t);
    if (tr.seg == 1) {
      fetch_mid(tr);
      return true;
    }
    load_store_f16(tr, buf);
    return false;
  };

  // ---- query fragments: rows j0 + 16*mt + n16, B operand of S^T = K Q^T, stored channel order ----
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
      qf[mt][ks] = __builtin_bit_cast(f16x8, to_stored(w.x, w.y, w.z, w.w));
    }
  }

  f32x4 acc[2][8];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[mt][c] = f32x4{0, 0, 0, 0};
  float m_run[2] = {kNegBig, kNegBig}, l_run[2] = {0.0f, 0.0f};
  const float sl2 = p.scale_log2;
  const float tau_raw = kTau / sl2;  // the lazy-rescale margin in raw score units

  auto compute = [&](int t, int buf) {
    const TileRef tr = tile_of(t);
    // S^T for both M tiles (raw scores q.k); each K fragment feeds both
    f32x4 s[2][4];
    const f32x4 zero4 = {0, 0, 0, 0};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16x8 a = *reinterpret_cast<const f16x8*>(&kt[buf][16 * kb + n16][32 * ks + 8 * g]);
        s[0][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[0][ks], ks ? s[0][kb] : zero4, 0, 0, 0);
        s[1][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[1][ks], ks ? s[1][kb] : zero4, 0, 0, 0);
      }
    // every key of a full cache tile is visible to every query of the block
    const bool full = tr.seg != 3 && tr.cnt == kKT;
    f16x8 pa[2][2];  // PV A operands: [M tile][key-block pair]
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      float x[4][4];
      if (full) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) x[kb][i] = s[mt][kb][i];
      } else {
        const int jq = j0 + 16 * mt + n16;  // this lane's query (column n16)
        // key kk of the tile is visible when kk < cnt and, in the chunk, base + kk <= jq
        const int lim = tr.seg == 3 ? (jq - tr.base + 1 < tr.cnt ? jq - tr.base + 1 : tr.cnt) : tr.cnt;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) x[kb][i] = 16 * kb + 4 * g + i < lim ? s[mt][kb][i] : -INFINITY;
      }
      float lmax = kNegBig;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        lmax = fmaxf(fmaxf(lmax, fmaxf(x[kb][0], x[kb][1])), fmaxf(x[kb][2], x[kb][3]));
      lmax = fmaxf(lmax, __shfl_xor(lmax, 16, 64));
      lmax = fmaxf(lmax, __shfl_xor(lmax, 32, 64));
      // running max m_run in raw score units; probabilities exp2((x - m) * scale)
      if (__builtin_amdgcn_ballot_w64(lmax - m_run[mt] > tau_raw) != 0) {
        const float m_new = fmaxf(m_run[mt], lmax);
        const float alpha = __builtin_amdgcn_exp2f((m_run[mt] - m_new) * sl2);
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
      const float nm = -m_run[mt] * sl2;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pv = __builtin_amdgcn_exp2f(fmaf(x[kb][i], sl2, nm));
          ps += pv;
          ph[kb][i] = static_cast<_Float16>(pv);
        }
      l_run[mt] += ps;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
        pa[mt][pp] = f16x8{ph[2 * pp][0], ph[2 * pp][1], ph[2 * pp][2], ph[2 * pp][3],
                           ph[2 * pp + 1][0], ph[2 * pp + 1][1], ph[2 * pp + 1][2], ph[2 * pp + 1][3]};
    }
    // O += P V.  B operand via tr16 reads of V rows: source lane s of group g
    // points at key 32 pp + 16 half + 4 g + (s >> 2), channels 16 c + 4 (s & 3);
    // lane n then holds stored channel 16 c + n of the four keys.
    const int vr0 = 4 * g + (n16 >> 2), vcol = 4 * (n16 & 3);
#pragma unroll
    for (int pp = 0; pp < 2; ++pp)
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const f16x4 lo = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            reinterpret_cast<lds_i16x4*>((__attribute__((address_space(3))) uint16_t*)&vt[buf][32 * pp + vr0][16 * c + vcol])));
        const f16x4 hi = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            reinterpret_cast<lds_i16x4*>((__attribute__((address_space(3))) uint16_t*)&vt[buf][32 * pp + 16 + vr0][16 * c + vcol])));
        const f16x8 bv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        acc[0][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[0][pp], bv, acc[0][c], 0, 0, 0);
        acc[1][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[1][pp], bv, acc[1][c], 0, 0, 0);
      }
  };

  if (begin_tile(0, 0)) store_mid(0);
  __syncthreads();
  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    // the next tile goes to the other buffer, last read by the previous tile's compute
    const bool mid_next = t + 1 < n_tiles && begin_tile(t + 1, buf ^ 1);
    if (active) compute(t, buf);
    if (mid_next) store_mid(buf ^ 1);
    __syncthreads();
  }

  if (!active) return;
  // ---- normalize and store: accumulator lane (stored channel n16, g), register i <-> row 4g + i ----
  const int ch = 8 * (n16 >> 3) + stored_channel(n16 & 7);
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
        for (int c = 0; c < 8; ++c) orow[16 * c + ch] = f2h(acc[mt][c][i] * inv);
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
