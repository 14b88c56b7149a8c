// Ragged tiered prefill attention on matrix cores (gfx950).
//
// Row b of the batch appends a chunk of Sq tokens to its cache
// [sink | middle | recent]; query j of the chunk attends to the whole cache
// and to chunk tokens 0..j (bottom-right causal, as the model's SDPA over
// the reference's materialized tiers, fade/cache.py:347-379,683-842).
//
// Workgroup = (query blocks and head pass, kv head, batch row): one or two
// groups of 4 waves (interleaved: wave w belongs to group w % NQB), group q
// serving the q-th 32-query block; wave w of a group serves query head kvh*G + 4*pass + w (G = Hq/Hkv <= 8: one pass of up
// to 4 heads for G <= 4, two passes for G = 5..8), its 32 query rows as one
// 32-row M tile.  With G = 1 or 2 the four waves of a group cover 4 or 2
// query blocks instead (wave w: head w % G of block w / G), so no wave idles.  With two groups, the first stages and dequantizes each
// tile's K and the second its V, so one dequantization serves 64 queries per
// head.  The row's key
// sequence is walked in 64-token tiles that never straddle a tier (sink,
// middle, recent, then the chunk).  The threads fetch a tile (thread =
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
// Per tile and wave (one 32-row M tile; 32x32x16 f16 MFMAs, which on gfx950
// run at twice the rate of 16x16x32):
//   S^T = K Q^T     A = K rows (32 keys x 16 channels), B = Q^T (registers);
//                   lane (n, h) = (query n, half h), register i <-> key
//                   32 kb + 8 (i / 4) + 4 h + i % 4
//   online softmax  a query's 64 scores: lane-local over 32, one exchange with
//                   lane n ^ 32
//   O += P V        A = P straight from the S^T registers: registers
//                   8 (s & 1) .. + 7 of key block s >> 1 are the k slots of
//                   k-step s; B = 16-byte reads of V^T rows
//
// V is kept transposed in LDS (row = channel, natural order) with key k at
// position swap23(k) (bits 2 and 3 exchanged), so that the eight keys of one
// PV k slot group are adjacent.  Middle tiles reach that layout without a
// pass through fp16 rows: wave w stages the codes and scales of keys
// 16 w .. 16 w + 15, and a ds_read_b64_tr_b4 hands each lane one channel of
// those 16 keys, which it dequantizes (fp16(code * scale), as the reference)
// into two 16-byte runs of its V^T row.  fp16 tiles (a few per row) are
// written transposed directly.
#include <math.h>

#include "fade_common.h"
#include "lds_dma.h"

namespace fade {
namespace prefill {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;

constexpr int kThreads = 256;
constexpr int kQB = 32;       // queries per workgroup
constexpr int kKT = 64;       // keys per tile
// halves per K row in LDS: D + 8 (16-byte reads of 16 rows: distinct banks at D = 128)
template <int D>
constexpr int kKPitch = D + 8;
// waves per SIMD the register allocation is sized for: 1 at head_dim 256 (512 registers), else 2
template <int D>
constexpr int kWavesPerEu = D > 128 ? 1 : 2;
constexpr int kVtPitch = 72;  // halves per V^T row in LDS (16-byte accesses of 8 consecutive rows: distinct banks)
constexpr float kNegBig = -1.0e30f;
// The running max moves only when a score exceeds it by kTau = 8 (log2 units),
// i.e. when a probability exceeds kTauP = 2^kTau.
constexpr float kTauP = 256.0f;

struct Tier {
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_sb, k_sh, k_ss, v_sb, v_sh, v_ss;
};

struct PParams {
  int64_t B, Hq, Hkv, Sq;
  int G;       // query heads per kv head (Hq / Hkv), <= 8
  int passes;  // workgroups per (query block, kv head): ceil(G / 4)
  int hpw;     // query heads per group of 4 waves: 4, or G = 1 / 2 (then 4 / 2 query blocks per group)
  const uint16_t* q;
  int64_t q_sb, q_sh, q_ss;
  uint16_t* out;
  int64_t o_sb, o_sh, o_ss;
  float scale_log2;
  const int32_t* lens;
  const int32_t* order;
  Tier sink, recent, chunk;
  int has_mid;
  int mid_fp16;                           // the middle tier is fp16 rows [B,Hkv,cap,128] (kq / vq)
  int64_t mid_cap, sink_cap, recent_cap;  // padded tier capacities: per-row lengths are clamped to them
  const uint8_t* kq;
  const uint16_t* ks;
  const uint8_t* vq;
  const uint16_t* vs;
  const int32_t* pages;  // paged middle: block table [B][ppr] of 64-token pages (one middle tile each)
  int64_t ppr;
  int mask_mode;          // FADE_MASK_*: bottom-right over the chunk, top-left over the row, none
  int chunk_len;          // chunk keys (Sq under FADE_MASK_BOTTOM_RIGHT)
  int D;                  // head_dim: a multiple of 8 up to the instance's capacity (packed middle: of 32)
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
// 32x32x16 MFMA on eight 16-bit values per lane of the instance's dtype
// (BF: bfloat16, else fp16), as bit patterns.
template <bool BF>
__device__ __forceinline__ f32x16 mfma32x32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
// Codes of a pair as fp16 72 + c (one dword of nib_to_f16) times two scales
// (bfloat16 bit patterns, low half first) -> the bf16 pair
// (bf16(c_lo * s_lo), bf16(c_hi * s_hi)): c * s is exact in fp32 (4-bit code,
// 8-bit significand), so one rounding, as the reference's bf16 dequantization.
__device__ __forceinline__ uint32_t dequant_pair_bf16(uint32_t o72, uint32_t s2) {
  const f16x2 m72 = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
  const f16x2 c = __builtin_bit_cast(f16x2, o72) + m72;  // exact
  return pack_bf16(static_cast<float>(c.x) * __uint_as_float(s2 << 16),
                   static_cast<float>(c.y) * __uint_as_float(s2 & 0xFFFF0000u));
}

// Position of key k (0..63) of a tile in a V^T row: bits 2 and 3 exchanged.
__host__ __device__ constexpr int swap23(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

// Head dims up to the capacity DP = 32, 64, 128 or 256: QK^T takes DP/16
// k-steps, PV DP/32 column blocks; a fetch thread covers DP/4 channels of a
// token (fp16 tiles), and DP/32 threads stage a middle token's code bytes, 16
// (32 channels) each (at DP = 256 in two passes of 32 tokens, the same
// channels, so the same K scales).  A head_dim D < DP (p.D) leaves the channels past D as
// zeros in the K rows and the query (so they add nothing to the scores) and
// never stores them; V channels past D feed only output columns that are not
// stored.  fp16 rows move in 8-channel units, packed rows in 32-channel ones.
// NQB query blocks of 32 per workgroup (4 waves each).  With NQB = 2 the two
// groups of 4 waves split the tile staging: waves 0-3 stage and dequantize K,
// waves 4-7 V, so each middle tile's dequantization serves 64 queries per head.
// BF: q, out, the fp16-layout tiers and the middle tier's scales are bfloat16;
// middle codes dequantize to bf16(code * scale), the MFMAs take bfloat16
// operands (the probabilities too), accumulating in fp32.
// DP = 256 runs NQB = 1 at one wave per SIMD: its O accumulators alone take 128
// registers per lane, and its LDS (two 33 KB K and two 36 KB V^T buffers) one
// workgroup per CU.
template <int DP, int NQB, bool BF>
__global__ __launch_bounds__(kThreads * NQB) __attribute__((amdgpu_waves_per_eu(kWavesPerEu<DP>, kWavesPerEu<DP>)))
void prefill_kernel(PParams p) {
  static_assert(DP <= 128 || NQB == 1, "head_dim 256 runs one query block per workgroup");
  constexpr int D = DP;           // channel capacity of the LDS rows and MFMA tiles
  constexpr int KROW = D / 2;     // staged bytes of one token's packed 4-bit codes
  constexpr int CPT = D / 4;      // channels per fetch thread (fp16 tiles)
  constexpr int KTHR = D / 32;    // threads (16 code bytes each) per middle token
  constexpr int UPR = D / 32;     // 16-byte units per staged V code row
  constexpr int NKS = D / 16;     // QK^T k-steps
  constexpr int NCB = D / 32;     // PV column blocks
  constexpr int KP = kKPitch<D>;
  constexpr int TPP = kThreads / KTHR < kKT ? kThreads / KTHR : kKT;  // middle tokens one K staging pass covers
  constexpr int KPS = kKT / TPP;                  // K staging passes (2 at D = 256)
  constexpr int VPS = (16 * UPR + 63) / 64;       // V staging loads per lane (2 at D = 256)
  constexpr int VWB = 16 * KROW > 1024 ? 16 * KROW : 1024;  // staged V code bytes of one wave's 16 keys
  const int Dr = p.D;             // the rows' channels (<= D)
  const int krow = Dr / 2;        // bytes of one token's packed codes in HBM
  const int qb = blockIdx.x / p.passes;
  const int h0 = 4 * (blockIdx.x - qb * p.passes);  // first query head (within the group) of this workgroup
  const int64_t kvh = blockIdx.y;
  int64_t b = blockIdx.z;
  if (p.order) {
    const int o = __builtin_amdgcn_readfirstlane(p.order[blockIdx.z]);
    b = o < 0 ? 0 : (o >= p.B ? p.B - 1 : o);
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // groups interleaved: wave w is wave w / NQB of group w % NQB (1% faster
  // than groups of consecutive waves)
  const int wq = wave / NQB, qblk = wave % NQB;  // wave within its group, the group's query block
  const int gtid = (wq << 6) | lane;             // thread within its group of 4 waves
  // staging roles: K (codes, scales) and V (codes, scales) of every tile
  const bool do_k = NQB == 1 || qblk == 0, do_v = NQB == 1 || qblk == NQB - 1;
  const int n16 = lane & 15, g = lane >> 4;
  const int G = p.G - h0 < 4 ? p.G - h0 : 4;  // query heads this workgroup serves
  // wave wq of a group serves head wq % hpw of the group's query block wq / hpw
  const int hpw = p.hpw, lhpw = hpw == 4 ? 2 : (hpw == 2 ? 1 : 0);
  const int qpg = 4 >> lhpw;                     // query blocks per group
  const int wh = wq & (hpw - 1), wsub = wq >> lhpw;
  const int64_t bkv = b * p.Hkv + kvh;
  // per-row tier lengths, clamped to the padded capacities (no read past a tier)
  auto clampi = [](int x, int64_t cap) { return x < 0 ? 0 : (x > cap ? static_cast<int>(cap) : x); };
  const int ns = clampi(__builtin_amdgcn_readfirstlane(p.lens[3 * b + 0]), p.sink_cap);
  const int nm = clampi(__builtin_amdgcn_readfirstlane(p.lens[3 * b + 1]), p.mid_cap);
  const int nr = clampi(__builtin_amdgcn_readfirstlane(p.lens[3 * b + 2]), p.recent_cap);
  const int Sq = static_cast<int>(p.Sq);
  const int jw = qb * kQB * NQB * qpg;                 // the workgroup's first query
  const int jwn = Sq - jw < kQB * NQB * qpg ? Sq - jw : kQB * NQB * qpg;  // its queries
  const int j0 = jw + kQB * (qblk + NQB * wsub);       // this wave's query block
  const int mode = p.mask_mode;
  // chunk keys any query of the workgroup can see (bottom-right: chunk keys 0..j)
  const int cv = mode == FADE_MASK_BOTTOM_RIGHT ? jw + jwn : p.chunk_len;
  // Key tiles never straddle a tier: sink, middle, recent, chunk tiles in turn.
  const int nts = (ns + kKT - 1) / kKT, ntm = (nm + kKT - 1) / kKT, ntr = (nr + kKT - 1) / kKT;
  const int ntc = (cv + kKT - 1) / kKT;
  int n_tiles = nts + ntm + ntr + ntc;
  if (mode == FADE_MASK_TOP_LEFT) {
    // query j sees keys 0..j of the row's sequence: only the tiles that start
    // at or before the block's last query (a prefix of the tile order)
    const int jmax = jw + jwn - 1;
    auto upto = [&](int nt, int off) {
      if (jmax < off) return 0;
      const int c = (jmax - off) / kKT + 1;
      return c < nt ? c : nt;
    };
    n_tiles = upto(nts, 0) + upto(ntm, ns) + upto(ntr, ns + nm) + upto(ntc, ns + nm + nr);
  }
  struct TileRef {
    int seg, base, cnt, gbase;  // segment (0 sink, 1 middle, 2 recent, 3 chunk), first key, keys,
                                // first key's index in the row's sequence
  };
  auto tile_of = [&](int t) {
    TileRef r;
    int len;
    if (t < nts) {
      r.seg = 0; r.base = kKT * t; len = ns; r.gbase = r.base;
    } else if (t < nts + ntm) {
      r.seg = 1; r.base = kKT * (t - nts); len = nm; r.gbase = ns + r.base;
    } else if (t < nts + ntm + ntr) {
      r.seg = 2; r.base = kKT * (t - nts - ntm); len = nr; r.gbase = ns + nm + r.base;
    } else {
      r.seg = 3; r.base = kKT * (t - nts - ntm - ntr); len = cv; r.gbase = ns + nm + nr + r.base;
    }
    r.cnt = len - r.base < kKT ? len - r.base : kKT;
    return r;
  };

  __shared__ __attribute__((aligned(16))) uint16_t kt[2][kKT][KP];
  __shared__ __attribute__((aligned(16))) uint16_t vtt[2][D][kVtPitch];
  __shared__ __attribute__((aligned(16))) float rowf[4 * NQB][32];  // per-wave factors of the 32 query rows
  // middle-tile staging: thread tid's 16 bytes of K codes of pass i at
  // 16 (tid + kThreads i) (token tid / KTHR + TPP i, channels 32 (tid % KTHR) ..);
  // keys 16 w + rho (rho < 16) in stg_v[VWB w ..], 16-byte unit u of row rho at unit
  // UPR rho + (u ^ ((rho >> 1) & (UPR - 1))); their V scales in dwords
  // 64 w + l, key 16 w + (l & 15) (a 2-byte direct load fills one dword per lane)
  __shared__ __attribute__((aligned(16))) uint8_t stg_k[KPS * kThreads * 16];
  __shared__ __attribute__((aligned(16))) uint8_t stg_v[4 * VWB];
  __shared__ __attribute__((aligned(16))) uint32_t stg_s[kThreads];

  // ---- tile fetch: thread = token r of the tile, channels CPT*cp .. CPT*cp+CPT-1 ----
  const int r = gtid >> 2, cp = gtid & 3;
  // middle K staging: thread = tokens mr + TPP i, channels 32*mc .. 32*mc+31 (threads gtid < TPP KTHR)
  const int mr = gtid / KTHR, mc = gtid % KTHR;
  const bool kstage = do_k && (TPP * KTHR == kThreads || gtid < TPP * KTHR);
  // fp16 rows of each segment (0 sink, 1 fp16 middle tier, 2 recent, 3 chunk)
  // of this (row, kv head): K and V row pointers and row strides in halves.
  // They sit in LDS, read (one broadcast per tile) by the few fp16 tiles of a
  // row, so the tile loop keeps no scalar registers for them.
  __shared__ __attribute__((aligned(16))) int64_t segd[4][4];
  if (tid == 0) {
    auto put = [&](int sg, const Tier t) {
      segd[sg][0] = reinterpret_cast<int64_t>(t.k + b * t.k_sb + kvh * t.k_sh);
      segd[sg][1] = reinterpret_cast<int64_t>(t.v + b * t.v_sb + kvh * t.v_sh);
      segd[sg][2] = t.k_ss;
      segd[sg][3] = t.v_ss;
    };
    put(0, p.sink);
    put(2, p.recent);
    put(3, p.chunk);
    // fp16 middle tier: [B, Hkv, cap, D] contiguous
    segd[1][0] = reinterpret_cast<int64_t>(reinterpret_cast<const uint16_t*>(p.kq) + bkv * p.mid_cap * Dr);
    segd[1][1] = reinterpret_cast<int64_t>(reinterpret_cast<const uint16_t*>(p.vq) + bkv * p.mid_cap * Dr);
    segd[1][2] = Dr;
    segd[1][3] = Dr;
  }
  const uint8_t* kq = p.kq + bkv * p.mid_cap * krow;
  const uint8_t* vq = p.vq + bkv * p.mid_cap * krow;
  const uint16_t* vsr = p.vs + bkv * p.mid_cap;

  // K scales of this thread's 32 staged channels as fp16 pairs, in the stored order
  uint32_t ksc[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint4 w = make_uint4(0, 0, 0, 0);
    if (p.has_mid && !p.mid_fp16 && kstage && 32 * mc < Dr) w = *reinterpret_cast<const uint4*>(p.ks + bkv * Dr + 32 * mc + 8 * i);
    const u32x4 st = to_stored(w.x, w.y, w.z, w.w);
#pragma unroll
    for (int e = 0; e < 4; ++e) ksc[4 * i + e] = st[e];
  }
  int fok = 0;  // bit i: this thread's staged middle row of pass i is a real token of the tile
  // staging slots of this wave's lanes (a direct load writes lane l's bytes at base + l * size)
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  const uint32_t stk = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8*)&stg_k[16 * 64 * wq])));
  const uint32_t stv = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8*)&stg_v[VWB * wq])));
  const uint32_t sts = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8*)&stg_s[64 * wq])));
  // Middle tile: codes and V scale to the staging area.  Nothing waits for
  // these loads before store_mid(), so they fly during the current tile's compute.
  auto fetch_mid = [&](const TileRef& tr) {
    // the tile's rows: from row tr.base of this (row, kv head)'s padded tensors,
    // or from row 0 of its page's (page, kv head) block in the pools
    const uint8_t* kq_t = kq;
    const uint8_t* vq_t = vq;
    const uint16_t* vs_t = vsr;
    int row0 = tr.base;
    if (p.pages != nullptr) {
      const int64_t blk = static_cast<int64_t>(p.pages[b * p.ppr + (tr.base >> 6)]) * p.Hkv + kvh;
      kq_t = p.kq + blk * kKT * krow;
      vq_t = p.vq + blk * kKT * krow;
      vs_t = p.vs + blk * kKT;
      row0 = 0;
    }
    fok = 0;
#pragma unroll
    for (int i = 0; i < KPS; ++i) {
      const bool ok = mr + TPP * i < tr.cnt;
      fok |= ok ? 1 << i : 0;
      const int key = row0 + (ok ? mr + TPP * i : tr.cnt - 1);  // rows past the tile: a valid row, zeroed in store_mid()
      if (kstage && 32 * mc < Dr) lds_dma16(kq_t + static_cast<int64_t>(key) * krow + 16 * mc, stk + 16 * kThreads * i);
    }
    // V: unit ul = l + 64 i < 16 UPR of wave w (lane l, load i) fills unit ul
    // of the wave's block: row rho = ul / UPR, source unit
    // (ul % UPR) ^ ((rho >> 1) & (UPR - 1)).  Rows past the tile read the last
    // valid key (finite; their probabilities are zero).
    if (do_v) {
#pragma unroll
      for (int i = 0; i < VPS; ++i) {
        const int ul = lane + 64 * i;
        const int vr = ul / UPR;
        const int vk = 16 * wq + vr;
        const int vu = (ul % UPR) ^ ((vr >> 1) & (UPR - 1));  // the unit's 32 channels in the row
        if ((16 * UPR >= 64 * (i + 1) || ul < 16 * UPR) && 32 * vu < Dr)
          lds_dma16(vq_t + static_cast<int64_t>(row0 + (vk < tr.cnt ? vk : tr.cnt - 1)) * krow + 16 * vu, stv + 1024 * i);
      }
      const int sk2 = 16 * wq + (lane & 15);
      lds_dma2(vs_t + row0 + (sk2 < tr.cnt ? sk2 : tr.cnt - 1), sts);
    }
  };
  // staged codes -> fp16(code * scale) rows of K and V in LDS buffer buf
  auto store_mid = [&](int buf) {
    // the staging loads are the only vector-memory operations in flight here
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const f16x2 m72 = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
    if (do_k) {
#pragma unroll
    for (int pi = 0; pi < KPS; ++pi) {
    uint4 kraw = make_uint4(0, 0, 0, 0);
    if (kstage && ((fok >> pi) & 1) && 32 * mc < Dr)
      kraw = *reinterpret_cast<const uint4*>(&stg_k[16 * (gtid + kThreads * pi)]);
    // codes -> fp16 72 + c -> c -> fp16(c * scale), already in the stored channel order
    const uint32_t kw[4] = {kraw.x, kraw.y, kraw.z, kraw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t o[4];
      u32x4 kd;
      nib_to_f16(kw[i], o);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        kd[e] = BF ? dequant_pair_bf16(o[e], ksc[4 * i + e])
                   : __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, o[e]) + m72) *
                                                      __builtin_bit_cast(f16x2, ksc[4 * i + e]));
      if (kstage) *reinterpret_cast<u32x4*>(&kt[buf][mr + TPP * pi][32 * mc + 8 * i]) = kd;
    }
    }
    }
    if (!do_v) return;
    // V.  Scales of the wave's keys by row rho (low 16 bits of dword 64 w + rho).
    uint32_t sc[16];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const uint4 d = *reinterpret_cast<const uint4*>(&stg_s[64 * wq + 4 * q4]);
      sc[4 * q4] = d.x;
      sc[4 * q4 + 1] = d.y;
      sc[4 * q4 + 2] = d.z;
      sc[4 * q4 + 3] = d.w;
    }
    // As source lane s' = n16 of group g this lane points the tr4 read at row
    // rho(s') = swap23(o(s')), o(s') = 2 (s' & 3) + ((s' >> 2) & 1) + 8 (s' >> 3),
    // channel unit cu = 4 q + g: lane n then receives channel 16 cu + (n ^ 1)
    // of those rows, nibble s' <-> position offset o(s'), so the fp16 pairs
    // come out as position pairs (2 j, 2 j + 1), rows (swap23(2 j), + 1).
    const int so = swap23(2 * (n16 & 3) + ((n16 >> 2) & 1) + 8 * (n16 >> 3));
    const uint8_t* vrow = &stg_v[VWB * wq + KROW * so];
    // channel units of 16: D/16 of them, four per pass of the lane groups
    // (D = 32: groups 2 and 3 repeat units 0 and 1 and store nothing)
#pragma unroll
    for (int q = 0; q < (D / 16 + 3) / 4; ++q) {
      const int cu = (4 * q + g) % (D / 16);
      const bool cu_ok = 4 * q + g < D / 16;
      const i32x2 xv = __builtin_amdgcn_ds_read_tr4_b64_v2i32(reinterpret_cast<lds_i32x2*>(
          const_cast<lds_u8*>((const lds_u8*)(vrow + 16 * ((cu >> 1) ^ ((so >> 1) & (UPR - 1))) + 8 * (cu & 1)))));
      const int ch = 16 * cu + (n16 ^ 1);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        uint32_t o[4];
        nib_to_f16(static_cast<uint32_t>(xv[half]), o);
        u32x4 vd;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int ra = swap23(8 * half + 2 * j);
          const uint32_t s2 = __builtin_amdgcn_perm(sc[ra + 1], sc[ra], 0x05040100u);
          vd[j] = BF ? dequant_pair_bf16(o[j], s2)
                     : __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, o[j]) + m72) * __builtin_bit_cast(f16x2, s2));
        }
        if (cu_ok) *reinterpret_cast<u32x4*>(&vtt[buf][ch][16 * wq + 8 * half]) = vd;
      }
    }
  };
  // fp16 tile (sink, recent or chunk: a few per row; an fp16 middle tier): loaded and stored at once
  auto load_store_f16 = [&](const TileRef& tr, int buf) {
    constexpr int NU = CPT / 8;  // 16-byte units per thread
    uint4 fk[NU], fv[NU];
    const int key = tr.base + r;
    if (r < tr.cnt) {
      typedef int64_t i64x2 __attribute__((ext_vector_type(2)));
      const i64x2 ptr = *reinterpret_cast<const i64x2*>(&segd[tr.seg][0]);
      const i64x2 ss = *reinterpret_cast<const i64x2*>(&segd[tr.seg][2]);
      const uint16_t* kp = reinterpret_cast<const uint16_t*>(ptr.x) + key * ss.x;
      const uint16_t* vp = reinterpret_cast<const uint16_t*>(ptr.y) + key * ss.y;
      const uint4* k4 = reinterpret_cast<const uint4*>(kp + CPT * cp);
      const uint4* v4 = reinterpret_cast<const uint4*>(vp + CPT * cp);
#pragma unroll
      for (int i = 0; i < NU; ++i) {
        const bool in = CPT * cp + 8 * i < Dr;  // units past the head_dim stay zero
        fk[i] = fv[i] = make_uint4(0, 0, 0, 0);
        if (do_k && in) fk[i] = k4[i];
        if (do_v && in) fv[i] = v4[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < NU; ++i) fk[i] = fv[i] = make_uint4(0, 0, 0, 0);
    }
    const int pr = swap23(r);
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      if (do_k)
        *reinterpret_cast<u32x4*>(&kt[buf][r][CPT * cp + 8 * i]) = to_stored(fk[i].x, fk[i].y, fk[i].z, fk[i].w);
      if (do_v) {
        const uint32_t vw[4] = {fv[i].x, fv[i].y, fv[i].z, fv[i].w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          vtt[buf][CPT * cp + 8 * i + e][pr] = static_cast<uint16_t>(vw[e >> 1] >> (16 * (e & 1)));
      }
    }
  };
  // Tile t into LDS buffer buf: fp16 tiles complete here; a middle tile only
  // starts (returns true) and completes in store_mid().
  auto begin_tile = [&](int t, int buf) {
    const TileRef tr = tile_of(t);
    if (tr.seg == 1 && !p.mid_fp16) {
      fetch_mid(tr);
      return true;
    }
    load_store_f16(tr, buf);
    return false;
  };

  // ---- query fragments: B operand of S^T = K Q^T; lane (n32, h) holds query
  // row j0 + n32, channels 16 ks + 8 h .. + 7 in the stored order ----
  const int n32 = lane & 31, h = lane >> 5;
  const bool active = wh < G && j0 < Sq;
  const int64_t hq = kvh * p.G + h0 + (active ? wh : 0);
  u32x4 qf[NKS];
  {
    const int j = j0 + n32;
    const uint16_t* qr = p.q + b * p.q_sb + hq * p.q_sh + static_cast<int64_t>(j < Sq ? j : Sq - 1) * p.q_ss;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const uint4 w = (active && j < Sq && 16 * ks + 8 * h < Dr) ? *reinterpret_cast<const uint4*>(qr + 16 * ks + 8 * h)
                                                                : make_uint4(0, 0, 0, 0);
      qf[ks] = to_stored(w.x, w.y, w.z, w.w);
    }
  }

  // O accumulators: acc[cb] lane (n32, h), register i <-> query row 8 (i / 4) + 4 h + i % 4,
  // channel 32 cb + n32
  f32x16 acc[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[cb][i] = 0.0f;
  float m_run = kNegBig, l_run = 0.0f;  // of query row n32 (the same in both halves; l_run over this half's keys)
  const float sl2 = p.scale_log2;
  float* const rf = &rowf[wave][0];

  auto compute = [&](int t, int buf) {
    const TileRef tr = tile_of(t);
    // S^T (raw scores q.k) for key blocks kb = 0, 1
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[kb][i] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(&kt[buf][32 * kb + n32][16 * ks + 8 * h]);
        s[kb] = mfma32x32<BF>(a, qf[ks], s[kb]);
      }
    }
    // bottom-right: every key of a full cache tile is visible to every query of
    // the block; top-left: a full tile that ends at or before the block's first query
    const bool full = tr.cnt == kKT && (mode == FADE_MASK_NONE || (mode == FADE_MASK_BOTTOM_RIGHT && tr.seg != 3) ||
                                        (mode == FADE_MASK_TOP_LEFT && tr.gbase + kKT - 1 <= j0));
    if (!full) {
      const int jq = j0 + n32;
      // key kk of the tile is visible when kk < cnt and, bottom-right, in the chunk base + kk <= jq;
      // top-left, gbase + kk <= jq
      int lim = tr.cnt;
      if (mode == FADE_MASK_BOTTOM_RIGHT && tr.seg == 3) lim = jq - tr.base + 1 < tr.cnt ? jq - tr.base + 1 : tr.cnt;
      if (mode == FADE_MASK_TOP_LEFT) lim = jq - tr.gbase + 1 < tr.cnt ? jq - tr.gbase + 1 : tr.cnt;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (32 * kb + 8 * (i >> 2) + 4 * h + (i & 3) >= lim) s[kb][i] = -INFINITY;
    }
    // probabilities exp2((x - m) * scale) against the running max m (raw score
    // units), as fp16 (bfloat16 in a BF instance): PV A operands, k-step s =
    // registers 8 (s & 1) .. + 7 of key block s >> 1
    u32x4 pa[4];
    auto probs = [&]() {
      const float nm = -m_run * sl2;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          if constexpr (BF) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              pa[2 * kb + hf][j] = pack_bf16(__builtin_amdgcn_exp2f(fmaf(s[kb][8 * hf + 2 * j], sl2, nm)),
                                             __builtin_amdgcn_exp2f(fmaf(s[kb][8 * hf + 2 * j + 1], sl2, nm)));
          } else {
            f16x8 ph;
#pragma unroll
            for (int j = 0; j < 8; ++j) ph[j] = static_cast<_Float16>(__builtin_amdgcn_exp2f(fmaf(s[kb][8 * hf + j], sl2, nm)));
            pa[2 * kb + hf] = __builtin_bit_cast(u32x4, ph);
          }
        }
    };
    probs();
    // The running max moves only when a score exceeds it by more than kTau
    // (log2 units), i.e. when a probability exceeds 2^kTau (inf included): a
    // packed max over the probabilities finds those tiles (fp16; bfloat16 as
    // unsigned 16-bit patterns, which order like the non-negative values);
    // the exact fp32 max is taken on them alone.
    bool over;
    if constexpr (BF) {
      const u16x8 pm = __builtin_elementwise_max(
          __builtin_elementwise_max(__builtin_bit_cast(u16x8, pa[0]), __builtin_bit_cast(u16x8, pa[1])),
          __builtin_elementwise_max(__builtin_bit_cast(u16x8, pa[2]), __builtin_bit_cast(u16x8, pa[3])));
      uint16_t mx = pm[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) mx = mx > pm[j] ? mx : pm[j];
      over = mx > 0x4380u;  // bfloat16 2^8
    } else {
      const f16x8 pm = __builtin_elementwise_max(
          __builtin_elementwise_max(__builtin_bit_cast(f16x8, pa[0]), __builtin_bit_cast(f16x8, pa[1])),
          __builtin_elementwise_max(__builtin_bit_cast(f16x8, pa[2]), __builtin_bit_cast(f16x8, pa[3])));
      const f16x2 pm2 =
          __builtin_elementwise_max(__builtin_elementwise_max(pm.s01, pm.s23), __builtin_elementwise_max(pm.s45, pm.s67));
      over = static_cast<float>(pm2.x) > kTauP || static_cast<float>(pm2.y) > kTauP;
    }
    if (__builtin_amdgcn_ballot_w64(over) != 0) {
      float lmax = kNegBig;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; i += 2) lmax = fmaxf(lmax, fmaxf(s[kb][i], s[kb][i + 1]));
      lmax = fmaxf(lmax, __shfl_xor(lmax, 32, 64));
      const float m_new = fmaxf(m_run, lmax);
      const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * sl2);
      m_run = m_new;
      l_run *= alpha;
      // the accumulator rows of this lane belong to other lanes' queries: via LDS
      if (h == 0) rf[n32] = alpha;
      __builtin_amdgcn_s_waitcnt(kLgkm0);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 a4 = *reinterpret_cast<const f32x4*>(&rf[8 * q + 4 * h]);
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[cb][4 * q + i] *= a4[i];
      }
      probs();
    }
    // the row sum of the same 16-bit probabilities PV multiplies: fp32 dot products with 1
    {
      float ps = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const u32x4 w = pa[k];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t we = w[e];
          if constexpr (BF) {
            const bf16x2 one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
            ps = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, we), one, ps, false);
          } else {
            const f16x2 one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
            ps = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, we), one, ps, false);
          }
        }
      }
      l_run += ps;
    }
    // O += P V.  B operand: lane (n32, h) reads channel 32 cb + n32 at V^T
    // positions 16 s + 8 h .. + 7 (keys 16 s + 8 (j >> 2) + 4 h + (j & 3)).
#pragma unroll
    for (int ks2 = 0; ks2 < 4; ++ks2)
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const u32x4 bv = *reinterpret_cast<const u32x4*>(&vtt[buf][32 * cb + n32][16 * ks2 + 8 * h]);
        acc[cb] = mfma32x32<BF>(pa[ks2], bv, acc[cb]);
      }
  };

  __syncthreads();  // segd
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
  // ---- normalize and store: 1 / l of each query row through LDS ----
  {
    const float lt = l_run + __shfl_xor(l_run, 32, 64);
    if (h == 0) rf[n32] = 1.0f / lt;
    __builtin_amdgcn_s_waitcnt(kLgkm0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 inv4 = *reinterpret_cast<const f32x4*>(&rf[8 * q + 4 * h]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = j0 + 8 * q + 4 * h + i;
        if (j < Sq) {
          uint16_t* orow = p.out + b * p.o_sb + hq * p.o_sh + static_cast<int64_t>(j) * p.o_ss;
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb)
            if (32 * cb + n32 < Dr) orow[32 * cb + n32] = f2w<BF>(acc[cb][4 * q + i] * inv4[i]);
        }
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
  if (a->D < 8 || a->D > 256 || a->D % 8 != 0)
    return einval("fade_tiered_prefill_attn: head_dim must be a multiple of 8 in [8, 256], got %lld", (long long)a->D);
  if (a->B <= 0 || a->Hq <= 0 || a->Hkv <= 0 || a->Sq <= 0)
    return einval("fade_tiered_prefill_attn: B, Hq, Hkv and Sq must be positive");
  if (a->Hq % a->Hkv != 0 || a->Hq / a->Hkv > 8)
    return einval("fade_tiered_prefill_attn: needs Hq %% Hkv == 0 and Hq/Hkv <= 8 (got %lld/%lld)",
                  (long long)a->Hq, (long long)a->Hkv);
  if (a->B > 65535 || a->Hkv > 65535 || a->Sq > (1 << 24)) return einval("fade_tiered_prefill_attn: shape too large");
  if (a->q == nullptr || a->out == nullptr || a->lens == nullptr)
    return einval("fade_tiered_prefill_attn: null q, out or lens");
  if (!aligned16(a->q) || (a->q_sb | a->q_sh | a->q_ss) % 8)
    return einval("fade_tiered_prefill_attn: q rows must be 16-byte aligned");
  if (a->dtype != FADE_DTYPE_F16 && a->dtype != FADE_DTYPE_BF16)
    return einval("fade_tiered_prefill_attn: dtype must be FADE_DTYPE_F16 or FADE_DTYPE_BF16, got %d", a->dtype);
  if (a->mask_mode != FADE_MASK_BOTTOM_RIGHT && a->mask_mode != FADE_MASK_TOP_LEFT && a->mask_mode != FADE_MASK_NONE)
    return einval("fade_tiered_prefill_attn: unknown mask_mode %d", a->mask_mode);
  if (a->mask_mode == FADE_MASK_BOTTOM_RIGHT && a->chunk.len != a->Sq)
    return einval("fade_tiered_prefill_attn: chunk tier must hold Sq tokens");
  if (a->chunk.len < 0 || a->chunk.len > (1 << 24)) return einval("fade_tiered_prefill_attn: bad chunk length");
  if (!tier_ok(a->sink) || !tier_ok(a->recent) || !tier_ok(a->chunk))
    return einval("fade_tiered_prefill_attn: fp16 tiers need 16-byte aligned rows");
  const fade_mid_tier& m = a->mid;
  const bool has_mid = m.len > 0 && m.fmt != FADE_MID_NONE;
  const bool mid_fp16 = has_mid && m.fmt == FADE_MID_FP16;
  if (has_mid && mid_fp16) {
    if (!m.k_codes || !m.v_codes || !aligned16(m.k_codes) || !aligned16(m.v_codes))
      return einval("fade_tiered_prefill_attn: fp16 middle tier pointers missing or misaligned");
    if (m.pages != nullptr) return einval("fade_tiered_prefill_attn: an fp16 middle tier cannot be paged");
  } else if (has_mid) {
    if (m.fmt != FADE_MID_SYM || m.k_bits != 4 || m.v_bits != 4)
      return einval("fade_tiered_prefill_attn: the middle tier must be FADE_MID_SYM 4-bit or FADE_MID_FP16");
    if (a->D % 32 != 0)
      return einval("fade_tiered_prefill_attn: a packed middle tier needs head_dim %% 32 == 0 (got %lld); "
                    "pass it as an fp16 middle tier", (long long)a->D);
    if (!m.k_codes || !m.v_codes || !m.k_scale || !m.v_scale || !aligned16(m.k_codes) || !aligned16(m.v_codes) ||
        (reinterpret_cast<uintptr_t>(m.k_scale) & 15))
      return einval("fade_tiered_prefill_attn: middle tier pointers missing or misaligned");
    if (m.pages != nullptr && (m.page_stride != 0 || m.pages_per_row * kKT < m.len))
      return einval("fade_tiered_prefill_attn: a paged middle tier needs separate pools and pages_per_row * 64 >= len");
  }
  PParams p{};
  p.B = a->B;
  p.Hq = a->Hq;
  p.Hkv = a->Hkv;
  p.Sq = a->Sq;
  p.G = static_cast<int>(a->Hq / a->Hkv);
  p.passes = (p.G + 3) / 4;
  p.hpw = p.G >= 3 ? 4 : p.G;
  const int qpg = 4 / p.hpw;  // query blocks per group of 4 waves
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
  p.mid_fp16 = mid_fp16 ? 1 : 0;
  p.mid_cap = has_mid ? m.len : 0;
  p.sink_cap = a->sink.len;
  p.recent_cap = a->recent.len;
  p.kq = static_cast<const uint8_t*>(m.k_codes);
  p.ks = static_cast<const uint16_t*>(m.k_scale);
  p.vq = static_cast<const uint8_t*>(m.v_codes);
  p.vs = static_cast<const uint16_t*>(m.v_scale);
  p.pages = has_mid ? m.pages : nullptr;
  p.ppr = has_mid ? m.pages_per_row : 0;
  p.mask_mode = a->mask_mode;
  p.chunk_len = static_cast<int>(a->chunk.len);
  p.D = static_cast<int>(a->D);
  // two groups of 4 waves once one group's query blocks do not cover the chunk
  // (one at head_dim > 128)
  const int nqb = a->Sq > kQB * qpg && a->D <= 128 ? 2 : 1;
  const dim3 grid(static_cast<unsigned>(cdiv(a->Sq, kQB * nqb * qpg) * p.passes), static_cast<unsigned>(a->Hkv),
                  static_cast<unsigned>(a->B));
  const bool bf = a->dtype == FADE_DTYPE_BF16;
#define FADE_PREFILL_LAUNCH(DD)                                                                                        \
  if (bf && nqb == 2) hipLaunchKernelGGL((prefill_kernel<DD, 2, true>), grid, dim3(2 * kThreads), 0, as_stream(stream), p); \
  else if (bf) hipLaunchKernelGGL((prefill_kernel<DD, 1, true>), grid, dim3(kThreads), 0, as_stream(stream), p);           \
  else if (nqb == 2) hipLaunchKernelGGL((prefill_kernel<DD, 2, false>), grid, dim3(2 * kThreads), 0, as_stream(stream), p); \
  else hipLaunchKernelGGL((prefill_kernel<DD, 1, false>), grid, dim3(kThreads), 0, as_stream(stream), p);
  // the smallest instance whose capacity covers the head_dim
  if (a->D <= 32) { FADE_PREFILL_LAUNCH(32) }
  else if (a->D <= 64) { FADE_PREFILL_LAUNCH(64) }
  else if (a->D <= 128) { FADE_PREFILL_LAUNCH(128) }
  else if (bf) hipLaunchKernelGGL((prefill_kernel<256, 1, true>), grid, dim3(kThreads), 0, as_stream(stream), p);
  else hipLaunchKernelGGL((prefill_kernel<256, 1, false>), grid, dim3(kThreads), 0, as_stream(stream), p);
#undef FADE_PREFILL_LAUNCH
  return check_launch("fade_tiered_prefill_attn");
}
