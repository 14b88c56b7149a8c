// Packed-tier decode attention kernel template (included by decode_int4.hip,
// fp16 instances, and decode_int4_bf16.hip, bf16 instances).
#pragma once

// Matrix-core decode attention over a packed middle tier for GQA groups of up
// to four query heads per kv head, gfx950: the reference INT4 format
// (per-channel K scales, per-token V scales; fade/quant.py:61-92), the rotated
// 2-bit format, the reference K4 + literal grouped INT2 V format
// (fade/quant.py:130-150) and the asymmetric group-32 build formats.
//
// Workgroup = NW wavefronts serving one (batch row, kv head, split).  Each
// wave runs its own online softmax over the tiles it takes: two fixed ones,
// then tiles claimed one at a time from an LDS counter, so faster waves take
// more.  The waves are merged through LDS, and the last workgroup of a
// (batch row, kv head) to finish merges the splits (no second launch).
//
// Block-diagonal tile layout.  A packed tile is 64 tokens = four 16-token
// sub-tiles s.  QK^T runs on int8 MFMA 16x16x64 whose k dimension carries 16
// channels of each of the four sub-tiles (k = 16*sigma + j) and whose 16
// columns are (head h, sub-tile s) = 4h + s; the query operand is zero unless
// s == sigma, so C[m][4h+s] = score(head h, token 16s + m).  With four heads
// every lane then owns four real scores:
//
//   lane = 16g + 4h + s, register i   <->   head h, token 16s + 4g + i
//
// which is also, unchanged, the A operand layout of the f16 MFMA 16x16x32 of
// P*V (rows 4h+s, k slots 8g..8g+7 = sub-tiles (sa, sb) x 4 tokens), and the
// PV accumulator lands as lane (n, g), register i  <->  head g, sub-tile i,
// channel n: the sum over sub-tiles is lane-local.  Softmax work per token
// is therefore done once, by one lane (not by 16 lanes of mostly padding).
//
// K codes: lane l loads the 64-byte row of token l straight into VGPRs; the
// two's-complement nibbles become int8 16*c with one AND (high nibbles) or a
// shift+AND (low nibbles), and the factor 16 is folded into the score scale.
// The query times the per-channel K scale is quantized per head to 16 bits
// and split into two int8 digits (hi*256 + lo); score = hi_acc*256 + lo_acc.
//
// V codes: HBM -> LDS by direct loads (swizzled 16-byte units), transposed
// by ds_read_b64_tr_b4 so that each lane receives one channel of 16 tokens,
// turned into fp16 64 + u (u = c + 8 in mantissa bits 4..7) with a shift and
// an AND-OR; P is pre-multiplied by the per-token V scale, and the constant
// 72 per token is removed at the end through an MFMA-accumulated 72 * sum(P').
//
// 2-bit variant (rotated backend, fade/rotated_quant.py:35-88,106-187: K per
// channel, V per token, four codes per byte MSB-first): K codes become int8
// 64*c (shift + AND per code position); a tr4 read now gives each lane two
// channels of 16 tokens (one nibble = two codes), each code becomes the fp16
// value 4 + u (u = c + 2 in mantissa bits 8..9), the per-token offset is 6.
//
// Asymmetric group-32 formats (build format; per-token scale and zero for
// each 32-channel group, unsigned codes): the K operand carries the codes as
// offset binary (16*(u - 8) or 64*(u - 2), one extra XOR folded into the
// AND), the QK^T MFMAs accumulate each channel group separately, and the
// score is sum_g s_g * qsc * (hi*256 + lo + 128*sum(q digits of g)) plus
// sum_g z_g * sum(q of g).  On the V side P is multiplied by each group's
// per-token scale (four P' operands) and the zero points accumulate
// lane-locally as sum_t p_t * z_t,g.  The query digits are read from LDS
// per tile (registers go to the per-group accumulators instead).
//
// fp16 tokens (sink + recent) form 16-token tiles handled with f16 MFMAs in
// the same fragment layout (sub-tile 0 only).
//
// Eight heads per pass (H8, GQA 5-8, symmetric formats).  A 64-token tile is
// two 32-token groups of two 16-token sub-tiles; QK^T's 16 columns are
// (head h, sub-tile s) = 2h + s and its k dimension carries 32 channels of
// each of the two sub-tiles (lane half g & 1 takes channel half 64 (g & 1),
// k-step ks its channels 16 ks .. 16 ks + 15), so a lane owns eight scores:
//
//   lane = 16g + 2h + s, register i of group q   <->   head h, token 32q + 16s + 4g + i
//
// The PV operand and MFMAs are those of four heads (rows 2h + s instead of
// 4h + s; groups 0 and 1 are the a0 / a1 token halves), and the accumulator
// register i of lane (n, g) holds head 2g + i / 2: the sum over sub-tiles is
// still lane-local.  Each kv tile is read once for up to eight heads, at the
// MFMA and V-conversion cost of four and twice the softmax work.
#include <math.h>

#include "decode_common.h"
#include "lds_dma.h"

namespace fade {
namespace decode {
namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
typedef __attribute__((address_space(3))) uint8_t lds_u8;

constexpr int kHeads = 4;               // query heads per kv head the layout serves
constexpr int kTile = 64;                // tokens of a packed tile
constexpr int kMini = 16;                // tokens of an fp16 tile
constexpr int kGroups = 4;               // 32-channel groups of the asymmetric formats
// One ring stage holds one tile: K codes at 0 (fp16 tile: K rows [16][256 B]),
// V codes at 4096 (fp16 tile: V rows [16][256 B]), then the per-token metadata:
// reference formats: V scales, one dword per token, at 8192;
// asymmetric formats: K scale | K zero | V scale | V zero, [64 tokens][4 groups]
// fp16 each, right after the V codes.
constexpr int kStageK = 0, kStageV = 4096;
enum { kFmtSym = 0, kFmtAsym = 1, kFmtLit = 2 };
template <int KB, int VB, int FMT>
struct Stage {
  static constexpr int kMeta = FMT == kFmtAsym ? kStageV + 1024 * VB : (FMT == kFmtLit ? kStageV + 8192 : 8192);
  static constexpr int kBytes = FMT == kFmtAsym ? (kMeta + 2048 > 8192 ? kMeta + 2048 : 8192) : kMeta + 256;
  // direct-to-LDS loads per packed tile (K and V codes in 1 KB loads, then the
  // metadata: one 2-byte or dword load, or eight dword loads) and per fp16 tile
  static constexpr int kOps = KB + VB + (FMT == kFmtAsym ? 8 : 1);
  static constexpr int kOpsF16 = FMT == kFmtSym ? 9 : 8;
};
constexpr int kQdZero = 8 * 2 * 4 * 16;  // zero operand after the [ks][digit][head][16 B] query digits
constexpr float kQMax = 32000.0f;
constexpr float kNegBig = -1.0e30f;      // running-max sentinel (finite: no inf - inf)
constexpr float kTau = 8.0f;             // the running max moves only when a score exceeds it by kTau (log2)

__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(a))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(b))) << 16);
}

// 16-bit operands of the instance's dtype (BF: bfloat16, else fp16), as bit
// patterns: a probability pair, and the f32-accumulating MFMAs of PV and of
// the fp16-tier tiles.
template <bool BF>
__device__ __forceinline__ uint32_t pack_w(float a, float b) {
  if constexpr (BF) return pack_bf16(a, b);
  else return pack_f16(a, b);
}
template <bool BF>
__device__ __forceinline__ f32x4 mfma32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
template <bool BF>
__device__ __forceinline__ f32x4 mfma16(i32x2 a, i32x2 b, f32x4 c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4, a), __builtin_bit_cast(bf16x4, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
}

// Output column n of channel tile c (PV accumulator) <-> head-dim channel.
// 8-bit (literal INT2 V): channel 16c + n.
// 4-bit: a tr4 read gives lane n the nibble of channel 16c + (n ^ 1).  2-bit:
// chunk c/2 of 32 channels, lane n holds the codes of channels
// 4(n/2) + 2(1 - n%2) + {0, 1} (first / second code of the nibble = c%2).
template <int BITS>
__device__ __forceinline__ int out_channel(int c, int n) {
  if (BITS == 8) return 16 * c + n;  // tr8 reads: lane n holds channel 16c + n
  if (BITS == 4) return 16 * c + (n ^ 1);
  return 32 * (c >> 1) + 4 * (n >> 1) + 2 * (1 - (n & 1)) + (c & 1);
}

// Two's-complement 2-bit codes of eight nibbles (first code in bits 2..3 of a
// nibble, second in bits 0..1) -> fp16 pairs (nibble j, nibble j+4) of value
// 6 + c: the code goes to mantissa bits 8..9 of 4.0 (0x4400) with its sign bit
// flipped (c + 2); mask = 0x03000300, cst = 0x46004600.  bfloat16 (BF): bits
// 5..6 of 4.0 (0x4080, one code step = 1.0 as well); mask = 0x00600060,
// cst = 0x40C040C0.
template <bool BF>
__device__ __forceinline__ void v2_nibbles_to_f16(uint32_t w, uint32_t mask, uint32_t cst, uint32_t (&of)[4],
                                                  uint32_t (&os)[4]) {
  if constexpr (BF) {
    of[0] = ((w << 3) & mask) ^ cst;
    of[1] = ((w >> 1) & mask) ^ cst;
    of[2] = ((w >> 5) & mask) ^ cst;
    of[3] = ((w >> 9) & mask) ^ cst;
    os[0] = ((w << 5) & mask) ^ cst;
    os[1] = ((w << 1) & mask) ^ cst;
    os[2] = ((w >> 3) & mask) ^ cst;
    os[3] = ((w >> 7) & mask) ^ cst;
  } else {
    of[0] = ((w << 6) & mask) ^ cst;
    of[1] = ((w << 2) & mask) ^ cst;
    of[2] = ((w >> 2) & mask) ^ cst;
    of[3] = ((w >> 6) & mask) ^ cst;
    os[0] = ((w << 8) & mask) ^ cst;
    os[1] = ((w << 4) & mask) ^ cst;
    os[2] = (w & mask) ^ cst;
    os[3] = ((w >> 4) & mask) ^ cst;
  }
}

// Eight two's-complement nibbles -> fp16 pairs (nibble j, nibble j+4) of value
// 72 + c: the nibble goes to mantissa bits 4..7 of 64.0 (0x5400, one code step
// = 1.0) and its top bit is flipped (c + 8, offset binary).  mask = 0x00F000F0
// and cst = 0x54805480 arrive in registers so that each pair is one v_bitop3
// ((a & mask) ^ cst) after a shift.  bfloat16 (BF): mantissa bits 1..4 of
// 64.0 (0x4280, one code step = 1.0 as well); mask = 0x001E001E,
// cst = 0x42904290.
template <bool BF>
__device__ __forceinline__ void v_nibbles_to_f16(uint32_t w, uint32_t mask, uint32_t cst, uint32_t (&o)[4]) {
  if constexpr (BF) {
    o[0] = ((w << 1) & mask) ^ cst;
    o[1] = ((w >> 3) & mask) ^ cst;
    o[2] = ((w >> 7) & mask) ^ cst;
    o[3] = ((w >> 11) & mask) ^ cst;
  } else {
    o[0] = ((w << 4) & mask) ^ cst;
    o[1] = (w & mask) ^ cst;
    o[2] = ((w >> 4) & mask) ^ cst;
    o[3] = ((w >> 8) & mask) ^ cst;
  }
}

struct FpRow {
  const uint16_t* k;
  const uint16_t* v;
};

// Tile loads: non-temporal (read once per launch) unless NT is false (the two
// head passes of GQA 5-8 read every tile twice).
template <bool NT>
__device__ __forceinline__ void tile_dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  if constexpr (NT) lds_dma16_nt(sbase, voff, lds);
  else lds_dma16(sbase, voff, lds);
}
template <bool NT>
__device__ __forceinline__ void tile_dma16(const void* g, uint32_t lds) {
  if constexpr (NT) lds_dma16_nt(g, lds);
  else lds_dma16(g, lds);
}
template <bool NT>
__device__ __forceinline__ void tile_dma4(const void* sbase, uint32_t voff, uint32_t lds) {
  if constexpr (NT) lds_dma4_nt(sbase, voff, lds);
  else lds_dma4(sbase, voff, lds);
}
template <bool NT>
__device__ __forceinline__ void tile_dma2(const void* sbase, uint32_t voff, uint32_t lds) {
  if constexpr (NT) lds_dma2_nt(sbase, voff, lds);
  else lds_dma2(sbase, voff, lds);
}
template <bool NT>
__device__ __forceinline__ void tile_dma2(const void* g, uint32_t lds) {
  if constexpr (NT) lds_dma2_nt(g, lds);
  else lds_dma2(g, lds);
}

__device__ __forceinline__ float half_of(uint32_t dw, int hi) {
  return h2f(static_cast<uint16_t>(hi ? dw >> 16 : dw & 0xFFFFu));
}

// Literal INT2 V rows (128 B, eight 16-byte units) in LDS: unit u of row r
// sits at unit u ^ lit_swz(r), so that the 16 rows one tr8 read pass touches
// (rows 16a + 4g + i, a and g in {0, 1} or {2, 3} ...) fall in distinct banks.
__device__ __forceinline__ int lit_swz(int r) { return ((r >> 1) & 3) | ((r >> 2) & 4); }

// LDS: two ring stages per wave (8.25 KB for the reference INT4 / 2-bit
// formats, 8 or 10 KB for the asymmetric ones, 12.25 KB for literal INT2 V).
// NW waves per workgroup (4, 6 or 8; see packed_kernel); registers are sized
// for two waves per SIMD.
// s_waitcnt vmcnt(c) for a run-time c = i A + j F (i + j <= NS: loads of
// i packed and j fp16 tiles): s_waitcnt takes an immediate, so every count
// the ring can reach has its own instruction.
template <int A, int F, int NS, int I = 0, int J = 0>
__device__ __forceinline__ void wait_vm_dispatch(int c) {
  if constexpr (I > NS) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // not reached: every count is listed
  } else if constexpr (I + J > NS) {
    wait_vm_dispatch<A, F, NS, I + 1, 0>(c);
  } else {
    static_assert(I * A + J * F <= 63, "more loads in flight than vmcnt counts");
    if (c == I * A + J * F) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(I * A + J * F));
      return;
    }
    wait_vm_dispatch<A, F, NS, I, J + 1>(c);
  }
}

// NS: ring stages per wave (tiles in flight while one is computed: NS - 1).
// BF: the query, the fp16-tier K/V, the symmetric formats' scales and the
// output are bfloat16 (else fp16); probabilities and V codes then enter the
// PV MFMAs as bfloat16 too.
// H8: eight query heads per pass (GQA 5-8, symmetric formats; partials and
// split counter laid out as the two-pass instance's, heads 4..7 in the second
// pass's slot).
template <int KB, int VB, int FMT, int NW, bool DET, bool TWO, bool H8, bool BF, bool ROT, int NS>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_packed_kernel(
    Params p) {
  constexpr int kWaves = NW, kThreads = 64 * NW;
  static_assert(!H8 || (FMT == kFmtSym && !TWO), "eight heads per pass: symmetric formats, one pass");
  constexpr int kHP = H8 ? 8 : kHeads;  // query heads a workgroup serves
  constexpr int kNX = H8 ? 8 : 4;       // scores per lane and packed tile
  constexpr int kQdBytes = H8 ? 4 * 2 * 8 * 2 * 16 : 8 * 2 * 4 * 16;  // query digits, then 16 zero bytes
  constexpr int kNKs = H8 ? 4 : 8;      // query-digit k-steps held in registers
  constexpr bool ASYM = FMT == kFmtAsym;  // asymmetric group-32 formats
  constexpr bool LIT = FMT == kFmtLit;    // K4 + literal grouped INT2 V (int8 codes)
  using S = Stage<KB, VB, FMT>;
  constexpr int kOps = S::kOps, kOpsF16 = S::kOpsF16, kMeta = S::kMeta;
  constexpr int kRowK = 16 * KB, kRowV = 16 * VB;  // packed row bytes of one token
  constexpr bool kNT = !TWO;                       // tiles are read once per launch
  const int split = blockIdx.x;
  // blockIdx.y = (kv head, head pass): a pass serves up to 4 of the kv head's
  // G query heads, from head h0 of the group (G = 5..8 takes two passes)
  // (TWO: the two-pass instance, for G = 5..8; one pass otherwise)
  const int64_t kvh = TWO ? blockIdx.y >> 1 : blockIdx.y, b = blockIdx.z;
  const int h0 = TWO ? 4 * static_cast<int>(blockIdx.y & 1) : 0;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, g = lane >> 4;
  // head / sub-tile of this lane's scores
  const int hq = H8 ? n16 >> 1 : n16 >> 2, sq = H8 ? n16 & 1 : n16 & 3;
  const int G = TWO ? (p.G - h0 < kHeads ? p.G - h0 : kHeads) : p.G;  // query heads of this pass
  const int64_t bkv = b * p.Hkv + kvh;                    // the kv pair: tier addressing
  // split counter / partials of this pass (H8: the first of the two-pass slots)
  const int64_t slot = TWO ? 2 * bkv + (h0 >> 2) : (H8 ? 2 * bkv : bkv);
  // Mc: rows of the middle tensors per (batch row, kv head); M, ns, F: this
  // row's middle, sink and fp16 token counts (per-row lengths when given,
  // clamped to the capacities)
  const int64_t Mc = p.mid.len;
  int64_t M = Mc, ns = p.sink.len, F = p.total - Mc;
  int64_t nFt = p.n_f16_tiles;
  if (p.lens != nullptr) {
    const int64_t ls = __builtin_amdgcn_readfirstlane(p.lens[3 * b]);
    const int64_t lm = __builtin_amdgcn_readfirstlane(p.lens[3 * b + 1]);
    const int64_t lr = __builtin_amdgcn_readfirstlane(p.lens[3 * b + 2]);
    ns = ls < 0 ? 0 : (ls < p.sink.len ? ls : p.sink.len);
    M = lm < 0 ? 0 : (lm < Mc ? lm : Mc);
    F = ns + (lr < 0 ? 0 : (lr < p.recent.len ? lr : p.recent.len));
    nFt = (F + kMini - 1) / kMini;
  }
  const int64_t nT = nFt + (M + kTile - 1) / kTile;
  // rotated middle tier: split 0 takes the fp16 tiles, splits 1.. the middle
  // tiles, so that every split's partial lies in one basis
  static_assert(!ROT || FMT == kFmtSym, "the rotated backend's middle tier is symmetric");
  static_assert(!BF || FMT != kFmtAsym, "asymmetric tiers come from fp16 caches only");
  constexpr bool rot = ROT;  // the ROT instances serve p.rot != nullptr
  const int64_t t0 = !rot ? static_cast<int64_t>(split) * p.tiles_per_split
                          : (split == 0 ? 0 : nFt + static_cast<int64_t>(split - 1) * p.tiles_per_split);
  const int64_t t1 = rot && split == 0 ? nFt : (t0 + p.tiles_per_split < nT ? t0 + p.tiles_per_split : nT);
  // Tiles of the split: the first two of each wave are t0 + wave and
  // t0 + NW + wave; after that waves claim tiles t0 + 2 NW + c in order
  // through an LDS counter, so that a wave that runs faster (e.g. the older
  // wave of a SIMD, which wins issue arbitration) takes more of them.  The
  // DET instance (p.deterministic) has wave w walk t0 + w, t0 + w + NW, ...
  // instead, so the order of every fp32 sum is fixed.
  const int n = p.n_splits;
  __shared__ int claim_s;
  if (tid == 0) claim_s = 0;

  __shared__ __attribute__((aligned(16))) uint8_t ring[NS][kWaves][S::kBytes];
  __shared__ __attribute__((aligned(16))) uint32_t qraw_s[kHP][kD / 2];  // fp16 query rows
  __shared__ __attribute__((aligned(16))) uint32_t ksraw_s[ASYM ? 1 : kHeads][kD / 2];  // K scales (waves 0..3)
  __shared__ __attribute__((aligned(16))) uint8_t qd_s[kQdBytes + 16];
  __shared__ float qsc_s[kHP];
  __shared__ int qoff_s[4][kGroups];    // asymmetric: 128 * sum of the query digits of a group
  __shared__ float qg_s[4][kGroups];    // asymmetric: sum of the query of a group (log2 domain)
  __shared__ float red_m[kWaves][kHP], red_l[kWaves][kHP];
  __shared__ float qrot_s[ROT ? kHP : 1][ROT ? kD : 1];  // q R^T (rotated tier)
  __shared__ int last_s;

  // Paged middle tier: per-token tensors are pools [page][Hkv][64][...] and
  // the split's page ids (middle tiles mt_lo .. of this row) sit in LDS, read
  // with plain loads before any tile DMA is in flight.  Unpaged: the row's
  // block of Mc token rows.
  const bool paged = !LIT && p.mid.pages != nullptr;
  __shared__ int32_t pages_s[kPageSlots];
  const int64_t mt_lo = (t0 > nFt ? t0 : nFt) - nFt;
  if (paged) {
    const int64_t mt_hi = (t1 > nFt ? t1 : nFt) - nFt;
    const int64_t cnt = mt_hi - mt_lo < kPageSlots ? mt_hi - mt_lo : kPageSlots;
    for (int64_t i = tid; i < cnt; i += kThreads) pages_s[i] = p.mid.pages[b * p.mid.pages_per_row + mt_lo + i];
    __syncthreads();
  }
  const int64_t rb0 = paged ? 0 : bkv * Mc;  // token-row base of the row's block
  const uint8_t* kc = p.mid.k_codes + rb0 * kRowK;
  // literal INT2 V: [v_rows][128] int8 codes and [v_rows / 64][128] scales per
  // (batch row, kv head), v_rows = the middle length padded to 64 (pad rows are 0)
  const uint8_t* vc = p.mid.v_codes + (LIT ? bkv * p.mid.v_rows : rb0) * kRowV;
  // reference formats: V scale per token; asymmetric: [token][4 groups] scale / zero
  const uint16_t* vsg =
      LIT ? p.mid.v_scale + bkv * (p.mid.v_rows / kTile) * kD : p.mid.v_scale + rb0 * (ASYM ? kGroups : 1);
  const uint16_t* ksg = ASYM ? p.mid.k_scale + rb0 * kGroups : nullptr;
  const uint16_t* kzg = ASYM ? p.mid.k_zero + rb0 * kGroups : nullptr;
  const uint16_t* vzg = ASYM ? p.mid.v_zero + rb0 * kGroups : nullptr;
  const int64_t Hkv = p.Hkv;
  const int64_t pstride = (!ASYM && paged) ? p.mid.page_stride : 0;
  // fp16 tiers as (uniform) locals: the lambdas below must not read the kernel
  // arguments through a pointer (that becomes a per-lane global load whose
  // compiler-inserted vmcnt wait would also wait for the tile prefetches).
  const uint16_t* const sk = p.sink.k + b * p.sink.k_sb + kvh * p.sink.k_sh;
  const uint16_t* const sv = p.sink.v + b * p.sink.v_sb + kvh * p.sink.v_sh;
  const int64_t sk_ss = p.sink.k_ss, sv_ss = p.sink.v_ss;
  const uint16_t* const rk = p.recent.k + b * p.recent.k_sb + kvh * p.recent.k_sh;
  const uint16_t* const rv = p.recent.v + b * p.recent.v_sb + kvh * p.recent.v_sh;
  const int64_t rk_ss = p.recent.k_ss, rv_ss = p.recent.v_ss;
  const float scale_log2 = p.scale_log2;
  auto fp16row = [&](int64_t f) {
    FpRow r;
    if (f < ns) {
      r.k = sk + f * sk_ss;
      r.v = sv + f * sv_ss;
    } else {
      r.k = rk + (f - ns) * rk_ss;
      r.v = rv + (f - ns) * rv_ss;
    }
    return r;
  };
  lds_u8* spr[NS];   // this wave's ring stages
  uint32_t str[NS];  // their LDS addresses (wave-uniform)
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    spr[s] = (lds_u8*)&ring[s][wave][0];
    str[s] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(spr[s])));
  }

  // ---- loads of one tile into a ring stage (kOps per packed tile, kOpsF16 per fp16 tile) ----
  // Packed tile, 4-bit codes: 16-byte unit q of K row r at LDS unit 4r + (q ^ ((r >> 2) & 3)),
  // of V row r at 4r + (q ^ ((r >> 4) ^ (r >> 2)) & 3); rows past the tier are
  // clamped to its last row (masked later).  fp16 tile: K row r unit u at
  // 16r + (u ^ r), V rows unswizzled.
  uint32_t voff[4], koff[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    voff[k] = (16 * k + (lane >> 2)) * 64 + 16 * ((lane & 3) ^ ((k ^ (lane >> 4)) & 3));
    koff[k] = (16 * k + (lane >> 2)) * 64 + 16 * ((lane & 3) ^ ((lane >> 4) & 3));
  }
  // kp / vp: the tile's K codes (K rows of an fp16 tile) / everything else;
  // a stage's K part is refilled as soon as the tile in it has read its K codes
  auto issue = [&](int64_t tt, uint32_t st, bool kp, bool vp) {
    if (tt >= nFt) {
      const int64_t m0 = (tt - nFt) * kTile;  // the tile's first token of the row's middle
      int64_t r0 = m0;                        // its first row in the tensors
      int64_t ob = -1;                        // byte offset of its (page, kv head) block, strided pools
      if (paged) {
        const int64_t slot = tt - nFt - mt_lo;
        const int64_t blk = static_cast<int64_t>(pages_s[slot < kPageSlots ? slot : kPageSlots - 1]) * Hkv + kvh;
        r0 = blk * kTile;
        if (pstride) ob = blk * pstride;
      }
      const uint8_t* kb = ob >= 0 ? kc + ob : kc + r0 * kRowK;
      const uint8_t* vb = ob >= 0 ? vc + ob : vc + r0 * kRowV;
      const int lim = m0 + kTile > M ? static_cast<int>(M - 1 - m0) : kTile - 1;
      if (kp && KB == 4) {
        uint32_t ko[4] = {koff[0], koff[1], koff[2], koff[3]};
        if (lim < kTile - 1) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int r = 16 * k + (lane >> 2);
            const int rr = r < lim ? r : lim;
            ko[k] = rr * 64 + 16 * ((lane & 3) ^ ((lane >> 4) & 3));
          }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) tile_dma16<kNT>(kb, ko[k], st + kStageK + 1024 * k);
      } else if (kp) {
        // 32-byte K rows in natural order
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int r = 32 * k + (lane >> 1);
          const int rr = r < lim ? r : lim;
          tile_dma16<kNT>(kb, rr * 32 + 16 * (lane & 1), st + kStageK + 1024 * k);
        }
      }
      if (!vp) return;
      if (VB == 8) {
        // 8 KB of int8 codes; the padded tier has all 64 rows of the tile
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int r = 8 * k + (lane >> 3);
          tile_dma16<kNT>(vb, r * 128 + 16 * ((lane & 7) ^ lit_swz(r)), st + kStageV + 1024 * k);
        }
      } else if (VB == 4) {
        uint32_t vo[4] = {voff[0], voff[1], voff[2], voff[3]};
        if (lim < kTile - 1) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int r = 16 * k + (lane >> 2);
            const int rr = r < lim ? r : lim;
            vo[k] = rr * 64 + 16 * ((lane & 3) ^ ((k ^ (lane >> 4)) & 3));
          }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) tile_dma16<kNT>(vb, vo[k], st + kStageV + 1024 * k);
      } else {
        // 32-byte V rows: row r unit u at 2r + (u ^ ((r >> 4) & 1)) (spreads the tr4 reads over more banks)
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int r = 32 * k + (lane >> 1);
          const int rr = r < lim ? r : lim;
          tile_dma16<kNT>(vb, rr * 32 + 16 * ((lane & 1) ^ ((r >> 4) & 1)), st + kStageV + 1024 * k);
        }
      }
      if constexpr (ASYM) {
        // [token][4 groups] fp16 = 8 bytes per token; dword loads (lane = token pair half)
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int r = 32 * k + (lane >> 1);
          const uint32_t o = 8u * (r < lim ? r : lim) + 4u * (lane & 1);
          tile_dma4<kNT>(ksg + 4 * r0, o, st + kMeta + 256 * k);
          tile_dma4<kNT>(kzg + 4 * r0, o, st + kMeta + 512 + 256 * k);
          tile_dma4<kNT>(vsg + 4 * r0, o, st + kMeta + 1024 + 256 * k);
          tile_dma4<kNT>(vzg + 4 * r0, o, st + kMeta + 1536 + 256 * k);
        }
      } else if constexpr (LIT) {
        tile_dma4<kNT>(vsg + (m0 / kTile) * kD, 4u * lane, st + kMeta);  // the tile's scale row
      } else {
        const uint32_t so = 2u * (lane < lim ? lane : lim);
        tile_dma2<kNT>(ob >= 0 ? reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(vsg) + ob) : vsg + r0, so,
                 st + kMeta);
      }
    } else {
      const int64_t f0 = tt * kMini;
      const int vf = static_cast<int>(F - f0 < kMini ? F - f0 : kMini);
      const int u = lane & 15;
      const uint16_t* vr = nullptr;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int row = 4 * k + (lane >> 4);
        const FpRow fr = fp16row(f0 + (row < vf ? row : vf - 1));
        if (kp) tile_dma16<kNT>(fr.k + 8 * (u ^ row), st + kStageK + 1024 * k);
        vr = fr.v;
      }
      if (!vp) return;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int row = 4 * k + (lane >> 4);
        const FpRow fr = fp16row(f0 + (row < vf ? row : vf - 1));
        tile_dma16<kNT>(fr.v + 8 * u, st + kStageV + 1024 * k);
      }
      if constexpr (FMT == kFmtSym) tile_dma2<kNT>(vr, st + kMeta);  // filler: as many loads as a packed tile
    }
  };

  // ---- prologue: query rows (and K scales) first, then the first two tiles ----
  {
#pragma unroll
    for (int h = wave; h < kHP; h += kWaves) {
      const uint32_t qa = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8*)&qraw_s[h][0])));
      if (h < G) lds_dma4(p.q + b * p.q_sb + (kvh * p.G + h0 + h) * p.q_sh + 2 * lane, qa);
      else qraw_s[h][lane] = 0u;
    }
    if (!ASYM && wave < kHeads) {
      const uint32_t ka = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_u8*)&ksraw_s[wave][0])));
      lds_dma4(p.mid.k_scale + bkv * kD + 2 * lane, ka);
    }
  }
  auto ops_t = [&](int64_t t) { return t < t1 ? (t < nFt ? kOpsF16 : kOps) : 0; };
  // s_waitcnt needs an immediate: the outstanding-op counts that can occur
  auto wait_vm = [&](int c) { wait_vm_dispatch<kOps, kOpsF16, NS>(c); };
  // ---- rotated middle tier: q R^T of the pass's heads, for the middle splits ----
  // f16 MFMA 16x16x32: C[channel 16 mt + row][head] = sum_k R[16 mt + row][k] q[head][k],
  // with R carried at scale 2^10 as hi = fp16(2^10 R) and lo = fp16(2^10 R - hi)
  // (about 2^-22 relative: an fp32 product), accumulated in fp32.  This wave's
  // R rows are loaded ahead of the first two tiles by loads the compiler does
  // not track, so that nothing waits for the tiles: the wait below for the
  // query covers them, and the registers are read only after it.
  constexpr int kMt = ROT ? (kD / 16 + kWaves - 1) / kWaves : 1;  // 16-channel blocks per wave
  const int ar = lane & 15, kq = lane >> 4;  // q R^T: A row / B column (head), and k group
  f32x4 rr[kMt][4][2];
  if constexpr (ROT) {
    if (rot && split > 0) {
#pragma unroll
      for (int i = 0; i < kMt; ++i) {
        const int mt = wave + i * kWaves < kD / 16 ? wave + i * kWaves : kD / 16 - 1;
        const float* rrow = p.rot + (16 * mt + ar) * kD + 8 * kq;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(rr[i][ks][0]) : "v"(rrow + 32 * ks) : "memory");
          asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(rr[i][ks][1]) : "v"(rrow + 32 * ks + 4) : "memory");
        }
      }
    }
  }
  // the ring's tiles, oldest first from stage 0: the wave's first NS tiles
  int64_t tq[NS];
  int c_first = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    tq[s] = t0 + s * kWaves + wave;
    if (tq[s] < t1) issue(tq[s], str[s], true, true);
    c_first += ops_t(tq[s]);
  }
  wait_vm(c_first);  // the query (and K-scale, and R) loads have landed
  __builtin_amdgcn_wave_barrier();
  if constexpr (ROT) {
    if (rot && split > 0) {
#pragma unroll
      for (int i = 0; i < kMt; ++i)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) asm volatile("" : "+v"(rr[i][ks][0]), "+v"(rr[i][ks][1]));
      __syncthreads();  // every wave's query row has landed
#pragma unroll
      for (int i = 0; i < kMt; ++i) {
        const int mt = wave + i * kWaves;
        if (mt < kD / 16) {
          f32x4 c = {0, 0, 0, 0};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const uint4 bq = ar < kHP ? *reinterpret_cast<const uint4*>(
                                               reinterpret_cast<const uint16_t*>(&qraw_s[ar][0]) + 32 * ks + 8 * kq)
                                         : make_uint4(0u, 0u, 0u, 0u);
            const u32x4 bqv = {bq.x, bq.y, bq.z, bq.w};
            if constexpr (BF) {
              // bf16 pieces hi + mid + lo of 2^10 R (about 2^-24 relative)
              u32x4 hi, mi, lo;
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                float v0 = rr[i][ks][j >> 1][2 * (j & 1)] * 1024.0f, v1 = rr[i][ks][j >> 1][2 * (j & 1) + 1] * 1024.0f;
                const uint32_t h2 = pack_bf16(v0, v1);
                v0 -= bf2f(static_cast<uint16_t>(h2 & 0xFFFFu));
                v1 -= bf2f(static_cast<uint16_t>(h2 >> 16));
                const uint32_t m2 = pack_bf16(v0, v1);
                v0 -= bf2f(static_cast<uint16_t>(m2 & 0xFFFFu));
                v1 -= bf2f(static_cast<uint16_t>(m2 >> 16));
                hi[j] = h2;
                mi[j] = m2;
                lo[j] = pack_bf16(v0, v1);
              }
              c = mfma32<true>(hi, bqv, c);
              c = mfma32<true>(mi, bqv, c);
              c = mfma32<true>(lo, bqv, c);
            } else {
              f16x8 hi, lo;
#pragma unroll
              for (int j = 0; j < 8; ++j) {
                const float v = rr[i][ks][j >> 2][j & 3] * 1024.0f;  // exact
                hi[j] = static_cast<_Float16>(v);
                lo[j] = static_cast<_Float16>(v - static_cast<float>(hi[j]));
              }
              c = mfma32<false>(__builtin_bit_cast(u32x4, hi), bqv, c);
              c = mfma32<false>(__builtin_bit_cast(u32x4, lo), bqv, c);
            }
          }
          if (ar < kHP) {
#pragma unroll
            for (int j = 0; j < 4; ++j) qrot_s[ar][16 * mt + 4 * kq + j] = c[j] * (1.0f / 1024.0f);
          }
        }
      }
      __syncthreads();
    }
  }

  // ---- query digits: wave w handles heads w, w + NW, ... (channels 2*lane, 2*lane+1) ----
  if (tid < 4) reinterpret_cast<uint32_t*>(&qd_s[kQdBytes])[tid] = 0u;
#pragma unroll
  for (int h = wave; h < kHP; h += kWaves) {
    const uint32_t qq = qraw_s[h][lane];
    float qf0 = w2f<BF>(static_cast<uint16_t>(qq & 0xFFFFu)), qf1 = w2f<BF>(static_cast<uint16_t>(qq >> 16));
    if constexpr (ROT) {
      if (rot && split > 0) {  // the middle tiles are scored with q R^T
        qf0 = qrot_s[h][2 * lane];
        qf1 = qrot_s[h][2 * lane + 1];
      }
    }
    if constexpr (!ASYM) {
      const uint32_t ks = ksraw_s[h & 3][lane];  // every row holds the kv head's K scales
      qf0 *= w2f<BF>(static_cast<uint16_t>(ks & 0xFFFFu));
      qf1 *= w2f<BF>(static_cast<uint16_t>(ks >> 16));
    }
    const float mx = group_max<64>(fmaxf(fabsf(qf0), fabsf(qf1)));
    const float inv = mx > 0.0f ? kQMax / mx : 0.0f;
    const int qi[2] = {static_cast<int>(rintf(qf0 * inv)), static_cast<int>(rintf(qf1 * inv))};
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      // channel d -> k-step d/16, operand byte j (see the K operand assembly below)
      const int d = 2 * lane + e;
      const int ksd = d >> 4, r = d & 15;
      const int j = KB == 4 ? 4 * (2 * (r >> 3) + (r & 1)) + ((r & 7) >> 1) : 4 * (r & 3) + (r >> 2);
      const int hi = (qi[e] + 128) >> 8;
      const int lo = qi[e] - 256 * hi;
      if constexpr (H8) {
        // [k-step (16 ks .. of channel half d >> 6)][digit][head][half][16 B]
        const int ks8 = (d >> 4) & 3, half = d >> 6;
        qd_s[(((2 * ks8 + 0) * 8 + h) * 2 + half) * 16 + j] = static_cast<uint8_t>(hi & 0xFF);
        qd_s[(((2 * ks8 + 1) * 8 + h) * 2 + half) * 16 + j] = static_cast<uint8_t>(lo & 0xFF);
      } else {
        qd_s[(2 * ksd + 0) * 64 + h * 16 + j] = static_cast<uint8_t>(hi & 0xFF);
        qd_s[(2 * ksd + 1) * 64 + h * 16 + j] = static_cast<uint8_t>(lo & 0xFF);
      }
    }
    if constexpr (ASYM) {
      // per 32-channel group (16 lanes): the digit sum restores the offset-binary
      // K operand (16*(u-8) or 64*(u-2) -> 16*u or 64*u: + 128 * sum of digits),
      // and the query sum multiplies the zero points
      int si = qi[0] + qi[1];
      float sf = qf0 + qf1;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        si += __shfl_xor(si, o, 64);
        sf += __shfl_xor(sf, o, 64);
      }
      if ((lane & 15) == 0) {
        qoff_s[h][lane >> 4] = 128 * si;
        qg_s[h][lane >> 4] = sf * p.scale_log2;
      }
    }
    // the K operand carries 16*c (4-bit) or 64*c (2-bit)
    if (lane == 0) qsc_s[h] = mx > 0.0f ? (mx / kQMax) * p.scale_log2 * (KB == 4 ? 0.0625f : 0.015625f) : 0.0f;
  }
  __syncthreads();

  const float qsc = qsc_s[hq];
  // query operands of the QK^T MFMAs (zero unless this lane's column block
  // matches its k group): registers for the reference formats, LDS reads per
  // tile for the asymmetric ones
  // (H8: column block 2h + s takes k groups 2s, 2s + 1, the two channel halves)
  const bool qlane = (H8 ? (g >> 1) == sq : sq == g) && (hq < G);
  const lds_u8* const qd_l =
      (const lds_u8*)&qd_s[0] + (qlane ? (H8 ? (2 * hq + (g & 1)) * 16 : hq * 16) : kQdBytes);
  const int qstride = qlane ? (H8 ? 256 : 64) : 0;
  i32x4 qdh[ASYM ? 1 : kNKs], qdl[ASYM ? 1 : kNKs];
  if constexpr (!ASYM) {
#pragma unroll
    for (int ks = 0; ks < kNKs; ++ks) {
      qdh[ks] = *reinterpret_cast<const __attribute__((address_space(3))) i32x4*>(qd_l + (2 * ks) * qstride);
      qdl[ks] = *reinterpret_cast<const __attribute__((address_space(3))) i32x4*>(qd_l + (2 * ks + 1) * qstride);
    }
  }
  auto qdig = [&](int ks, int digit) -> i32x4 {
    if constexpr (ASYM)
      return *reinterpret_cast<const __attribute__((address_space(3))) i32x4*>(qd_l + (2 * ks + digit) * qstride);
    else
      return digit ? qdl[ks] : qdh[ks];
  };
  int qoff[kGroups];
  float qgv[kGroups];
  if constexpr (ASYM) {
#pragma unroll
    for (int gi = 0; gi < kGroups; ++gi) {
      qoff[gi] = qoff_s[hq][gi];
      qgv[gi] = qg_s[hq][gi];
    }
  }
  const uint16_t* q16 = reinterpret_cast<const uint16_t*>(&qraw_s[hq][0]);

  float m_run = kNegBig, l_run = 0.0f;
  f32x4 acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = f32x4{0, 0, 0, 0};
  // offset accumulators (one per channel group for the asymmetric formats) and
  // the lane-local zero-point sums of the asymmetric formats
  constexpr int kOffs = ASYM ? kGroups : 1;
  f32x4 acc_off[kOffs];
  float zacc[kGroups];
#pragma unroll
  for (int gi = 0; gi < kOffs; ++gi) acc_off[gi] = f32x4{0, 0, 0, 0};
#pragma unroll
  for (int gi = 0; gi < kGroups; ++gi) zacc[gi] = 0.0f;

  // Online-softmax step for this lane's kNX log2-domain scores x (absolute);
  // pr = the unnormalized probabilities relative to the running max.
  auto softmax = [&](float (&x)[kNX], float (&pr)[kNX]) {
    float lmax = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    if constexpr (H8) lmax = fmaxf(lmax, fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
    if (__builtin_amdgcn_ballot_w64(lmax - m_run > kTau) != 0) {
      // the max over the lanes of this lane's head
      float tmax = lmax;
      tmax = fmaxf(tmax, __shfl_xor(tmax, 1, 64));
      if constexpr (!H8) tmax = fmaxf(tmax, __shfl_xor(tmax, 2, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
      if constexpr (H8) {
        // accumulator registers 0, 1 of lane (n, g) belong to head 2g, 2 and 3 to 2g + 1
        const float a0s = __shfl(alpha, 4 * g, 64), a1s = __shfl(alpha, 4 * g + 2, 64);
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] *= f32x4{a0s, a0s, a1s, a1s};
#pragma unroll
        for (int gi = 0; gi < kOffs; ++gi) acc_off[gi] *= f32x4{a0s, a0s, a1s, a1s};
      } else {
        const float ag = __shfl(alpha, 4 * g, 64);  // accumulator rows of lane (n, g) belong to head g
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] *= ag;
#pragma unroll
        for (int gi = 0; gi < kOffs; ++gi) acc_off[gi] *= ag;
      }
      if constexpr (ASYM) {
#pragma unroll
        for (int gi = 0; gi < kGroups; ++gi) zacc[gi] *= alpha;
      }
    }
#pragma unroll
    for (int i = 0; i < kNX; ++i) pr[i] = __builtin_amdgcn_exp2f(x[i] - m_run);
    float ps = (pr[0] + pr[1]) + (pr[2] + pr[3]);
    if constexpr (H8) ps += (pr[4] + pr[5]) + (pr[6] + pr[7]);
    l_run += ps;
  };

  // ---- fp16 tile (16 tokens) from a ring stage ----
  auto fp16_tile = [&](int64_t t, const lds_u8* sp, auto&& after_k) {
    const int64_t f0 = t * kMini;
    const int vf = static_cast<int>(F - f0 < kMini ? F - f0 : kMini);
    // QK^T in the plain layout: k = 32 channels (8 per lane group), columns
    // 4h + s (H8: 2h + s) repeat head h for every s; the s != 0 copies are masked below.
    f32x4 c4 = {0, 0, 0, 0};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x4 a = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
          sp + kStageK + 256 * n16 + 16 * ((4 * ks + g) ^ n16));
      const uint4 bq = *reinterpret_cast<const uint4*>(q16 + 32 * ks + 8 * g);
      c4 = mfma32<BF>(a, u32x4{bq.x, bq.y, bq.z, bq.w}, c4);
    }
    after_k();  // the stage's K rows have been read
    float x[kNX], pr[kNX];
#pragma unroll
    for (int i = 0; i < kNX; ++i) x[i] = (i < 4 && sq == 0 && 4 * g + i < vf) ? c4[i & 3] * scale_log2 : -INFINITY;
    softmax(x, pr);
    const uint32_t pk0 = sq == 0 ? pack_w<BF>(pr[0], pr[1]) : 0u;
    const uint32_t pk1 = sq == 0 ? pack_w<BF>(pr[2], pr[3]) : 0u;
    const i32x2 a4 = {static_cast<int>(pk0), static_cast<int>(pk1)};
    const __attribute__((address_space(3))) uint16_t* v16 =
        reinterpret_cast<const __attribute__((address_space(3))) uint16_t*>(sp + kStageV);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int col = out_channel<VB>(c, n16);
      const i32x2 vb = {static_cast<int>(v16[(4 * g + 0) * kD + col] | (static_cast<uint32_t>(v16[(4 * g + 1) * kD + col]) << 16)),
                        static_cast<int>(v16[(4 * g + 2) * kD + col] | (static_cast<uint32_t>(v16[(4 * g + 3) * kD + col]) << 16))};
      acc[c] = mfma16<BF>(a4, vb, acc[c]);
    }
  };

  // ---- packed tile from a ring stage ----
  // tr4 read addresses: as source lane s' = n16 of group g this lane fetches
  // row 16*sigma + 4g + i, where slot k = ((s'&3)<<1)|((s'>>2)&1) of pair s'>>3
  // gives sigma = 2*(s'>>3) + (k>>2), i = k&3.
  uint32_t vrd[4];
  {
    const int kk = ((n16 & 3) << 1) | ((n16 >> 2) & 1);
    const int sigma = 2 * (n16 >> 3) + (kk >> 2);
    const int r = 16 * sigma + 4 * g + (kk & 3);
    if (VB == 8) {
      // tr8: output lane p, byte j <- byte p % 8 of source lane 2j + p / 8.  Source
      // lane s reads half s & 1 of channel unit c of the row holding slot
      // pi(s >> 1), pi = (0 2 1 3 4 6 5 7), so that the fp16 pairs below come out
      // in slot order; slot k <-> token 16 (k >> 2) + 4g + (k & 3) (+32 for a1).
      const int j = n16 >> 1;
      const int k = (j & 4) | ((j & 1) << 1) | ((j >> 1) & 1);
      const int r0 = 16 * (k >> 2) + 4 * g + (k & 3);
      vrd[0] = kStageV + 128 * r0 + 8 * (n16 & 1);
      vrd[1] = lit_swz(r0);
      vrd[2] = kStageV + 128 * (r0 + 32) + 8 * (n16 & 1);
      vrd[3] = lit_swz(r0 + 32);
    } else if (VB == 4) {
      const int sw = (sigma ^ g) & 3;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) vrd[qq] = kStageV + 16 * (4 * r + (qq ^ sw));
    } else {
      // chunk c4 (8 bytes) of row r: unit c4/2 at position (c4/2) ^ (sigma & 1)
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) vrd[c4] = kStageV + 32 * r + 16 * ((c4 >> 1) ^ (sigma & 1)) + 8 * (c4 & 1);
    }
  }
  uint32_t krd[4];  // K row `lane`, 16-byte unit q (H8: [group][u], row 32q + 16(g >> 1) + n16, unit 2(g & 1) + u)
#pragma unroll
  for (int qq = 0; qq < 4; ++qq) {
    if constexpr (H8) {
      const int r = 32 * (qq >> 1) + 16 * (g >> 1) + n16, u = 2 * (g & 1) + (qq & 1);
      krd[qq] = KB == 4 ? kStageK + 16 * (4 * r + (u ^ ((r >> 2) & 3))) : kStageK + 32 * r + 16 * (g & 1);
    } else {
      krd[qq] = KB == 4 ? kStageK + 16 * (4 * lane + (qq ^ ((lane >> 2) & 3))) : kStageK + 32 * lane + 16 * (qq & 1);
    }
  }
  // this lane's tokens 16*sq + 4g + i: V scales (reference) or the four
  // [token][group] metadata arrays (asymmetric), 8 bytes per token
  const uint32_t vs_rd = ASYM ? kMeta + 8 * (16 * sq + 4 * g) : kMeta + 4 * (16 * sq + 4 * g);
  const uint32_t z = 0u;
  uint32_t vmask, vcst;  // register-resident constants of the V code conversion
  if constexpr (BF) {  // bfloat16 values (no asymmetric instance)
    if (VB == 4) {
      asm volatile("s_mov_b32 %0, 0x001E001E" : "=s"(vmask));
      asm volatile("v_mov_b32 %0, 0x42904290" : "=v"(vcst));
    } else {
      asm volatile("s_mov_b32 %0, 0x00600060" : "=s"(vmask));
      asm volatile("v_mov_b32 %0, 0x40C040C0" : "=v"(vcst));
    }
  } else if (VB == 8) {
    asm volatile("s_mov_b32 %0, 0x03000300" : "=s"(vmask));
    asm volatile("v_mov_b32 %0, 0x46004600" : "=v"(vcst));
  } else if (VB == 4) {
    asm volatile("s_mov_b32 %0, 0x00F000F0" : "=s"(vmask));
    if (ASYM) asm volatile("v_mov_b32 %0, 0x54005400" : "=v"(vcst));
    else asm volatile("v_mov_b32 %0, 0x54805480" : "=v"(vcst));
  } else {
    asm volatile("s_mov_b32 %0, 0x03000300" : "=s"(vmask));
    if (ASYM) asm volatile("v_mov_b32 %0, 0x44004400" : "=v"(vcst));
    else asm volatile("v_mov_b32 %0, 0x46004600" : "=v"(vcst));
  }
  // per-token offset of the V values: 72 / 6 (two's complement codes) or
  // 64 / 4 (unsigned codes of the asymmetric formats), fp16 or bfloat16
  const uint32_t offv = BF ? (VB == 4 ? 0x42904290u : 0x40C040C0u)
                           : (VB == 4 ? (ASYM ? 0x54005400u : 0x54805480u) : (ASYM ? 0x44004400u : 0x46004600u));
  // literal INT2 V: the tile's per-channel scales of this lane's output channels
  const uint32_t lsc_rd = kMeta + 2 * n16;
  const u32x4 boff = {offv, offv, offv, offv};
  // K codes -> int8 operand: two's complement (x & m) or offset binary ((x & m) ^ 0x80)
  constexpr uint32_t kFlip = ASYM ? 0x80808080u : 0u;

  auto packed_tile = [&](int64_t t, const lds_u8* sp, auto&& after_k) {
    float x[kNX], pr[kNX];
    if constexpr (H8) {
      // QK^T of the two 32-token groups: A = K codes of token 32q + 16(g >> 1) + n16,
      // channel half g & 1; k-step ks = channels 64 (g & 1) + 16 ks .. + 15
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        i32x4 chi = {0, 0, 0, 0}, clo = {0, 0, 0, 0};
        if (KB == 4) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const u32x4 kv = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + krd[2 * q + u]);
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
              const int ks = 2 * u + h2;
              const uint32_t w0 = kv[2 * h2], w1 = kv[2 * h2 + 1];
              const i32x4 a = {static_cast<int>(w0 & 0xF0F0F0F0u), static_cast<int>((w0 << 4) & 0xF0F0F0F0u),
                               static_cast<int>(w1 & 0xF0F0F0F0u), static_cast<int>((w1 << 4) & 0xF0F0F0F0u)};
              chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig(ks, 0), chi, 0, 0, 0);
              clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig(ks, 1), clo, 0, 0, 0);
            }
          }
        } else {
          const u32x4 kv = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + krd[2 * q]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t w = kv[e];
            const i32x4 a = {static_cast<int>(w & 0xC0C0C0C0u), static_cast<int>((w << 2) & 0xC0C0C0C0u),
                             static_cast<int>((w << 4) & 0xC0C0C0C0u), static_cast<int>((w << 6) & 0xC0C0C0C0u)};
            chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig(e, 0), chi, 0, 0, 0);
            clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig(e, 1), clo, 0, 0, 0);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * q + i] = static_cast<float>(chi[i] * 256 + clo[i]) * qsc;
      }
    } else if constexpr (!ASYM) {
      // QK^T: A = K codes of token `lane` as int8 (16*c or 64*c)
      i32x4 chi = {0, 0, 0, 0}, clo = {0, 0, 0, 0};
      if (KB == 4) {
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const u32x4 kv = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + krd[qq]);
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            const int ks = 2 * qq + h2;
            const uint32_t w0 = kv[2 * h2], w1 = kv[2 * h2 + 1];
            const i32x4 a = {static_cast<int>(w0 & 0xF0F0F0F0u), static_cast<int>((w0 << 4) & 0xF0F0F0F0u),
                             static_cast<int>(w1 & 0xF0F0F0F0u), static_cast<int>((w1 << 4) & 0xF0F0F0F0u)};
            chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig(ks, 0), chi, 0, 0, 0);
            clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig(ks, 1), clo, 0, 0, 0);
          }
        }
      } else {
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
          const u32x4 kv = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + krd[qq]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // k-step 4qq+e: dword i, byte j <-> channel 16ks + 4j + i
            const int ks = 4 * qq + e;
            const uint32_t w = kv[e];
            const i32x4 a = {static_cast<int>(w & 0xC0C0C0C0u), static_cast<int>((w << 2) & 0xC0C0C0C0u),
                             static_cast<int>((w << 4) & 0xC0C0C0C0u), static_cast<int>((w << 6) & 0xC0C0C0C0u)};
            chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig(ks, 0), chi, 0, 0, 0);
            clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig(ks, 1), clo, 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = static_cast<float>(chi[i] * 256 + clo[i]) * qsc;
    } else {
      // per-group integer dot products, combined with the token's group scale and zero
      const u32x4 ks01 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + vs_rd);
      const u32x4 ks23 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + vs_rd + 16);
      const u32x4 kz01 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + vs_rd + 512);
      const u32x4 kz23 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + vs_rd + 528);
      // token i, group gi: dword 2*(i&1) + (gi>>1) of the (i>>1) vector, half gi&1
      auto meta = [&](const u32x4& v01, const u32x4& v23, int i, int gi) {
        const uint32_t dw = (i < 2 ? v01 : v23)[2 * (i & 1) + (gi >> 1)];
        return half_of(dw, gi & 1);
      };
      float xs[4] = {0, 0, 0, 0}, xz[4] = {0, 0, 0, 0};
      auto group_done = [&](int gi, const i32x4& chi, const i32x4& clo) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float dg = static_cast<float>(chi[i] * 256 + clo[i] + qoff[gi]);
          xs[i] = fmaf(meta(ks01, ks23, i, gi), dg, xs[i]);
          xz[i] = fmaf(meta(kz01, kz23, i, gi), qgv[gi], xz[i]);
        }
      };
      if (KB == 4) {
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {  // 16-byte unit qq = channel group qq
          const u32x4 kv = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + krd[qq]);
          i32x4 chi = {0, 0, 0, 0}, clo = {0, 0, 0, 0};
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            const int ks = 2 * qq + h2;
            const uint32_t w0 = kv[2 * h2], w1 = kv[2 * h2 + 1];
            const i32x4 a = {static_cast<int>((w0 & 0xF0F0F0F0u) ^ kFlip),
                             static_cast<int>(((w0 << 4) & 0xF0F0F0F0u) ^ kFlip),
                             static_cast<int>((w1 & 0xF0F0F0F0u) ^ kFlip),
                             static_cast<int>(((w1 << 4) & 0xF0F0F0F0u) ^ kFlip)};
            chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig(ks, 0), chi, 0, 0, 0);
            clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig(ks, 1), clo, 0, 0, 0);
          }
          group_done(qq, chi, clo);
        }
      } else {
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
          const u32x4 kv = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + krd[qq]);
#pragma unroll
          for (int e2 = 0; e2 < 2; ++e2) {  // channel group 2qq + e2 = k-steps 4qq + 2e2 + {0, 1}
            i32x4 chi = {0, 0, 0, 0}, clo = {0, 0, 0, 0};
#pragma unroll
            for (int e1 = 0; e1 < 2; ++e1) {
              const int e = 2 * e2 + e1, ks = 4 * qq + e;
              const uint32_t w = kv[e];
              const i32x4 a = {static_cast<int>((w & 0xC0C0C0C0u) ^ kFlip),
                               static_cast<int>(((w << 2) & 0xC0C0C0C0u) ^ kFlip),
                               static_cast<int>(((w << 4) & 0xC0C0C0C0u) ^ kFlip),
                               static_cast<int>(((w << 6) & 0xC0C0C0C0u) ^ kFlip)};
              chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig(ks, 0), chi, 0, 0, 0);
              clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig(ks, 1), clo, 0, 0, 0);
            }
            group_done(2 * qq + e2, chi, clo);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = fmaf(xs[i], qsc, xz[i]);
    }
    after_k();  // the stage's K codes have been read
    const int64_t m0 = (t - nFt) * kTile;
    if (m0 + kTile > M) {
      const int valid = static_cast<int>(M - m0);
#pragma unroll
      for (int i = 0; i < kNX; ++i)
        if (32 * (i >> 2) * (H8 ? 1 : 0) + 16 * sq + 4 * g + (i & 3) >= valid) x[i] = -INFINITY;
    }
    softmax(x, pr);
    // P' = P * v_scale: one operand pair (a0, a1) per V scale group
    constexpr int kPs = ASYM ? kGroups : 1;
    u32x4 a0[kPs], a1[kPs];
    if constexpr (LIT) {
      // per-channel V scales apply after the tile's PV products
      const uint32_t pk0 = pack_w<BF>(pr[0], pr[1]), pk1 = pack_w<BF>(pr[2], pr[3]);
      a0[0] = u32x4{sq == 0 ? pk0 : z, sq == 0 ? pk1 : z, sq == 1 ? pk0 : z, sq == 1 ? pk1 : z};
      a1[0] = u32x4{sq == 2 ? pk0 : z, sq == 2 ? pk1 : z, sq == 3 ? pk0 : z, sq == 3 ? pk1 : z};
    } else if constexpr (H8) {
      // group q's probabilities times their tokens' V scales: the a0 / a1 token halves
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const u32x4 sv = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + vs_rd + 128 * q);
        const uint32_t pk0 = pack_w<BF>(pr[4 * q] * w2f<BF>(static_cast<uint16_t>(sv[0])),
                                        pr[4 * q + 1] * w2f<BF>(static_cast<uint16_t>(sv[1])));
        const uint32_t pk1 = pack_w<BF>(pr[4 * q + 2] * w2f<BF>(static_cast<uint16_t>(sv[2])),
                                        pr[4 * q + 3] * w2f<BF>(static_cast<uint16_t>(sv[3])));
        const u32x4 aq = {sq == 0 ? pk0 : z, sq == 0 ? pk1 : z, sq == 1 ? pk0 : z, sq == 1 ? pk1 : z};
        if (q == 0) a0[0] = aq;
        else a1[0] = aq;
      }
    } else if constexpr (!ASYM) {
      // scales sit in the low halves of the stage's scale dwords
      const u32x4 sv = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + vs_rd);
      const uint32_t pk0 =
          pack_w<BF>(pr[0] * w2f<BF>(static_cast<uint16_t>(sv[0])), pr[1] * w2f<BF>(static_cast<uint16_t>(sv[1])));
      const uint32_t pk1 =
          pack_w<BF>(pr[2] * w2f<BF>(static_cast<uint16_t>(sv[2])), pr[3] * w2f<BF>(static_cast<uint16_t>(sv[3])));
      a0[0] = u32x4{sq == 0 ? pk0 : z, sq == 0 ? pk1 : z, sq == 1 ? pk0 : z, sq == 1 ? pk1 : z};
      a1[0] = u32x4{sq == 2 ? pk0 : z, sq == 2 ? pk1 : z, sq == 3 ? pk0 : z, sq == 3 ? pk1 : z};
    } else {
      const u32x4 vs01 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + vs_rd + 1024);
      const u32x4 vs23 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + vs_rd + 1040);
      const u32x4 vz01 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + vs_rd + 1536);
      const u32x4 vz23 = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(sp + vs_rd + 1552);
      auto meta = [&](const u32x4& v01, const u32x4& v23, int i, int gi) {
        const uint32_t dw = (i < 2 ? v01 : v23)[2 * (i & 1) + (gi >> 1)];
        return half_of(dw, gi & 1);
      };
#pragma unroll
      for (int gi = 0; gi < kGroups; ++gi) {
        const uint32_t pk0 = pack_f16(pr[0] * meta(vs01, vs23, 0, gi), pr[1] * meta(vs01, vs23, 1, gi));
        const uint32_t pk1 = pack_f16(pr[2] * meta(vs01, vs23, 2, gi), pr[3] * meta(vs01, vs23, 3, gi));
        a0[gi] = u32x4{sq == 0 ? pk0 : z, sq == 0 ? pk1 : z, sq == 1 ? pk0 : z, sq == 1 ? pk1 : z};
        a1[gi] = u32x4{sq == 2 ? pk0 : z, sq == 2 ? pk1 : z, sq == 3 ? pk0 : z, sq == 3 ? pk1 : z};
#pragma unroll
        for (int i = 0; i < 4; ++i) zacc[gi] = fmaf(pr[i], meta(vz01, vz23, i, gi), zacc[gi]);
      }
    }
    // channel tile c lies in 32-channel group c >> 1 (both code widths)
    if (VB == 8) {
      // literal INT2 V: ternary int8 codes c -> fp16 6 + c (low two bits, sign
      // bit flipped, into mantissa bits 8..9 of 4.0).  Each tile's products
      // are offset-corrected (6 * sum P) and scaled per channel before they
      // join the running accumulator.
      f32x4 toff = {0, 0, 0, 0};
      toff = mfma32<BF>(a0[0], boff, toff);
      toff = mfma32<BF>(a1[0], boff, toff);
      const __attribute__((address_space(3))) uint16_t* lsc =
          reinterpret_cast<const __attribute__((address_space(3))) uint16_t*>(sp + lsc_rd);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const i32x2 x0 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            reinterpret_cast<lds_i32x2*>(const_cast<lds_u8*>(sp) + vrd[0] + 16 * (c ^ vrd[1])));
        const i32x2 x1 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            reinterpret_cast<lds_i32x2*>(const_cast<lds_u8*>(sp) + vrd[2] + 16 * (c ^ vrd[3])));
        const uint32_t w0 = static_cast<uint32_t>(x0[0]), w1 = static_cast<uint32_t>(x0[1]);
        const uint32_t w2 = static_cast<uint32_t>(x1[0]), w3 = static_cast<uint32_t>(x1[1]);
        // bytes (0, 2) -> slots (0, 1), bytes (1, 3) -> slots (2, 3); the code's
        // low two bits to mantissa bits 8..9 (fp16) or 5..6 (bfloat16)
        constexpr int kSa = BF ? 5 : 8, kSb = BF ? 3 : 0;
        const u32x4 b0 = {((w0 << kSa) & vmask) ^ vcst, ((w0 >> kSb) & vmask) ^ vcst, ((w1 << kSa) & vmask) ^ vcst,
                          ((w1 >> kSb) & vmask) ^ vcst};
        const u32x4 b1 = {((w2 << kSa) & vmask) ^ vcst, ((w2 >> kSb) & vmask) ^ vcst, ((w3 << kSa) & vmask) ^ vcst,
                          ((w3 >> kSb) & vmask) ^ vcst};
        f32x4 tc = {0, 0, 0, 0};
        tc = mfma32<BF>(a0[0], b0, tc);
        tc = mfma32<BF>(a1[0], b1, tc);
        const float sc = w2f<BF>(lsc[16 * c]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[c][i] = fmaf(sc, tc[i] - toff[i], acc[c][i]);
      }
    } else if (VB == 4) {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int gp = ASYM ? c >> 1 : 0;
        const i32x2 xv = __builtin_amdgcn_ds_read_tr4_b64_v2i32(
            reinterpret_cast<lds_i32x2*>(const_cast<lds_u8*>(sp) + vrd[c >> 1] + 8 * (c & 1)));
        uint32_t b0[4], b1[4];
        v_nibbles_to_f16<BF>(static_cast<uint32_t>(xv[0]), vmask, vcst, b0);
        v_nibbles_to_f16<BF>(static_cast<uint32_t>(xv[1]), vmask, vcst, b1);
        acc[c] = mfma32<BF>(a0[gp], u32x4{b0[0], b0[1], b0[2], b0[3]}, acc[c]);
        acc[c] = mfma32<BF>(a1[gp], u32x4{b1[0], b1[1], b1[2], b1[3]}, acc[c]);
      }
    } else {
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        const int gp = ASYM ? c4 : 0;
        const i32x2 xv = __builtin_amdgcn_ds_read_tr4_b64_v2i32(
            reinterpret_cast<lds_i32x2*>(const_cast<lds_u8*>(sp) + vrd[c4]));
        uint32_t f0[4], s0[4], f1[4], s1[4];
        v2_nibbles_to_f16<BF>(static_cast<uint32_t>(xv[0]), vmask, vcst, f0, s0);
        v2_nibbles_to_f16<BF>(static_cast<uint32_t>(xv[1]), vmask, vcst, f1, s1);
        acc[2 * c4] = mfma32<BF>(a0[gp], u32x4{f0[0], f0[1], f0[2], f0[3]}, acc[2 * c4]);
        acc[2 * c4] = mfma32<BF>(a1[gp], u32x4{f1[0], f1[1], f1[2], f1[3]}, acc[2 * c4]);
        acc[2 * c4 + 1] = mfma32<BF>(a0[gp], u32x4{s0[0], s0[1], s0[2], s0[3]}, acc[2 * c4 + 1]);
        acc[2 * c4 + 1] = mfma32<BF>(a1[gp], u32x4{s1[0], s1[1], s1[2], s1[3]}, acc[2 * c4 + 1]);
      }
    }
    if constexpr (!LIT) {
#pragma unroll
      for (int gp = 0; gp < kPs; ++gp) {
        acc_off[gp] = mfma32<BF>(a0[gp], boff, acc_off[gp]);
        acc_off[gp] = mfma32<BF>(a1[gp], boff, acc_off[gp]);
      }
    }
  };

  // ---- main loop: NS stages, NS - 1 tiles in flight behind the one computed ----
  // step s: tile tq[s] (the oldest) sits in stage s, the tiles of the other
  // stages are in flight behind it; afterwards stage s is refilled with a
  // newly claimed tile.  Claims only grow, so once the oldest tile is past the
  // split (>= t1) so is every tile behind it, and nothing is in flight.
  auto step = [&](int s) -> bool {
    const int64_t cur = tq[s];
    if (cur >= t1) return false;
    lds_u8* const sp = spr[s];
    const uint32_t st = str[s];
    // the tile that refills this stage, known before `cur` is computed
    int64_t nt;
    if constexpr (DET) {  // wave w walks tiles t0 + w, t0 + w + NW, ... : cur's NS-th successor
      nt = cur + NS * kWaves;
    } else {
      int c = 0;
      if (lane == 0) c = __hip_atomic_fetch_add(&claim_s, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      nt = t0 + NS * kWaves + __builtin_amdgcn_readfirstlane(c);
    }
    int behind = 0;  // loads issued after cur's
#pragma unroll
    for (int j = 1; j < NS; ++j) behind += ops_t(tq[(s + j) % NS]);
    wait_vm(behind);  // `cur` landed
    __builtin_amdgcn_wave_barrier();
    // once cur's K codes have been read from the stage, nt's K codes are loaded
    // into it: they fly during the rest of cur's compute
    auto refill_k = [&]() {
      if (nt < t1) {
        __builtin_amdgcn_s_waitcnt(kLgkm0);
        __builtin_amdgcn_wave_barrier();
        issue(nt, st, true, false);
      }
    };
    if (cur < nFt) fp16_tile(cur, sp, refill_k);
    else packed_tile(cur, sp, refill_k);
    __builtin_amdgcn_s_waitcnt(kLgkm0);  // every LDS read of this stage has returned
    __builtin_amdgcn_wave_barrier();
    if (nt < t1) issue(nt, st, false, true);
    tq[s] = nt;
    return true;
  };
  for (bool more = true; more;) {
#pragma unroll
    for (int s = 0; s < NS; ++s)
      if (more) more = step(s);
  }

  // ---- merge the wavefronts of the workgroup ----
  float lsum = l_run;  // summed over the lanes of this lane's head
  lsum += __shfl_xor(lsum, 1, 64);
  if constexpr (!H8) lsum += __shfl_xor(lsum, 2, 64);
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  // zero-point sums of head hq (score lanes), then of head g (accumulator lanes)
  float zs[kGroups];
  if constexpr (ASYM) {
#pragma unroll
    for (int gi = 0; gi < kGroups; ++gi) {
      float zz = zacc[gi];
      zz += __shfl_xor(zz, 1, 64);
      zz += __shfl_xor(zz, 2, 64);
      zz += __shfl_xor(zz, 16, 64);
      zz += __shfl_xor(zz, 32, 64);
      zs[gi] = __shfl(zz, 4 * g, 64);
    }
  }
  if (g == 0 && sq == 0) {
    red_m[wave][hq] = m_run;
    red_l[wave][hq] = lsum;
  }
  __syncthreads();
  float* red_o = reinterpret_cast<float*>(&ring[0][0][0]);  // [wave][kHP heads][128] (NW * 2 or 4 KB)
  if constexpr (H8) {
    // accumulator registers 0, 1 of lane (n, g): head 2g; 2, 3: head 2g + 1
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int h = 2 * g + e;
      float Mg = red_m[0][h];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) Mg = fmaxf(Mg, red_m[w][h]);
      const float wsc = exp2f(red_m[wave][h] - Mg);
      const float off = acc_off[0][2 * e] + acc_off[0][2 * e + 1];
#pragma unroll
      for (int c = 0; c < 8; ++c)
        red_o[(wave * kHP + h) * kD + out_channel<VB>(c, n16)] = ((acc[c][2 * e] + acc[c][2 * e + 1]) - off) * wsc;
    }
  } else {
    float Mg = red_m[0][g];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) Mg = fmaxf(Mg, red_m[w][g]);
    const float wsc = exp2f(red_m[wave][g] - Mg);
    float off[kOffs];
#pragma unroll
    for (int gp = 0; gp < kOffs; ++gp) off[gp] = (acc_off[gp][0] + acc_off[gp][1]) + (acc_off[gp][2] + acc_off[gp][3]);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float o = ((acc[c][0] + acc[c][1]) + (acc[c][2] + acc[c][3])) - off[ASYM ? c >> 1 : 0];
      if constexpr (ASYM) o += zs[c >> 1];
      red_o[(wave * 4 + g) * kD + out_channel<VB>(c, n16)] = o * wsc;
    }
  }
  __syncthreads();
  for (int idx = tid; idx < G * kD; idx += kThreads) {
    const int h = idx >> 7, d = idx & (kD - 1);
    float Mh = red_m[0][h];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) Mh = fmaxf(Mh, red_m[w][h]);
    float o = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      o += red_o[(w * kHP + h) * kD + d];
      L += red_l[w][h] * exp2f(red_m[w][h] - Mh);
    }
    if (n == 1) {
      p.out[b * p.o_sb + (kvh * p.G + h0 + h) * p.o_sh + d] = f2w<BF>(o / L);
    } else {
      // H8: heads 4..7 in the second pass's slot (the two-pass layout)
      const int64_t pi = ((slot + (h >> 2)) * n + split) * 4 + (h & 3);
      store_sys(&p.ws_acc[pi * kD + d], o);
      if (d == 0) store_sys2(&p.ws_ml[2 * pi], Mh, L);
    }
  }
  if (n == 1) return;

  // ---- the last workgroup of this (batch row, kv head) merges the splits ----
  // Cross-workgroup protocol (the XCDs' L2s are separate caches):
  // - writers: every (m, l, acc) partial is a system-scope store (global_store
  //   ... sc0 sc1: written through the L2 to memory); every wave waits for the
  //   completion of its own stores (vmcnt(0); the workgroup barrier alone does
  //   not wait for other waves' stores), then thread 0 increments the counter.
  //   No release fence: its buffer_wbl2 writes back an XCD's whole L2 for the
  //   sake of non-atomic stores, which this merge has none of (an agent-scope
  //   release cost 12 us per call at config 1);
  // - the workgroup whose increment returns n - 1 has seen every other
  //   increment, each issued after its partials reached memory; it acquires
  //   (buffer_inv sc1) before the barrier that lets its waves issue the partial
  //   loads, which are system-scope loads (sc0 sc1: fetched from memory, never
  //   an L2 line of an earlier call).
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&p.counters[slot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prev == static_cast<uint32_t>(n - 1);
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    last_s = last;
  }
  __syncthreads();
  if (!last_s) return;
  {
    // thread tid merges items (head, channel) tid + e * kThreads; the loads of
    // a batch of 16 splits for all its items issue before any is used
    constexpr int kB = 16, kE = (kHP * kD + kThreads - 1) / kThreads;
    // rotated tier: thread (channel c, quarter dq) of 4 kD virtual threads needs
    // R[32 dq .. 32 dq + 31][c]; loaded first, so that they fly with the partials
    constexpr int kV = (4 * kD + kThreads - 1) / kThreads;
    float rr[ROT ? kV : 1][ROT ? 32 : 1];
    if constexpr (ROT) {
      {
#pragma unroll
        for (int iv = 0; iv < kV; ++iv) {
          const int vt = tid + iv * kThreads;
          if (vt < 4 * kD) {
#pragma unroll
            for (int d = 0; d < 32; ++d) rr[iv][d] = p.rot[(32 * (vt >> 7) + d) * kD + (vt & (kD - 1))];
          }
        }
      }
    }
    // rotated tier: of = split 0 (fp16 tiers, plain basis), o = the middle splits (rotated basis)
    float Mh[kE], o[kE], L[kE], of[kE];
#pragma unroll
    for (int e = 0; e < kE; ++e) {
      Mh[e] = kNegBig;
      o[e] = 0.0f;
      L[e] = 0.0f;
      of[e] = 0.0f;
    }
    for (int s0 = 0; s0 < n; s0 += kB) {
      float mm[kE][kB], ll[kE][kB], aa[kE][kB];
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        if (s0 + j < n) {  // wave-uniform: only the splits that exist are loaded
#pragma unroll
          for (int e = 0; e < kE; ++e) {
            const int idx = tid + e * kThreads;
            const int h = idx < G * kD ? idx >> 7 : 0, d = idx & (kD - 1);
            const int64_t pi = ((slot + (h >> 2)) * n + s0 + j) * 4 + (h & 3);
            load_sys2(&p.ws_ml[2 * pi], mm[e][j], ll[e][j]);
            aa[e][j] = load_sys(&p.ws_acc[pi * kD + d]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < kE; ++e) {
            mm[e][j] = kNegBig;
            ll[e][j] = 0.0f;
            aa[e][j] = 0.0f;
          }
        }
      }
#pragma unroll
      for (int e = 0; e < kE; ++e) {
        float bm = kNegBig;
#pragma unroll
        for (int j = 0; j < kB; ++j)
          if (s0 + j < n) bm = fmaxf(bm, mm[e][j]);
        const float Mn = fmaxf(Mh[e], bm);
        const float r = exp2f(Mh[e] - Mn);
        o[e] *= r;
        L[e] *= r;
        of[e] *= r;
#pragma unroll
        for (int j = 0; j < kB; ++j) {
          if (s0 + j < n) {
            const float w = exp2f(mm[e][j] - Mn);
            L[e] += ll[e][j] * w;
            if (rot && s0 + j == 0) of[e] += aa[e][j] * w;
            else o[e] += aa[e][j] * w;
          }
        }
        Mh[e] = Mn;
      }
    }
    if (rot) {
      // out = (of + o R) / L: o [head][d] to LDS, then 512 virtual threads
      // (channel c, quarter dq) sum d over [32 dq, 32 dq + 32) for every head
      float* ro = reinterpret_cast<float*>(&ring[0][0][0]);  // [kHP][kD] o, then [4 dq][kHP][kD] partial products
      float* pp = ro + kHP * kD;
#pragma unroll
      for (int e = 0; e < kE; ++e) {
        const int idx = tid + e * kThreads;
        if (idx < kHP * kD) ro[idx] = idx < G * kD ? o[e] : 0.0f;
      }
      __syncthreads();
#pragma unroll
      for (int iv = 0; iv < kV; ++iv) {
        const int vt = tid + iv * kThreads;
        if (vt < 4 * kD) {
          const int c = vt & (kD - 1), dq = vt >> 7;
          float sh[kHP];
#pragma unroll
          for (int h = 0; h < kHP; ++h) sh[h] = 0.0f;
#pragma unroll
          for (int d = 0; d < 32; ++d)
#pragma unroll
            for (int h = 0; h < kHP; ++h) sh[h] = fmaf(ro[h * kD + 32 * dq + d], rr[iv][d], sh[h]);
#pragma unroll
          for (int h = 0; h < kHP; ++h) pp[(dq * kHP + h) * kD + c] = sh[h];
        }
      }
      __syncthreads();
#pragma unroll
      for (int e = 0; e < kE; ++e) {
        const int idx = tid + e * kThreads;
        if (idx < G * kD) {
          const int h = idx >> 7, c = idx & (kD - 1);
          const float v = of[e] + ((pp[h * kD + c] + pp[(kHP + h) * kD + c]) +
                                   (pp[(2 * kHP + h) * kD + c] + pp[(3 * kHP + h) * kD + c]));
          p.out[b * p.o_sb + (kvh * p.G + h0 + h) * p.o_sh + c] = f2w<BF>(v / L[e]);
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < kE; ++e) {
        const int idx = tid + e * kThreads;
        if (idx < G * kD)
          p.out[b * p.o_sb + (kvh * p.G + h0 + (idx >> 7)) * p.o_sh + (idx & (kD - 1))] = f2w<BF>(o[e] / L[e]);
      }
    }
  }
  if (tid == 0) __hip_atomic_store(&p.counters[slot], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


}  // namespace
}  // namespace decode
}  // namespace fade
