// Shared definitions of the tiered decode attention kernels.
#pragma once

#include "fade_common.h"

namespace fade {
namespace decode {

constexpr int kD = 128;   // head_dim of the matrix-core attention kernels (the portable one: 32..256)
constexpr int kMaxG = 8;  // max query heads per kv head

struct Fp16Tier {
  const uint16_t* k;
  const uint16_t* v;
  int64_t len;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
};

struct MidTier {
  int fmt, k_bits, v_bits, group;
  int64_t len, v_rows;
  const uint8_t* k_codes;
  const uint16_t* k_scale;
  const uint16_t* k_zero;
  const uint8_t* v_codes;
  const uint16_t* v_scale;
  const uint16_t* v_zero;
  const int32_t* pages;  // optional [B][pages_per_row] page of each 64-token tile (paged pools)
  int64_t pages_per_row;
  int64_t page_stride;  // paged SYM: bytes between (page, kv head) blocks of every tensor, or 0
};

// Page slots a workgroup of the INT4 kernel holds (its split's middle tiles).
constexpr int kPageSlots = 256;

struct Params {
  int64_t B, Hq, Hkv;
  int G;
  int D;  // head_dim: kD for the matrix-core kernels; 32, 64, 128 or 256 for the portable one
  const uint16_t* q;
  int64_t q_sb, q_sh;
  float scale_log2;  // sm_scale * log2(e): softmax runs in the exp2 domain
  Fp16Tier sink, recent;
  MidTier mid;
  int64_t total;             // sink.len + mid.len + recent.len
  int64_t tokens_per_split;  // multiple of the kernel tile
  int n_splits;
  float* ws_ml;   // [B][Hq][n_splits][2]  (m, l); INT4 kernel: [B*Hkv][n_splits][4][2]
  float* ws_acc;  // [B][Hq][n_splits][D] unnormalized output; INT4 kernel: [B*Hkv][n_splits][4][kD]
  // output (the INT4 kernel; the portable kernel with one split) and split
  // counters (INT4 kernel)
  uint16_t* out;
  int64_t o_sb, o_sh;
  uint32_t* counters;       // [B*Hkv*passes] finished splits; zero between calls
  // INT4 kernel only
  int64_t n_f16_tiles;      // 16-token fp16 tiles ahead of the packed 64-token tiles
  int64_t tiles_per_split;  // tiles (either kind) per split
  const int32_t* lens;      // optional [B][3] per-row sink / middle / recent lengths
  int32_t deterministic;    // INT4 kernel: fixed round-robin tile order instead of claims
  int passes;               // INT4 kernel: head passes per kv head, ceil(G / 4): 1 or 2
  // INT4 kernel, FADE_MID_SYM: the rotated backend's R (fp32 [kD][kD]); the
  // middle tier then holds codes of x R^T.  Split 0 takes the fp16 tiles,
  // splits 1.. the middle tiles (scored with q R^T); the merge returns
  // fp16 part + (middle part) R.  nullptr: no rotation.
  const float* rot;
  // dtype of every 16-bit float of the call (query, output, fp16-tier K/V, the
  // symmetric and literal-INT2 formats' scales, an fp16-format middle tier):
  // 0 fp16, 1 bfloat16.  The asymmetric format's scale and zero are fp16.
  int bf16;
  // GQA 5..8 on an unrotated symmetric tier: eight heads per pass whatever the
  // size (else only where every resident workgroup gets at least 8 tiles)
  int force_h8;
};

// Signed symmetric code of channel d in a packed row (fade/quant.py:26-43,
// fade/rotated_quant.py:35-48 layouts).
__device__ __forceinline__ int sym_code_at(const uint8_t* row, int d, int bits) {
  if (bits == 4) {
    const int byte = row[d >> 1];
    const int n = (d & 1) ? (byte & 0xF) : (byte >> 4);
    return n - ((n & 8) << 1);
  }
  const int byte = row[d >> 2];
  const int n = (byte >> (6 - 2 * (d & 3))) & 3;
  return n - ((n & 2) << 1);
}

// Unsigned code of channel d in an asymmetric packed row.
__device__ __forceinline__ int asym_code_at(const uint8_t* row, int d, int bits) {
  if (bits == 4) {
    const int byte = row[d >> 1];
    return (d & 1) ? (byte & 0xF) : (byte >> 4);
  }
  const int byte = row[d >> 2];
  return (byte >> (6 - 2 * (d & 3))) & 3;
}

__global__ void decode_combine_kernel(const float* __restrict__ ws_ml,
                                      const float* __restrict__ ws_acc, int n_splits, int64_t Hq,
                                      uint16_t* __restrict__ out, int64_t o_sb, int64_t o_sh, int bf16);

int launch_valu(const Params& p, hipStream_t st);
// Matrix-core kernel; returns FADE_EINVAL when the middle format is not handled.
int launch_mfma(const Params& p, hipStream_t st);
bool mfma_supports(const Params& p);
// Packed-tier kernel for GQA groups of <= 4 heads (reference INT4 and rotated
// 2-bit formats, asymmetric group-32 formats), with the split merge fused in
// (no combine launch).
bool int4_supports(const Params& p);
int int4_fp16_tiles(const Params& p);
int64_t int4_tiles(const Params& p);
int int4_resident_wgs(const Params& p);  // resident workgroups of the kernel instance for p
int int4_grid_passes(const Params& p);   // head passes the instance's grid carries per kv head
bool eight_heads_pay(const Params& p);   // GQA 5..8, symmetric tier: one eight-head pass rather than two
int launch_int4(const Params& p, hipStream_t st);
// A packed-kernel instance: the kernel, its wavefronts per workgroup, and its
// slot in the resident-workgroup cache (fp16 instances 0..35, bf16 36..71,
// the two-pass symmetric instances of small GQA 5..8 caches 72..79).
struct PackedChoice {
  void (*k)(Params);
  int waves;
  int index;
  int grid_passes;  // head passes in the grid's y dimension (2: the two-pass instance; 1 otherwise)
};
constexpr int kPackedSlots = 80;
// The bfloat16 instance for a middle tier int4_supports accepted (reference
// INT4, rotated 4- or 2-bit, K4 + literal INT2 V; decode_int4_bf16.hip).
PackedChoice packed_kernel_bf16(const Params& p);
int mfma_tile();
// Number of 64-token tiles the matrix-core kernel walks (fp16 tokens, then packed).
int64_t mfma_tiles(const Params& p);
int64_t mfma_target_wgs(const Params& p);  // workgroups of one machine-wide wave at the call's head dim

// Split partials and their merge reads: system-scope accesses (sc0 sc1), which
// go past the XCD's L2 to memory (stores written through, loads fetched), so a
// partial whose store has completed is in memory for a merging workgroup on
// any XCD; per instruction, with no whole-cache write-back or invalidate.
__device__ __forceinline__ void store_sys(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ float load_sys(const float* p) {
  return __builtin_bit_cast(float, __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_SYSTEM));
}
// (m, l) of one partial as one 8-byte access
__device__ __forceinline__ void store_sys2(float* p, float a, float b) {
  const uint64_t v = static_cast<uint64_t>(__builtin_bit_cast(uint32_t, a)) |
                     (static_cast<uint64_t>(__builtin_bit_cast(uint32_t, b)) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void load_sys2(const float* p, float& a, float& b) {
  const uint64_t v =
      __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  a = __builtin_bit_cast(float, static_cast<uint32_t>(v));
  b = __builtin_bit_cast(float, static_cast<uint32_t>(v >> 32));
}

}  // namespace decode
}  // namespace fade
