// Host side of the packed-tier decode attention (fp16 instances; the kernel
// template is in decode_packed.h, the bf16 instances in decode_int4_bf16.hip).
#include "decode_packed.h"

namespace fade {
namespace decode {
namespace {

bool aligned(const void* x, uintptr_t a) { return (reinterpret_cast<uintptr_t>(x) & (a - 1)) == 0; }

bool fp16_tier_ok(const Fp16Tier& t) {
  if (t.len == 0) return true;
  return aligned(t.k, 16) && aligned(t.v, 16) && ((t.k_sb | t.k_sh | t.k_ss | t.v_sb | t.v_sh | t.v_ss) % 8 == 0);
}

}  // namespace

bool int4_supports(const Params& p) {
  const MidTier& m = p.mid;
  // G = 5..8 runs as two head passes (the kv tiles are read once per pass);
  // measured faster than the general matrix-core kernel at most shapes
  if (m.len <= 0 || p.G > 8 || p.D != kD) return false;
  if (p.bf16 && m.fmt == FADE_MID_ASYM) return false;  // no bf16 cache holds the asymmetric format
  const bool bits_ok = (m.k_bits == 4 || m.k_bits == 2) && (m.v_bits == 4 || m.v_bits == 2);
  if (m.fmt == FADE_MID_SYM) {
    if (!bits_ok) return false;
    if (m.k_bits != m.v_bits) return false;
    if (!aligned(m.k_scale, 4) || !aligned(m.v_scale, 2)) return false;
  } else if (m.fmt == FADE_MID_K4V2G) {
    // K as the reference INT4 format; V literal int8 codes in 64-token groups
    if (m.group != kTile || m.v_rows < m.len || m.v_rows % kTile) return false;
    if (!aligned(m.k_scale, 4) || !aligned(m.v_scale, 4)) return false;
  } else if (m.fmt == FADE_MID_ASYM) {
    if (!bits_ok || m.group != 32) return false;
    if (!aligned(m.k_scale, 4) || !aligned(m.k_zero, 4) || !aligned(m.v_scale, 4) || !aligned(m.v_zero, 4))
      return false;
  } else {
    return false;
  }
  if (!fp16_tier_ok(p.sink) || !fp16_tier_ok(p.recent)) return false;
  if (!aligned(p.q, 16) || p.q_sb % 8 || p.q_sh % 8) return false;
  return aligned(m.k_codes, 16) && aligned(m.v_codes, 16);
}

int int4_fp16_tiles(const Params& p) {
  const int64_t F = p.total - p.mid.len;
  return static_cast<int>(cdiv(F, kMini));
}

int64_t int4_tiles(const Params& p) { return int4_fp16_tiles(p) + cdiv(p.mid.len, kTile); }

namespace {

// index: the template instance, format slot * 4 + DET * 2 + MANY (bf16: + 36);
// 72..79: the two-pass symmetric instances of small GQA 5..8 caches
typedef PackedChoice Choice;

int cu_count() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        n > 0)
      cus = n;
    else
      (void)hipGetLastError();
  }
  return cus > 0 ? cus : 256;
}

}  // namespace

// GQA 5..8 on a symmetric tier: at least 8 tiles per resident workgroup of the
// eight-head instance (two 4-wave workgroups per CU for 4-bit codes, one
// 8-wave workgroup for 2-bit).
bool eight_heads_pay(const Params& p) {
  const int64_t resident = static_cast<int64_t>(cu_count()) * (p.mid.k_bits == 4 ? 2 : 1);
  return int4_tiles(p) * p.B * p.Hkv >= 8 * resident;
}

namespace {

// The kernel instance for a middle tier int4_supports accepted (wave counts
// measured best on MI355X): the reference INT4 format runs two 4-wave
// workgroups per CU; the others one workgroup per CU, of eight waves where two
// stages per wave fit the 160 KB of LDS, six for the 10 and 12.25 KB stages.
// GQA 5..8 (MANY): the unrotated symmetric formats serve all eight heads in
// one pass (H8, each kv tile read once) when that gives every resident
// workgroup at least 8 tiles; below that (small caches) two head passes keep
// twice the workgroups busy and measured faster (B=8, 28/4 heads, S=4096:
// 16.4 against 19.3 us; B=16, S=8192: 31.4 against 25.4 us).  The other
// formats run two head passes (the rotated 4-bit instance with eight heads
// spills registers in its R merge).
// `index` keys the resident-workgroup cache per template instance, so an
// instance whose registers or LDS differ gets its own occupancy.
template <bool DET, bool MANY>
Choice packed_kernel_t(const Params& p) {
  const int kb = p.mid.k_bits, vb = p.mid.v_bits;
  constexpr int v = (DET ? 2 : 0) + (MANY ? 1 : 0);
  constexpr int gp = MANY ? 2 : 1;
  if (MANY && p.mid.fmt == FADE_MID_SYM && p.rot == nullptr && !p.force_h8 && !eight_heads_pay(p))
    return kb == 4 ? Choice{decode_packed_kernel<4, 4, kFmtSym, 4, DET, true, false, false, false, 2>, 4, 72 + (DET ? 1 : 0), 2}
                   : Choice{decode_packed_kernel<2, 2, kFmtSym, 8, DET, true, false, false, false, 2>, 8, 74 + (DET ? 1 : 0), 2};
  if (p.mid.fmt == FADE_MID_K4V2G)
    return {decode_packed_kernel<4, 8, kFmtLit, 6, DET, MANY, false, false, false, 2>, 6, 4 * 6 + v, gp};
  if (p.mid.fmt == FADE_MID_SYM) {
    if (p.rot != nullptr) {  // rotated backend: q R^T in the prologue, the middle part times R in the merge
      if (kb == 4) return {decode_packed_kernel<4, 4, kFmtSym, 4, DET, MANY, false, false, true, 2>, 4, 4 * 7 + v, gp};
      return {decode_packed_kernel<2, 2, kFmtSym, 8, DET, MANY, false, false, true, 2>, 8, 4 * 8 + v, gp};
    }
    if (kb == 4)  // two workgroups per CU
      return {decode_packed_kernel<4, 4, kFmtSym, 4, DET, false, MANY, false, false, 2>, 4, 4 * 0 + v, 1};
    return {decode_packed_kernel<2, 2, kFmtSym, 8, DET, false, MANY, false, false, 2>, 8, 4 * 1 + v, 1};
  }
  if (kb == 4 && vb == 4)
    return {decode_packed_kernel<4, 4, kFmtAsym, 6, DET, MANY, false, false, false, 2>, 6, 4 * 2 + v, gp};
  if (kb == 4 && vb == 2)
    return {decode_packed_kernel<4, 2, kFmtAsym, 8, DET, MANY, false, false, false, 2>, 8, 4 * 3 + v, gp};
  if (kb == 2 && vb == 2)
    return {decode_packed_kernel<2, 2, kFmtAsym, 8, DET, MANY, false, false, false, 2>, 8, 4 * 4 + v, gp};
  return {decode_packed_kernel<2, 4, kFmtAsym, 6, DET, MANY, false, false, false, 2>, 6, 4 * 5 + v, gp};
}

Choice packed_kernel(const Params& p) {
  if (p.bf16) return packed_kernel_bf16(p);
  if (p.passes > 1) return p.deterministic ? packed_kernel_t<true, true>(p) : packed_kernel_t<false, true>(p);
  return p.deterministic ? packed_kernel_t<true, false>(p) : packed_kernel_t<false, false>(p);
}

}  // namespace

int int4_resident_wgs(const Params& p) {
  static int cached[kPackedSlots] = {};
  const Choice c = packed_kernel(p);
  if (cached[c.index] > 0) return cached[c.index];
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, c.k, 64 * c.waves, 0) != hipSuccess || cus <= 0 ||
      per_cu <= 0) {
    (void)hipGetLastError();
    return 256;
  }
  cached[c.index] = cus * per_cu;
  return cached[c.index];
}

int int4_grid_passes(const Params& p) { return packed_kernel(p).grid_passes; }

int launch_int4(const Params& p, hipStream_t st) {
  const Choice c = packed_kernel(p);
  const dim3 grid(static_cast<unsigned>(p.n_splits), static_cast<unsigned>(p.Hkv * c.grid_passes),
                  static_cast<unsigned>(p.B));
  hipLaunchKernelGGL(c.k, grid, dim3(64 * c.waves), 0, st, p);
  return check_launch("fade_tiered_decode_attn(packed)");
}

}  // namespace decode
}  // namespace fade
