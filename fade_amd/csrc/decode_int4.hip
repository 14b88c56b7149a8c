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

// index: the template instance, format slot * 4 + DET * 2 + TWO (bf16: + 36)
typedef PackedChoice Choice;

// The kernel instance for a middle tier int4_supports accepted (wave counts
// measured best on MI355X): the reference INT4 format runs two 4-wave
// workgroups per CU; the others one workgroup per CU, of eight waves where two
// stages per wave fit the 160 KB of LDS, six for the 10 and 12.25 KB stages.
// `index` keys the resident-workgroup cache per template instance, so an
// instance whose registers or LDS differ gets its own occupancy.
template <bool DET, bool TWO>
Choice packed_kernel_t(const Params& p) {
  const int kb = p.mid.k_bits, vb = p.mid.v_bits;
  constexpr int v = (DET ? 2 : 0) + (TWO ? 1 : 0);
  if (p.mid.fmt == FADE_MID_K4V2G) return {decode_packed_kernel<4, 8, kFmtLit, 6, DET, TWO, false, false, 2>, 6, 4 * 6 + v};
  if (p.mid.fmt == FADE_MID_SYM) {
    if (p.rot != nullptr) {  // rotated backend: q R^T in the prologue, the middle part times R in the merge
      if (kb == 4) return {decode_packed_kernel<4, 4, kFmtSym, 4, DET, TWO, false, true, 2>, 4, 4 * 7 + v};
      return {decode_packed_kernel<2, 2, kFmtSym, 8, DET, TWO, false, true, 2>, 8, 4 * 8 + v};
    }
    if (kb == 4) return {decode_packed_kernel<4, 4, kFmtSym, 4, DET, TWO, false, false, 2>, 4, 4 * 0 + v};  // two workgroups per CU
    return {decode_packed_kernel<2, 2, kFmtSym, 8, DET, TWO, false, false, 2>, 8, 4 * 1 + v};
  }
  if (kb == 4 && vb == 4) return {decode_packed_kernel<4, 4, kFmtAsym, 6, DET, TWO, false, false, 2>, 6, 4 * 2 + v};
  if (kb == 4 && vb == 2) return {decode_packed_kernel<4, 2, kFmtAsym, 8, DET, TWO, false, false, 2>, 8, 4 * 3 + v};
  if (kb == 2 && vb == 2) return {decode_packed_kernel<2, 2, kFmtAsym, 8, DET, TWO, false, false, 2>, 8, 4 * 4 + v};
  return {decode_packed_kernel<2, 4, kFmtAsym, 6, DET, TWO, false, false, 2>, 6, 4 * 5 + v};
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

int launch_int4(const Params& p, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(p.n_splits), static_cast<unsigned>(p.Hkv * p.passes),
                  static_cast<unsigned>(p.B));
  const Choice c = packed_kernel(p);
  hipLaunchKernelGGL(c.k, grid, dim3(64 * c.waves), 0, st, p);
  return check_launch("fade_tiered_decode_attn(packed)");
}

}  // namespace decode
}  // namespace fade
