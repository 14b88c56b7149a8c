// bfloat16 instances of the packed-tier decode attention kernel
// (decode_packed.h), in a translation unit of their own so that the fp16 and
// bf16 instances compile in parallel.  A bfloat16 cache holds the reference
// INT4 format, the rotated 4- or 2-bit format or K4 + literal INT2 V (the
// asymmetric format quantizes fp16 tensors only).
#include "decode_packed.h"

namespace fade {
namespace decode {
namespace {

// Same wave counts and head-pass choices as the fp16 instances
// (decode_int4.hip); slots 36.. of the resident-workgroup cache.
template <bool DET, bool MANY>
PackedChoice packed_bf16_t(const Params& p) {
  constexpr int v = 36 + (DET ? 2 : 0) + (MANY ? 1 : 0);
  const int kb = p.mid.k_bits;
  if (MANY && p.mid.fmt == FADE_MID_SYM && p.rot == nullptr && !p.force_h8 && !eight_heads_pay(p))
    return kb == 4 ? PackedChoice{decode_packed_kernel<4, 4, kFmtSym, 4, DET, true, false, true, false, 2>, 4, 76 + (DET ? 1 : 0), 2}
                   : PackedChoice{decode_packed_kernel<2, 2, kFmtSym, 8, DET, true, false, true, false, 2>, 8, 78 + (DET ? 1 : 0), 2};
  if (p.mid.fmt == FADE_MID_K4V2G)
    return {decode_packed_kernel<4, 8, kFmtLit, 6, DET, MANY, false, true, false, 2>, 6, 4 * 6 + v, MANY ? 2 : 1};
  if (p.rot != nullptr) {
    if (kb == 4) return {decode_packed_kernel<4, 4, kFmtSym, 4, DET, MANY, false, true, true, 2>, 4, 4 * 7 + v, MANY ? 2 : 1};
    return {decode_packed_kernel<2, 2, kFmtSym, 8, DET, MANY, false, true, true, 2>, 8, 4 * 8 + v, MANY ? 2 : 1};
  }
  if (kb == 4) return {decode_packed_kernel<4, 4, kFmtSym, 4, DET, false, MANY, true, false, 2>, 4, 4 * 0 + v, 1};
  return {decode_packed_kernel<2, 2, kFmtSym, 8, DET, false, MANY, true, false, 2>, 8, 4 * 1 + v, 1};
}

}  // namespace

PackedChoice packed_kernel_bf16(const Params& p) {
  if (p.passes > 1) return p.deterministic ? packed_bf16_t<true, true>(p) : packed_bf16_t<false, true>(p);
  return p.deterministic ? packed_bf16_t<true, false>(p) : packed_bf16_t<false, false>(p);
}

}  // namespace decode
}  // namespace fade
