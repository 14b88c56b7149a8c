// bfloat16 instances of the packed-tier decode attention kernel
// (decode_packed.h), in a translation unit of their own so that the fp16 and
// bf16 instances compile in parallel.  A bfloat16 cache holds the reference
// INT4 format, the rotated 4- or 2-bit format or K4 + literal INT2 V (the
// asymmetric format quantizes fp16 tensors only).
#include "decode_packed.h"

namespace fade {
namespace decode {
namespace {

// Same wave counts as the fp16 instances (decode_int4.hip); slots 36.. of the
// resident-workgroup cache.
template <bool DET, bool TWO>
PackedChoice packed_bf16_t(const Params& p) {
  constexpr int v = 36 + (DET ? 2 : 0) + (TWO ? 1 : 0);
  const int kb = p.mid.k_bits;
  if (p.mid.fmt == FADE_MID_K4V2G) return {decode_packed_kernel<4, 8, kFmtLit, 6, DET, TWO, true, false, 2>, 6, 4 * 6 + v};
  if (p.rot != nullptr) {
    if (kb == 4) return {decode_packed_kernel<4, 4, kFmtSym, 4, DET, TWO, true, true, 2>, 4, 4 * 7 + v};
    return {decode_packed_kernel<2, 2, kFmtSym, 8, DET, TWO, true, true, 2>, 8, 4 * 8 + v};
  }
  if (kb == 4) return {decode_packed_kernel<4, 4, kFmtSym, 4, DET, TWO, true, false, 2>, 4, 4 * 0 + v};
  return {decode_packed_kernel<2, 2, kFmtSym, 8, DET, TWO, true, false, 2>, 8, 4 * 1 + v};
}

}  // namespace

PackedChoice packed_kernel_bf16(const Params& p) {
  if (p.passes > 1) return p.deterministic ? packed_bf16_t<true, true>(p) : packed_bf16_t<false, true>(p);
  return p.deterministic ? packed_bf16_t<true, false>(p) : packed_bf16_t<false, false>(p);
}

}  // namespace decode
}  // namespace fade
