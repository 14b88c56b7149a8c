// Eviction re-RoPE of surviving keys as one gather + read-modify-write pass.
//
// The reference (fade/cache.py:911-935) un-RoPEs every cached row at its old
// position in fp32, casts to fp16, index_selects the kept rows, re-RoPEs them
// at contiguous positions and casts again -- about a dozen passes over all S
// rows.  Un-RoPE is row-wise, so this kernel touches only the kept rows:
// each thread owns the pair (i, i + D/2) of one kept row, which is exactly
// the pair that rotate_half mixes, and performs both rotations in registers
// with the reference's rounding (three separately rounded fp32 ops per
// rotation, fp16 rounding in between; compiled with -ffp-contract=off).
// V rows are gathered in the same launch.
#include "fade_common.h"

namespace fade {
namespace {

__global__ void rerope_gather_kernel(const uint16_t* __restrict__ k, int64_t ksb, int64_t ksh,
                                     int64_t kss, const uint16_t* __restrict__ v, int64_t vsb,
                                     int64_t vsh, int64_t vss, int64_t H, int64_t S, int D,
                                     const int64_t* __restrict__ keep, int64_t n_kept,
                                     const float* __restrict__ cos_old,
                                     const float* __restrict__ sin_old,
                                     const float* __restrict__ cos_new,
                                     const float* __restrict__ sin_new, uint16_t* __restrict__ k_out,
                                     uint16_t* __restrict__ v_out) {
  const int half = D / 2;
  const int rows_per_block = blockDim.x / half;
  const int i = threadIdx.x % half;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * rows_per_block + threadIdx.x / half;
  const int64_t bh = blockIdx.y;
  if (j >= n_kept) return;
  const int64_t src = keep[j];
  uint16_t* ko = k_out + (bh * n_kept + j) * D;
  uint16_t* vo = v_out ? v_out + (bh * n_kept + j) * D : nullptr;
  if (src < 0 || src >= S) {  // never produced by the host; keep the access in bounds
    ko[i] = ko[i + half] = 0;
    if (vo) vo[i] = vo[i + half] = 0;
    return;
  }
  const uint16_t* kr = k + (bh / H) * ksb + (bh % H) * ksh + src * kss;
  const float a = h2f(kr[i]);         // k[i]
  const float b = h2f(kr[i + half]);  // k[i + D/2]
  // inverse: k*cos - rotate_half(k)*sin, rotate_half(k) = [-k2, k1]
  const float* co = cos_old + src * D;
  const float* so = sin_old + src * D;
  const float u_lo = round_f16(a * co[i] - (-b) * so[i]);
  const float u_hi = round_f16(b * co[i + half] - a * so[i + half]);
  // apply: k*cos + rotate_half(k)*sin at the new position
  const float* cn = cos_new + j * D;
  const float* sn = sin_new + j * D;
  ko[i] = f2h(u_lo * cn[i] + (-u_hi) * sn[i]);
  ko[i + half] = f2h(u_hi * cn[i + half] + u_lo * sn[i + half]);
  if (vo) {
    const uint16_t* vr = v + (bh / H) * vsb + (bh % H) * vsh + src * vss;
    vo[i] = vr[i];
    vo[i + half] = vr[i + half];
  }
}

}  // namespace
}  // namespace fade

using namespace fade;

FADE_API int fade_rerope_gather(const void* k_f16, int64_t ksb, int64_t ksh, int64_t kss,
                                const void* v_f16, int64_t vsb, int64_t vsh, int64_t vss, int64_t B,
                                int64_t H, int64_t S, int64_t D, const int64_t* keep_idx,
                                int64_t n_kept, const float* cos_old, const float* sin_old,
                                const float* cos_new, const float* sin_new, void* k_out_f16,
                                void* v_out_f16, void* stream) {
  if (D <= 0 || D % 2 != 0 || D > 512)
    return einval("fade_rerope_gather: head_dim must be even and <= 512, got %lld", (long long)D);
  if (n_kept < 0 || n_kept > S)
    return einval("fade_rerope_gather: n_kept=%lld out of range for S=%lld", (long long)n_kept, (long long)S);
  if ((v_f16 == nullptr) != (v_out_f16 == nullptr))
    return einval("fade_rerope_gather: v and v_out must both be given or both be NULL");
  const int64_t BH = B * H;
  if (BH == 0 || n_kept == 0) return FADE_OK;
  if (BH > 65535) return einval("fade_rerope_gather: B*H=%lld exceeds 65535", (long long)BH);
  const int half = static_cast<int>(D / 2);
  const int rpb = half >= 256 ? 1 : 256 / half;
  const dim3 grid(static_cast<unsigned>(cdiv(n_kept, rpb)), static_cast<unsigned>(BH));
  hipLaunchKernelGGL(rerope_gather_kernel, grid, dim3(rpb * half), 0, as_stream(stream),
                     static_cast<const uint16_t*>(k_f16), ksb, ksh, kss,
                     static_cast<const uint16_t*>(v_f16), vsb, vsh, vss, H, S, static_cast<int>(D),
                     keep_idx, n_kept, cos_old, sin_old, cos_new, sin_new,
                     static_cast<uint16_t*>(k_out_f16), static_cast<uint16_t*>(v_out_f16));
  return check_launch("fade_rerope_gather");
}
