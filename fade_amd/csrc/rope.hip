// Eviction re-RoPE of surviving keys as one gather + read-modify-write pass.
//
// The reference (fade/cache.py:911-935) un-RoPEs every cached row at its old
// position in fp32, casts to fp16, index_selects the kept rows, re-RoPEs them
// at contiguous positions and casts again -- about a dozen passes over all S
// rows.  Un-RoPE is row-wise, so this kernel touches only the kept rows:
// each thread owns the pair (i, i + D/2) of one kept row, which is exactly
// the pair that rotate_half mixes, and performs both rotations in registers
// with the reference's rounding (three separately rounded fp32 ops per
// rotation, a rounding to the cache dtype -- fp16, bf16 or none for fp32 -- in between;
// compiled with -ffp-contract=off).  V rows are gathered in the same launch.
#include "fade_common.h"

namespace fade {
namespace {

template <typename T>
__global__ void rerope_gather_kernel(const T* __restrict__ k, int64_t ksb, int64_t ksh,
                                     int64_t kss, const T* __restrict__ v, int64_t vsb,
                                     int64_t vsh, int64_t vss, int64_t H, int64_t S, int D,
                                     const int64_t* __restrict__ keep, int64_t n_kept,
                                     const float* __restrict__ cos_old,
                                     const float* __restrict__ sin_old,
                                     const float* __restrict__ cos_new,
                                     const float* __restrict__ sin_new, T* __restrict__ k_out,
                                     T* __restrict__ v_out) {
  const int half = D / 2;
  const int rows_per_block = blockDim.x / half;
  const int i = threadIdx.x % half;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * rows_per_block + threadIdx.x / half;
  const int64_t bh = blockIdx.y;
  if (j >= n_kept) return;
  const int64_t src = keep[j];
  T* ko = k_out + (bh * n_kept + j) * D;
  T* vo = v_out ? v_out + (bh * n_kept + j) * D : nullptr;
  if (src < 0 || src >= S) {  // never produced by the host; keep the access in bounds
    ko[i] = ko[i + half] = from_f32<T>(0.0f);
    if (vo) vo[i] = vo[i + half] = from_f32<T>(0.0f);
    return;
  }
  const T* kr = k + (bh / H) * ksb + (bh % H) * ksh + src * kss;
  const float a = to_f32(kr[i]);         // k[i]
  const float b = to_f32(kr[i + half]);  // k[i + D/2]
  // inverse: k*cos - rotate_half(k)*sin, rotate_half(k) = [-k2, k1]
  const float* co = cos_old + src * D;
  const float* so = sin_old + src * D;
  const float u_lo = round_to<T>(a * co[i] - (-b) * so[i]);
  const float u_hi = round_to<T>(b * co[i + half] - a * so[i + half]);
  // apply: k*cos + rotate_half(k)*sin at the new position
  const float* cn = cos_new + j * D;
  const float* sn = sin_new + j * D;
  ko[i] = from_f32<T>(u_lo * cn[i] + (-u_hi) * sn[i]);
  ko[i + half] = from_f32<T>(u_hi * cn[i + half] + u_lo * sn[i + half]);
  if (vo) {
    const T* vr = v + (bh / H) * vsb + (bh % H) * vsh + src * vss;
    vo[i] = vr[i];
    vo[i + half] = vr[i + half];
  }
}

// Four element pairs (i .. i+3, i+D/2 .. i+D/2+3) per thread: the same
// arithmetic per element as the kernel above, with 4-element K/V accesses and
// 16-byte table reads (D/2 a multiple of 4; K/V rows 4-element aligned).
template <typename T>
struct alignas(4 * sizeof(T)) Vec4 {
  T e[4];
};
template <typename T>
__global__ void rerope_gather_vec4_kernel(const T* __restrict__ k, int64_t ksb, int64_t ksh, int64_t kss,
                                          const T* __restrict__ v, int64_t vsb, int64_t vsh, int64_t vss, int64_t H,
                                          int64_t S, int D, const int64_t* __restrict__ keep, int64_t n_kept,
                                          const float* __restrict__ cos_old, const float* __restrict__ sin_old,
                                          const float* __restrict__ cos_new, const float* __restrict__ sin_new,
                                          T* __restrict__ k_out, T* __restrict__ v_out) {
  const int half = D / 2, tpr = half / 4;  // threads per row
  const int rows_per_block = blockDim.x / tpr;
  const int i = 4 * (threadIdx.x % tpr);
  const int64_t j = static_cast<int64_t>(blockIdx.x) * rows_per_block + threadIdx.x / tpr;
  const int64_t bh = blockIdx.y;
  if (j >= n_kept) return;
  const int64_t src = keep[j];
  T* ko = k_out + (bh * n_kept + j) * D;
  T* vo = v_out ? v_out + (bh * n_kept + j) * D : nullptr;
  Vec4<T> klo, khi, vlo, vhi;
  if (src < 0 || src >= S) {  // never produced by the host; keep the access in bounds
#pragma unroll
    for (int e = 0; e < 4; ++e) klo.e[e] = khi.e[e] = from_f32<T>(0.0f);
    *reinterpret_cast<Vec4<T>*>(ko + i) = klo;
    *reinterpret_cast<Vec4<T>*>(ko + i + half) = khi;
    if (vo) {
      *reinterpret_cast<Vec4<T>*>(vo + i) = klo;
      *reinterpret_cast<Vec4<T>*>(vo + i + half) = khi;
    }
    return;
  }
  const T* kr = k + (bh / H) * ksb + (bh % H) * ksh + src * kss;
  const Vec4<T> a4 = *reinterpret_cast<const Vec4<T>*>(kr + i);
  const Vec4<T> b4 = *reinterpret_cast<const Vec4<T>*>(kr + i + half);
  const float4 col = *reinterpret_cast<const float4*>(cos_old + src * D + i);
  const float4 coh = *reinterpret_cast<const float4*>(cos_old + src * D + i + half);
  const float4 sol = *reinterpret_cast<const float4*>(sin_old + src * D + i);
  const float4 soh = *reinterpret_cast<const float4*>(sin_old + src * D + i + half);
  const float4 cnl = *reinterpret_cast<const float4*>(cos_new + j * D + i);
  const float4 cnh = *reinterpret_cast<const float4*>(cos_new + j * D + i + half);
  const float4 snl = *reinterpret_cast<const float4*>(sin_new + j * D + i);
  const float4 snh = *reinterpret_cast<const float4*>(sin_new + j * D + i + half);
  const float co_l[4] = {col.x, col.y, col.z, col.w}, co_h[4] = {coh.x, coh.y, coh.z, coh.w};
  const float so_l[4] = {sol.x, sol.y, sol.z, sol.w}, so_h[4] = {soh.x, soh.y, soh.z, soh.w};
  const float cn_l[4] = {cnl.x, cnl.y, cnl.z, cnl.w}, cn_h[4] = {cnh.x, cnh.y, cnh.z, cnh.w};
  const float sn_l[4] = {snl.x, snl.y, snl.z, snl.w}, sn_h[4] = {snh.x, snh.y, snh.z, snh.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a = to_f32(a4.e[e]), b = to_f32(b4.e[e]);
    const float u_lo = round_to<T>(a * co_l[e] - (-b) * so_l[e]);
    const float u_hi = round_to<T>(b * co_h[e] - a * so_h[e]);
    klo.e[e] = from_f32<T>(u_lo * cn_l[e] + (-u_hi) * sn_l[e]);
    khi.e[e] = from_f32<T>(u_hi * cn_h[e] + u_lo * sn_h[e]);
  }
  *reinterpret_cast<Vec4<T>*>(ko + i) = klo;
  *reinterpret_cast<Vec4<T>*>(ko + i + half) = khi;
  if (vo) {
    const T* vr = v + (bh / H) * vsb + (bh % H) * vsh + src * vss;
    vlo = *reinterpret_cast<const Vec4<T>*>(vr + i);
    vhi = *reinterpret_cast<const Vec4<T>*>(vr + i + half);
    *reinterpret_cast<Vec4<T>*>(vo + i) = vlo;
    *reinterpret_cast<Vec4<T>*>(vo + i + half) = vhi;
  }
}

}  // namespace
}  // namespace fade

using namespace fade;

namespace fade {
namespace {
template <typename T>
int rerope_gather(const char* fn, const void* k, int64_t ksb, int64_t ksh, int64_t kss, const void* v, int64_t vsb,
                  int64_t vsh, int64_t vss, int64_t B, int64_t H, int64_t S, int64_t D, const int64_t* keep_idx,
                  int64_t n_kept, const float* cos_old, const float* sin_old, const float* cos_new,
                  const float* sin_new, void* k_out, void* v_out, void* stream) {
  if (D <= 0 || D % 2 != 0 || D > 512) return einval("%s: head_dim must be even and <= 512, got %lld", fn, (long long)D);
  if (n_kept < 0 || n_kept > S)
    return einval("%s: n_kept=%lld out of range for S=%lld", fn, (long long)n_kept, (long long)S);
  if ((v == nullptr) != (v_out == nullptr)) return einval("%s: v and v_out must both be given or both be NULL", fn);
  const int64_t BH = B * H;
  if (BH == 0 || n_kept == 0) return FADE_OK;
  if (BH > 65535) return einval("%s: B*H=%lld exceeds 65535", fn, (long long)BH);
  const int half = static_cast<int>(D / 2);
  auto al = [](const void* p, int b) { return (reinterpret_cast<uintptr_t>(p) % b) == 0; };
  const int vb = 4 * static_cast<int>(sizeof(T));  // bytes of 4 elements
  if (half % 4 == 0 && half / 4 <= 256 && al(k, vb) && al(k_out, vb) && (ksb | ksh | kss) % 4 == 0 &&
      (v == nullptr || (al(v, vb) && al(v_out, vb) && (vsb | vsh | vss) % 4 == 0)) && al(cos_old, 16) &&
      al(sin_old, 16) && al(cos_new, 16) && al(sin_new, 16)) {
    const int tpr = half / 4, rpb4 = 256 / tpr;
    const dim3 grid4(static_cast<unsigned>(cdiv(n_kept, rpb4)), static_cast<unsigned>(BH));
    hipLaunchKernelGGL(rerope_gather_vec4_kernel<T>, grid4, dim3(rpb4 * tpr), 0, as_stream(stream),
                       static_cast<const T*>(k), ksb, ksh, kss, static_cast<const T*>(v), vsb, vsh, vss, H, S,
                       static_cast<int>(D), keep_idx, n_kept, cos_old, sin_old, cos_new, sin_new,
                       static_cast<T*>(k_out), static_cast<T*>(v_out));
    return check_launch(fn);
  }
  const int rpb = half >= 256 ? 1 : 256 / half;
  const dim3 grid(static_cast<unsigned>(cdiv(n_kept, rpb)), static_cast<unsigned>(BH));
  hipLaunchKernelGGL(rerope_gather_kernel<T>, grid, dim3(rpb * half), 0, as_stream(stream), static_cast<const T*>(k),
                     ksb, ksh, kss, static_cast<const T*>(v), vsb, vsh, vss, H, S, static_cast<int>(D), keep_idx,
                     n_kept, cos_old, sin_old, cos_new, sin_new, static_cast<T*>(k_out), static_cast<T*>(v_out));
  return check_launch(fn);
}
}  // namespace
}  // namespace fade

FADE_API int fade_rerope_gather(const void* k_f16, int64_t ksb, int64_t ksh, int64_t kss,
                                const void* v_f16, int64_t vsb, int64_t vsh, int64_t vss, int64_t B,
                                int64_t H, int64_t S, int64_t D, const int64_t* keep_idx,
                                int64_t n_kept, const float* cos_old, const float* sin_old,
                                const float* cos_new, const float* sin_new, void* k_out_f16,
                                void* v_out_f16, void* stream) {
  return rerope_gather<uint16_t>("fade_rerope_gather", k_f16, ksb, ksh, kss, v_f16, vsb, vsh, vss, B, H, S, D,
                                 keep_idx, n_kept, cos_old, sin_old, cos_new, sin_new, k_out_f16, v_out_f16, stream);
}

FADE_API int fade_rerope_gather_dtype(const void* k, int64_t ksb, int64_t ksh, int64_t kss, const void* v,
                                      int64_t vsb, int64_t vsh, int64_t vss, int64_t B, int64_t H, int64_t S,
                                      int64_t D, const int64_t* keep_idx, int64_t n_kept, const float* cos_old,
                                      const float* sin_old, const float* cos_new, const float* sin_new,
                                      void* k_out, void* v_out, int32_t dtype, void* stream) {
  const char* fn = "fade_rerope_gather_dtype";
  switch (dtype) {
    case FADE_DTYPE_F16:
      return rerope_gather<uint16_t>(fn, k, ksb, ksh, kss, v, vsb, vsh, vss, B, H, S, D, keep_idx, n_kept, cos_old,
                                     sin_old, cos_new, sin_new, k_out, v_out, stream);
    case FADE_DTYPE_BF16:
      return rerope_gather<Bf16>(fn, k, ksb, ksh, kss, v, vsb, vsh, vss, B, H, S, D, keep_idx, n_kept, cos_old,
                                 sin_old, cos_new, sin_new, k_out, v_out, stream);
    case FADE_DTYPE_F32:
      return rerope_gather<float>(fn, k, ksb, ksh, kss, v, vsb, vsh, vss, B, H, S, D, keep_idx, n_kept, cos_old,
                                  sin_old, cos_new, sin_new, k_out, v_out, stream);
    default: return einval("%s: unknown dtype %d", fn, dtype);
  }
}
