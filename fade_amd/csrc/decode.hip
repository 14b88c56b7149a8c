// Tiered decode attention: one query token per (batch, query head) against
// the cache laid out as  sink (fp16) | middle (packed codes) | recent (fp16),
// without materializing fp16 K/V (the reference dequantizes and torch.cat's
// the whole cache every step: fade/cache.py:683-842).
//
// Work split (flash-decoding): one workgroup per (split of the token range,
// kv head, batch row) serves the whole GQA group of Hq/Hkv query heads, so
// each KV byte is read once.  Each workgroup writes an unnormalized partial
// (m, l, acc[D]) in the log2 domain; decode_combine_kernel merges the splits.
// Head dims 32, 64, 128 and 256 (the matrix-core kernels take 128 only).
//
// This file holds the portable VALU kernel (any middle format) and the
// combine pass.  decode_mfma.hip holds the matrix-core kernel for the
// packed symmetric formats.
#include <math.h>

#include "decode_common.h"

namespace fade {
namespace decode {
namespace {

constexpr int kTile = 64;
constexpr int kThreads = 256;

// D/4 dequantized K values of token t of a row whose sink and middle tiers
// hold ns and nm tokens, channels [D/4*quarter, D/4*(quarter+1)).
template <int D>
__device__ void load_kq(const Params& p, int64_t b, int64_t kvh, int64_t t, int64_t ns, int64_t nm, int quarter,
                        const float* ks_s, float* out) {
  constexpr int CQ = D / 4;
  const int d0 = CQ * quarter;
  const Fp16Tier* seg = nullptr;
  int64_t r = t;
  if (t < ns) {
    seg = &p.sink;
  } else if (t < ns + nm) {
    const int64_t m = t - ns;
    const int64_t row = (b * p.Hkv + kvh) * p.mid.len + m;
    switch (p.mid.fmt) {
      case FADE_MID_FP16: {
        const uint16_t* src = reinterpret_cast<const uint16_t*>(p.mid.k_codes) + row * D + d0;
        for (int j = 0; j < CQ; ++j) out[j] = h2f(src[j]);
        return;
      }
      case FADE_MID_SYM:
      case FADE_MID_K4V2G: {
        const int bits = p.mid.fmt == FADE_MID_SYM ? p.mid.k_bits : 4;
        const uint8_t* src = p.mid.k_codes + row * (D * bits / 8);
        for (int j = 0; j < CQ; ++j) {
          const int d = d0 + j;
          out[j] = round_f16(static_cast<float>(sym_code_at(src, d, bits)) * ks_s[d]);
        }
        return;
      }
      default: {  // FADE_MID_ASYM
        const int bits = p.mid.k_bits, g = p.mid.group;
        const uint8_t* src = p.mid.k_codes + row * (D * bits / 8);
        for (int j = 0; j < CQ; ++j) {
          const int d = d0 + j;
          const float s = h2f(p.mid.k_scale[row * (D / g) + d / g]);
          const float z = h2f(p.mid.k_zero[row * (D / g) + d / g]);
          out[j] = round_f16(static_cast<float>(asym_code_at(src, d, bits)) * s + z);
        }
        return;
      }
    }
  } else {
    seg = &p.recent;
    r = t - ns - nm;
  }
  const uint16_t* src = seg->k + b * seg->k_sb + kvh * seg->k_sh + r * seg->k_ss + d0;
  for (int j = 0; j < CQ; ++j) out[j] = h2f(src[j]);
}

// Dequantized V channels d0 .. d0 + N - 1 of token t (tiers as in load_kq).
template <int D, int N>
__device__ void load_vn(const Params& p, int64_t b, int64_t kvh, int64_t t, int64_t ns, int64_t nm, int d0,
                        float* v) {
  const Fp16Tier* seg = nullptr;
  int64_t r = t;
  if (t < ns) {
    seg = &p.sink;
  } else if (t < ns + nm) {
    const int64_t m = t - ns;
    const int64_t bkv = b * p.Hkv + kvh;
    const int64_t row = bkv * p.mid.len + m;
    switch (p.mid.fmt) {
      case FADE_MID_FP16: {
        const uint16_t* src = reinterpret_cast<const uint16_t*>(p.mid.v_codes) + row * D + d0;
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = h2f(src[j]);
        return;
      }
      case FADE_MID_SYM: {
        const int bits = p.mid.v_bits;
        const uint8_t* src = p.mid.v_codes + row * (D * bits / 8);
        const float s = h2f(p.mid.v_scale[row]);
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = round_f16(static_cast<float>(sym_code_at(src, d0 + j, bits)) * s);
        return;
      }
      case FADE_MID_K4V2G: {
        const int8_t* src = reinterpret_cast<const int8_t*>(p.mid.v_codes) + (bkv * p.mid.v_rows + m) * D + d0;
        const int64_t G = p.mid.v_rows / p.mid.group;
        const uint16_t* sc = p.mid.v_scale + (bkv * G + m / p.mid.group) * D + d0;
#pragma unroll
        for (int j = 0; j < N; ++j) v[j] = round_f16(static_cast<float>(src[j]) * h2f(sc[j]));
        return;
      }
      default: {  // FADE_MID_ASYM
        const int bits = p.mid.v_bits, g = p.mid.group;
        const uint8_t* src = p.mid.v_codes + row * (D * bits / 8);
#pragma unroll
        for (int j = 0; j < N; ++j) {
          const int d = d0 + j;
          const float s = h2f(p.mid.v_scale[row * (D / g) + d / g]);
          const float z = h2f(p.mid.v_zero[row * (D / g) + d / g]);
          v[j] = round_f16(static_cast<float>(asym_code_at(src, d, bits)) * s + z);
        }
        return;
      }
    }
  } else {
    seg = &p.recent;
    r = t - ns - nm;
  }
  const uint16_t* src = seg->v + b * seg->v_sb + kvh * seg->v_sh + r * seg->v_ss + d0;
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = h2f(src[j]);
}

// Portable kernel, head_dim D (32, 64, 128 or 256).  Tile of 64 tokens:
//   A) thread (quarter = wave, token = lane) dots its D/4 channels with all heads;
//   B) wave h finishes head h's scores for the 64 tokens, online softmax;
//   C) thread (heads wave / wave+4, channels CPL*lane .. + CPL-1) accumulates P*V.
template <int D>
__global__ __launch_bounds__(kThreads) void decode_valu_kernel(Params p) {
  constexpr int CQ = D / 4;                   // channels per wave in A
  constexpr int CPL = D >= 64 ? D / 64 : 1;   // channels per lane in C
  constexpr int LANES = D / CPL;              // lanes holding channels in C
  const int split = blockIdx.x;
  const int64_t kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = p.G;

  __shared__ float q_s[kMaxG][D];
  __shared__ float ks_s[D];
  __shared__ float sc_s[4][kMaxG][kTile];
  __shared__ float p_s[kMaxG][kTile];
  __shared__ float alpha_s[kMaxG];

  for (int i = tid; i < G * D; i += kThreads) {
    const int h = i / D, d = i % D;
    q_s[h][d] = h2f(p.q[b * p.q_sb + (kvh * G + h) * p.q_sh + d]);
  }
  if (p.mid.fmt == FADE_MID_SYM || p.mid.fmt == FADE_MID_K4V2G)
    for (int d = tid; d < D; d += kThreads) ks_s[d] = h2f(p.mid.k_scale[(b * p.Hkv + kvh) * D + d]);
  __syncthreads();

  // the row's tier lengths: the tiers' own, or per row (lens, clamped to the padded tiers)
  int64_t ns = p.sink.len, nm = p.mid.len, nr = p.recent.len;
  if (p.lens != nullptr) {
    auto clampl = [](int64_t x, int64_t cap) { return x < 0 ? 0 : (x > cap ? cap : x); };
    ns = clampl(p.lens[3 * b], p.sink.len);
    nm = clampl(p.lens[3 * b + 1], p.mid.len);
    nr = clampl(p.lens[3 * b + 2], p.recent.len);
  }
  const int64_t total = ns + nm + nr;
  const int64_t t_begin = static_cast<int64_t>(split) * p.tokens_per_split;
  const int64_t t_end = t_begin + p.tokens_per_split < total ? t_begin + p.tokens_per_split : total;

  float m_run[2] = {-INFINITY, -INFINITY};
  float l_lane[2] = {0.0f, 0.0f};
  float acc[2][CPL];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int c = 0; c < CPL; ++c) acc[hh][c] = 0.0f;

  for (int64_t ts = t_begin; ts < t_end; ts += kTile) {
    {  // A
      const int64_t t = ts + lane;
      float part[kMaxG];
#pragma unroll
      for (int h = 0; h < kMaxG; ++h) part[h] = 0.0f;
      if (t < t_end) {
        float kv[CQ];
        load_kq<D>(p, b, kvh, t, ns, nm, wave, ks_s, kv);
        for (int h = 0; h < G; ++h) {
          float s = 0.0f;
#pragma unroll
          for (int j = 0; j < CQ; ++j) s += q_s[h][CQ * wave + j] * kv[j];
          part[h] = s;
        }
      }
      for (int h = 0; h < G; ++h) sc_s[wave][h][lane] = part[h];
    }
    __syncthreads();
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {  // B
      const int h = wave + 4 * hh;
      if (h < G) {
        const int64_t t = ts + lane;
        float s = -INFINITY;
        if (t < t_end)
          s = (sc_s[0][h][lane] + sc_s[1][h][lane] + sc_s[2][h][lane] + sc_s[3][h][lane]) * p.scale_log2;
        const float m_new = fmaxf(m_run[hh], group_max<64>(s));
        float alpha = 1.0f, pv = 0.0f;
        if (m_new != -INFINITY) {
          alpha = exp2f(m_run[hh] - m_new);
          pv = exp2f(s - m_new);
        }
        l_lane[hh] = l_lane[hh] * alpha + pv;
        p_s[h][lane] = pv;
        if (lane == 0) alpha_s[h] = alpha;
        m_run[hh] = m_new;
      }
    }
    __syncthreads();
    if (lane < LANES) {  // C
      const int nv = static_cast<int>(t_end - ts < kTile ? t_end - ts : kTile);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int h = wave + 4 * hh;
        if (h < G)
#pragma unroll
          for (int c = 0; c < CPL; ++c) acc[hh][c] *= alpha_s[h];
      }
      for (int lt = 0; lt < nv; ++lt) {
        float v[CPL];
        load_vn<D, CPL>(p, b, kvh, ts + lt, ns, nm, CPL * lane, v);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int h = wave + 4 * hh;
          if (h < G) {
            const float pp = p_s[h][lt];
#pragma unroll
            for (int c = 0; c < CPL; ++c) acc[hh][c] += pp * v[c];
          }
        }
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int h = wave + 4 * hh;
    if (h < G) {
      const float l = group_sum<64>(l_lane[hh]);
      const int64_t idx = (b * p.Hq + kvh * G + h) * p.n_splits + split;
      if (lane == 0) {
        p.ws_ml[2 * idx] = m_run[hh];
        p.ws_ml[2 * idx + 1] = l;
      }
      if (lane < LANES)
#pragma unroll
        for (int c = 0; c < CPL; ++c) p.ws_acc[idx * D + CPL * lane + c] = acc[hh][c];
    }
  }
}

}  // namespace

// Merge the n_splits partials of each (b, hq) into the fp16 output; one
// thread per channel (blockDim.x = head_dim D).
__global__ __launch_bounds__(256) void decode_combine_kernel(const float* __restrict__ ws_ml,
                                                             const float* __restrict__ ws_acc,
                                                             int n_splits, int64_t Hq,
                                                             uint16_t* __restrict__ out,
                                                             int64_t o_sb, int64_t o_sh) {
  const int64_t bh = blockIdx.x;
  const int d = threadIdx.x, D = blockDim.x;
  const float* ml = ws_ml + bh * n_splits * 2;
  float M = -INFINITY;
  for (int s = 0; s < n_splits; ++s) M = fmaxf(M, ml[2 * s]);
  float L = 0.0f, o = 0.0f;
  if (M != -INFINITY) {
    for (int s = 0; s < n_splits; ++s) {
      const float m = ml[2 * s];
      if (m == -INFINITY) continue;
      const float w = exp2f(m - M);
      L += ml[2 * s + 1] * w;
      o += ws_acc[(bh * n_splits + s) * D + d] * w;
    }
  }
  out[(bh / Hq) * o_sb + (bh % Hq) * o_sh + d] = f2h(o / L);
}

int launch_valu(const Params& p, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(p.n_splits), static_cast<unsigned>(p.Hkv),
                  static_cast<unsigned>(p.B));
  switch (p.D) {
    case 32: hipLaunchKernelGGL(decode_valu_kernel<32>, grid, dim3(kThreads), 0, st, p); break;
    case 64: hipLaunchKernelGGL(decode_valu_kernel<64>, grid, dim3(kThreads), 0, st, p); break;
    case 128: hipLaunchKernelGGL(decode_valu_kernel<128>, grid, dim3(kThreads), 0, st, p); break;
    case 256: hipLaunchKernelGGL(decode_valu_kernel<256>, grid, dim3(kThreads), 0, st, p); break;
    default: return einval("fade_tiered_decode_attn: head_dim must be 32, 64, 128 or 256, got %d", p.D);
  }
  return check_launch("fade_tiered_decode_attn(valu)");
}

}  // namespace decode
}  // namespace fade
