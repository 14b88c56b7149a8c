// Host side of the tiered decode attention: validation, split planning,
// kernel choice and the combine launch.
#include "decode_common.h"

using namespace fade;
using namespace fade::decode;

namespace {

int64_t total_tokens(const fade_decode_args* a) { return a->sink.len + a->mid.len + a->recent.len; }

// Split the token range into n_splits pieces (multiples of the kernel's token
// tile) so that B*Hkv*n_splits workgroups fill the 256 CUs: the matrix-core
// kernel runs two 4-wave workgroups per CU, so ~512 workgroups is one full
// wave of the machine (measured best for configs 1 and 2); the portable
// kernel wants more, smaller workgroups.
void plan_splits(const fade_decode_args* a, int tile, int64_t* n_splits, int64_t* tps,
                 int64_t total_override = -1, int64_t target_wgs = 2048) {
  const int64_t total = total_override >= 0 ? total_override : total_tokens(a);
  const int64_t pairs = a->B * a->Hkv;
  int64_t want = a->n_splits > 0 ? a->n_splits : (target_wgs + pairs / 2) / (pairs > 0 ? pairs : 1);
  const int64_t max_splits = cdiv(total, tile) > 0 ? cdiv(total, tile) : 1;
  if (want > max_splits) want = max_splits;
  if (want < 1) want = 1;
  int64_t t = cdiv(cdiv(total, want), tile) * tile;
  if (t < tile) t = tile;
  *tps = t;
  *n_splits = cdiv(total, t) > 0 ? cdiv(total, t) : 1;
}

int64_t ml_bytes(const fade_decode_args* a, int64_t n) {
  return ((a->B * a->Hq * n * 2 * 4 + 255) / 256) * 256;
}

int validate(const fade_decode_args* a) {
  if (a == nullptr) return einval("fade_tiered_decode_attn: null args");
  if (a->D != kD) return einval("fade_tiered_decode_attn: head_dim must be %d, got %lld", kD, (long long)a->D);
  if (a->B <= 0 || a->Hq <= 0 || a->Hkv <= 0)
    return einval("fade_tiered_decode_attn: B, Hq, Hkv must be positive");
  if (a->Hq % a->Hkv != 0)
    return einval("fade_tiered_decode_attn: Hq=%lld is not a multiple of Hkv=%lld", (long long)a->Hq, (long long)a->Hkv);
  if (a->Hq / a->Hkv > kMaxG)
    return einval("fade_tiered_decode_attn: at most %d query heads per kv head, got %lld", kMaxG,
                  (long long)(a->Hq / a->Hkv));
  if (a->B > 65535 || a->Hkv > 65535) return einval("fade_tiered_decode_attn: B or Hkv too large");
  if (a->sink.len < 0 || a->mid.len < 0 || a->recent.len < 0)
    return einval("fade_tiered_decode_attn: negative tier length");
  if (total_tokens(a) <= 0) return einval("fade_tiered_decode_attn: the cache is empty");
  if (a->q == nullptr || a->out == nullptr) return einval("fade_tiered_decode_attn: null q/out");
  if (a->sink.len > 0 && (a->sink.k == nullptr || a->sink.v == nullptr))
    return einval("fade_tiered_decode_attn: sink tier has null K/V");
  if (a->recent.len > 0 && (a->recent.k == nullptr || a->recent.v == nullptr))
    return einval("fade_tiered_decode_attn: recent tier has null K/V");
  const fade_mid_tier& m = a->mid;
  if (m.len > 0) {
    if (m.k_codes == nullptr || m.v_codes == nullptr)
      return einval("fade_tiered_decode_attn: middle tier has null codes");
    switch (m.fmt) {
      case FADE_MID_FP16:
        break;
      case FADE_MID_SYM:
        if ((m.k_bits != 4 && m.k_bits != 2) || (m.v_bits != 4 && m.v_bits != 2))
          return einval("fade_tiered_decode_attn: SYM bits must be 4 or 2");
        if (m.k_scale == nullptr || m.v_scale == nullptr)
          return einval("fade_tiered_decode_attn: SYM middle tier needs scales");
        break;
      case FADE_MID_K4V2G:
        if (m.group < 1 || m.v_rows < m.len || m.v_rows % m.group != 0)
          return einval("fade_tiered_decode_attn: K4V2G needs group>0 and padded rows %% group == 0");
        if (m.k_scale == nullptr || m.v_scale == nullptr)
          return einval("fade_tiered_decode_attn: K4V2G middle tier needs scales");
        break;
      case FADE_MID_ASYM:
        if ((m.k_bits != 4 && m.k_bits != 2) || (m.v_bits != 4 && m.v_bits != 2))
          return einval("fade_tiered_decode_attn: ASYM bits must be 4 or 2");
        if (m.group != 16 && m.group != 32 && m.group != 64)
          return einval("fade_tiered_decode_attn: ASYM group must be 16, 32 or 64");
        if (!m.k_scale || !m.k_zero || !m.v_scale || !m.v_zero)
          return einval("fade_tiered_decode_attn: ASYM middle tier needs scale and zero");
        break;
      default:
        return einval("fade_tiered_decode_attn: unknown middle format %d", m.fmt);
    }
  }
  if (a->kernel < 0 || a->kernel > 2) return einval("fade_tiered_decode_attn: kernel must be 0, 1 or 2");
  return FADE_OK;
}

Params to_params(const fade_decode_args* a) {
  Params p{};
  p.B = a->B;
  p.Hq = a->Hq;
  p.Hkv = a->Hkv;
  p.G = static_cast<int>(a->Hq / a->Hkv);
  p.q = static_cast<const uint16_t*>(a->q);
  p.q_sb = a->q_sb;
  p.q_sh = a->q_sh;
  p.scale_log2 = a->sm_scale * 1.4426950408889634f;
  auto tier = [](const fade_fp16_tier& t) {
    Fp16Tier r{};
    r.k = static_cast<const uint16_t*>(t.k);
    r.v = static_cast<const uint16_t*>(t.v);
    r.len = t.len;
    r.k_sb = t.k_sb; r.k_sh = t.k_sh; r.k_ss = t.k_ss;
    r.v_sb = t.v_sb; r.v_sh = t.v_sh; r.v_ss = t.v_ss;
    return r;
  };
  p.sink = tier(a->sink);
  p.recent = tier(a->recent);
  const fade_mid_tier& m = a->mid;
  p.mid.fmt = m.len > 0 ? m.fmt : FADE_MID_NONE;
  p.mid.k_bits = m.k_bits;
  p.mid.v_bits = m.v_bits;
  p.mid.group = m.group;
  p.mid.len = m.len;
  p.mid.v_rows = m.v_rows;
  p.mid.k_codes = static_cast<const uint8_t*>(m.k_codes);
  p.mid.k_scale = static_cast<const uint16_t*>(m.k_scale);
  p.mid.k_zero = static_cast<const uint16_t*>(m.k_zero);
  p.mid.v_codes = static_cast<const uint8_t*>(m.v_codes);
  p.mid.v_scale = static_cast<const uint16_t*>(m.v_scale);
  p.mid.v_zero = static_cast<const uint16_t*>(m.v_zero);
  p.total = total_tokens(a);
  return p;
}

bool use_mfma(const fade_decode_args* a, const Params& p) {
  if (a->kernel == 1) return false;
  return mfma_supports(p);
}

}  // namespace

FADE_API int fade_tiered_decode_workspace_bytes(const fade_decode_args* a, int64_t* bytes) {
  int rc = validate(a);
  if (rc) return rc;
  if (bytes == nullptr) return einval("fade_tiered_decode_workspace_bytes: null output");
  const Params p = to_params(a);
  const bool mfma = use_mfma(a, p);
  int64_t n, tps;
  plan_splits(a, mfma ? mfma_tile() : 64, &n, &tps, mfma ? mfma_tiles(p) * mfma_tile() : -1, mfma ? 512 : 2048);
  *bytes = ml_bytes(a, n) + a->B * a->Hq * n * kD * 4;
  return FADE_OK;
}

FADE_API int fade_tiered_decode_attn(const fade_decode_args* a, void* stream) {
  int rc = validate(a);
  if (rc) return rc;
  Params p = to_params(a);
  const bool mfma = use_mfma(a, p);
  if (a->kernel == 2 && !mfma)
    return einval("fade_tiered_decode_attn: the matrix-core kernel does not handle middle format %d", p.mid.fmt);
  int64_t n, tps;
  plan_splits(a, mfma ? mfma_tile() : 64, &n, &tps, mfma ? mfma_tiles(p) * mfma_tile() : -1, mfma ? 512 : 2048);
  const int64_t need = ml_bytes(a, n) + a->B * a->Hq * n * kD * 4;
  if (a->workspace == nullptr || a->workspace_bytes < need)
    return einval("fade_tiered_decode_attn: workspace too small (%lld < %lld bytes)",
                  (long long)a->workspace_bytes, (long long)need);
  if (n > 65535) return einval("fade_tiered_decode_attn: too many splits");
  p.n_splits = static_cast<int>(n);
  p.tokens_per_split = tps;
  p.ws_ml = static_cast<float*>(a->workspace);
  p.ws_acc = reinterpret_cast<float*>(static_cast<char*>(a->workspace) + ml_bytes(a, n));
  hipStream_t st = as_stream(stream);
  rc = mfma ? launch_mfma(p, st) : launch_valu(p, st);
  if (rc) return rc;
  const int64_t rows = a->B * a->Hq;
  hipLaunchKernelGGL(decode_combine_kernel, dim3(static_cast<unsigned>(rows)), dim3(kD), 0, st,
                     p.ws_ml, p.ws_acc, p.n_splits, a->Hq, static_cast<uint16_t*>(a->out), a->o_sb,
                     a->o_sh);
  return check_launch("fade_tiered_decode_attn(combine)");
}
