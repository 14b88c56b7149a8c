// Host side of the tiered decode attention: validation, split planning,
// kernel choice and the combine launch.
#include <mutex>

#include "decode_common.h"

using namespace fade;
using namespace fade::decode;

// The library's own decode scratch (fade_tiered_decode_attn_noalloc): 16 MiB on
// every GPU the library runs on, held until the process ends.  Host code never
// uses this name as an address: the per-device address comes from
// hipGetSymbolAddress (scratch_for below).
constexpr int64_t kScratchBytes = 16ll << 20;
constexpr int64_t kScratchCounterBytes = 256ll << 10;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

int64_t total_tokens(const fade_decode_args* a) { return a->sink.len + a->mid.len + a->recent.len; }

// Split the token range into n_splits pieces (multiples of the kernel's token
// tile) so that B*Hkv*n_splits workgroups fill the 256 CUs: the matrix-core
// kernel runs two 4-wave workgroups per CU, so ~512 workgroups is one full
// wave of the machine (measured best for configs 1 and 2); the portable
// kernel wants more, smaller workgroups.
void plan_splits(const fade_decode_args* a, int tile, int64_t* n_splits, int64_t* tps,
                 int64_t total_override = -1, int64_t target_wgs = 2048, int64_t min_tiles = 1) {
  const int64_t total = total_override >= 0 ? total_override : total_tokens(a);
  const int64_t pairs = a->B * a->Hkv;
  int64_t want = a->n_splits > 0 ? a->n_splits : (target_wgs + pairs / 2) / (pairs > 0 ? pairs : 1);
  const int64_t max_splits = cdiv(total, tile) > 0 ? cdiv(total, tile) : 1;
  // automatic split counts keep at least min_tiles tiles per split
  if (a->n_splits <= 0 && want > cdiv(total, tile * min_tiles)) want = cdiv(total, tile * min_tiles);
  if (want > max_splits) want = max_splits;
  if (want < 1) want = 1;
  int64_t t = cdiv(cdiv(total, want), tile) * tile;
  if (t < tile) t = tile;
  *tps = t;
  *n_splits = cdiv(total, t) > 0 ? cdiv(total, t) : 1;
}

int64_t round256(int64_t x) { return ((x + 255) / 256) * 256; }

// Workspace: [counters: B*Hkv*P u32][ml: rows*n*2 f32][acc: rows*n*D f32], rows
// covering both partial layouts (B*Hq per query head, or B*Hkv*4*P); P =
// ceil((Hq/Hkv) / 4) head passes of the INT4 kernel.
struct WsLayout {
  int64_t counters, ml, acc, total;
};
WsLayout ws_layout(const fade_decode_args* a, int64_t n) {
  const int64_t P = (a->Hq / a->Hkv + 3) / 4;
  const int64_t rows = a->B * (a->Hq > a->Hkv * 4 * P ? a->Hq : a->Hkv * 4 * P);
  WsLayout w;
  w.counters = 0;
  w.ml = round256(a->B * a->Hkv * P * 4);
  w.acc = w.ml + round256(rows * n * 2 * 4);
  w.total = w.acc + rows * n * a->D * 4;
  return w;
}

int validate(const fade_decode_args* a) {
  if (a == nullptr) return einval("fade_tiered_decode_attn: null args");
  if (a->D < 8 || a->D > 256 || a->D % 8 != 0)
    return einval("fade_tiered_decode_attn: head_dim must be a multiple of 8 in [8, 256], got %lld", (long long)a->D);
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
    if (m.pages != nullptr) {
      if (m.fmt != FADE_MID_SYM && m.fmt != FADE_MID_ASYM)
        return einval("fade_tiered_decode_attn: paged middle tiers are FADE_MID_SYM or FADE_MID_ASYM");
      if (m.pages_per_row < cdiv(m.len, 64))
        return einval("fade_tiered_decode_attn: pages_per_row=%lld < %lld tiles of the middle tier",
                      (long long)m.pages_per_row, (long long)cdiv(m.len, 64));
      if (m.page_stride != 0) {
        const int64_t need = 64 * 16 * (m.k_bits > m.v_bits ? m.k_bits : m.v_bits);
        if (m.fmt != FADE_MID_SYM || m.page_stride < need || m.page_stride % 16 != 0)
          return einval("fade_tiered_decode_attn: page_stride needs FADE_MID_SYM, a multiple of 16 and >= %lld",
                        (long long)need);
      }
    }
  }
  if (a->kernel < 0 || a->kernel > 4) return einval("fade_tiered_decode_attn: kernel must be 0, 1, 2, 3 or 4");
  if (a->dtype != FADE_DTYPE_F16 && a->dtype != FADE_DTYPE_BF16)
    return einval("fade_tiered_decode_attn: dtype must be FADE_DTYPE_F16 or FADE_DTYPE_BF16, got %d", a->dtype);
  if (a->dtype == FADE_DTYPE_BF16) {
    if (a->mid.len > 0 && a->mid.fmt == FADE_MID_ASYM)
      return einval("fade_tiered_decode_attn: the asymmetric middle format holds fp16 tensors; bfloat16 calls "
                    "take FADE_MID_SYM, FADE_MID_K4V2G or FADE_MID_FP16");
  }
  if (a->rotation != nullptr && a->mid.len > 0) {
    if (a->mid.fmt != FADE_MID_SYM)
      return einval("fade_tiered_decode_attn: a rotation applies to a FADE_MID_SYM middle tier");
    if (reinterpret_cast<uintptr_t>(a->rotation) & 15)
      return einval("fade_tiered_decode_attn: rotation must be 16-byte aligned");
  }
  return FADE_OK;
}

Params to_params(const fade_decode_args* a) {
  Params p{};
  p.B = a->B;
  p.Hq = a->Hq;
  p.Hkv = a->Hkv;
  p.G = static_cast<int>(a->Hq / a->Hkv);
  p.D = static_cast<int>(a->D);
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
  p.mid.pages = m.pages;
  p.mid.pages_per_row = m.pages_per_row;
  p.mid.page_stride = m.pages != nullptr ? m.page_stride : 0;
  p.total = total_tokens(a);
  p.lens = a->lens;
  p.deterministic = a->deterministic;
  p.passes = static_cast<int>((p.G + 3) / 4);
  p.rot = m.len > 0 ? a->rotation : nullptr;  // no middle tokens: nothing is rotated
  p.bf16 = a->dtype == FADE_DTYPE_BF16 ? 1 : 0;
  p.force_h8 = a->kernel == 4 ? 1 : 0;
  return p;
}

enum class Kern { kValu, kMfma, kInt4 };

// kernel: 0 auto, 1 portable VALU, 2 matrix-core (INT4 kernel when it applies),
// 3 the general matrix-core kernel.
Kern choose(const fade_decode_args* a, const Params& p) {
  if (a->kernel == 1) return Kern::kValu;
  if (a->kernel != 3 && int4_supports(p)) return Kern::kInt4;
  if (mfma_supports(p)) return Kern::kMfma;
  return Kern::kValu;
}

struct Plan {
  Kern k;
  int64_t n, tps, n_f16_tiles, tiles_per_split;
};

Plan make_plan(const fade_decode_args* a, const Params& p) {
  Plan pl{};
  pl.k = choose(a, p);
  if (pl.k == Kern::kInt4) {
    // One machine-wide wave of resident workgroups; tiles of either kind cost
    // about the same bytes (8 KB), so splits take equal tile counts.
    const int64_t nT = int4_tiles(p);
    const int64_t pairs = a->B * a->Hkv * int4_grid_passes(p);  // workgroups per split
    int64_t want = a->n_splits > 0 ? a->n_splits : (int4_resident_wgs(p) + pairs / 2) / pairs;
    pl.n_f16_tiles = int4_fp16_tiles(p);
    pl.tps = 0;
    if (p.rot != nullptr) {
      // rotated middle tier: split 0 = the fp16 tiles, then middle splits of equal tile counts
      const int64_t nMt = nT - pl.n_f16_tiles;
      int64_t ms = want - 1;
      if (ms > nMt) ms = nMt;
      if (ms < 1) ms = 1;
      if (p.mid.pages != nullptr && ms < cdiv(nMt, kPageSlots)) ms = cdiv(nMt, kPageSlots);
      pl.tiles_per_split = cdiv(nMt, ms);
      pl.n = 1 + cdiv(nMt, pl.tiles_per_split);
      return pl;
    }
    if (want > nT) want = nT;
    if (want < 1) want = 1;
    // paged middle tier: a split's page ids fit the workgroup's kPageSlots
    if (p.mid.pages != nullptr && want < cdiv(nT, kPageSlots)) want = cdiv(nT, kPageSlots);
    pl.tiles_per_split = cdiv(nT, want);
    pl.n = cdiv(nT, pl.tiles_per_split);
    return pl;
  }
  if (pl.k == Kern::kMfma) {
    plan_splits(a, mfma_tile(), &pl.n, &pl.tps, mfma_tiles(p) * mfma_tile(), mfma_target_wgs(p));
    return pl;
  }
  // Portable kernel: at least four 64-token tiles per split, about 1024
  // workgroups (2048 at head_dim 128).  Measured at head dims 32, 64, 128 and
  // 256, 14/2 and 32/8 heads, B = 4 and 16: below that the per-split set-up
  // and partials outweigh the added parallelism.
  plan_splits(a, 64, &pl.n, &pl.tps, -1, p.D == 128 ? 2048 : 1024, 4);
  return pl;
}


// Partial-result bytes (ml + acc) of a plan with n splits, after the counters.
int64_t partial_bytes(const fade_decode_args* a, int64_t n) {
  const WsLayout w = ws_layout(a, n);
  return w.total - w.ml;
}

// The kernels of a validated plan, with the split counters at `counters` and the
// partial results at `partials` (ml, then acc, as ws_layout places them after
// its counter region).
int run_plan(const fade_decode_args* a, Params& p, const Plan& pl, uint32_t* counters, char* partials,
             hipStream_t st) {
  if ((a->kernel == 2 || a->kernel == 3 || a->kernel == 4) && pl.k == Kern::kValu)
    return einval("fade_tiered_decode_attn: the matrix-core kernels do not handle this middle tier (format %d)",
                  p.mid.fmt);
  if (p.rot != nullptr && pl.k != Kern::kInt4)
    return einval("fade_tiered_decode_attn: a rotated middle tier needs the matrix-core INT4 kernel "
                  "(FADE_MID_SYM with 4- or 2-bit K and V, GQA <= 8)");
  if (a->mid.pages != nullptr && pl.k != Kern::kInt4)
    return einval("fade_tiered_decode_attn: paged middle tiers need the matrix-core INT4 "
                  "kernel (middle tier FADE_MID_SYM or FADE_MID_ASYM, GQA <= 8)");
  if (pl.n > 65535) return einval("fade_tiered_decode_attn: too many splits");
  const WsLayout ws = ws_layout(a, pl.n);
  p.n_splits = static_cast<int>(pl.n);
  p.tokens_per_split = pl.tps;
  p.ws_ml = reinterpret_cast<float*>(partials);
  p.ws_acc = reinterpret_cast<float*>(partials + (ws.acc - ws.ml));
  p.out = static_cast<uint16_t*>(a->out);
  p.o_sb = a->o_sb;
  p.o_sh = a->o_sh;
  p.counters = counters;
  if (pl.k == Kern::kInt4) {
    p.n_f16_tiles = pl.n_f16_tiles;
    p.tiles_per_split = pl.tiles_per_split;
    return launch_int4(p, st);
  }
  const int rc = pl.k == Kern::kMfma ? launch_mfma(p, st) : launch_valu(p, st);
  if (rc) return rc;
  if (pl.k == Kern::kValu && p.n_splits == 1) return 0;  // the portable kernel wrote the output
  const int64_t rows = a->B * a->Hq;
  hipLaunchKernelGGL(decode_combine_kernel, dim3(static_cast<unsigned>(rows)), dim3(static_cast<unsigned>(p.D)), 0, st, p.ws_ml,
                     p.ws_acc, p.n_splits, a->Hq, static_cast<uint16_t*>(a->out), a->o_sb, a->o_sh, p.bf16);
  return check_launch("fade_tiered_decode_attn(combine)");
}

// ---- the library's own decode scratch (fade_tiered_decode_attn_noalloc) ----
// One array per GPU the library runs on, held until the process ends:
// [split counters: kScratchCounterBytes][partial results].  The counters sit
// in a region of their own, so no call's partials ever land on them; every
// decode call leaves the counters it used at zero, and the region is zeroed
// once, by the first call on each device (stream-ordered before its kernels).

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch` on each device

__global__ void zero_words_kernel(uint32_t* p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Device address of this device's `scratch` (looked up once per device, with
// that device current); on the first call the counter region is zeroed on `st`.
int scratch_for(hipStream_t st, char** out) {
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) {
    (void)hipGetLastError();
    set_error("fade_tiered_decode_attn_noalloc: hipGetDevice failed");
    return FADE_ERUNTIME;
  }
  int dev = cur;
  if (st != nullptr) {
    hipDevice_t d = 0;
    if (hipStreamGetDevice(st, &d) != hipSuccess) {
      (void)hipGetLastError();
      set_error("fade_tiered_decode_attn_noalloc: hipStreamGetDevice failed");
      return FADE_ERUNTIME;
    }
    dev = static_cast<int>(d);
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("fade_tiered_decode_attn_noalloc: device %d beyond the %d the library tracks", dev, kMaxDevices);
    return FADE_ERUNTIME;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur && hipSetDevice(dev) != hipSuccess) {
      (void)hipGetLastError();
      set_error("fade_tiered_decode_attn_noalloc: hipSetDevice(%d) failed", dev);
      return FADE_ERUNTIME;
    }
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    int rc = FADE_OK;
    if (e != hipSuccess || ptr == nullptr) {
      set_error("fade_tiered_decode_attn_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      (void)hipGetLastError();
      rc = FADE_ERUNTIME;
    } else {
      const int64_t words = kScratchCounterBytes / 4;
      hipLaunchKernelGGL(zero_words_kernel, dim3(static_cast<unsigned>(cdiv(words, 256))), dim3(256), 0, st,
                         static_cast<uint32_t*>(ptr), words);
      rc = check_launch("fade_tiered_decode_attn_noalloc(zero counters)");
      if (rc == FADE_OK) g_scratch_ptr[dev] = ptr;
    }
    if (dev != cur) (void)hipSetDevice(cur);
    if (rc) return rc;
  }
  *out = static_cast<char*>(g_scratch_ptr[dev]);
  return FADE_OK;
}

}  // namespace

FADE_API int fade_tiered_decode_workspace_bytes(const fade_decode_args* a, int64_t* bytes) {
  int rc = validate(a);
  if (rc) return rc;
  if (bytes == nullptr) return einval("fade_tiered_decode_workspace_bytes: null output");
  const Params p = to_params(a);
  const Plan pl = make_plan(a, p);
  *bytes = ws_layout(a, pl.n).total;
  return FADE_OK;
}

FADE_API int fade_tiered_decode_attn(const fade_decode_args* a, void* stream) {
  int rc = validate(a);
  if (rc) return rc;
  Params p = to_params(a);
  const Plan pl = make_plan(a, p);
  const WsLayout ws = ws_layout(a, pl.n);
  if (a->workspace == nullptr || a->workspace_bytes < ws.total)
    return einval("fade_tiered_decode_attn: workspace too small (%lld < %lld bytes)",
                  (long long)a->workspace_bytes, (long long)ws.total);
  char* wsb = static_cast<char*>(a->workspace);
  return run_plan(a, p, pl, reinterpret_cast<uint32_t*>(wsb + ws.counters), wsb + ws.ml, as_stream(stream));
}

FADE_API int fade_tiered_decode_attn_noalloc(const fade_decode_args* a, void* stream) {
  int rc = validate(a);
  if (rc) return rc;
  Params p = to_params(a);
  const int64_t passes = (a->Hq / a->Hkv + 3) / 4;
  if (a->B * a->Hkv * passes * 4 > kScratchCounterBytes)
    return einval("fade_tiered_decode_attn_noalloc: B*Hkv*ceil(Hq/Hkv/4) = %lld split counters exceed the "
                  "library scratch's %lld",
                  (long long)(a->B * a->Hkv * passes), (long long)(kScratchCounterBytes / 4));
  // the planner's split count, halved until the partial results fit the scratch
  const int64_t cap = kScratchBytes - kScratchCounterBytes;
  fade_decode_args b = *a;
  Plan pl = make_plan(&b, p);
  while (partial_bytes(&b, pl.n) > cap && pl.n > 1) {
    b.n_splits = static_cast<int32_t>(pl.n / 2);
    const Plan smaller = make_plan(&b, p);
    if (smaller.n >= pl.n) break;  // e.g. a paged tier's minimum split count
    pl = smaller;
  }
  if (partial_bytes(&b, pl.n) > cap)
    return einval("fade_tiered_decode_attn_noalloc: %lld bytes of partial results exceed the library scratch's "
                  "%lld (%lld splits)",
                  (long long)partial_bytes(&b, pl.n), (long long)cap, (long long)pl.n);
  hipStream_t st = as_stream(stream);
  char* base = nullptr;
  rc = scratch_for(st, &base);
  if (rc) return rc;
  return run_plan(&b, p, pl, reinterpret_cast<uint32_t*>(base), base + kScratchCounterBytes, st);
}
