// Device-side tier reassignment (fade/cache.py:881-1057, shared tiers, the
// reference INT4 middle format).
//
// The reference materializes the whole layer in position order (dequantized
// middle included), reads the number of kept tokens back to the host, un-RoPEs
// every row, index_selects the kept rows, re-RoPEs them, then splits the
// survivors with three more nonzero() calls (each a host sync) and
// requantizes the middle tier.  Here:
//
//   plan    one workgroup per row of tiers scans it (two passes over per-thread runs and
//           one block scan) and writes, per source token j, its destination
//           (sink / recent / middle slot) and its rank among the kept
//           tokens, the new position arrays and the tier counts;
//   gather  one thread per (kept token, channel pair i, i + D/2) reads the source
//           row in place -- sink or recent fp16, or a middle row dequantized
//           in registers as fp16(fp16(code) * fp16(scale)) -- un-RoPEs /
//           re-RoPEs K with the reference's rounding when tokens were
//           evicted (three separately rounded fp32 ops per rotation, fp16 in
//           between; -ffp-contract=off) and stores K and V straight into the
//           new tiers (the middle into an fp16 staging tensor that the
//           quantizers then encode).
//
// Destination writes are bounded by the capacities the host allocated; a
// slot beyond them is skipped and flagged in counts[3] (never an
// out-of-range store).
#include "fade_common.h"

namespace fade {
namespace {

constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int64_t kTierFp16 = 0, kTierInt4 = 1, kTierInt2 = 2, kTierEvict = 3;
constexpr int kClsShift = 28;
constexpr int32_t kSlotMask = (1 << kClsShift) - 1;

// Exclusive scan of a 64-bit value over the block (lane shuffles + LDS).
__device__ __forceinline__ uint64_t block_exclusive_scan(uint64_t v, uint64_t* wtot, uint64_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t u = __shfl_up(inc, o, 64);
    if (lane >= o) inc += u;
  }
  if (lane == 63) wtot[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    uint64_t w = lane < kPlanWaves ? wtot[lane] : 0;
    uint64_t winc = w;
#pragma unroll
    for (int o = 1; o < kPlanWaves; o <<= 1) {
      const uint64_t u = __shfl_up(winc, o, 64);
      if (lane >= o) winc += u;
    }
    if (lane < kPlanWaves) wtot[lane] = winc - w;  // exclusive wave offsets
    if (lane == kPlanWaves - 1) *total = winc;
  }
  __syncthreads();
  return wtot[wave] + inc - v;
}

// counts = {n_fp16, n_int4, n_kept, status}; status bit 0: an INT2 token,
// bit 1: a value outside {FP16, INT4, INT2, EVICT}.
__global__ __launch_bounds__(kPlanThreads) void plan_kernel(const int64_t* __restrict__ tiers, int64_t tiers_rs,
                                                            int64_t S, int64_t n_sink,
                                                            const int64_t* __restrict__ pos_old, int64_t pos_old_rs,
                                                            int32_t* __restrict__ dst, int32_t* __restrict__ newpos,
                                                            int32_t* __restrict__ src_of,
                                                            int64_t* __restrict__ pos_sink,
                                                            int64_t* __restrict__ pos_recent,
                                                            int64_t* __restrict__ pos_mid, int32_t* __restrict__ counts) {
  __shared__ uint64_t wtot[kPlanWaves];
  __shared__ uint64_t total_s;
  __shared__ int status_s;
  // one workgroup per plan row (batch row of a per-row assignment)
  const int64_t row = blockIdx.x;
  tiers += row * tiers_rs;
  dst += row * S;
  newpos += row * S;
  src_of += row * S;
  pos_sink += row * S;
  pos_recent += row * S;
  pos_mid += row * S;
  counts += 4 * row;
  if (threadIdx.x == 0) status_s = 0;
  const int64_t per = (S + kPlanThreads - 1) / kPlanThreads;
  const int64_t j0 = static_cast<int64_t>(threadIdx.x) * per;
  const int64_t j1 = j0 + per < S ? j0 + per : S;
  uint32_t nf = 0, ni = 0;
  int bad = 0;
  for (int64_t j = j0; j < j1; ++j) {
    const int64_t v = tiers[j];
    if (v == kTierFp16) ++nf;
    else if (v == kTierInt4) ++ni;
    else if (v == kTierInt2) bad |= 1;
    else if (v != kTierEvict) bad |= 2;
  }
  __syncthreads();  // status_s initialised
  if (bad) atomicOr(&status_s, bad);
  const uint64_t ex = block_exclusive_scan(static_cast<uint64_t>(nf) | (static_cast<uint64_t>(ni) << 32), wtot, &total_s);
  const uint64_t tot = total_s;
  const int64_t n_fp16 = static_cast<int64_t>(tot & 0xFFFFFFFFu), n_int4 = static_cast<int64_t>(tot >> 32);
  const int64_t n_kept = n_fp16 + n_int4;
  const bool evicted = n_kept < S;
  int64_t f = static_cast<int64_t>(ex & 0xFFFFFFFFu), m = static_cast<int64_t>(ex >> 32);
  for (int64_t j = j0; j < j1; ++j) {
    const int64_t v = tiers[j];
    int32_t d = -1, np = -1;
    if (v == kTierFp16 || v == kTierInt4) {
      np = static_cast<int32_t>(f + m);
      src_of[f + m] = static_cast<int32_t>(j);
      const int64_t p = evicted ? f + m : pos_old[pos_old_rs * row + j];
      if (v == kTierFp16) {
        if (f < n_sink) {
          d = static_cast<int32_t>(f);
          pos_sink[f] = p;
        } else {
          d = (1 << kClsShift) | static_cast<int32_t>(f - n_sink);
          pos_recent[f - n_sink] = p;
        }
        ++f;
      } else {
        d = (2 << kClsShift) | static_cast<int32_t>(m);
        pos_mid[m] = p;
        ++m;
      }
    }
    dst[j] = d;
    newpos[j] = np;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    counts[0] = static_cast<int32_t>(n_fp16);
    counts[1] = static_cast<int32_t>(n_int4);
    counts[2] = static_cast<int32_t>(n_kept);
    counts[3] = status_s;
  }
}

__device__ __forceinline__ float nib(uint32_t byte, bool high) {
  const int c = high ? static_cast<int>(byte >> 4) : static_cast<int>(byte & 0xF);
  return static_cast<float>(c - ((c & 8) << 1));
}

// One thread per (kept token, channel pair i, i + D/2) of one (b, h); the
// grid covers `rows` kept ranks (the host's count, or S when it has none).
// With mid_colmax, the workgroup's middle rows also leave their per-channel
// max |K| (after the RoPE rewrite, as fp16 values), reduced in LDS and
// folded into part blockIdx.x % colmax_parts by an atomic max on the float's
// bits (order-preserving for values >= 0).
__global__ __launch_bounds__(256) void gather_kernel(FadeReassignArgs a) {
  const int D = static_cast<int>(a.D), half = D / 2;
  const int rows_per_block = blockDim.x / half;
  const int i = threadIdx.x % half;
  const int64_t rank = static_cast<int64_t>(blockIdx.x) * rows_per_block + threadIdx.x / half;
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / a.H, h = bh % a.H;
  // the plan of this batch row (a shared assignment has one)
  const int64_t pr = a.plan_rows > 1 ? b : 0;
  const int32_t* counts = a.counts + 4 * pr;
  int32_t* status = a.counts + 4 * pr + 3;
  const int32_t* dst = a.dst + pr * a.S;
  const int32_t* newpos = a.newpos + pr * a.S;
  float cm0 = 0.0f, cm1 = 0.0f;  // |K| of channels i and i + half if this thread wrote a middle row
  do {  // `break` = this thread writes nothing (every thread still reaches the column-max reduction)
    if (rank >= counts[2] || rank >= a.S) break;
    const int64_t j = a.src_of[pr * a.S + rank];
    if (j < 0 || j >= a.S) break;
    const int32_t d = dst[j];
    if (d < 0) break;
    const int cls = d >> kClsShift;
    const int64_t slot = d & kSlotMask;
    // this row's partition of the position order into sink | middle | recent,
    // and its token count (tokens were evicted from it iff it keeps fewer)
    int64_t nso = a.n_sink_old, nmo = a.n_mid_old, Sb = a.S;
    if (a.src_lens != nullptr) {
      nso = a.src_lens[3 * b];
      nmo = a.src_lens[3 * b + 1];
      const int64_t nro = a.src_lens[3 * b + 2];
      Sb = nso + nmo + nro;
      if (nso < 0 || nso > a.n_sink_old || nmo < 0 || nmo > a.n_mid_old || nro < 0 || nro > a.n_rec_cap || j >= Sb) {
        atomicOr(status, 16);  // a kept token the row does not have
        break;
      }
    }
    // source pair
    float k0, k1;
    uint16_t v0, v1;
    if (j < nso || j >= nso + nmo) {
      const bool sink = j < nso;
      const int64_t r = sink ? j : j - nso - nmo;
      const uint16_t* kb = static_cast<const uint16_t*>(sink ? a.sink_k : a.rec_k);
      const uint16_t* vb = static_cast<const uint16_t*>(sink ? a.sink_v : a.rec_v);
      const int64_t off = sink ? b * a.sink_sb + h * a.sink_sh + r * a.sink_ss : b * a.rec_sb + h * a.rec_sh + r * a.rec_ss;
      k0 = h2f(kb[off + i]);
      k1 = h2f(kb[off + i + half]);
      v0 = vb[off + i];
      v1 = vb[off + i + half];
    } else {
      // reference INT4: K per-channel scale [B,H,1,D], V per-token scale [B,H,mid,1]
      const int64_t r = j - nso;
      const uint8_t* kq = static_cast<const uint8_t*>(a.mid_kq) + (bh * a.n_mid_old + r) * half;
      const uint8_t* vq = static_cast<const uint8_t*>(a.mid_vq) + (bh * a.n_mid_old + r) * half;
      const uint16_t* ks = static_cast<const uint16_t*>(a.mid_ks) + bh * D;
      const float vs = h2f(static_cast<const uint16_t*>(a.mid_vs)[bh * a.n_mid_old + r]);
      const bool hi0 = (i & 1) == 0, hi1 = ((i + half) & 1) == 0;  // even channel: high nibble
      k0 = round_f16(nib(kq[i >> 1], hi0) * h2f(ks[i]));
      k1 = round_f16(nib(kq[(i + half) >> 1], hi1) * h2f(ks[i + half]));
      v0 = f2h(nib(vq[i >> 1], hi0) * vs);
      v1 = f2h(nib(vq[(i + half) >> 1], hi1) * vs);
    }
    uint16_t ko0, ko1;
    if (counts[2] < Sb) {
      // un-RoPE at the old position (k*cos - rotate_half(k)*sin), fp16, then
      // RoPE at the new one (k*cos + rotate_half(k)*sin), fp16
      const int64_t po = a.pos_old[a.pos_old_rs * b + j], pn = newpos[j];
      if (po < 0 || po >= a.table_rows || pn < 0 || pn >= a.table_rows) {
        atomicOr(status, 4);
        break;
      }
      const float* co = a.cos_tab + po * D;
      const float* so = a.sin_tab + po * D;
      const float u0 = round_f16(k0 * co[i] - (-k1) * so[i]);
      const float u1 = round_f16(k1 * co[i + half] - k0 * so[i + half]);
      const float* cn = a.cos_tab + pn * D;
      const float* sn = a.sin_tab + pn * D;
      ko0 = f2h(u0 * cn[i] + (-u1) * sn[i]);
      ko1 = f2h(u1 * cn[i + half] + u0 * sn[i + half]);
    } else {
      ko0 = f2h(k0);
      ko1 = f2h(k1);
    }
    uint16_t *kd, *vd;
    int64_t off;
    if (cls == 0) {
      if (slot >= a.cap_sink) { atomicOr(status, 8); break; }
      kd = static_cast<uint16_t*>(a.out_sink_k);
      vd = static_cast<uint16_t*>(a.out_sink_v);
      off = (bh * a.cap_sink + slot) * D;
    } else if (cls == 1) {
      if (slot >= a.cap_rec) { atomicOr(status, 8); break; }
      kd = static_cast<uint16_t*>(a.out_rec_k);
      vd = static_cast<uint16_t*>(a.out_rec_v);
      off = b * a.out_rec_sb + h * a.out_rec_sh + slot * a.out_rec_ss;
    } else {
      if (slot >= a.cap_mid) { atomicOr(status, 8); break; }
      kd = static_cast<uint16_t*>(a.out_mid_k);
      vd = static_cast<uint16_t*>(a.out_mid_v);
      off = (bh * a.cap_mid + slot) * D;
    }
    kd[off + i] = ko0;
    kd[off + i + half] = ko1;
    vd[off + i] = v0;
    vd[off + i + half] = v1;
    if (cls == 2) {
      cm0 = fabsf(h2f(ko0));
      cm1 = fabsf(h2f(ko1));
    }
  } while (false);
  if (a.mid_colmax == nullptr) return;
  __shared__ float red[2][256];
  red[0][threadIdx.x] = cm0;
  red[1][threadIdx.x] = cm1;
  __syncthreads();
  if (static_cast<int>(threadIdx.x) < half) {
    float m0 = 0.0f, m1 = 0.0f;
    for (int t = i; t < static_cast<int>(blockDim.x); t += half) {
      m0 = fmaxf(m0, red[0][t]);
      m1 = fmaxf(m1, red[1][t]);
    }
    unsigned int* cp = reinterpret_cast<unsigned int*>(a.mid_colmax + (bh * a.colmax_parts + blockIdx.x % a.colmax_parts) * D);
    if (m0 > 0.0f || m0 != m0) atomicMax(cp + i, __float_as_uint(m0));
    if (m1 > 0.0f || m1 != m1) atomicMax(cp + i + half, __float_as_uint(m1));
  }
}

}  // namespace
}  // namespace fade

using namespace fade;

FADE_API int fade_reassign_plan(const int64_t* tiers, int64_t tiers_row_stride, int64_t rows, int64_t S,
                                int64_t n_sink, const int64_t* pos_old, int64_t pos_old_row_stride, int32_t* dst,
                                int32_t* newpos,
                                int32_t* src_of, int64_t* pos_sink, int64_t* pos_recent, int64_t* pos_mid,
                                int32_t* counts, void* stream) {
  const char* fn = "fade_reassign_plan";
  if (S < 0 || n_sink < 0) return einval("%s: negative S or n_sink", fn);
  if (rows < 1 || rows > 65535) return einval("%s: rows=%lld out of range", fn, (long long)rows);
  if (S >= (1LL << 30)) return einval("%s: S=%lld too large", fn, (long long)S);
  if (counts == nullptr) return einval("%s: null counts", fn);
  if (S > 0 && (tiers == nullptr || pos_old == nullptr || dst == nullptr || newpos == nullptr || src_of == nullptr ||
                pos_sink == nullptr || pos_recent == nullptr || pos_mid == nullptr))
    return einval("%s: null pointer", fn);
  hipLaunchKernelGGL(plan_kernel, dim3(static_cast<unsigned>(rows)), dim3(kPlanThreads), 0, as_stream(stream), tiers,
                     tiers_row_stride, S, n_sink, pos_old, pos_old_row_stride, dst, newpos, src_of, pos_sink, pos_recent,
                     pos_mid, counts);
  return check_launch(fn);
}

FADE_API int fade_reassign_gather(const FadeReassignArgs* args, void* stream) {
  const char* fn = "fade_reassign_gather";
  if (args == nullptr) return einval("%s: null argument", fn);
  const FadeReassignArgs& a = *args;
  if (a.D <= 0 || a.D % 2 != 0 || a.D > 512) return einval("%s: head_dim must be even and <= 512", fn);
  if (a.B < 0 || a.H < 0 || a.S < 0 || a.n_sink_old < 0 || a.n_mid_old < 0 || a.n_rec_cap < 0)
    return einval("%s: inconsistent tier lengths", fn);
  if (a.dst == nullptr || a.newpos == nullptr || a.src_of == nullptr || a.counts == nullptr || a.pos_old == nullptr)
    return einval("%s: null plan pointer", fn);
  if (a.n_mid_old > 0 && (a.mid_kq == nullptr || a.mid_ks == nullptr || a.mid_vq == nullptr || a.mid_vs == nullptr))
    return einval("%s: null middle tier", fn);
  // without src_lens, token j >= sink + middle rows is recent row j - sink - middle: none
  // when S is at most sink + middle (a zero-padded layout whose positions are row 0's)
  const int64_t rec_tail = a.S - a.n_sink_old - a.n_mid_old;
  const int64_t rec_rows = a.src_lens != nullptr ? a.n_rec_cap : (rec_tail > 0 ? rec_tail : 0);
  if ((a.n_sink_old > 0 && (a.sink_k == nullptr || a.sink_v == nullptr)) ||
      (rec_rows > 0 && (a.rec_k == nullptr || a.rec_v == nullptr)))
    return einval("%s: null fp16 tier", fn);
  if ((a.cap_sink > 0 && (a.out_sink_k == nullptr || a.out_sink_v == nullptr)) ||
      (a.cap_rec > 0 && (a.out_rec_k == nullptr || a.out_rec_v == nullptr)) ||
      (a.cap_mid > 0 && (a.out_mid_k == nullptr || a.out_mid_v == nullptr)))
    return einval("%s: null output", fn);
  if (a.table_rows > 0 && (a.cos_tab == nullptr || a.sin_tab == nullptr)) return einval("%s: null RoPE table", fn);
  if (a.mid_colmax != nullptr && (a.colmax_parts < 1 || a.colmax_parts > 65535))
    return einval("%s: colmax_parts must be 1..65535 with mid_colmax", fn);
  const int64_t BH = a.B * a.H;
  if (BH == 0 || a.S == 0) return FADE_OK;
  if (BH > 65535) return einval("%s: B*H=%lld exceeds 65535", fn, (long long)BH);
  if (a.plan_rows != 1 && a.plan_rows != a.B) return einval("%s: plan_rows must be 1 or B", fn);
  const int half = static_cast<int>(a.D / 2);
  const int rpb = half >= 256 ? 1 : 256 / half;
  const int64_t rows = a.rows > 0 && a.rows < a.S ? a.rows : a.S;
  const dim3 grid(static_cast<unsigned>(cdiv(rows, rpb)), static_cast<unsigned>(BH));
  hipLaunchKernelGGL(gather_kernel, grid, dim3(rpb * half), 0, as_stream(stream), a);
  return check_launch(fn);
}
