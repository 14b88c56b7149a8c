/*
 * fade_hip.h -- C ABI of libfade_hip.so, the MI355X (gfx950) kernels behind
 * the FADE tiered-KV hot path.
 *
 * Conventions
 *   - Every tensor argument is a device pointer.  Sizes and strides are
 *     int64 element counts; the last (head_dim) axis is always unit-stride.
 *   - "stream" is a hipStream_t (NULL = the legacy default stream).  All
 *     work is enqueued asynchronously on it; nothing allocates device
 *     memory.  Entry points that need scratch take a caller-provided
 *     workspace whose size the matching *_workspace_bytes() call returns.
 *   - Return value: FADE_OK (0) or a negative code; fade_hip_last_error()
 *     returns a message for the calling thread's last failure.
 *     FADE_EINVAL marks a bad argument (the Python layer raises ValueError,
 *     as the reference does for shape errors); FADE_ERUNTIME a HIP failure
 *     (RuntimeError).
 *   - fp16 tensors are IEEE binary16 (torch.float16); fp32 are IEEE binary32.
 *
 * Reference interfaces replaced (Omodaka9375/fade, pure Python + Triton)
 * are cited per entry point as file:line.  The reference has no FFI: the
 * binding a maintainer would add is the ctypes layer in fade_amd/_lib.py.
 */
#ifndef FADE_HIP_H
#define FADE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FADE_OK 0
#define FADE_ERUNTIME (-1)
#define FADE_EINVAL (-22)

#define FADE_ABI_VERSION 2  /* 2: fade_decode_args and fade_prefill_args end with dtype */

/* Quantization axes. */
#define FADE_AXIS_CHANNEL 0 /* one scale per (b, h, d): reduce over S (K)  */
#define FADE_AXIS_TOKEN 1   /* one scale per (b, h, s): reduce over D (V)  */

/* element type of the *_dtype quantizer entry points (input, scale, output) */
#define FADE_DTYPE_F16 0
#define FADE_DTYPE_BF16 1
#define FADE_DTYPE_F32 2

/* Middle-tier formats understood by the attention kernels. */
#define FADE_MID_NONE 0 /* no middle tier                                      */
#define FADE_MID_FP16 1 /* fp16 K/V (flash-decode comparator)                  */
#define FADE_MID_SYM 2  /* symmetric packed codes, K per-channel scale [B,H,1,D],
                           V per-token scale [B,H,S,1]; bits 4 (nibbles, high =
                           even index) or 2 (four per byte, first in bits 7:6).
                           fade/quant.py:61-92, fade/rotated_quant.py:106-173   */
#define FADE_MID_K4V2G 3 /* K as FADE_MID_SYM 4-bit; V literal grouped INT2:
                           int8 codes [B,H,S_pad,D], scale [B,H,S_pad/64,D]
                           (fade/cache.py:983-988, fade/quant.py:130-150)       */
#define FADE_MID_ASYM 4 /* per-token asymmetric groups along D (build format):
                           codes [B,H,S,D*bits/8], scale/zero [B,H,S,D/group]   */

int fade_hip_abi_version(void);
const char* fade_hip_last_error(void);

/* ---------------- bit packing (fade/quant.py:26-58, rotated_quant.py:35-69) */
/* q: int8 codes, n_rows x D contiguous; packed: n_rows x D*bits/8.  bits 4|2 */
int fade_pack_codes(const void* q_i8, int64_t n_rows, int64_t D, int32_t bits, void* packed_u8,
                    void* stream);
int fade_unpack_codes(const void* packed_u8, int64_t n_rows, int64_t D, int32_t bits, void* q_i8,
                      void* stream);

/* ---------------- symmetric INT4 on fp16 (fade/quant.py:61-92) ------------ */
/* K [B,H,S,D] fp16 with strides (sb, sh, ss) -> packed [B,H,S,D/2] u8 and
 * scale [B,H,1,D] fp16.  Two passes over S (column absmax, then codes). */
int fade_quant_k_int4_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D, int64_t* bytes);
int fade_quant_k_int4(const void* k_f16, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                      int64_t sh, int64_t ss, void* packed_u8, void* scale_f16, void* workspace,
                      int64_t workspace_bytes, void* stream);
/* fade_quant_k_int4's second pass alone (fade/quant.py:61-75), for K whose
 * column absmax another kernel already gathered (fade_reassign_gather's
 * mid_colmax): colmax fp32 [B*H][parts][D], each part a max of |K| over some
 * of the rows; the absmax of channel d is the max over the parts.  Codes and
 * scales equal fade_quant_k_int4's when the parts cover every row. */
int fade_quant_k_int4_from_colmax(const void* k_f16, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                                  int64_t sh, int64_t ss, const float* colmax, int64_t parts, void* packed_u8,
                                  void* scale_f16, void* stream);
/* V [B,H,S,D] fp16 -> packed [B,H,S,D/2] u8 and scale [B,H,S,1] fp16. */
int fade_quant_v_int4(const void* v_f16, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                      int64_t sh, int64_t ss, void* packed_u8, void* scale_f16, void* stream);

/* Dequantize symmetric packed codes: out = fp16(code * scale)
 * (fade/quant.py:124-127, rotated_quant.py:142-143).  axis selects the
 * scale layout ([B,H,1,D] for CHANNEL, [B,H,S,1] for TOKEN); bits 4|2. */
int fade_dequant_sym(const void* packed_u8, const void* scale_f16, int32_t bits, int32_t axis,
                     int64_t B, int64_t H, int64_t S, int64_t D, void* out_f16, void* stream);

/* fade_quant_k_int4 / fade_quant_v_int4 / fade_dequant_sym for any of the
 * dtypes the reference's quantizers take (fade/quant.py:61-92, 124-127;
 * tests/test_quant.py:110-141 run them on bfloat16 and float32): the scale
 * is emitted in the input's dtype, and each op rounds to that dtype as
 * torch's per-op arithmetic does (bf16: clamp(min=1e-8), reciprocal, *qmax,
 * x*inv each rounded to bf16; fp32: one IEEE rounding per op).  dtype is a
 * FADE_DTYPE_*; FADE_DTYPE_F16 gives the fp16 entry points' results. */
int fade_quant_k_int4_dtype(const void* k, int32_t dtype, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                            int64_t sh, int64_t ss, void* packed_u8, void* scale, void* workspace,
                            int64_t workspace_bytes, void* stream);
int fade_quant_v_int4_dtype(const void* v, int32_t dtype, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                            int64_t sh, int64_t ss, void* packed_u8, void* scale, void* stream);
/* out = dtype(code * scale), scale and out both of `dtype`. */
int fade_dequant_sym_dtype(const void* packed_u8, const void* scale, int32_t dtype, int32_t bits, int32_t axis,
                           int64_t B, int64_t H, int64_t S, int64_t D, void* out, void* stream);

/* ---------------- grouped INT2, reference literal (fade/quant.py:95-176) --- */
/* x [B,H,S,D] fp16 (rows >= S read as zero, i.e. pad_to_group fused) ->
 * codes int8 [B,H,S_pad,D], scale [B,H,S_pad/group,D] fp16. */
int fade_quant_int2_grouped(const void* x_f16, int64_t B, int64_t H, int64_t S, int64_t S_pad,
                            int64_t D, int64_t sb, int64_t sh, int64_t ss, int64_t group,
                            void* codes_i8, void* scale_f16, void* stream);
/* codes [B,H,S_pad,D] -> out [B,H,S_out,D] fp16 (rows beyond S_out trimmed). */
int fade_dequant_int2_grouped(const void* codes_i8, const void* scale_f16, int64_t B, int64_t H,
                              int64_t S_pad, int64_t D, int64_t group, int64_t S_out,
                              void* out_f16, void* stream);
/* The same two for a bfloat16 or float32 cache (fade/quant.py:95-176 on a
 * tensor of that dtype): each op rounds to the dtype, the scale and the
 * dequantized output are of it.  dtype is a FADE_DTYPE_*. */
int fade_quant_int2_grouped_dtype(const void* x, int32_t dtype, int64_t B, int64_t H, int64_t S, int64_t S_pad,
                                  int64_t D, int64_t sb, int64_t sh, int64_t ss, int64_t group, void* codes_i8,
                                  void* scale, void* stream);
int fade_dequant_int2_grouped_dtype(const void* codes_i8, const void* scale, int32_t dtype, int64_t B, int64_t H,
                                    int64_t S_pad, int64_t D, int64_t group, int64_t S_out, void* out,
                                    void* stream);

/* ---------------- rotated symmetric on fp32 (fade/rotated_quant.py:106-173) */
/* x_rot [B,H,S,D] fp32 contiguous (x.float() @ R.T) -> packed codes at
 * bits 4|2 (3 = raw int8) and fp16 scale ([B,H,1,D] or [B,H,S,1]). */
int fade_quant_rotated_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D, int32_t axis,
                                       int64_t* bytes);
int fade_quant_rotated(const float* x_rot, int64_t B, int64_t H, int64_t S, int64_t D,
                       int32_t bits, int32_t axis, void* packed, void* scale_f16, void* workspace,
                       int64_t workspace_bytes, void* stream);
/* fade_quant_rotated with the scale stored as scale_dtype (FADE_DTYPE_*): the
 * reference computes absmax / qmax in fp32 and casts it to the input's dtype
 * (fade/rotated_quant.py:129-131, 171-173), one rounding; for bfloat16 and
 * float32 K/V. */
int fade_quant_rotated_dtype(const float* x_rot, int64_t B, int64_t H, int64_t S, int64_t D, int32_t bits,
                             int32_t axis, void* packed, void* scale, int32_t scale_dtype, void* workspace,
                             int64_t workspace_bytes, void* stream);

/* Fused rotate + quantize (fade/rotated_quant.py:106-131 K, 148-173 V) for
 * fp16 x [B,H,S,128] (element strides sb/sh/ss, rows 16-byte aligned) and
 * R fp32 [128,128] row-major on the device: x_rot = x @ R^T on f16 matrix
 * cores with R split hi/lo (fp32-GEMM accuracy), then the same quantizer and
 * layouts as fade_quant_rotated.  Codes can differ from an fp32 GEMM's only
 * where x_rot * inv lies within GEMM rounding of a half-integer.
 * Workspace: axis CHANNEL only, size from the _workspace_bytes query. */
int fade_rotate_quant_workspace_bytes(int64_t B, int64_t H, int64_t S, int64_t D, int32_t axis,
                                      int64_t* bytes);
int fade_rotate_quant(const void* x_f16, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                      int64_t sh, int64_t ss, const float* R, int32_t bits, int32_t axis,
                      void* packed, void* scale_f16, void* workspace, int64_t workspace_bytes,
                      void* stream);

/* ---------------- asymmetric per-token groups (build format, no reference
 * counterpart: BASELINE's "asymmetric group-32 scale/zero") ------------- */
int fade_quant_asym(const void* x_f16, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sb,
                    int64_t sh, int64_t ss, int32_t bits, int32_t group, void* packed_u8,
                    void* scale_f16, void* zero_f16, void* stream);
int fade_dequant_asym(const void* packed_u8, const void* scale_f16, const void* zero_f16,
                      int32_t bits, int32_t group, int64_t B, int64_t H, int64_t S, int64_t D,
                      void* out_f16, void* stream);

/* ---------------- eviction re-RoPE (fade/cache.py:911-935, 283-311) ------- */
/* For each kept row j (keep_idx[j] ascending, int64):
 *   k_out[b,h,j] = fp16(apply(fp16(inverse(k[b,h,keep_idx[j]], cos_old[keep_idx[j]],
 *                  sin_old[keep_idx[j]])), cos_new[j], sin_new[j]))
 *   v_out[b,h,j] = v[b,h,keep_idx[j]]
 * cos/sin tables fp32 [S,D] (old) and [n_kept,D] (new).  v may be NULL. */
int fade_rerope_gather(const void* k_f16, int64_t ksb, int64_t ksh, int64_t kss, const void* v_f16,
                       int64_t vsb, int64_t vsh, int64_t vss, int64_t B, int64_t H, int64_t S,
                       int64_t D, const int64_t* keep_idx, int64_t n_kept, const float* cos_old,
                       const float* sin_old, const float* cos_new, const float* sin_new,
                       void* k_out_f16, void* v_out_f16, void* stream);
/* fade_rerope_gather for a bfloat16 or float32 cache: the same fp32 ops,
 * rounded to the cache dtype where the reference casts to k.dtype
 * (fade/cache.py:311, 935; no rounding for float32).  dtype is a FADE_DTYPE_*. */
int fade_rerope_gather_dtype(const void* k, int64_t ksb, int64_t ksh, int64_t kss, const void* v, int64_t vsb,
                             int64_t vsh, int64_t vss, int64_t B, int64_t H, int64_t S, int64_t D,
                             const int64_t* keep_idx, int64_t n_kept, const float* cos_old, const float* sin_old,
                             const float* cos_new, const float* sin_new, void* k_out, void* v_out, int32_t dtype,
                             void* stream);

/* ---------------- device-side tier reassignment --------------------------- */
/* fade/cache.py:881-1057 (apply_tier_assignment, shared tiers) for the
 * reference INT4 middle tier, without materializing the layer.
 *
 * fade_reassign_plan: tiers int64 [rows][S] (TIER_FP16 0 / INT4 1 / INT2 2 /
 * EVICT 3; row stride 0 and rows 1 for a shared assignment, fade/cache.py:881;
 * rows B for a per-row one, fade/cache.py:1059) in the cache's position
 * order, pos_old int64 [S] (row stride 0) or [rows][S].  Per row, writes dst int32 [S]
 * (-1 evicted, else cls << 28 | slot with cls 0 sink, 1 recent, 2 middle; the
 * first n_sink FP16 tokens are the sink), newpos int32 [S] (rank among kept
 * tokens), src_of int32 [S] (source index of each kept rank), the new positions of each tier (pos_sink / pos_recent / pos_mid,
 * capacity S each: old positions, or 0..n_kept-1 when tokens are evicted) and
 * counts int32 [4] = {n_fp16, n_int4, n_kept, status} (status bit 0: INT2
 * tokens present -- not handled here; bit 1: an unknown tier value); every
 * per-row output is [rows][S] ([rows][4] for counts). */
int fade_reassign_plan(const int64_t* tiers, int64_t tiers_row_stride, int64_t rows, int64_t S,
                       int64_t n_sink, const int64_t* pos_old, int64_t pos_old_row_stride, int32_t* dst,
                       int32_t* newpos, int32_t* src_of, int64_t* pos_sink, int64_t* pos_recent,
                       int64_t* pos_mid, int32_t* counts, void* stream);

/* fade_reassign_gather: moves every kept token of the current tiers (in
 * position order: sink rows, middle rows, recent rows) to its destination;
 * one pass over the kept tokens (src_of), at most counts[2] of them.
 * Middle rows are dequantized as fp16(fp16(code) * fp16(scale)); K rows are
 * un-RoPE'd at pos_old and re-RoPE'd at newpos (fp16 between, as the
 * reference) when counts[2] < S, using cos/sin tables fp32 [table_rows, D]
 * indexed by position.  Sink and middle outputs are contiguous
 * [B,H,cap,D]; the recent output has element strides.  Writes beyond a
 * capacity are skipped and set status bit 3 (bit 2: a position outside the
 * tables). */
typedef struct FadeReassignArgs {
  int64_t B, H, D, S;
  int64_t n_sink_old, n_mid_old; /* rows of the sink / middle tensors.  Without src_lens,
                                    token j of the position order is sink row j, middle row
                                    j - sink or recent row j - sink - middle; S may be below
                                    sink + middle (+ recent) rows, as in the reference's
                                    zero-padded per-sequence layout, whose positions are row
                                    0's (fade/cache.py:1161-1167) */
  const int32_t* src_lens;       /* optional device [B][3]: each row's current sink / middle /
                                    recent tokens (a ragged layout); row b's position order is
                                    its own sink | middle | recent, tokens past them absent */
  int64_t plan_rows;             /* 1: one shared plan; B: the plan of row b */
  int64_t pos_old_rs;            /* row stride of pos_old (0: shared) */
  int64_t n_rec_cap;             /* with src_lens: rows of the recent tensors */
  const void* sink_k;
  const void* sink_v;
  int64_t sink_sb, sink_sh, sink_ss; /* element strides shared by sink K and V */
  const void* mid_kq;                /* [B,H,mid,D/2] u8, high nibble = even channel */
  const void* mid_ks;                /* [B,H,1,D] fp16 */
  const void* mid_vq;                /* [B,H,mid,D/2] u8 */
  const void* mid_vs;                /* [B,H,mid,1] fp16 */
  const void* rec_k;
  const void* rec_v;
  int64_t rec_sb, rec_sh, rec_ss;
  const int32_t* dst;
  const int32_t* newpos;
  const int32_t* src_of;
  int64_t rows;    /* kept tokens if the caller knows the count, else 0 (grid covers S) */
  int32_t* counts; /* from fade_reassign_plan; status ORed into counts[3] */
  const int64_t* pos_old;
  const float* cos_tab;
  const float* sin_tab;
  int64_t table_rows;
  void* out_sink_k;
  void* out_sink_v;
  int64_t cap_sink;
  void* out_rec_k;
  void* out_rec_v;
  int64_t out_rec_sb, out_rec_sh, out_rec_ss, cap_rec;
  void* out_mid_k;
  void* out_mid_v;
  int64_t cap_mid;
  float* mid_colmax;     /* optional device fp32 [B*H][colmax_parts][D], zero-filled by the
                            caller: per-channel max of |K| over the middle rows written (as
                            their fp16 values), spread over the parts; with it
                            fade_quant_k_int4_from_colmax quantizes the middle in one pass */
  int64_t colmax_parts;  /* parts of mid_colmax (>= 1 when it is given) */
} FadeReassignArgs;
int fade_reassign_gather(const FadeReassignArgs* args, void* stream);

/* ---------------- tiered decode attention --------------------------------- */
/* fp16 tier (sink or recent): K/V [B,Hkv,len,D] with element strides. */
typedef struct fade_fp16_tier {
  const void* k;
  const void* v;
  int64_t len;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
} fade_fp16_tier;

/* Middle tier; all tensors contiguous in the layouts listed above. */
typedef struct fade_mid_tier {
  int32_t fmt;    /* FADE_MID_* */
  int32_t k_bits; /* 4 or 2 (SYM/ASYM) */
  int32_t v_bits; /* 4 or 2 (SYM/ASYM) */
  int32_t group;  /* ASYM group along D; K4V2G group along S (64) */
  int64_t len;    /* tokens */
  int64_t v_rows; /* K4V2G: padded row count of the V codes (>= len) */
  const void* k_codes;
  const void* k_scale;
  const void* k_zero;
  const void* v_codes;
  const void* v_scale;
  const void* v_zero;
  /* Optional paged layout (decode only; FADE_MID_SYM or FADE_MID_ASYM): pages
   * is device int32 [B][pages_per_row], the page of each 64-token middle tile
   * of a row.  Every per-token tensor (codes, SYM V scale, ASYM scale/zero) is
   * then a pool [n_pages][Hkv][64][...] shared by the rows; the SYM K scale
   * stays [B,Hkv,1,D].  len = the longest row's middle (per-row lengths come
   * from the decode args' lens). */
  const int32_t* pages;
  int64_t pages_per_row;
  /* Paged FADE_MID_SYM only: bytes between consecutive (page, kv head) blocks
   * of k_codes, v_codes and v_scale (which may then interleave in one pool,
   * e.g. [K codes | V codes | V scales] per block: one request stream per
   * tile); 0 = each tensor's own block size. */
  int64_t page_stride;
} fade_mid_tier;

typedef struct fade_decode_args {
  int64_t B, Hq, Hkv, D;       /* D a multiple of 8 in [8, 256] (the matrix-core kernels take
                                  128, the general one also 64 and 256 for FADE_MID_SYM 4-bit, FADE_MID_FP16
                                  and FADE_MID_NONE; other cases run the portable
                                  kernel, which reads every middle format and per-row lens, not
                                  pages or a rotation); Hq % Hkv == 0; Hq/Hkv <= 8 */
  const void* q;               /* [B,Hq,1,D] fp16 */
  int64_t q_sb, q_sh;
  void* out;                   /* [B,Hq,1,D] fp16 */
  int64_t o_sb, o_sh;
  float sm_scale;              /* usually 1/sqrt(D) */
  fade_fp16_tier sink;         /* tokens [0, sink.len) */
  fade_mid_tier mid;           /* next mid.len tokens */
  fade_fp16_tier recent;       /* last recent.len tokens */
  int32_t n_splits;            /* 0 = choose automatically */
  int32_t kernel;              /* 0 = auto, 1 = portable VALU kernel, 2 = matrix-core kernels
                                  only, 3 = the general matrix-core kernel (no INT4 fast path),
                                  4 = as 2, with Hq/Hkv = 5..8 on an unrotated FADE_MID_SYM tier
                                  served eight heads per pass whatever the size (0 and 2 take
                                  that instance where every resident workgroup gets at least 8
                                  tiles, two head passes below) */
  void* workspace;             /* zero-filled before its first use.  Its first
                                  round256(4*B*Hkv*P) bytes (P = 1 for Hq/Hkv <= 4, else 2)
                                  hold per-(row, kv head, head pass) split counters, which
                                  every call leaves at zero again; partial results follow
                                  them.  Later calls with the same B*Hkv*P can reuse it as it
                                  is, whatever their other sizes; before a call with another
                                  B*Hkv*P, zero its first round256(4*B*Hkv*P) bytes (an
                                  earlier call's partials may lie there). */
  int64_t workspace_bytes;
  const int32_t* lens;         /* optional device [B][3]: sink, middle, recent tokens of each
                                  row (ragged batch; each at most the tier's len, which is then
                                  the padded capacity of its tensors; every row >= 1 token).
                                  NULL: every row has the tiers' full lengths.  Ragged rows
                                  need the matrix-core INT4 kernel (SYM / ASYM formats; for
                                  Hq/Hkv = 5..8 it runs two head passes). */
  int32_t deterministic;       /* nonzero: bitwise-reproducible results.  The matrix-core INT4
                                  kernel's waves then walk their split's tiles in a fixed
                                  round-robin order instead of claiming them as they finish
                                  (the order of the fp32 sums then no longer depends on timing);
                                  the other kernels are deterministic either way. */
  const float* rotation;       /* optional device fp32 [128][128] R, row-major, of the rotated
                                  backend (fade/rotated_quant.py:41-45,134-187): the middle tier
                                  (FADE_MID_SYM, 4- or 2-bit) holds codes of K R^T and V R^T,
                                  while q, sink and recent are in the model's basis.  Middle
                                  tokens are scored with q R^T (computed in the kernel) and their
                                  values summed in the rotated basis; the result is the fp16
                                  tiers' part + (middle part) R.  Needs the matrix-core INT4
                                  kernel.  NULL: no rotation. */
  int32_t dtype;               /* FADE_DTYPE_F16 (0, zero-initialized arguments) or
                                  FADE_DTYPE_BF16: the type of q, out, the sink / recent K/V,
                                  an fp16-format middle tier and the FADE_MID_SYM /
                                  FADE_MID_K4V2G scales (the reference's cache keeps every
                                  tier and scale in the model's dtype).  FADE_MID_ASYM (fp16
                                  scale / zero by format) takes FADE_DTYPE_F16 only. */
} fade_decode_args;

/* Replaces dequantize + torch.cat (fade/cache.py:683-842) + SDPA and the
 * Triton fused_int4_sdpa decode path (fade/kernels/fused_int4_attn.py:277-342). */
int fade_tiered_decode_workspace_bytes(const fade_decode_args* args, int64_t* bytes);
int fade_tiered_decode_attn(const fade_decode_args* args, void* stream);

/* fade_tiered_decode_attn without a workspace: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments, kernels
 * and results as fade_tiered_decode_attn; args->workspace and workspace_bytes
 * are ignored.  The split counters and partial results live in the library's
 * own scratch: one 16 MiB array per GPU (256 KiB of counters, at most 65536
 * (row, kv head, head pass) slots, then partial results), held until the
 * process ends.  The split count is halved until the partial results fit;
 * FADE_EINVAL when even one split does not.  Nothing is allocated or freed.
 * Every call on a GPU shares that GPU's scratch: calls that overlap on one GPU
 * (other streams, other threads) race and must not be issued.  The first call
 * on a device zeroes the counter region on its stream; every call leaves the
 * counters at zero again. */
int fade_tiered_decode_attn_noalloc(const fade_decode_args* args, void* stream);

/* ---------------- ragged tiered prefill attention -------------------------- */
/* Masks of fade_tiered_prefill_attn (fade_prefill_args.mask_mode). */
#define FADE_MASK_BOTTOM_RIGHT 0 /* the cache fully visible, chunk causal: query j sees chunk keys 0..j */
#define FADE_MASK_TOP_LEFT 1     /* query j sees keys 0..j of the row's whole key sequence
                                    [sink | middle | recent | chunk], as the reference's fused
                                    kernel applies is_causal (fade/kernels/fused_int4_attn.py:165-169) */
#define FADE_MASK_NONE 2         /* every key visible to every query */
/* A chunk of Sq new tokens per batch row attends to that row's cache
 * [sink | middle | recent] followed by the chunk itself, bottom-right causal:
 * query j of row b sees cache tokens and chunk tokens 0..j (mask_mode
 * FADE_MASK_BOTTOM_RIGHT, chunk.len = Sq).  The two other masks take any chunk
 * length, 0 included (queries without keys of their own, as the reference's
 * fused_int4_sdpa over one packed tensor, fade/kernels/fused_int4_attn.py:277-342);
 * every row must then see at least one key.  Tier tensors are
 * padded along S (row b uses the first lens[3b+0..2] tokens of sink / middle /
 * recent); the middle tier is FADE_MID_SYM 4-bit (padded, or paged: mid.pages,
 * separate pools, pages_per_row * 64 >= mid.len; D % 32 == 0), FADE_MID_FP16
 * or FADE_MID_NONE.  D a multiple of 8 in [8, 256], Hq/Hkv <= 8.  `order` (optional, device int32 [B]) lists batch rows in the
 * order their workgroups are dispatched (longest first balances the tail).
 * Replaces the reference's prefill path: update() returning the materialized
 * tiers (fade/cache.py:347-379,683-842) followed by causal SDPA in the model. */
typedef struct fade_prefill_args {
  int64_t B, Hq, Hkv, D, Sq;
  const void* q;  /* [B,Hq,Sq,D] fp16 */
  int64_t q_sb, q_sh, q_ss;
  void* out;      /* [B,Hq,Sq,D] fp16 */
  int64_t o_sb, o_sh, o_ss;
  float sm_scale;
  const int32_t* lens;  /* device [B][3]: sink, middle, recent tokens of each row */
  const int32_t* order; /* device [B] or NULL */
  fade_fp16_tier sink;  /* len = padded capacity */
  fade_mid_tier mid;    /* len = padded capacity (rows of the code tensors) */
  fade_fp16_tier recent;
  fade_fp16_tier chunk; /* the chunk's own K/V, len = Sq (other masks: any length) */
  int32_t mask_mode;    /* FADE_MASK_*; 0 (zero-initialized arguments) = bottom-right */
  int32_t dtype;        /* FADE_DTYPE_F16 (0) or FADE_DTYPE_BF16: q, out, the fp16-layout tiers
                           (sink, recent, chunk, an fp16-format middle) and the packed middle
                           tier's scales; middle codes dequantize to dtype(code * scale) */
} fade_prefill_args;

int fade_tiered_prefill_attn(const fade_prefill_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FADE_HIP_H */
