/*
 * kvq.h -- C ABI (version 6) of the MI355X (gfx950) quantized-KV decode path.
 *
 * libkvq.so exports three groups of entry points: quantize-on-append, split-K
 * decode attention and error reporting.  Every entry point
 *   - takes plain device pointers, sizes and strides (no framework types);
 *   - never allocates, never synchronises, and enqueues its work on the
 *     hipStream_t it is given;
 *   - returns KVQ_OK or a KVQ_ERR_* code.  kvq_last_error() then returns a
 *     message for the calling thread.
 *
 * The reference (zilangchen/LLM_KVCache_Quantization) has no C/C++ layer.  Its
 * path is PyTorch + Triton.  Each entry point below names the reference Python
 * interface it replaces.  The Python mirror in
 * llm_kvcache_quantization_amd/ keeps those interfaces' names, arguments and
 * exceptions, and calls this ABI through ctypes.
 */
#ifndef KVQ_H_
#define KVQ_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* kvq_stream_t; /* == hipStream_t */

/* status codes */
#define KVQ_OK 0
#define KVQ_ERR_INVALID 1     /* bad argument: shape, stride, size or null pointer */
#define KVQ_ERR_UNSUPPORTED 2 /* valid request outside what this build implements */
#define KVQ_ERR_LAUNCH 3      /* HIP reported an error when the kernel was enqueued */

/* element dtypes for scales */
#define KVQ_DTYPE_F16 0
#define KVQ_DTYPE_F32 1

/* KV cache formats (one per K and one per V) */
#define KVQ_FMT_INT8_SYM 1  /* int8 codes [..., D]; fp16/fp32 scale per (token, group) */
#define KVQ_FMT_INT4_SYM 2  /* packed nibbles [..., D/2], byte = ((c[2i]+8)<<4)|(c[2i+1]+8),
                               codes in [-7,7]; fp16/fp32 scale per (token, group) */
#define KVQ_FMT_INT4_ASYM 3 /* packed nibbles as above, codes in [-8,7]; static fp16 scale
                               and zero-point per (kv head, group of 32); optional fp16
                               side-band holding n_outlier channels per K head verbatim */

#define KVQ_FMT_INT4_KIVI 4  /* packed nibbles as INT4_SYM, codes in [-8,7], value c * s + z
                               with fp32 s, z (src/quant/asymmetric_quant.py:24-196,
                               src/cache/kivi_style_cache.py): K per (b, h, channel)
                               [B,H,D] (scale_stride_b/_h/_g, channels contiguous) or, ABI 6,
                               per (b, h, token) [B,H,T] like V (scale_stride_t 1,
                               scale_stride_g 0: the reference's MixedKVCache K at 4 bits,
                               src/cache/mixed_kv_cache.py:159-162); V per (b, h, token)
                               [B,H,T] (scale_stride_b/_h/_t, tokens contiguous); zero_point
                               has the scale's strides */
#define KVQ_FMT_INT8_KIVI 5  /* int8 codes [..., D] in [-128,127], value c * s + z, the
                                parameters as INT4_KIVI (the reference's quant_bits=8 KIVI
                                cache); append: range floor 255 * 2^-14, s = range / 255,
                                z = min + 128 s */
#define KVQ_FMT_FP16 6       /* fp16 values [..., D] as stored (a 16-bit side of the
                                reference's mixed / allocator caches); an append copies the
                                row (codes = the fp16 rows, byte strides, no scales) */

/* code layouts (kvq_kv_view.layout, kvq_append_params.codes_layout) */
#define KVQ_LAYOUT_ROWS 0   /* token-major: the code bytes of token t start at t * stride_t */
#define KVQ_LAYOUT_TILE32 1 /* INT4_ASYM V only (with INT4_ASYM K, or INT8_SYM K with a
                               static group-32 scale): 32-token tiles of 2048 bytes, tile i at
                               i * 32 * stride_t (stride_t must be 64).  Within a tile, byte
                               ((L * 8 + 2 p + k) * 4 + 2 a + j) holds packed byte 4 c + 2 k + j
                               of token T(g, p, a), where L = 16 g + c (g < 4, c < 16),
                               T(g, p, a) = 16 (p / 2) + 4 g + 2 (p % 2) + a (p < 4, a, k, j < 2):
                               the 32 bytes of L are one lane's PV operand on gfx950 */

/* A read-only view of one layer's quantized K or V cache. */
typedef struct kvq_kv_view {
  const void* codes;     /* code byte of (b=0, h=0, t=0, d=0) */
  int64_t stride_b;      /* bytes */
  int64_t stride_h;      /* bytes */
  int64_t stride_t;      /* bytes; the D (or D/2) code bytes of a token are contiguous */
  const void* scale;     /* INT8_SYM/INT4_SYM: [B,H,T,G] (any strides, 0 allowed);
                            INT4_ASYM: [H,G] (only stride_h / stride_g are read);
                            INT4_KIVI (fp32): K [B,H,D] (stride_b / _h / _g = 1, 16-byte
                            aligned rows), V [B,H,T] (stride_b / _h / _t = 1) */
  int64_t scale_stride_b, scale_stride_h, scale_stride_t, scale_stride_g; /* elements */
  int32_t scale_dtype;   /* KVQ_DTYPE_F16 or KVQ_DTYPE_F32 (F32 is rounded to fp16 in-kernel);
                            K and V per-token scales must have the same dtype */
  int32_t n_outlier;     /* INT4_ASYM K only: 0 or 4 */
  const void* zero_point;         /* INT4_ASYM: fp16 [H,G]; INT4_KIVI: fp32; same strides
                                     as scale */
  const int32_t* outlier_idx;     /* [H, n_outlier] channel indices, distinct, in [0, D) */
  const void* outlier_val;        /* fp16 [B,H,T,n_outlier] */
  int64_t outlier_stride_b, outlier_stride_h, outlier_stride_t; /* elements */
  int32_t layout;                 /* KVQ_LAYOUT_ROWS or KVQ_LAYOUT_TILE32 */
  int32_t reserved;               /* 0 */
} kvq_kv_view;

/* Decode attention (q_len == 1), split-K with an in-kernel GQA head group.
 *
 * Replaces:
 *   decode_attn_int8(q, k_cache, v_cache, k_scale, v_scale, context_lens, sm_scale)
 *     src/kernels/triton_decode_attn_int8.py:306-519   (formats INT8_SYM / INT8_SYM)
 *   decode_attn_int4(q, k_cache_int4, v_cache_int4, k_scale, v_scale, context_lens, ...)
 *     src/kernels/triton_decode_attn_int4.py:62-121    (formats INT4_SYM / INT4_SYM,
 *     read packed in place instead of unpacking the whole cache to int8)
 *   and the per-head inv_tau query scaling of src/engine/patch_model.py:711-746.
 * The INT4_ASYM formats (and INT8_SYM K with INT4_ASYM V) have no reference kernel;
 * they follow the asymmetric formula of src/quant/asymmetric_quant.py:24-196 with
 * static group parameters.
 *
 * out[b, h, :] = softmax_t(sm_scale * q'[b,h] . khat[b, h/n_rep, t]) @ vhat[b, h/n_rep, t]
 * for t < context_lens[b] (clamped to [0, capacity]); rows with an empty context are 0.
 * q' = fp16(q * inv_tau[h]) when inv_tau is given.  Requires head_dim == 128 and
 * q_heads / kv_heads <= 16.  INT4_ASYM requires group_size == 32; the scale formats
 * require group_size in {8, 16, 32, 64, 128}.
 *
 * Kernel choice (the same results either way, within the stated tolerance): the tiled
 * kernel (8-wave work-groups, single-launch merge of the split partials) serves
 *  - INT4_ASYM K with TILE32 V;
 *  - INT8_SYM K whose scale view is static (stride 0, or size 1, over b and t; 128-byte dense
 *    rows) with TILE32 INT4_ASYM V (group 32) or a static INT8_SYM V in dense rows (any
 *    group size);
 *  - per-token INT8_SYM / INT4_SYM scales on both sides in dense rows (groups of 16 or more),
 *    INT8_SYM K with per-token scales and INT4_KIVI or FP16 V;
 *  - the KIVI family (INT4_KIVI, INT8_KIVI, FP16 on either side), per-token INT4_KIVI K with
 *    INT4_KIVI, INT8_SYM or FP16 V, and FP16 K with INT8_SYM V.
 * Every other combination runs the row-layout split-K kernel and a combine launch.
 */
typedef struct kvq_decode_params {
  const void* q;          /* fp16 [B, Hq, D], d contiguous */
  int64_t q_stride_b, q_stride_h;     /* elements */
  const void* inv_tau;    /* fp16 [Hq] or NULL */
  int32_t k_format, v_format;
  kvq_kv_view k, v;
  const int32_t* context_lens;        /* device int32 [B], or NULL: every row has context_len */
  int32_t batch, q_heads, kv_heads, head_dim, group_size;
  int64_t capacity;       /* token dimension of the cache views */
  float sm_scale;
  int32_t chunk_tokens;   /* split size in tokens (work-groups per (b, kv head) =
                             ceil(capacity / chunk_tokens)); 0 = choose automatically */
  void* workspace;        /* device scratch of kvq_decode_workspace_bytes() bytes, zero-filled
                             before its first use: its first B * kv_heads * 128 bytes hold
                             work-group arrival counters that every call leaves zero, so one
                             workspace serves any later call with the same batch * kv_heads
                             that fits in it; calls sharing a workspace must be ordered on
                             one stream */
  int64_t workspace_bytes;
  void* out;              /* fp16 [B, Hq, D], d contiguous */
  int64_t out_stride_b, out_stride_h; /* elements */
  int32_t context_len;    /* context of every row when context_lens is NULL (ABI 4) */
  int32_t v_group_size;   /* ABI 6: the group size of INT8_SYM / INT4_SYM V when it differs from
                             group_size (the reference's MixedKVCache v_group_size); 0 = the
                             same as group_size.  Tiled per-token kernels only */
  /* fp16 residual window (ABI 5; src/cache/kivi_style_cache.py:102-113, 354-404): the
     res_tokens most recent tokens of every row kept unquantized, fp16 [B, kv_heads, >=
     res_tokens, D] with dense 256-byte token rows, attended together with the row's
     quantized context (any order within the window).  0 = none.  KIVI-family formats
     (INT4_KIVI, INT8_KIVI, FP16) on the tiled kernel with at most 64 work-groups per
     (b, kv head); at most 65536 tokens (the merging work-group attends the window with VALU
     dot products, so a long window lengthens the launch). */
  const void* res_k;
  const void* res_v;
  int64_t res_stride_b, res_stride_h;   /* elements */
  int32_t res_tokens;
  int32_t pad1;           /* 0 */
} kvq_decode_params;

int kvq_decode_attn(const kvq_decode_params* p, kvq_stream_t stream);

/* kvq_decode_attn without a caller workspace, for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops and harnesses that forbid
 * hipMalloc).  No counterpart in the reference, whose Triton wrapper allocates per call.
 *
 * p->workspace / p->workspace_bytes are ignored: the split-K partials and merge counters
 * live in a fixed 16 MiB device array (KVQ_NOALLOC_SCRATCH_BYTES) that libkvq.so holds on
 * every GPU it runs on until the process ends.  Calls whose kvq_decode_workspace_bytes(p)
 * exceeds it return KVQ_ERR_UNSUPPORTED.  The call enqueues one small fill kernel that
 * clears the merge counters, then the kernels of kvq_decode_attn, with bit-identical
 * results.  It calls no hipMalloc / hipFree.  Every call on one GPU shares that GPU's
 * array: calls that may overlap on one GPU (different streams without ordering) race. */
#define KVQ_NOALLOC_SCRATCH_BYTES (16LL << 20)
int kvq_decode_attn_noalloc(const kvq_decode_params* p, kvq_stream_t stream);

/* split size kvq_decode_attn will use for p (p->chunk_tokens if nonzero) */
int32_t kvq_decode_chunk_tokens(const kvq_decode_params* p);
/* bytes of workspace kvq_decode_attn needs for p */
int64_t kvq_decode_workspace_bytes(const kvq_decode_params* p);

/* Quantize-on-append of new K and V rows into a cache layer.
 *
 * Replaces the quantize + pack + slice-write part of:
 *   INT8KVCache.append   src/cache/int8_cache.py:350-488
 *     (quantize_symmetric_int8_with_scale src/quant/int8_basic.py:111-164,
 *      quantize_symmetric_int8 (percentile 100) int8_basic.py:18-108)
 *   INT4KVCache.append   src/cache/int4_cache.py:392-589
 *     (quantize_symmetric_int4_with_scale src/quant/int4_basic.py:115-159,
 *      _apply_outlier_rescue int4_cache.py:360-390, pack_int4 int4_basic.py:230-272)
 *   the static-parameter asymmetric INT4 K quantizer of
 *     src/kernels/triton_quantize_pack_int4.py:18-62 (INT4_ASYM; per group instead of
 *     per channel, plus the fp16 outlier-channel side-band, which has no reference).
 * Codes are bit-exact with those torch formulas: IEEE fp32 division, round half to
 * even; INT8 rounds the quotient to fp16 before rounding to an integer.
 */
typedef struct kvq_append_params {
  int32_t format;         /* KVQ_FMT_* */
  const void* x;          /* fp16 [B, H, S_new, D], d contiguous */
  int64_t x_stride_b, x_stride_h, x_stride_s;   /* elements */
  int32_t batch, heads, seq_new, head_dim, group_size;
  /* static parameters per (head, group); NULL static_scale = dynamic (absmax) scales */
  const void* static_scale;
  int32_t static_scale_dtype;                   /* KVQ_DTYPE_* */
  int64_t static_stride_h, static_stride_g;     /* elements */
  const void* static_zp;                        /* INT4_ASYM: fp16, same strides */
  /* scale policy (INT8_SYM and INT4_SYM with a static scale) */
  int32_t adaptive;        /* scale = max(static * margin, dynamic) */
  float adaptive_margin;
  int32_t mixed_rescue;    /* INT4_SYM: scale = max(scale, dynamic) */
  float rescue_quantile;   /* INT4_SYM: 0 = off; else fp32(1 - outlier_rescue_ratio) */
  int32_t rescue_all;      /* INT4_SYM: ratio >= 1: scale = max(scale, dynamic) everywhere */
  /* destination */
  void* codes;             /* code byte of (b=0, h=0, t=0) */
  int64_t codes_stride_b, codes_stride_h, codes_stride_t;   /* bytes */
  void* scale_out;         /* per-token scale [B,H,T,G] or NULL */
  int32_t scale_out_dtype;
  int64_t so_stride_b, so_stride_h, so_stride_t, so_stride_g; /* elements */
  int32_t n_outlier;       /* INT4_ASYM: 0 or 4 */
  const int32_t* outlier_idx;     /* [H, n_outlier] */
  void* outlier_out;              /* fp16 [B,H,T,n_outlier] */
  int64_t oo_stride_b, oo_stride_h, oo_stride_t;            /* elements */
  int64_t write_pos;       /* first token slot written */
  int64_t capacity;        /* token slots in the destination */
  int32_t* status;         /* device int32[2] or NULL: [0] |= 1 if x had NaN/Inf,
                              [1] += number of clipped elements */
  int32_t codes_layout;    /* KVQ_LAYOUT_ROWS, or KVQ_LAYOUT_TILE32 for INT4_ASYM
                              (codes_stride_t must then be 64 and capacity a multiple of 32) */
  int32_t reserved;        /* 0 */
  void* scratch;           /* device scratch of kvq_append_scratch_bytes() bytes (16-byte
                              aligned; no initial contents needed) when that is nonzero, else
                              NULL.  Needed by the INT4_SYM group rescue over more than 4096
                              (row, group) scales; calls sharing it must be ordered */
  int64_t scratch_bytes;
  /* INT4_KIVI (src/cache/kivi_style_cache.py:407-605): K with static_scale / static_zp fp32
     [B,H,D] (static_stride_b / _h, static_stride_g = the channel stride) quantized as
     clamp(rint((x - z_d) / s_d), -8, 7); V with static_scale NULL: per-token parameters
     from the token's min / max over its 128 channels, s = max(max - min, 15 * 2^-14) / 15,
     z = min + 8 s, written as fp32 to scale_out (so_stride_b/_h/_t) and zp_out (same strides) */
  int64_t static_stride_b;  /* elements */
  void* zp_out;
  /* INT8_SYM / INT4_SYM without a static scale (ABI 4): 0 = the group's absmax; else
     fp32(percentile / 100) in (0, 1): the group's torch.quantile of |x| at that level
     (linear interpolation in fp32, src/quant/int8_basic.py:78-83, int4_basic.py:84-90) */
  float dyn_quantile;
  /* KIVI V (ABI 5): 0 = the token's min / max; with dyn_quantile = fp32(p / 100) > 0 this is
     fp32((100 - p) / 100): the range is torch.quantile at these two levels over the token's
     128 channels (src/quant/asymmetric_quant.py:97-103).  0 for every other use. */
  float dyn_quantile_lo;
} kvq_append_params;

/* Appends K and V of one layer with one launch (either pointer may be NULL).  The INT4_SYM
 * group rescue takes torch.quantile's threshold over the dynamic group scales of the whole
 * call (src/cache/int4_cache.py:384-390): up to 4096 (row, group) scales inside the launch,
 * beyond that by an exact radix select over p->scratch (a few short launches first). */
int kvq_quant_append(const kvq_append_params* k, const kvq_append_params* v,
                     kvq_stream_t stream);
/* bytes of scratch kvq_quant_append needs for p (0: none) */
int64_t kvq_append_scratch_bytes(const kvq_append_params* p);

/* Decode step of one layer in one launch: quantize-on-append of one new token per
 * (b, kv head) followed by the decode attention of p over the cache that now holds it.
 *
 * Replaces the append + attention pair of the reference's decode step,
 *   cache.append(layer, k, v)            src/engine/patch_model.py:755
 *   decode_attn_*(q, caches..., ctx)     src/engine/patch_model.py:837-957
 * with the codes and the output bit-identical to kvq_quant_append then kvq_decode_attn,
 * except that for the per-token, KIVI and mixed row formats (the writer runs the row
 * quantizer) a writer holding at least kShed + 3 tiles of the split (1 + 3 tiles, with the
 * INT4 group rescue 3 + 3) hands its first kShed tiles to waves of other SIMDs: the codes
 * stay bit-identical and the output then agrees within the attention's stated tolerance.
 * Supported for the formats the tiled kernel serves (see kvq_decode_attn), with k_new /
 * v_new of seq_new 1 sharing write_pos and naming the very code buffers and strides p
 * reads:
 *  - INT4_ASYM K with TILE32 V, static INT8 K with TILE32 INT4_ASYM V or static INT8 V
 *    rows: a static scale table and no scale policy (adaptive, rescue, scale_out); an
 *    INT4_ASYM side must name p's static tables and outlier side-band, an INT8_SYM side
 *    quantizes with its own table (fp16 or fp32), as kvq_quant_append would;
 *  - the row formats (per-token INT8_SYM / INT4_SYM scales in dense rows with groups of 16
 *    or more, INT4_KIVI / INT8_KIVI, FP16 sides): any policy kvq_quant_append takes; the
 *    INT4_SYM group rescue with a threshold (rescue_quantile > 0 without rescue_all), which
 *    spans every row of the append, only with at most 32 rows (batch * heads) and its lower
 *    rank within 32 of the top of the (row, group) scales; scale_out / zp_out and KIVI K's
 *    static parameters must be the buffers p reads.  The decode kernel's writer wave runs
 *    the append kernel's row arithmetic (and finds the rescue threshold itself).
 * Anything else returns KVQ_ERR_UNSUPPORTED (or KVQ_ERR_INVALID), and the caller makes the
 * two calls instead.  The status words are updated as kvq_quant_append does. */
int kvq_append_decode_attn(const kvq_decode_params* p, const kvq_append_params* k_new,
                           const kvq_append_params* v_new, kvq_stream_t stream);

/* Measurement aid, with no counterpart in the reference: reads `bytes` (a multiple of 16)
 * of device memory at buf (16-byte aligned) once, with the non-temporal 16-byte loads the
 * decode kernels use for cache codes, over `work_groups` work-groups of 512 threads, and
 * writes nothing to sink (work_groups words) in practice.  Timing it over the bytes of a
 * decode launch gives the read ceiling that launch is measured against. */
int kvq_stream_read(const void* buf, int64_t bytes, uint32_t* sink, int32_t work_groups,
                    kvq_stream_t stream);

/* message for the last non-OK return on this thread ("" if none) */
const char* kvq_last_error(void);
/* ABI version (increments on incompatible changes to the structs above); this is 6 */
int32_t kvq_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* KVQ_H_ */
