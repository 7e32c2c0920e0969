/*
 * starkv.h — C ABI of the MI355X (gfx950) STAR-KV decode- and
 * prefill-attention library (libstarkv.so, built from star-kv_amd/csrc/).
 *
 * Every entry point takes plain pointers and sizes, returns an int status
 * (0 = OK, negative = argument validation error, positive = HIP error code)
 * and never throws.  Device pointers are HIP device addresses; "host" arrays
 * are read during the call only.  Work is enqueued asynchronously on the
 * given hipStream_t (pass torch.cuda.current_stream().cuda_stream).  No entry
 * point allocates device memory: scratch comes from a caller-owned workspace
 * sized by the matching *_workspace_bytes query.  Calls are re-entrant (no
 * mutable global state); two calls that share one workspace must be ordered
 * on one stream.
 */
#ifndef STARKV_H_
#define STARKV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Bumped on every change of a struct layout or of an entry point's meaning;
 * the Python binding refuses a library of another version. */
#define STARKV_ABI_VERSION 5

/* element types */
enum {
  STARKV_F16 = 1,
  STARKV_BF16 = 2,
  STARKV_F32 = 3,
  STARKV_I8 = 4,
  STARKV_U8 = 5
};

/* status codes */
enum {
  STARKV_OK = 0,
  STARKV_ERR_NULL = -1,       /* a required pointer is NULL */
  STARKV_ERR_SHAPE = -2,      /* inconsistent or unsupported sizes */
  STARKV_ERR_DTYPE = -3,      /* unsupported element type */
  STARKV_ERR_ALIGN = -4,      /* pointer / stride alignment */
  STARKV_ERR_RANK = -5,       /* latent rank outside 1..128 (K) or 1..8192 (V) */
  STARKV_ERR_WORKSPACE = -6,  /* workspace NULL or smaller than required */
  STARKV_ERR_LIMIT = -7,      /* exceeds a compiled limit (heads, items, positions) */
  STARKV_ERR_FORMAT = -8      /* unknown quantisation format */
};

/* quantised latent formats */
enum {
  STARKV_FMT_DENSE = 0,      /* fp16 / bf16 latent, reference layout */
  STARKV_FMT_INT4_REF = 1,   /* reference nibbles: rank j in byte j>>1 (lo = even),
                                value (nib-8)*s, one fp16 scale per token
                                (bx_quant.py:75-86) */
  STARKV_FMT_INT8_SYM = 2,   /* int8 q*s, one fp16 scale per token (per (b,h,s) for K) */
  STARKV_FMT_INT4_G64 = 3    /* int4 asymmetric, groups of 64 ranks, fp16 scale+zero
                                per (b,s,group), x = n*s + z rounded once to fp16 */
};

int starkv_abi_version(void);
const char* starkv_status_string(int status);

/* ---------------------------------------------------------------------
 * RoPE tables.  Replaces the per-program cos/sin recomputation of
 * get_freq_multi_tokens (abx_rope_batched.py:40-48) and the theta=10000
 * constant of the Triton launch (abx_rope_batched.py:184).  inv_freq is the
 * host array of D/2 = 64 inverse frequencies as HF computes them
 * (default or llama3); attention_scaling multiplies cos and sin
 * (HF:models/llama/modeling_llama.py:125-126).
 * ------------------------------------------------------------------- */
size_t starkv_rope_table_bytes(int max_positions);
int starkv_rope_build(const float* inv_freq_host, float attention_scaling, int max_positions,
                      void* table, size_t table_bytes, void* stream);

/* ---------------------------------------------------------------------
 * starkv_rope_apply — replaces the query rotation of the reference attention
 * forward, _rope(query_states, cos, sin) (model.py:423, HF apply_rotary_pos_emb,
 * HF:models/llama/modeling_llama.py:130-153): in place, for i < 64,
 *   x[i]      <- x[i] c - x[i + 64] s,   x[i + 64] <- x[i + 64] c + x[i] s
 * with (c, s) the table's (attention-scaled) cos / sin of frequency i at
 * position pos0 + t.  x: act dtype [B, H, T, 128], element (b,h,t,d) at
 * x + b*stride_b + h*stride_h + t*stride_t + d.  pos0_device (optional): a
 * device int read at run time instead of pos0 (graph replay); rows whose
 * position then falls outside [0, rope_max_positions) are left unrotated and,
 * when error_flag (optional device int) is given, the kernel stores 1 there
 * (the library never clears it; the caller zeroes it and checks it after
 * synchronising).  Computed in fp32 and rounded once (the reference rounds
 * each of its three operations).  batch * n_heads * n_tokens * 64 must stay
 * below 2^32 - 256 (STARKV_ERR_LIMIT).
 * ------------------------------------------------------------------- */
typedef struct {
  int batch, n_heads, n_tokens, dtype;
  void* x; int64_t stride_b, stride_h, stride_t;
  const void* rope_table; int rope_max_positions;
  int pos0;
  const int* pos0_device;
  int* error_flag;
} starkv_rope_apply_desc;

int starkv_rope_apply(const starkv_rope_apply_desc* d, void* stream);

/* ---------------------------------------------------------------------
 * K-latent description shared by the K-logit and decode entry points.
 * KV head h has rank r_h = rank[h] (1..128); element (b, h, s, j) of the
 * latent lives at  base + b*stride_b + head_offset[h] + s*pos_stride[h] + j.
 * The reference cache [B, Hkv, S, r] (LlamaLoRaAttention_headwise.py:88-102)
 * is head_offset[h] = h*stride(1), pos_stride[h] = stride(2).
 * B_k (k_u^T, model.py:455) row j of head h lives at
 * bk + bk_head_offset[h] + j*bk_row_stride, 128 contiguous elements.
 *
 * Any rank 1..128 and any row layout in every format.  Dense rows that the
 * streaming K-logit kernels cannot read (a rank that is not a multiple of 8,
 * or rows not 16-byte aligned) are copied by starkv_k_logits into its
 * workspace first; quantised rows of any byte alignment are read as aligned
 * words joined in registers.
 * Quantised K (offsets and strides of data/data2 in bytes; every value
 * dequantised to fp16 before use, as the reference's
 * dequantise-then-multiply path does, LlamaLoRaAttention_headwise_quant.py:
 * 137-144):
 *   INT8_SYM  all ranks int8 in data, x = q * s, fp16 scale per (b,h,s) at
 *             scale + b*scale_stride_b + h*scale_stride_h + s.  Fastest
 *             layout (LatentCache's): 16-byte aligned data, rows and
 *             offsets; 16-byte aligned scale, scale strides multiples of 8
 *             and scale_stride_h >= round_up(seq_len, 8) -- each scale row
 *             is then read in 8-position pieces through round_up(seq_len, 8)
 *             (values past seq_len are ignored);
 *   INT4_REF  split == 0: all ranks int4 nibbles in data (rank 2k low nibble
 *             of byte k, x = (nibble - 8) * s), scale as above;
 *             split > 0 (multiple of 16): ranks [0, split) in data (int8 when
 *             split_format is STARKV_FMT_INT8_SYM, else int4 nibbles) with
 *             scale, ranks [split, rank[h]) as int4 nibbles in data2 at
 *             data2 + b*stride2_b + head_offset2[h] + s*pos_stride2[h] + byte
 *             with fp16 scales scale2 (b,h,s) at scale2 + b*scale2_stride_b +
 *             h*scale2_stride_h + s -- the split cache of
 *             LlamaLoRaAttention_headwise_quant.py:107-127 (upper 16 ranks).
 * ------------------------------------------------------------------- */
typedef struct {
  int n_kv_heads;
  const int* rank;                 /* host [Hkv] */
  const int64_t* head_offset;      /* host [Hkv], elements (bytes when quantised) */
  const int64_t* pos_stride;       /* host [Hkv], elements (bytes when quantised) */
  int64_t stride_b;                /* elements (bytes when quantised) */
  int format;                      /* STARKV_FMT_DENSE, STARKV_FMT_INT8_SYM or STARKV_FMT_INT4_REF */
  const void* data;                /* device */
  const void* scale;               /* quantised: fp16 scales of data */
  int64_t scale_stride_b, scale_stride_h;
  const void* bk;                  /* device, act dtype */
  const int64_t* bk_head_offset;   /* host [Hkv], elements */
  int64_t bk_row_stride;           /* elements */
  int split, split_format;         /* INT4_REF two-block cache (see above) */
  const void* data2;
  const int64_t* head_offset2;     /* host [Hkv], bytes */
  const int64_t* pos_stride2;      /* host [Hkv], bytes */
  int64_t stride2_b;               /* bytes */
  const void* scale2;
  int64_t scale2_stride_b, scale2_stride_h;
} starkv_klatent;

/* ---------------------------------------------------------------------
 * starkv_k_logits — replaces abx(a, b, x, dtype) (abx_rope_batched.py:135-186)
 * and the Triton _abx_fwd kernel (55-132):
 *   out[b, q, s] = scale * q_rot[b,q] . RoPE_s(X_k[b, q//gs, s] @ B_k[q//gs])  (+ mask)
 * q: [B, Hq, 128] act dtype (already rotated), element (b,q,d) at
 * q + b*q_stride_b + q*q_stride_h + d.  out: out_dtype (act dtype or F32),
 * element (b,q,s) at out + b*out_stride_b + q*out_stride_h + s.
 * Position s uses the angle of position s (the Triton kernel's semantics).
 * Workspace: starkv_k_logits_workspace_bytes is 0 when the K rows can be
 * streamed in place (dense: ranks multiples of 8 on 16-byte aligned rows;
 * int8 or the split format: always), else the size of a padded copy of the
 * dense K latent ([B][Hkv][S] rows of round_up(r, 8) elements, 16-byte pitch)
 * that the call writes before the logits.
 * ------------------------------------------------------------------- */
typedef struct {
  int batch, n_q_heads, head_dim, seq_len;
  int dtype;                        /* act dtype of q, X_k (dense), B_k */
  const void* q; int64_t q_stride_b, q_stride_h;
  starkv_klatent k;
  const void* rope_table; int rope_max_positions;
  float scale;
  const void* mask; int mask_dtype; int64_t mask_stride_b, mask_stride_h;   /* optional */
  void* out; int out_dtype; int64_t out_stride_b, out_stride_h;
} starkv_klogits_desc;

size_t starkv_k_logits_workspace_bytes(const starkv_klogits_desc* d);
int starkv_k_logits(const starkv_klogits_desc* d, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------
 * V-latent description.  Dense: element (b, s, j) at
 * data + b*stride_b + s*stride_s + j (reference cache [B, S, Rv],
 * LlamaLoRaAttention_headwise.py:96-102).  Quantised formats (any rank and
 * any byte alignment of rows -- the reference bx default, rank 1228 over a
 * 256-rank upper block, leaves 486-byte lower rows -- with the two-block
 * INT4_REF split a multiple of 8; strides of data/data2 in bytes, of scales
 * in fp16 elements; every value dequantised to fp16 exactly as the reference
 * kernel does, then rounded to bf16 for bf16 activations):
 *   INT4_REF (bx_quant.py:117-166 x1/x2): with 0 < split < rank, ranks
 *     [0, split) in data ((b,s,byte) at data + b*stride_b + s*stride_s +
 *     byte) with the fp16 per-token scale (b,s) at scale + b*scale_stride_b +
 *     s*scale_stride_s, ranks [split, rank) as int4 in data2/scale2 likewise;
 *     split_format says whether the upper block holds int4 nibbles
 *     (STARKV_FMT_INT4_REF, split/2 bytes per token) or int8
 *     (STARKV_FMT_INT8_SYM, split bytes per token).  Otherwise all ranks are
 *     int4 nibbles in data.
 *   INT8_SYM: all ranks int8 in data, per-token scale.
 *   INT4_G64: nibbles n (rank 2k low nibble of byte k) in data; fp16 scale
 *     and zero of (b, s, group g = rank/64) at scale / zero + b*scale_stride_b
 *     + s*scale_stride_s + g; x = n*s + z.  Row pitches (stride_s, and
 *     scale_stride_s in bytes) below 16 MB, else STARKV_ERR_LIMIT.
 * ------------------------------------------------------------------- */
typedef struct {
  int rank;
  int format;
  const void* data; int64_t stride_b, stride_s;
  const void* scale; int64_t scale_stride_b, scale_stride_s;
  int split; int split_format;
  const void* data2; int64_t stride2_b, stride2_s;
  const void* scale2; int64_t scale2_stride_b, scale2_stride_s;
  const void* zero;   /* INT4_G64 zero points */
  int capacity;       /* reserved (0) */
} starkv_vlatent;

/* ---------------------------------------------------------------------
 * starkv_pv_latent — replaces bx(b, x1, x2, scale_v_upper, scale_v_lower,
 * original_rank, upper_rank) (bx_quant.py:117-166) and the reference decode
 * line prob_v = P @ X_v (model.py:484):  out[b, h, j] = sum_s P[b,h,s] V[b,s,j].
 * p: act dtype, element (b,h,s) at p + b*p_stride_b + h*p_stride_h + s.
 * out: act dtype, element (b,h,j) at out + b*out_stride_b + h*out_stride_h + j.
 * Deterministic (fixed-order split-S reduction; no float atomics, unlike
 * bx_quant.py:113-114).
 * ------------------------------------------------------------------- */
typedef struct {
  int batch, n_heads, seq_len;
  int dtype;
  const void* p; int64_t p_stride_b, p_stride_h;
  starkv_vlatent v;
  void* out; int64_t out_stride_b, out_stride_h;
} starkv_pv_desc;

size_t starkv_pv_latent_workspace_bytes(const starkv_pv_desc* d);
int starkv_pv_latent(const starkv_pv_desc* d, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------
 * starkv_decode_attention — the fused decode step that replaces the
 * reference decode branch model.py:450-487 (abx -> /sqrt(D) -> +mask ->
 * softmax(fp32) -> P @ X_v -> per-head up-projection), i.e. the scope of the
 * reference's "attention us/layer" (latency.py:262-268):
 *   out[b, q, :] = U_v[q//gs] @ sum_s softmax_s(logit[b,q,s]) X_v[b, s, :]
 * uv: v_proj.U.weight [Hkv*128, Rv] act dtype, row i at uv + i*uv_row_stride.
 * out: [B, Hq, 128], element (b,q,d) at out + b*out_stride_b + q*out_stride_h
 * + d, of type out_dtype (0 = the act dtype, or STARKV_F32).
 * ------------------------------------------------------------------- */
typedef struct {
  int batch, n_q_heads, head_dim, seq_len;
  int dtype;
  const void* q; int64_t q_stride_b, q_stride_h;
  starkv_klatent k;
  starkv_vlatent v;
  const void* uv; int64_t uv_row_stride;
  const void* rope_table; int rope_max_positions;
  float scale;
  const void* mask; int mask_dtype; int64_t mask_stride_b, mask_stride_h;   /* optional */
  void* out; int out_dtype; int64_t out_stride_b, out_stride_h;
  /* optional: a device int; positions after *last_pos_device take the logit
   * -1e30, as an additive mask of -1e30 would give them (a context length
   * kept on the device, for steps replayed from one captured graph; no
   * counterpart in the reference, whose eager decode passes the length) */
  const int* last_pos_device;
} starkv_decode_desc;

size_t starkv_decode_workspace_bytes(const starkv_decode_desc* d);
int starkv_decode_attention(const starkv_decode_desc* d, void* workspace, size_t workspace_bytes, void* stream);

/* Same as starkv_decode_attention, and records events[0..3] (hipEvent_t) on
 * the stream before the K-logit kernel, after it, after the P.V kernel and
 * after the up-projection, so a caller can time each kernel on the stream it
 * runs on (the reference times with triton.testing.do_bench,
 * latency.py:221-223). */
int starkv_decode_attention_timed(const starkv_decode_desc* d, void* workspace, size_t workspace_bytes,
                                  void* stream, void* const* events);

/* ---------------------------------------------------------------------
 * starkv_decode_attention_noalloc — no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): the same decode as
 * starkv_decode_attention with the same descriptor and results, but its
 * workspace is a device array of STARKV_NOALLOC_SCRATCH_BYTES inside the
 * library, which each GPU the library runs on holds until the process ends.
 * Descriptors whose starkv_decode_workspace_bytes exceeds that size return
 * STARKV_ERR_LIMIT (B16 S32768 with the Llama-2-7B shape needs 123 MiB).
 * Runs on the current device (the stream must belong to it); calls that
 * overlap on one GPU share the array and race -- order them on one stream.
 * ------------------------------------------------------------------- */
#define STARKV_NOALLOC_SCRATCH_BYTES (128u << 20)
int starkv_decode_attention_noalloc(const starkv_decode_desc* d, void* stream);

/* ---------------------------------------------------------------------
 * Latent-cache writers.  Quantise (or copy) n_tokens new latent rows into a
 * preallocated cache at positions [pos0, pos0 + n_tokens), in place.
 * Replaces the per-step torch.cat of HF DynamicLayer.update
 * (HF:cache_utils.py:127-146, via model.py:411-419) and the quantise-on-write
 * of LlamaLoRaAttention_headwise_quant.py:107-127 (quantize_r_split_int8_
 * int4_packed, absent from the reference): int8 blocks s = fp16(amax/127),
 * q = clip(rint(x/s), -127, 127); int4 blocks s = fp16(amax/7),
 * n = clip(rint(x/s), -8, 7) stored as nibble n+8; group-64 asymmetric
 * z = fp16(min), s = fp16((max-z)/15), n = clip(rint((x-z)/s), 0, 15); a zero
 * scale becomes 1; divisions correctly rounded, rint half to even.
 * The cache is the same description the attention entry points read (for K
 * the B_k fields are ignored); capacity is the number of positions it holds.
 * src: act dtype; K row (b, h, t) of rank[h] elements at src +
 * b*src_stride_b + h*src_stride_h + t*src_stride_t, V row (b, t) of rank
 * elements at src + b*src_stride_b + t*src_stride_t.
 * ------------------------------------------------------------------- */
typedef struct {
  int batch, n_tokens, pos0, capacity;
  int dtype;
  const void* src; int64_t src_stride_b, src_stride_h, src_stride_t;
  starkv_klatent k;
  const int64_t* src_head_offset;   /* optional host [Hkv] (NULL: h*src_stride_h): element offset
                                       of head h's row, for sources with the heads back to back
                                       ([B, T, sum of ranks], as the latent projection writes them) */
  const int* pos0_device;   /* optional (NULL: use pos0): device int read by the kernel at
                               run time, for calls captured once in a HIP graph and replayed
                               at advancing positions; rows landing outside [0, capacity) are
                               then skipped by the kernel instead of rejected by the host */
  int* error_flag;          /* optional device int: the kernel stores 1 there when it skips a
                               row (never cleared by the library) */
} starkv_k_append_desc;

typedef struct {
  int batch, n_tokens, pos0, capacity;
  int dtype;
  const void* src; int64_t src_stride_b, src_stride_t;
  starkv_vlatent v;
  const int* pos0_device;   /* as in starkv_k_append_desc */
  int* error_flag;          /* as in starkv_k_append_desc */
} starkv_v_append_desc;

int starkv_k_append(const starkv_k_append_desc* d, void* stream);
int starkv_v_append(const starkv_v_append_desc* d, void* stream);

/* starkv_decode_append: starkv_k_append(k), starkv_v_append(v) and, when q
 * is not NULL, starkv_rope_apply(q) in one launch -- the three small writes
 * before a decode step's attention (the reference's DynamicLayer.update,
 * HF:cache_utils.py:127-146, and the query half of model.py:423), with the
 * same results, validation and status codes as the three calls; all three
 * descriptors must carry one dtype (STARKV_ERR_DTYPE).  For launch-bound
 * decode loops: one kernel instead of three. */
int starkv_decode_append(const starkv_k_append_desc* k, const starkv_v_append_desc* v,
                         const starkv_rope_apply_desc* q, void* stream);

/* ---------------------------------------------------------------------
 * starkv_prefill_attention — replaces the reference prefill branch
 * model.py:429-449 (materialise key_full = RoPE(X_k @ B_k) and
 * value_full = X_v @ U_v^T, repeat over GQA groups, then SDPA), with the
 * causal mask the reference leaves to the caller's attention_mask (without
 * one its SDPA call attends to future tokens):
 *   out[b, q, t, :] = sum_{s <= pos0 + t} softmax_s(scale * q_rot[b,q,t] . K[b,q//gs,s]) V[b,q//gs,s]
 *   K[b,h,s] = RoPE_s(X_k[b,h,s] @ B_k[h]),  V[b,h,s] = U_v[h] @ X_v[b,s]
 * over the pos0 + n_tokens cached positions (the n_tokens new queries sit at
 * positions pos0 .. pos0 + n_tokens - 1; the latents of every position up to
 * the last one must already be in the caches, e.g. by starkv_k_append /
 * starkv_v_append).  q: rotated queries, act dtype, element (b,q,t,d) at
 * q + b*q_stride_b + q*q_stride_h + t*q_stride_t + d (16-byte aligned, strides
 * multiples of 8).  out likewise with out_stride_*, act dtype.
 * K latent: STARKV_FMT_DENSE, STARKV_FMT_INT8_SYM or STARKV_FMT_INT4_REF (the
 * reference module's split cache, either upper-block format); V latent:
 * STARKV_FMT_DENSE, STARKV_FMT_INT4_G64, STARKV_FMT_INT8_SYM or
 * STARKV_FMT_INT4_REF (with or without its upper block); any rank and row
 * layout: latents (and a U_v) that the reconstruction kernels cannot read in
 * place -- ranks or pitches that are not multiples of 8, rows not aligned --
 * are first repacked into aligned rows of a multiple of 8 ranks in the
 * workspace (zero past the rank; nibble 8 for int4).  Quantised latents are
 * dequantised bit-exactly as in decode.  The workspace holds the
 * reconstructed K and V (2 x batch x Hkv x round_up(pos0 + n_tokens, 64) x
 * 128 fp16 elements, for either act dtype: bf16 activations attend in fp16,
 * exact for |values| up to 65504, with 8x finer rounding of K and V than
 * bf16 storage) and any repacked copies.
 * ------------------------------------------------------------------- */
typedef struct {
  int batch, n_q_heads, head_dim, n_tokens, pos0;
  int dtype;
  const void* q; int64_t q_stride_b, q_stride_h, q_stride_t;
  starkv_klatent k;
  starkv_vlatent v;
  const void* uv; int64_t uv_row_stride;
  const void* rope_table; int rope_max_positions;
  float scale;
  void* out; int64_t out_stride_b, out_stride_h, out_stride_t;
} starkv_prefill_desc;

size_t starkv_prefill_workspace_bytes(const starkv_prefill_desc* d);
int starkv_prefill_attention(const starkv_prefill_desc* d, void* workspace, size_t workspace_bytes, void* stream);

/* Same as starkv_prefill_attention, and records events[0..2] (hipEvent_t) on
 * the stream before the K / V reconstruction, after it and after the
 * attention kernel (per-kernel timing, as starkv_decode_attention_timed). */
int starkv_prefill_attention_timed(const starkv_prefill_desc* d, void* workspace, size_t workspace_bytes,
                                   void* stream, void* const* events);

/* ---------------------------------------------------------------------
 * The e2e decoder layer's own elementwise work.  No counterpart in the
 * reference's attention path: these replace, in the end-to-end harness, the
 * HF layers the reference's latency.py runs around the attention
 * (transformers models/llama/modeling_llama.py: LlamaRMSNorm.forward, the
 * residual adds of LlamaDecoderLayer.forward, LlamaMLP's act_fn(gate) * up),
 * one launch each instead of torch's several.  act() below rounds to the
 * activation dtype, as torch does after each fp16 / bf16 operation.
 *
 * starkv_rms_norm: for each of `rows` rows of `hidden` values,
 *   x' = act(x + residual)   (when residual is given; stored to residual_out when that is given)
 *   out = act(weight * act(x' * rsqrt(sum(x'^2) / hidden + eps)))   (sum and rsqrt in fp32)
 * Row r of x at x + r * x_stride (elements), likewise residual, residual_out
 * and out; weight [hidden].  hidden a multiple of 8 and <= 16384
 * (STARKV_ERR_LIMIT); every pointer 16-byte aligned and every stride a
 * multiple of 8 (STARKV_ERR_ALIGN).  out may alias x; residual_out may alias
 * x or residual.
 * ------------------------------------------------------------------- */
typedef struct {
  int rows, hidden, dtype;
  const void* x; int64_t x_stride;
  const void* residual; int64_t residual_stride;       /* optional */
  void* residual_out; int64_t residual_out_stride;     /* optional (requires residual) */
  const void* weight;
  float eps;
  void* out; int64_t out_stride;
} starkv_rms_norm_desc;

int starkv_rms_norm(const starkv_rms_norm_desc* d, void* stream);

/* starkv_silu_mul: out = act(act(g / (1 + exp(-g))) * u) elementwise over
 * `rows` rows of `width` values (gate row r at gate + r * gate_stride, up and
 * out likewise; fp32 inside).  width a multiple of 8; pointers 16-byte
 * aligned, strides multiples of 8 (STARKV_ERR_ALIGN). */
typedef struct {
  int rows, width, dtype;
  const void* gate; int64_t gate_stride;
  const void* up; int64_t up_stride;
  void* out; int64_t out_stride;
} starkv_silu_mul_desc;

int starkv_silu_mul(const starkv_silu_mul_desc* d, void* stream);

/* starkv_skinny_gemm: the decode-batch projections of the e2e decoder layer
 * (nn.Linear y = x W^T with m <= 16 rows, where the weight stream bounds the
 * time), fp32 accumulation, one rounding:
 *   epilogue 0: out[i][j]  = act(sum_k x[i][k] w[j][k])              (j < n)
 *   epilogue 1: out[i][j]  = act(sum_k x[i][k] w[j][k] + out[i][j])  (the residual add, in place)
 *   epilogue 2: g = act(x . w[j]), u = act(x . w[j + n/2]):
 *               out[i][j]  = act(act(g / (1 + exp(-g))) * u)        (j < n/2; LlamaMLP over the
 *               gate rows followed by the up rows of one merged weight)
 * x [m][k] row stride x_stride, w [n][k] row stride w_stride, out row stride
 * out_stride (elements).  With w_packed, w holds the weight packed as
 * [n/16][k/64][16][64] (element (j, kk) at ((j/16 * k/64 + kk/64) * 16 +
 * j%16) * 64 + kk%64; w_stride unused): each tile's range then streams
 * linearly.  With rms, x is the raw input of an RMSNorm whose weight the
 * caller folded into w (w[j][kk] = act(W[j][kk] * norm_weight[kk])): the sums
 * above are scaled by rsqrt(sum_kk x[i][kk]^2 / k + rms_eps) per row before
 * the epilogue (HF LlamaRMSNorm followed by the projection, without rounding
 * the normalised input).  k a multiple of 64, n a multiple of 16 (32 for
 * epilogue 2), m <= 16 (STARKV_ERR_LIMIT); x and w 16-byte aligned, strides
 * multiples of 8 (STARKV_ERR_ALIGN). */
typedef struct {
  int m, n, k, dtype, epilogue;
  const void* x; int64_t x_stride;
  const void* w; int64_t w_stride;
  void* out; int64_t out_stride;
  int w_packed;
  int rms; float rms_eps;
} starkv_skinny_gemm_desc;

int starkv_skinny_gemm(const starkv_skinny_gemm_desc* d, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* STARKV_H_ */
