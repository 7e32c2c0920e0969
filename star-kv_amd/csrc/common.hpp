// Shared device/host definitions of libstarkv (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/starkv.h"

namespace starkv {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int HEAD_DIM = 128;
constexpr int TILE = 32;            // positions per K-logit tile (the MFMA N dimension)
constexpr int KSTEP = 16;           // positions per P.V MFMA K-step
constexpr int PV_RG = 16;           // split partials per first-level reduction group

// ---------------------------------------------------------------------------
// K-logit launch plan (passed by value as a kernel argument, read with
// scalar loads).  Wave w of workgroup-plan g owns up to `maxi` "items"; an
// item is one 32-rank M-tile of one query head.
// ---------------------------------------------------------------------------
constexpr int K_MAXI = 4;          // items per wave (upper bound over kernel variants)
constexpr int K_MAX_WAVES = 64;    // waves in one batch's plan
constexpr int K_MAX_KV = 64;
constexpr int K_MAX_QH = 64;
constexpr int K1_WS_RING_BYTES = 163840 - 1024;      // warp-specialised K-logit LDS ring (+ 1 KB carry)
constexpr int K1_WS_RING_I8_BYTES = 163840 - 1536;   // the same for int8 latents (+ 1.5 KB carry)

// item word: qhead[0:8) kv[8:16) mtile[16:20) nvalid[20:26) last_of_q[26] valid[27]
__host__ __device__ inline uint32_t item_pack(int qh, int kv, int mt, int nv, int last) {
  return (uint32_t)qh | ((uint32_t)kv << 8) | ((uint32_t)mt << 16) | ((uint32_t)nv << 20) |
         ((uint32_t)(last ? 1 : 0) << 26) | (1u << 27);
}
__device__ inline int item_qh(uint32_t w) { return w & 0xff; }
__device__ inline int item_kv(uint32_t w) { return (w >> 8) & 0xff; }
__device__ inline int item_mt(uint32_t w) { return (w >> 16) & 0xf; }
__device__ inline int item_nv(uint32_t w) { return (w >> 20) & 0x3f; }
__device__ inline bool item_last(uint32_t w) { return (w >> 26) & 1; }
__device__ inline bool item_valid(uint32_t w) { return (w >> 27) & 1; }

struct KArgs {
  const void* q; int64_t q_sb, q_sh;
  const void* x; int64_t x_sb;
  const void* xscale; int64_t xs_sb, xs_sh;       // quantised K: fp16 scales of x per (b, h, s)
  const void* x2; int64_t x2_sb;                   // quantised K lower block (int4 nibbles, bytes)
  const void* xscale2; int64_t xs2_sb, xs2_sh;     // its fp16 scales
  int ksplit, k_a_int8;                            // ranks [0, ksplit) in x (int8 if k_a_int8, else int4)
  const void* bk; int64_t bk_rs;
  const uint4* rope;                               // RoPE operand table [tile][8][64] x 16 B
  const void* mask; int64_t m_sb, m_sh; int mask_dtype;
  const int* last_pos;                             // optional (device): positions past it take -1e30
  // logit (b, q, s) at out + b*o_sb + (s / 32)*o_st + q*o_sh + s % 32: rows
  // (o_st = 32) or 32-position tiles of all heads (o_sh = 32, o_st = Hq*32)
  void* out; int64_t o_sb, o_st, o_sh;
  float* chunkmax;                                 // [B][Hq][n_chunks] (optional)
  int S, Hq, n_chunks, tiles_per_chunk, n_wg;
  int maxi;                                        // items per wave of the launched variant (2 or 4)
  int ws;                                          // warp-specialised kernel (dense, 16-byte aligned latents)
  int ws_stage, ws_nst;                            // its LDS stage bytes and stage count
  int ws_i8;                                       // ... over int8 latents (per-(b,h,s) fp16 scales)
  float wscale;                                    // softmax scale (the RoPE table carries the attention scaling)
  int64_t xoff[K_MAX_KV];                          // per KV head: elements (dense) or bytes (quantised)
  int xpitch[K_MAX_KV];
  int64_t xoff2[K_MAX_KV];                         // lower block (bytes)
  int xpitch2[K_MAX_KV];
  int64_t bkoff[K_MAX_KV];
  uint32_t items[K_MAX_WAVES][K_MAXI];             // [workgroup plan * waves + wave][item]
  // grouped-query variant (k_logits_gqa.hip, 2 <= gs <= 8): K reconstructed
  // once per KV head; item 0 of consumer wave w = item_pack(kv * gs, kv, dim half, 0, 1)
  int gqa, gs;
  int16_t krank[K_MAX_KV];
};
constexpr int K1_GQ_CARRY_BYTES = 2 * 2 * 64 * 4 * 4;          // GQA: dim-half partial logits, 2 tiles x 2 heads
constexpr int K1_GQ_RING_BYTES = 81920 - K1_GQ_CARRY_BYTES;    // its LDS ring (two workgroups per CU)

// ---------------------------------------------------------------------------
// P.V launch arguments.
// ---------------------------------------------------------------------------
// V-latent storage of the P.V kernel (template parameter VQ)
constexpr int VQ_DENSE = 0;    // act-dtype rows; x strides in elements
constexpr int VQ_BLOCK = 1;    // per-token fp16 scale: ranks [0, split) in x (int4 nibbles, or int8 when
                               // a_int8), ranks [split, Rv) in x2 (int4 nibbles); x strides in bytes
constexpr int VQ_G64 = 2;      // int4 asymmetric: fp16 scale and zero per (b, s, 64-rank group)

struct PVArgs {
  const void* x; int64_t x_sb, x_ss;               // V latent (VQ_DENSE: elements; else bytes)
  const void* x2; int64_t x2_sb, x2_ss;            // VQ_BLOCK lower block (bytes)
  const void* xs; int64_t xs_sb, xs_ss;            // fp16 scales of x: (b, s[, g]) in elements
  const void* xs2; int64_t xs2_sb, xs2_ss;         // fp16 scales of x2
  const void* xz;                                  // VQ_G64 fp16 zero points (strides of xs)
  int split, a_int8;                               // VQ_BLOCK: first rank of x2; x holds int8
  int xnb, x2nb;                                   // quantised: bytes a row of x / x2 holds (unaligned rows)
  int qfast;                                       // quantised rows aligned for whole-chunk loads (host-side)
  const float* logits; int64_t l_sb, l_st, l_sh;   // fused path: fp32 logits, K1's layout (o_sb, o_st, o_sh)
  const float* chunkmax; int n_chunk1;             // fused path: per-chunk maxima
  const void* p; int64_t p_sb, p_sh;               // drop-in path: probabilities (act dtype)
  int p_vec;                                       // drop-in: P rows allow 16-byte loads
  // bq = b * n_hg + head group (32 heads each)
  float* part;                                     // [bq][n_c2][32][Rvp] fp32, or fp16 when part16
  int part16;                                      // fused: fp16 partials divided by their chunk's softmax sum
  float* psum;                                     // fused: [B*n_hg][n_c2][32] softmax partial sums
  float* part2; int n_grp;                         // drop-in two-level reduction: [B*n_hg][n_grp][32][Rvp]
  void* out; int64_t o_sb, o_sh;                   // drop-in: act-dtype [B][H][Rv]
  int S, H, n_hg, Rv, Rvp, n_cb, n_c2, c2_len;
};

// ---------------------------------------------------------------------------
// Latent-cache writer arguments (quant.hip).
// ---------------------------------------------------------------------------
struct KAppendArgs {
  const void* src; int64_t src_sb, src_sh, src_st;   // new rows (b, h, t), act dtype, elements
  int B, H, T, pos0, cap;
  const int* pos0_dev;                              // optional: position read at run time
  int* err;                                         // optional: set to 1 when a row is skipped
  int fmt;                                          // STARKV_FMT_DENSE or a quantised format
  void* data; int64_t stride_b;                     // dense: elements; quantised: bytes
  void* scale; int64_t sc_sb, sc_sh;
  int split, a_int8;                                // ranks [0, split) in data (int8 if a_int8)
  void* data2; int64_t stride2_b;                   // ranks [split, r) as int4
  void* scale2; int64_t sc2_sb, sc2_sh;
  int rank[K_MAX_KV];
  int64_t off[K_MAX_KV], pitch[K_MAX_KV];
  int64_t off2[K_MAX_KV], pitch2[K_MAX_KV];
  int64_t src_off[K_MAX_KV];                        // source row offset of head h (elements)
};

struct VAppendArgs {
  const void* src; int64_t src_sb, src_st;          // new rows (b, t), act dtype, elements
  int B, T, pos0, cap, R, vq;
  int gw;                                           // waves per row (group-64: one per group)
  const int* pos0_dev;                              // optional: position read at run time
  int* err;                                         // optional: set to 1 when a row is skipped
  void* data; int64_t stride_b, stride_s;
  void* scale; int64_t sc_sb, sc_ss;
  void* zero;                                       // VQ_G64 (strides of scale)
  int split, a_int8;
  void* data2; int64_t stride2_b, stride2_s;
  void* scale2; int64_t sc2_sb, sc2_ss;
};

// ---------------------------------------------------------------------------
// Up-projection arguments.
// ---------------------------------------------------------------------------
struct UPArgs {
  const float* part; const float* psum;            // P.V split partials and softmax sums (PVArgs layout)
  int part16;                                      // partials fp16, divided by their psum
  int n_c2, Rvp, n_hg;
  const void* uv; int64_t uv_rs;                   // [Hkv*128][Rv]
  void* out; int64_t o_sb, o_sh;                   // [B][Hq][128]
  int B, Hq, gs, Rv;
  int sw, n_sl;                                    // column slices of the V rank (sw columns each)
  int n_cs;                                        // chunk sets (contiguous ranges of the n_c2 chunks)
  float* ypart;                                    // [Hkv][n_sl][n_cs][B*gs][128] partial up-projections
  int out_f32;                                     // 1: fp32 output, 0: weight dtype
};

// ---------------------------------------------------------------------------
// In-place RoPE of query rows (rope.hip).
// ---------------------------------------------------------------------------
struct RopeApplyArgs {
  void* x; int64_t sb, sh, st;                     // [B][H][T][128], act dtype, elements
  int B, H, T, pos0, max_pos;
  const int* pos0_dev;                             // optional: position read at run time
  int* err;                                        // optional: set to 1 when a row is skipped
  const void* table;
};

// In-place rotation of [B][H][T][128] rows by the table: one thread per
// (row, frequency i < 64), computing both halves in fp32 and rounding once.
// ---------------------------------------------------------------------------
// Prefill arguments (prefill.hip).
// ---------------------------------------------------------------------------
constexpr int PF_K_POS = 256;    // positions per K-reconstruction workgroup
constexpr int PF_V_POS = 256;    // positions per V-reconstruction workgroup (two KV heads)
constexpr int PF_Q_POS = 256;    // queries per attention workgroup
struct PFArgs {
  int S, S_pad, Hkv, Hq, gs, T, pos0;              // S = pos0 + T positions reconstructed, S_pad = round_up(S, 64)
  int rc_nb, rc_blocks;                            // K reconstruction: position blocks per batch, times B
  int rv_nb, rv_blocks;                            // V reconstruction: the same for its blocks
  int rv_hpx;                                      // V reconstruction: head pairs per XCD (0: blocks per XCD)
  int fa_nqb, fa_nkvi;                             // attention: query blocks per head, B * Hkv
  // K latent: dense act dtype (offsets / pitches in elements) or int8 (bytes) with fp16 scales (b, h, s)
  const void* kx; int64_t kx_sb; int k_i8;
  const void* kscale; int64_t ks_sb, ks_sh;
  int krank[K_MAX_KV];
  int64_t kxoff[K_MAX_KV];
  int64_t kxpitch[K_MAX_KV];
  const void* bk; int64_t bk_rs;
  int64_t bkoff[K_MAX_KV];
  // K latent in the reference split format (k_ref): ranks [0, ksplit) in kx (int8 if k_a8, else
  // int4 nibbles), ranks [ksplit, r) int4 nibbles in kx2 (bytes); fp16 scales per (b, h, s) in
  // kscale / kscale2
  int k_ref, ksplit, k_a8;
  const void* kx2; int64_t kx2_sb;
  const void* kscale2; int64_t ks2_sb, ks2_sh;
  int64_t kxoff2[K_MAX_KV];
  int64_t kxpitch2[K_MAX_KV];
  // V latent: dense act dtype (elements) or group-64 int4 (bytes) with fp16 scale / zero (b, s, g)
  const void* vx; int64_t vx_sb, vx_ss; int v_g64, Rv;
  const void* vscale; const void* vzero; int64_t vs_sb, vs_ss;
  // ... or per-token blocks (v_blk: the reference int4 format with an optional int8 / int4 upper
  // block, or int8): ranks [0, vsplit) in vx (int8 if v_a8, else int4), [vsplit, Rv) int4 in vx2;
  // fp16 scales per (b, s) in vscale / vscale2
  int v_blk, vsplit, v_a8;
  const void* vx2; int64_t vx2_sb, vx2_ss;
  const void* vscale2; int64_t vs2_sb, vs2_ss;
  const void* uv; int64_t uv_rs;                   // [Hkv*128][Rv]
  const void* rope;                                // RoPE table (rope.hip layout)
  void* kbuf; void* vbuf;                          // [B][Hkv][S_pad][128] act dtype
  const void* q; int64_t q_sb, q_sh, q_st;         // rotated queries (b, qh, t)
  float scale_log2;                                // softmax scale * log2(e)
  void* out; int64_t o_sb, o_sh, o_st;             // (b, qh, t), act dtype
};
// Prefill inputs whose latent rank is not a multiple of 8, or whose rows are
// not aligned for the reconstruction kernels' chunk loads, are first copied
// into aligned workspace rows (prefill.hip repack_rows_kernel): row (b, h, s)
// of nel[h] elements (16-bit values, bytes or int4 nibbles) at src + b*src_sb
// + src_off[h] + s*src_pitch[h] (bytes) goes to dst + b*dst_sb + (h*S + s)*pitch,
// the elements past nel[h] up to the pitch set to the kind's zero (0, 0,
// nibble 8).
constexpr int RP_HALF = 0, RP_BYTE = 1, RP_NIB = 2;
struct RepackArgs {
  const uint8_t* src; int64_t src_sb;
  int64_t src_off[K_MAX_KV], src_pitch[K_MAX_KV];
  int nel[K_MAX_KV];
  uint8_t* dst; int64_t dst_sb; int pitch;         // pitch: bytes, a multiple of 16
  int kind, H, S;
};
int launch_repack(const RepackArgs& a, int B, hipStream_t st);

// ---------------------------------------------------------------------------
// The e2e decoder layer's RMSNorm and SiLU-multiply (layer_ops.hip).
// ---------------------------------------------------------------------------
constexpr int NORM_MAX_HIDDEN = 16384;
struct NormArgs {
  const void* x; int64_t xs;                       // rows of H act-dtype values, strides in elements
  const void* res; int64_t rs;                     // optional residual added first
  void* res_out; int64_t ros;                      // optional: the sum x + res
  const void* w;                                   // [H] weight
  void* out; int64_t os;
  int rows, H;
  float eps;
};
struct SiluMulArgs {
  const void* g; int64_t gs;
  const void* u; int64_t us;
  void* out; int64_t os;
  int rows, W;
};

constexpr int GEMM_STORE = 0, GEMM_ADD = 1, GEMM_SILU_MUL = 2;
constexpr int GEMM_MAX_M = 16, GEMM_MAX_WAVES = 8, GEMM_MAX_STAGES = 8, GEMM_PAIRS_PER_STAGE = 4;
struct GemmArgs {                                  // skinny_gemm.hip
  const void* x; int64_t xs;                       // [M][K] activations, row stride (elements)
  const void* w; int64_t ws;                       // [N][K] weight (nn.Linear layout), row stride
  void* out; int64_t os;                           // [M][N] (SILU_MUL: [M][half_rows])
  int M, N, K, half_rows;
  int wpk;                                         // w packed [N / 16][K / 64][16][64]
  int rms; float rms_eps;                          // x is an RMSNorm's raw input (weight folded into w)
  int nst, pps;                                    // LDS ring stages per wave, 64-k pairs per stage (launcher)
};

// A decode step's cache writes and query rotation in one launch (quant.hip)
struct StepAppendArgs {
  KAppendArgs k;
  VAppendArgs v;
  RopeApplyArgs r;
  int has_rope;
  int64_t nbk, nbv;                                // workgroups of the K and V writes (set by the launcher)
};

// these are passed by value as kernel arguments (at most 4 KiB)
static_assert(sizeof(KArgs) <= 4096 && sizeof(PFArgs) <= 4096 && sizeof(StepAppendArgs) <= 4096,
              "kernel argument size");

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
template <typename T> struct ElemTraits;
template <> struct ElemTraits<_Float16> { static constexpr int code = STARKV_F16; };
template <> struct ElemTraits<__bf16> { static constexpr int code = STARKV_BF16; };

__device__ inline float bf16_bits_to_float(uint32_t lo16) { return __uint_as_float(lo16 << 16); }

__device__ inline float to_f32(_Float16 h) { return (float)h; }
__device__ inline float to_f32(__bf16 h) { return (float)h; }

template <typename T> __device__ inline T from_f32(float f);
template <> __device__ inline _Float16 from_f32<_Float16>(float f) { return (_Float16)f; }
template <> __device__ inline __bf16 from_f32<__bf16>(float f) { return (__bf16)f; }
template <> __device__ inline float from_f32<float>(float f) { return f; }

__device__ inline float load_elem_f32(const void* p, int dtype, int64_t idx) {
  if (dtype == STARKV_F32) return ((const float*)p)[idx];
  if (dtype == STARKV_F16) return (float)((const _Float16*)p)[idx];
  return (float)((const __bf16*)p)[idx];
}

__device__ inline floatx16 mfma_f16(half8 a, half8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ inline floatx16 mfma_bf16(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// value of lane (l ^ 32): sum of the two halves of a wave64
__device__ inline float add_halves(float v) {
  auto x = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return __int_as_float(x[0]) + __int_as_float(x[1]);
}

__device__ inline float wave_max32(float v) {   // max over the 32 lanes of a half wave
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

typedef _Float16 kh2 __attribute__((ext_vector_type(2)));

// 16 quantised ranks -> 16 fp16 values, bit-exact fp16(n * s): the integer is
// biased into the fp16 pattern 1024 + n (exact), the bias removed (exact) and
// one correctly rounded packed-fp16 multiply by the scale.  int8: 16 bytes;
// int4: 8 bytes (rank 2k in the low nibble of byte k, value nibble - 8).
__device__ inline void dequant16(uint4 r, bool k8, uint16_t s16, uint4& lo, uint4& hi) {
  uint32_t pr[8];
  _Float16 bias;
  if (k8) {
    // n + 128 as a byte, placed under the exponent byte 0x64 by one v_perm per
    // pair (selector 4 picks byte 0 of the 0x64646464 source)
    const uint32_t w[4] = {r.x ^ 0x80808080u, r.y ^ 0x80808080u, r.z ^ 0x80808080u, r.w ^ 0x80808080u};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      pr[2 * k] = __builtin_amdgcn_perm(0x64646464u, w[k], 0x04010400u);
      pr[2 * k + 1] = __builtin_amdgcn_perm(0x64646464u, w[k], 0x04030402u);
    }
    bias = (_Float16)-1152.0f;
  } else {
    const uint32_t w[2] = {r.x, r.y};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t u = w[k >> 2] >> (8 * (k & 3));
      pr[k] = (u & 0xFu) | (((u >> 4) & 0xFu) << 16) | 0x64006400u;
    }
    bias = (_Float16)-1032.0f;
  }
  const kh2 s = __builtin_bit_cast(kh2, (uint32_t)s16 * 0x10001u), b2 = {bias, bias};
  uint32_t o[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    o[k] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(kh2, pr[k]) + b2) * s);
  lo = make_uint4(o[0], o[1], o[2], o[3]);
  hi = make_uint4(o[4], o[5], o[6], o[7]);
}

// ---------------------------------------------------------------------------
// Rows of any byte alignment: quantised latents whose rank or pitch is not a
// multiple of the vector width (the reference's bx default, 1228 V ranks over
// a 256-rank upper block, leaves 486-byte int4 rows).  ld_row_bytes<N> reads
// N bytes (4, 8 or 16) of a row from byte `off` on as aligned dwords joined
// with v_alignbyte.  Every dword address is clamped to the dword holding the
// row's last valid byte (row + nvalid - 1, nvalid >= 1), so no load touches a
// dword without a byte of the row: it stays on the row's own pages.  Bytes
// at or past nvalid come back unspecified; callers mask the ranks they hold.
// ---------------------------------------------------------------------------
template <int N>
__device__ inline void ld_row_bytes(const uint8_t* row, int off, int nvalid, uint32_t (&out)[N / 4]) {
  static_assert(N == 4 || N == 8 || N == 16, "4, 8 or 16 bytes");
  const uint64_t p = (uint64_t)row + (uint64_t)off;
  const uint64_t last = ((uint64_t)row + (uint64_t)(nvalid - 1)) & ~(uint64_t)3;
  const uint64_t base = p & ~(uint64_t)3;
  const uint32_t sh = (uint32_t)p & 3u;
  uint32_t d[N / 4 + 1];
#pragma unroll
  for (int i = 0; i <= N / 4; ++i) {
    const uint64_t q = base + 4u * (uint64_t)i;
    d[i] = *(const uint32_t*)(q < last ? q : last);
  }
#pragma unroll
  for (int i = 0; i < N / 4; ++i) out[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
}

// eight 16-bit values (rank order, two per dword): those at index >= nv become 0
__device__ inline uint4 mask_h8(uint4 f, int nv) {
  uint32_t w[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t m = (2 * k + 1 < nv) ? 0xFFFFFFFFu : (2 * k < nv) ? 0x0000FFFFu : 0u;
    w[k] &= m;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// launchers (return hipError_t as int; 0 on success)
int rope_table_tiles(int max_positions);
int launch_rope_table(const float* inv_freq_host, int max_positions, float scaling, void* table, hipStream_t st);
int launch_rope_apply(const RopeApplyArgs& a, int dtype, hipStream_t st);
int launch_rms_norm(const NormArgs& a, int dtype, hipStream_t st);
int launch_silu_mul(const SiluMulArgs& a, int dtype, hipStream_t st);
int launch_skinny_gemm(const GemmArgs& a, int dtype, int epi, hipStream_t st);
int launch_k_logits(const KArgs& a, int dtype, int fmt, bool out_f32, int out_dtype, bool fast, int B, hipStream_t st);
int launch_k_logits_ws(const KArgs& a, int dtype, bool out_f32, int out_dtype, int B, hipStream_t st);
int launch_k_logits_gqa(const KArgs& a, int dtype, bool out_f32, int out_dtype, int B, hipStream_t st);
int launch_pv(const PVArgs& a, int dtype, int vq, bool fused, bool fast, int B, hipStream_t st);
int pv_tiles_per_wave(int Rvp, bool fused, int vq);   // column tiles (of 32 ranks) per P.V wave
int pv_wide_tiles(int Rvp, bool fused, int vq);       // > 0: the 8-wave all-columns kernel, tiles per wave
// P.V workgroups resident per CU (the kernel's register budget): the wide
// dense variants (8 and 13 tiles) take one, the others two
constexpr int pv_wg_per_cu(int ntw, int vq) { return ntw >= 8 && vq == VQ_DENSE ? 1 : 2; }
int launch_up_proj(const UPArgs& a, int dtype, bool fast, hipStream_t st);
int up_slice_width(int n_kv, int Rv, int cus);        // V-rank columns per up-projection workgroup
int up_chunk_sets(int n_kv, int n_sl, int n_c2, int cus);   // chunk sets per (slice, KV head)
int launch_fill_i32(int* p, int n, int v, hipStream_t st);
int launch_k_append(const KAppendArgs& a, int dtype, hipStream_t st);
int launch_v_append(const VAppendArgs& a, int dtype, hipStream_t st);
int launch_step_append(const StepAppendArgs& a, int dtype, hipStream_t st);
int launch_prefill(const PFArgs& a, int dtype, int B, hipStream_t st, hipEvent_t mid);   // mid: after K/V

// In-place RoPE of one (query row, frequency i < 64) element pair by the
// table, in fp32 and rounded once; rows whose run-time position falls outside
// the table are left as they are and set the error flag.
// The (cos, sin) pair of (position p, frequency i) is fp16 element pair
// ((p/32*8 + i/8)*64 + (i%8)/4*32 + p%32)*8 + 2*(i%4) of the table.
template <typename T>
__device__ inline void rope_apply_row(const RopeApplyArgs& a, int64_t idx) {
  const int64_t rows = (int64_t)a.B * a.H * a.T;
  if (idx >= rows * 64) return;
  const int i = (int)(idx & 63);
  const int64_t row = idx >> 6;
  const int t = (int)(row % a.T);
  const int h = (int)((row / a.T) % a.H);
  const int b = (int)(row / ((int64_t)a.T * a.H));
  const int p = (a.pos0_dev ? *a.pos0_dev : a.pos0) + t;
  if (p < 0 || p >= a.max_pos) {                 // only a run-time position can land here
    if (a.err != nullptr) *a.err = 1;
    return;
  }
  T* x = (T*)a.x + b * a.sb + h * a.sh + (int64_t)t * a.st;
  const int64_t te = ((int64_t)((p >> 5) * 8 + (i >> 3)) * 64 + ((i & 7) >> 2) * 32 + (p & 31)) * 8 + 2 * (i & 3);
  const uint32_t cs = ((const uint32_t*)a.table)[te >> 1];
  const kh2 c2 = __builtin_bit_cast(kh2, cs);
  const float c = (float)c2[0], sn = (float)c2[1];
  const float x0 = to_f32(x[i]), x1 = to_f32(x[i + 64]);
  x[i] = (T)(x0 * c - x1 * sn);
  x[i + 64] = (T)(x1 * c + x0 * sn);
}

}  // namespace starkv
