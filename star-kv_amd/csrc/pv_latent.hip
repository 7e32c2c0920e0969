// K2: probabilities x V-latent on gfx950.
//
// Replaces the reference's P @ X_v (model.py:484) and the Triton _bx_fwd
// kernel (bx_quant.py:37-114):   o[b, q, j] = sum_s P[b, q, s] * X_v[b, s, j].
//
// X_v is one latent shared by every head, so a workgroup streams a
// (position chunk x column block) slab of X_v once for all 32 heads: the MFMA
// 32x32x16 A operand is P (32 heads x 16 positions), the B operand is X_v
// (16 positions x 32 ranks).  The four waves of a workgroup take the same
// positions and split the column tiles, so every wave owns its accumulators.
// X_v rows arrive with coalesced 16-byte non-temporal loads (two K-steps in
// flight per wave), are staged in wave-private LDS and are read back
// transposed with ds_read_b64_tr_b16, the gfx950 LDS transpose load: within
// each 16-lane group, lane j receives column j%4 of the rows addressed by
// lanes {j/4, 4+j/4, 8+j/4, 12+j/4}.
//
// Quantised latents are fetched as packed bytes (int4 nibbles or int8) with
// their fp16 scales, carried through the prefetch registers, and dequantised
// just before the LDS write with packed-fp16 arithmetic: an integer n is
// biased into the fp16 bit pattern 1024 + n (exact), the bias removed (exact),
// then one correctly rounded multiply by the scale (reference int4 / int8:
// fp16((n - 8) * s), bx_quant.py:83-86) or fused multiply-add with the zero
// point (group-64 int4: fp16(n * s + z), one rounding).  bf16 activations
// round that fp16 value once more to bf16, as torch_bx's .to(b.dtype) does
// (bx_quant.py:171-172).
//
// Fused mode: P = exp(logit - M) is formed in registers from the fp32 logits
// of K1 with M the global row max (from K1's chunk maxima); the softmax
// denominators are summed on the side and normalisation happens in K3.
// More than 32 heads take one more pass per group of 32 (blockIdx.y counts
// (batch, head group)).
// Drop-in mode (bx): P is read as given.
//
// Split-S: each workgroup writes its chunk's partial sums; they are added in
// fixed chunk order (deterministic; no float atomics, unlike the fp16 atomics
// into an uninitialised tensor of bx_quant.py:113-114, 147) by
// pv_reduce_kernel (drop-in) or by the up-projection kernel (fused decode).
#include "common.hpp"

namespace starkv {

typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 lds_fp16x4;

constexpr int PV_QDEPTH = 2;   // quantised latents: K-steps loaded ahead
constexpr int PV_WDEPTH = 3;   // the all-columns kernel: register stages of its software pipeline

__device__ inline uint2 lds_read_tr16(const uint16_t* p) {
  auto r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) lds_fp16x4*)(p));
  return __builtin_bit_cast(uint2, r);
}

__device__ inline uint4 ld_stream16(const void* p) {
  typedef unsigned u4v __attribute__((ext_vector_type(4)));
  const u4v t = __builtin_nontemporal_load((const u4v*)p);
  return make_uint4(t.x, t.y, t.z, t.w);
}

template <int NTW, int VQ>
struct PVStage {
  uint4 r[VQ == VQ_DENSE ? NTW : 1];   // dense: X_v chunks (16 B = 8 ranks) of this wave's slab
  uint2 q[VQ == VQ_DENSE ? 1 : NTW];   // quantised: the chunk's packed bytes (int4: .x)
  uint16_t s[VQ == VQ_DENSE ? 1 : NTW];  // fp16 scale bits of the chunk's row (and group)
  uint16_t z[VQ == VQ_G64 ? NTW : 1];  // fp16 zero-point bits (group-64 int4)
  float p[8];                          // fused: fp32 logits of the A operand
  uint4 praw;                          // drop-in: 8 probabilities of the A operand (act dtype)
};

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
__device__ inline h2v as_h2(uint32_t u) { return __builtin_bit_cast(h2v, u); }
__device__ inline uint32_t as_u32(h2v h) { return __builtin_bit_cast(uint32_t, h); }

// Eight dequantised fp16 values of one chunk, packed two per dword.  kind8:
// the bytes are int8 (x, y), else eight int4 nibbles in x, rank 2k in the low
// nibble of byte k.  Ranks in order (0..7), except group-64 int4: ranks
// 0 2 4 6 1 3 5 7 (pv_g64_rank maps an LDS column back to its rank).
// s2, z2: the fp16 scale / zero-point bits in both halves of a dword
template <int VQ>
__device__ inline uint4 dequant8(uint2 q, bool kind8, uint32_t s2, uint32_t z2) {
  const h2v s = as_h2(s2);
  uint32_t pr[4];
  _Float16 bias;
  if (VQ == VQ_BLOCK && kind8) {
    const uint32_t x = q.x ^ 0x80808080u, y = q.y ^ 0x80808080u;      // n + 128, unsigned
    pr[0] = (x & 0xFFu) | ((x << 8) & 0xFF0000u);
    pr[1] = ((x >> 16) & 0xFFu) | ((x >> 8) & 0xFF0000u);
    pr[2] = (y & 0xFFu) | ((y << 8) & 0xFF0000u);
    pr[3] = ((y >> 16) & 0xFFu) | ((y >> 8) & 0xFF0000u);
    bias = (_Float16)-1152.0f;                                       // 1024 + 128
  } else if (VQ == VQ_G64) {
    // even ranks (low nibbles) and odd ranks (high nibbles) as bytes; one
    // v_perm per pair of same-parity ranks places two of them under the
    // exponent byte 0x64 (selector 4 picks a byte of the 0x64646464 source)
    const uint32_t lo = q.x & 0x0F0F0F0Fu, hi = (q.x >> 4) & 0x0F0F0F0Fu;
    pr[0] = __builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u);     // ranks 0, 2
    pr[1] = __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u);     // ranks 4, 6
    pr[2] = __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u);     // ranks 1, 3
    pr[3] = __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u);     // ranks 5, 7
    bias = (_Float16)-1024.0f;
  } else {
    // low nibbles (even ranks) and high nibbles (odd ranks) as bytes; one
    // v_perm per pair puts byte k of each under a zero byte
    const uint32_t lo = q.x & 0x0F0F0F0Fu, hi = (q.x >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int k = 0; k < 4; ++k) pr[k] = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u + 0x00010001u * k);
    bias = (_Float16)-1032.0f;                                       // nibble - 8
  }
  const h2v b2 = {bias, bias};
  const uint32_t ebyte = VQ == VQ_G64 ? 0u : 0x64006400u;            // group-64: already in place
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const h2v n = as_h2(pr[k] | ebyte) + b2;                           // exact small integers
    if constexpr (VQ == VQ_G64) {
      const h2v zz = as_h2(z2);
      o[k] = as_u32(__builtin_elementwise_fma(n, s, zz));
    } else {
      o[k] = as_u32(n * s);
    }
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// group-64 int4 chunks sit in LDS as ranks 0 2 4 6 1 3 5 7: the rank of LDS
// column n (within a 32-column tile)
__device__ inline int pv_g64_rank(int n) { return (n & ~7) | ((n & 3) << 1) | ((n >> 2) & 1); }

__device__ inline uint4 f16x8_to_bf16x8(uint4 h) {
  const uint32_t w[4] = {h.x, h.y, h.z, h.w};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const h2v v = as_h2(w[k]);
    const __bf16 lo = (__bf16)(float)v[0], hi = (__bf16)(float)v[1];
    o[k] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// the maximum of one head's K1 chunk maxima cm[0, n) over c = j, j+8, ...:
// eight independent loads in flight per step (a load-then-max loop would wait
// out one memory latency per chunk: 32 of them at 256 chunks)
__device__ inline float chunk_max_part(const float* cm, int n, int j) {
  float m[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) m[u] = -INFINITY;
  int c = j;
  for (; c + 56 < n; c += 64) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = cm[c + 8 * u];
#pragma unroll
    for (int u = 0; u < 8; ++u) m[u] = fmaxf(m[u], v[u]);
  }
  for (; c < n; c += 8) m[0] = fmaxf(m[0], cm[c]);
#pragma unroll
  for (int u = 1; u < 8; ++u) m[0] = fmaxf(m[0], m[u]);
  return m[0];
}

template <typename VT, int NTW, bool FUSED, bool FAST, int VQ>
__global__ __launch_bounds__(256, pv_wg_per_cu(NTW, VQ)) void pv_kernel(const PVArgs a) {
  // K-steps of loads in flight per wave (register stages)
  constexpr int DEPTH = VQ == VQ_DENSE ? 2 : PV_QDEPTH;
  constexpr int PITCH = NTW * 32 + 8;            // elements per staged row (16-byte pad)
  constexpr int STAGE = 16 * PITCH;              // elements per staged K-step
  constexpr int CPR = NTW * 4;                   // 16-byte chunks per staged row
  // dense aligned rows are fetched cooperatively: the workgroup's 256 lanes
  // read each K-step's rows as contiguous 16-byte chunks (every 128-byte line
  // by one instruction) and write them into the owning wave's slab, one
  // barrier per K-step.  Per-wave column slabs would split lines between waves
  // and, with non-temporal loads, fetch the split lines twice.
  constexpr bool COOP = VQ == VQ_DENSE && FAST;
  __shared__ __attribute__((aligned(16))) uint16_t stage[4][2][STAGE];
  __shared__ float Ms[32];
  __shared__ float Ps[4][32];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  // blockIdx.y = (batch, group of 32 heads): the MFMA M dimension holds 32
  // heads, so more than 32 heads take one more pass over the latent
  const int cb = blockIdx.x % a.n_cb, c2 = blockIdx.x / a.n_cb, bq = blockIdx.y;
  const int b = bq / a.n_hg, h0 = (bq - b * a.n_hg) * 32;     // batch, first head of the group
  const int tile0 = (cb * 4 + wave) * NTW;                    // first 32-column tile of this wave
  const int nvt = max(0, min(NTW, a.Rvp / 32 - tile0));       // valid tiles (wave-uniform)
  const int col0 = tile0 * 32;
  const int H = a.H;

  if constexpr (FUSED) {
    const int q = tid >> 3, j = tid & 7;
    float m = -INFINITY;
    if (h0 + q < H) m = chunk_max_part(a.chunkmax + ((int64_t)b * H + h0 + q) * a.n_chunk1, a.n_chunk1, j);
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    if (j == 0) Ms[q] = h0 + q < H ? m : 0.f;
    __syncthreads();
  }
  const float Mq = FUSED ? Ms[n] : 0.f;
  const float MqL = -Mq * 1.4426950408889634f;  // exp(l - M) = exp2(l * log2(e) - M * log2(e))
  const bool qok = h0 + n < H;

  const int s_begin = c2 * a.c2_len;
  const int s_end = min(a.S, s_begin + a.c2_len);
  const int nks = (s_end - s_begin + KSTEP - 1) / KSTEP;

  floatx16 acc[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) acc[j] = floatx16{};
  float psum = 0.f;

  // ---- per-lane staging map: chunk c -> (row, 16-byte column chunk) of the
  // 16 x NTW*32 slab (cooperative: of the workgroup's 16 x 4*NTW*32 block;
  // soff then counts from stage[0][buf] and includes the owning wave)
  int goff[NTW], soff[NTW], grow[NTW], gcol[NTW];
  bool cok[NTW];
  const int cb0 = cb * 4 * CPR;                                  // first chunk column of the workgroup
  const int ncol = max(1, min(4 * CPR, a.Rv / 8 - cb0));         // chunk columns it covers (cooperative)
#pragma unroll
  for (int c = 0; c < NTW; ++c) {
    if constexpr (COOP) {
      const int f = min(c * 256 + tid, 16 * ncol - 1);           // lanes past the block repeat its last chunk
      const int row = f / ncol, cc = f % ncol;
      grow[c] = row;
      gcol[c] = (cb0 + cc) * 8;
      goff[c] = 0;
      soff[c] = (cc / CPR) * 2 * STAGE + row * PITCH + (cc % CPR) * 8;
      cok[c] = true;
    } else {
      const int f = c * 64 + lane;
      const int row = f / CPR, c16 = f % CPR;
      grow[c] = row;
      gcol[c] = col0 + c16 * 8;
      goff[c] = row * (int)a.x_ss + gcol[c];
      soff[c] = row * PITCH + c16 * 8;
      cok[c] = (c16 / 4 < nvt) && (gcol[c] < a.Rv);
    }
  }
  if constexpr (COOP) {
    // slab columns past the workgroup's block are never written: zero them
    // once (both buffers), so the discarded output columns stay finite
#pragma unroll 1
    for (int e = lane; e < 2 * 16 * CPR; e += 64) {
      const int bf = e / (16 * CPR), row = (e / CPR) % 16, c16 = e % CPR;
      if (wave * CPR + c16 >= ncol) *(uint4*)&stage[wave][bf][row * PITCH + c16 * 8] = make_uint4(0, 0, 0, 0);
    }
  }
  const VT* xb = (const VT*)a.x + b * a.x_sb + (int64_t)s_begin * a.x_ss;
  // quantised: byte offset of the chunk in its row, its block, int8 or int4, its group
  int qoff[NTW], qg[NTW];
  bool qlo[NTW], q8[NTW];
  const uint8_t* xq = (const uint8_t*)a.x + b * a.x_sb + (int64_t)s_begin * a.x_ss;
  const uint8_t* xq2 = (const uint8_t*)a.x2 + b * a.x2_sb + (int64_t)s_begin * a.x2_ss;
  const uint16_t* sq = (const uint16_t*)a.xs + b * a.xs_sb + (int64_t)s_begin * a.xs_ss;
  const uint16_t* sq2 = (const uint16_t*)a.xs2 + b * a.xs2_sb + (int64_t)s_begin * a.xs2_ss;
#pragma unroll
  for (int c = 0; c < NTW; ++c) {
    qlo[c] = VQ == VQ_BLOCK && gcol[c] >= a.split;
    q8[c] = VQ == VQ_BLOCK && !qlo[c] && a.a_int8;
    qoff[c] = qlo[c] ? (gcol[c] - a.split) / 2 : (q8[c] ? gcol[c] : gcol[c] / 2);
    qg[c] = gcol[c] / 64;
  }
  // dense (aligned) and group-64 loads: 32-bit byte offsets from the chunk's
  // first row, row * pitch by a 24-bit multiply (the host keeps row pitches
  // below 16 MB and a chunk below 2 GB); columns past the slab read column 0
  const uint32_t xp = (uint32_t)(VQ == VQ_DENSE ? a.x_ss * (int64_t)sizeof(VT) : a.x_ss);
  const uint32_t sp = (uint32_t)(a.xs_ss * 2);
  const char* xrow0 = (const char*)a.x + (b * a.x_sb + (int64_t)s_begin * a.x_ss) * (VQ == VQ_DENSE ? (int64_t)sizeof(VT) : 1);
  const char* srow0 = (const char*)a.xs + (b * a.xs_sb + (int64_t)s_begin * a.xs_ss) * 2;
  const char* zrow0 = (const char*)a.xz + (b * a.xs_sb + (int64_t)s_begin * a.xs_ss) * 2;
  uint32_t xco[NTW], sco[NTW];
#pragma unroll
  for (int c = 0; c < NTW; ++c) {
    xco[c] = !cok[c] ? 0u : VQ == VQ_DENSE ? (uint32_t)(gcol[c] * sizeof(VT)) : (uint32_t)qoff[c];
    sco[c] = cok[c] ? (uint32_t)qg[c] * 2 : 0u;
  }

  // Every load of a stage is issued unconditionally from a clamped, in-bounds
  // address: K-steps past the chunk re-read its last K-step, rows past s_end
  // its last row and columns past the slab column 0.  Those values reach only
  // products with P = 0 (positions >= s_end) or discarded output columns, so
  // nothing is zeroed, and with a fixed number of loads per stage (no branch
  // in the loop body) the compiler waits for exactly the older stage
  // (vmcnt(n)) instead of draining every load at the loop head.
  auto load = [&](PVStage<NTW, VQ>& st, int ks) {
    const int kc = min(ks, nks - 1);
    const int rmax = s_end - 1 - s_begin;                   // last valid row of the chunk
    if constexpr (VQ != VQ_DENSE) {
#pragma unroll
      for (int c = 0; c < NTW; ++c) {
        const int64_t r = min(kc * KSTEP + grow[c], rmax);
        if constexpr (VQ == VQ_BLOCK) {
          const bool lo = cok[c] && qlo[c];
          if (FAST) {
            const uint8_t* p = (lo ? xq2 + r * a.x2_ss : xq + r * a.x_ss) + (cok[c] ? qoff[c] : 0);
            st.q[c].x = *(const uint32_t*)p;
            st.q[c].y = *(const uint32_t*)(p + (q8[c] ? 4 : 0));
          } else {
            // rows of any alignment and length: 8 bytes from the chunk's first
            // byte (int4 uses the first 4); bytes past the row are unspecified
            // and land only in output columns >= Rv, which are discarded
            uint32_t w[2];
            ld_row_bytes<8>(lo ? xq2 + r * a.x2_ss : xq + r * a.x_ss, cok[c] ? qoff[c] : 0, lo ? a.x2nb : a.xnb, w);
            st.q[c] = make_uint2(w[0], w[1]);
          }
          st.s[c] = lo ? sq2[r * a.xs2_ss] : sq[r * a.xs_ss];
        } else if constexpr (!FAST) {
          const uint32_t ru = (uint32_t)r, so = __umul24(ru, sp) + sco[c];
          uint32_t w[1];
          ld_row_bytes<4>((const uint8_t*)xrow0 + (__umul24(ru, xp)), xco[c], a.xnb, w);
          st.q[c].x = w[0];
          st.q[c].y = 0;
          st.s[c] = *(const uint16_t*)(srow0 + so);
          st.z[c] = *(const uint16_t*)(zrow0 + so);
        } else {
          const uint32_t ru = (uint32_t)r, so = __umul24(ru, sp) + sco[c];
          st.q[c].x = *(const uint32_t*)(xrow0 + (__umul24(ru, xp) + xco[c]));
          st.q[c].y = 0;
          st.s[c] = *(const uint16_t*)(srow0 + so);
          st.z[c] = *(const uint16_t*)(zrow0 + so);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < NTW; ++c) {
      if constexpr (VQ != VQ_DENSE) break;
      if (FAST) {
        const uint32_t ru = (uint32_t)min(kc * KSTEP + grow[c], rmax);
        st.r[c] = ld_stream16(xrow0 + (__umul24(ru, xp) + xco[c]));
      } else {
        const int s0 = s_begin + ks * KSTEP;
        st.r[c] = make_uint4(0, 0, 0, 0);
        if (cok[c] && s0 + grow[c] < s_end) {
          const VT* p = xb + (int64_t)ks * KSTEP * a.x_ss + goff[c];
          uint16_t tmp[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) tmp[e] = (gcol[c] + e < a.Rv) ? ((const uint16_t*)p)[e] : (uint16_t)0;
          st.r[c] = make_uint4(tmp[0] | (tmp[1] << 16), tmp[2] | (tmp[3] << 16), tmp[4] | (tmp[5] << 16), tmp[6] | (tmp[7] << 16));
        }
      }
    }
    if constexpr (FUSED) {
      // rows past H read row H-1; the logits buffer holds S_pad >= s_end + 8
      // columns; 8 aligned positions never straddle a 32-position tile
      const int sa = s_begin + kc * KSTEP + 8 * hh;
      const float* lp = a.logits + b * a.l_sb + (int64_t)(sa >> 5) * a.l_st + min(h0 + n, H - 1) * a.l_sh + (sa & 31);
      const float4 u = *(const float4*)lp, v = *(const float4*)(lp + 4);
      st.p[0] = u.x; st.p[1] = u.y; st.p[2] = u.z; st.p[3] = u.w;
      st.p[4] = v.x; st.p[5] = v.y; st.p[6] = v.z; st.p[7] = v.w;
    } else {
      const int sa = s_begin + ks * KSTEP + 8 * hh;
      const VT* pp = (const VT*)a.p + b * a.p_sb + min(h0 + n, H - 1) * a.p_sh + sa;
      st.praw = make_uint4(0, 0, 0, 0);
      if (qok && ks < nks) {
        if (a.p_vec && sa + 8 <= s_end) {
          st.praw = *(const uint4*)pp;
        } else {
          uint16_t tmp[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) tmp[e] = sa + e < s_end ? ((const uint16_t*)pp)[e] : (uint16_t)0;
          st.praw = make_uint4(tmp[0] | (tmp[1] << 16), tmp[2] | (tmp[3] << 16), tmp[4] | (tmp[5] << 16), tmp[6] | (tmp[7] << 16));
        }
      }
    }
  };

  // transposed-read addressing: group g = lane/16, rho = lane%16
  const int g = lane >> 4, rho = lane & 15;
  const int tr_off = (8 * hh + (rho >> 2)) * PITCH + 16 * (g & 1) + 4 * (rho & 3);

  auto compute = [&](PVStage<NTW, VQ>& st, int ks, int buf) {
    uint16_t* sbuf = &stage[wave][buf][0];
#pragma unroll
    for (int c = 0; c < NTW; ++c) {
      if constexpr (COOP) {
        *(uint4*)&stage[0][buf][soff[c]] = st.r[c];
      } else if constexpr (VQ == VQ_DENSE) {
        *(uint4*)&sbuf[soff[c]] = st.r[c];
      } else {
        uint4 h = dequant8<VQ>(st.q[c], q8[c], (uint32_t)st.s[c] * 0x10001u,
                               VQ == VQ_G64 ? (uint32_t)st.z[VQ == VQ_G64 ? c : 0] * 0x10001u : 0u);
        if constexpr (__is_same(VT, __bf16)) h = f16x8_to_bf16x8(h);
        *(uint4*)&sbuf[soff[c]] = h;
      }
    }
    float pc[8];
    uint4 praw;
    if constexpr (FUSED) {
#pragma unroll
      for (int e = 0; e < 8; ++e) pc[e] = st.p[e];
    } else {
      praw = st.praw;
    }
    load(st, ks + DEPTH);                   // clamped past the chunk
    if constexpr (COOP) {
      // every wave's chunks of this K-step are in LDS (and every wave has
      // consumed the buffer's previous K-step, two steps ago)
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }

    const int sa = s_begin + ks * KSTEP + 8 * hh;
    float pv[8];
    if constexpr (FUSED) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // computed for every lane and selected (the logits past s_end are
        // unwritten workspace: their exponentials are discarded)
        const float ex = __builtin_amdgcn_exp2f(fmaf(pc[e], 1.4426950408889634f, MqL));
        pv[e] = (qok && sa + e < s_end) ? ex : 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) psum += pv[e];
    } else {
      const uint32_t w[4] = {praw.x, praw.y, praw.z, praw.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint16_t u = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
        pv[e] = to_f32(__builtin_bit_cast(VT, u));
      }
    }

    const uint16_t* sb = sbuf + tr_off;
    if constexpr (__is_same(VT, _Float16)) {
      half8 A;
#pragma unroll
      for (int e = 0; e < 8; ++e) A[e] = (_Float16)pv[e];
#pragma unroll
      for (int j = 0; j < NTW; ++j) {
        if (j < nvt) {
          const uint2 lo = lds_read_tr16(sb + 32 * j);
          const uint2 hi = lds_read_tr16(sb + 32 * j + 4 * PITCH);
          acc[j] = mfma_f16(A, __builtin_bit_cast(half8, make_uint4(lo.x, lo.y, hi.x, hi.y)), acc[j]);
        }
      }
    } else {
      bf16x8 Ah, Al;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const __bf16 h = (__bf16)pv[e];
        Ah[e] = h;
        Al[e] = (__bf16)(pv[e] - (float)h);
      }
#pragma unroll
      for (int j = 0; j < NTW; ++j) {
        if (j < nvt) {
          const uint2 lo = lds_read_tr16(sb + 32 * j);
          const uint2 hi = lds_read_tr16(sb + 32 * j + 4 * PITCH);
          const bf16x8 Bv = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
          acc[j] = mfma_bf16(Ah, Bv, acc[j]);
          acc[j] = mfma_bf16(Al, Bv, acc[j]);
        }
      }
    }
  };

  if ((COOP || nvt > 0) && nks > 0) {       // cooperative: every wave takes part in the barriers
    // K-steps in groups of DEPTH, each stage loaded DEPTH steps ahead; the
    // last group computes up to DEPTH - 1 K-steps past the chunk with P = 0
    // (no branch in the loop body)
    PVStage<NTW, VQ> st[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load(st[d], d);
    for (int ks = 0; ks < nks; ks += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) compute(st[d], ks + d, (ks + d) & 1);
    }
  }

  // ---- this chunk's partial sums: D[row q][col] -> part[bq][c2][q][col] (one
  // contiguous 32 x Rvp block per workgroup row of the grid).  Fused fp16
  // partials are divided by the head's softmax sum over the chunk (the same
  // in every wave: all waves form the same P): a convex combination of V
  // rows, so fp16 holds it without overflow or underflow into subnormals.
  const int Rvp = a.Rvp;
  if constexpr (FUSED) {
    const float ps = add_halves(psum);
    if (hh == 0) Ps[wave][n] = ps;
    __syncthreads();
    if (cb == 0 && tid < 32) a.psum[((int64_t)bq * a.n_c2 + c2) * 32 + tid] = Ps[0][tid];
  }
  if (FUSED && a.part16) {
    _Float16* part = (_Float16*)a.part + (((int64_t)bq * a.n_c2 + c2) * 32) * Rvp;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int q = 8 * (v >> 2) + 4 * hh + (v & 3);
      const float sq = Ps[wave][q];
      const float inv = sq > 0.f ? 1.0f / sq : 0.f;
#pragma unroll
      for (int j = 0; j < NTW; ++j)
        if (j < nvt)
          part[(int64_t)q * Rvp + col0 + 32 * j + (VQ == VQ_G64 ? pv_g64_rank(n) : n)] = (_Float16)(acc[j][v] * inv);
    }
    return;
  }
  float* part = a.part + (((int64_t)bq * a.n_c2 + c2) * 32) * Rvp;
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    if (j < nvt) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int q = 8 * (v >> 2) + 4 * hh + (v & 3);
        part[(int64_t)q * Rvp + col0 + 32 * j + (VQ == VQ_G64 ? pv_g64_rank(n) : n)] = acc[j][v];
      }
    }
  }
}

// Fused quantised P.V over all columns of the V latent in one workgroup.
//
// 8 waves split the column tiles (NTW each, Rvp <= 8 * NTW * 32), so a
// K-step's logits and scale / zero rows are fetched once per (chunk, batch,
// head group) instead of once per column block (blocks of one chunk run on
// different XCDs, each fetching them through its own L2), and the K-step's
// 32 x 16 exponentials are formed once instead of by every wave: thread
// (eh, head en, ee) forms P[en][8 eh + ee] and writes it into a
// double-buffered LDS A operand that every wave reads with one 16-byte load
// (the A layout of pv_kernel: lane (n, hh) holds positions 8 hh .. 8 hh + 7 of
// head n).  The K-step's scale / zero rows take the same route (at most two
// 16-bit loads per thread), so the global loads of a wave are its packed
// bytes.  Buffers of K-step ks+1 are written while K-step ks computes; one
// barrier per K-step publishes them.  X_v slabs stay wave-private as in
// pv_kernel (dequantised by the loading lane, read back transposed).
template <int NTW>
struct PVWStage {
  uint2 q[8];          // packed bytes of the lane's 8 chunks (int4: .x)
  float p;             // the thread's logit
  uint16_t sz[2];      // the thread's scale / zero items
};

template <typename VT, int NTW, bool FAST, int VQ>
__global__ __launch_bounds__(512, 1) void pv_wide_kernel(const PVArgs a) {
  constexpr int NWV = 8, DEPTH = PV_WDEPTH;
  constexpr int PITCH = NTW * 32 + 8;            // elements per staged row (16-byte pad)
  constexpr int STAGE = 16 * PITCH;              // elements per staged K-step
  constexpr int CPR = NTW * 4;                   // 8-rank chunks per staged row
  constexpr bool BF = __is_same(VT, __bf16);
  constexpr int NA = BF ? 2 : 1;                 // A operand pieces (bf16: high and low parts)
  static_assert(VQ != VQ_DENSE, "quantised latents only");
  __shared__ __attribute__((aligned(16))) uint16_t stage[NWV][2][STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t Ash[2][NA][512];   // [buf][piece][eh][en][ee]
  // scale / zero rows of a K-step, bits in both halves of a word: per
  // (group or block g, row parity hh) a 20-word block holding (scale, zero) of
  // rows hh, hh + 2, ..., hh + 14 -- the rows of a lane's chunks -- so a lane
  // reads its 16 words with four 16-byte loads (the 4 pad words keep the
  // groups of a half-wave on distinct banks)
  __shared__ __attribute__((aligned(16))) uint32_t Ssh[2][64 * 20];
  __shared__ float Ms[32];
  __shared__ float Ps2[2][32];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  const int c2 = blockIdx.x, bq = blockIdx.y;
  const int b = bq / a.n_hg, h0 = (bq - b * a.n_hg) * 32;    // batch, first head of the group
  const int tile0 = wave * NTW;                               // first 32-column tile of this wave
  const int nvt = max(0, min(NTW, a.Rvp / 32 - tile0));       // valid tiles (wave-uniform)
  const int col0 = tile0 * 32;
  const int H = a.H;
  const int eh = tid >> 8, en = (tid >> 3) & 31, ee = tid & 7;

  if (tid < 256) {
    const int q = tid >> 3, j = tid & 7;
    float m = -INFINITY;
    if (h0 + q < H) m = chunk_max_part(a.chunkmax + ((int64_t)b * H + h0 + q) * a.n_chunk1, a.n_chunk1, j);
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    if (j == 0) Ms[q] = h0 + q < H ? m : 0.f;
  }
  __syncthreads();
  const float MqL = -Ms[en] * 1.4426950408889634f;   // exp(l - M) = exp2(l * log2(e) - M * log2(e))
  const bool eok = h0 + en < H;

  const int s_begin = c2 * a.c2_len;
  const int s_end = min(a.S, s_begin + a.c2_len);
  const int nks = (s_end - s_begin + KSTEP - 1) / KSTEP;
  const int rmax = s_end - 1 - s_begin;                        // last valid row of the chunk

  floatx16 acc[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) acc[j] = floatx16{};
  float psum = 0.f;

  // ---- per-lane chunk map: lane (n, hh) takes the 8-rank column chunk n of
  // the wave's slab in rows 2c + hh, c = 0..7 (NCH chunks).  One load
  // instruction then reads 4*CPR contiguous bytes of each of two rows, and
  // the lane's column, scale group and slab offset are the same for every
  // chunk.  Lanes past the slab (n >= CPR) load column 0 and store into the
  // row's pad, which is never read.
  constexpr int NCH = 8;
  const int c16 = min(n, CPR);
  const int gcol = col0 + c16 * 8;
  const bool cok = n < CPR && c16 / 4 < nvt && gcol < a.Rv;
  const bool qlo = VQ == VQ_BLOCK && gcol >= a.split;
  const bool q8 = VQ == VQ_BLOCK && !qlo && a.a_int8;
  const int qoff = !cok ? 0 : qlo ? (gcol - a.split) / 2 : (q8 ? gcol : gcol / 2);
  // scale column of the chunk in the staged rows: group-64 int4 its group,
  // block formats its block (0 upper, 1 lower)
  const int qsel = VQ == VQ_G64 ? min(gcol / 64, 31) : (qlo ? 1 : 0);
  const int soff0 = hh * PITCH + c16 * 8;          // slab offset of chunk 0 (row hh)
  const uint8_t* xq = (const uint8_t*)a.x + b * a.x_sb + (int64_t)s_begin * a.x_ss;
  const uint8_t* xq2 = (const uint8_t*)a.x2 + b * a.x2_sb + (int64_t)s_begin * a.x2_ss;
  // Offsets from a stream's first row of the chunk are 32-bit, rows by a
  // 24-bit multiply: the host takes this kernel only when every row pitch is
  // below 16 MB, and keeps a chunk below 2 GB.  (64-bit row products cost
  // quarter-rate multiplies per chunk and K-step.)
  const uint32_t xp = (uint32_t)a.x_ss, xp2 = (uint32_t)a.x2_ss;

  // ---- scale / zero items of a K-step: nsz per row (group-64: ng scales then
  // ng zero points; block formats: the upper block's scale, the lower's);
  // thread item f = row * nsz + k for f = tid, tid + 512
  const int ng = VQ == VQ_G64 ? (a.Rv + 63) / 64 : 0;
  const int nsz = VQ == VQ_G64 ? 2 * ng : (a.split < a.Rv ? 2 : 1);
  int zrow[2], zsel[2], zg[2];
  bool zok[2];
  const uint16_t* zsrc[2];
  uint32_t zpitch[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int f0 = tid + 512 * u;
    zok[u] = f0 < 16 * nsz;
    const int f = min(f0, 16 * nsz - 1);
    zrow[u] = f / nsz;
    const int k = f % nsz;
    if constexpr (VQ == VQ_G64) {
      zsel[u] = k >= ng;
      zg[u] = k - zsel[u] * ng;
      zsrc[u] = (const uint16_t*)(zsel[u] ? a.xz : a.xs) + b * a.xs_sb + (int64_t)s_begin * a.xs_ss + zg[u];
      zpitch[u] = (uint32_t)a.xs_ss;
    } else {
      zsel[u] = 0;
      zg[u] = k;
      zsrc[u] = k ? (const uint16_t*)a.xs2 + b * a.xs2_sb + (int64_t)s_begin * a.xs2_ss
                  : (const uint16_t*)a.xs + b * a.xs_sb + (int64_t)s_begin * a.xs_ss;
      zpitch[u] = (uint32_t)(k ? a.xs2_ss : a.xs_ss);
    }
  }
  const float* lrow = a.logits + b * a.l_sb + min(h0 + en, H - 1) * a.l_sh;

  // Every load is issued from a clamped, in-bounds address (K-steps past the
  // chunk re-read its last K-step, rows past s_end its last row, chunks past
  // the slab column 0); those values meet P = 0 or discarded columns only.
  // The logit and the scale / zero items go first: they are consumed one
  // K-step before the packed bytes of the same stage.
  auto load = [&](PVWStage<NTW>& st, int ks) {
    const int kc = min(ks, nks - 1);
    // the logits buffer holds S_pad >= round_up(s_end, 16) positions
    const int sa = s_begin + kc * KSTEP + 8 * eh + ee;
    st.p = lrow[__umul24((uint32_t)(sa >> 5), (uint32_t)a.l_st) + (uint32_t)(sa & 31)];
#pragma unroll
    for (int u = 0; u < 2; ++u) st.sz[u] = zsrc[u][__umul24((uint32_t)min(kc * KSTEP + zrow[u], rmax), zpitch[u])];
    const bool lo = VQ == VQ_BLOCK && cok && qlo;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const uint32_t r = (uint32_t)min(kc * KSTEP + 2 * c + hh, rmax);
      if (FAST) {
        // one unsigned 32-bit offset from the stream's (uniform) base
        const uint32_t o = (lo ? __umul24(r, xp2) : __umul24(r, xp)) + (uint32_t)qoff;
        const uint8_t* base = lo ? xq2 : xq;
        st.q[c].x = *(const uint32_t*)(base + o);
        st.q[c].y = (VQ == VQ_BLOCK && q8) ? *(const uint32_t*)(base + (o + 4u)) : 0u;
      } else {
        const uint8_t* rowp = lo ? xq2 + __umul24(r, xp2) : xq + __umul24(r, xp);
        // rows of any alignment and length; bytes past the row land only in
        // output columns >= Rv, which are discarded
        if constexpr (VQ == VQ_BLOCK) {
          uint32_t w[2];
          ld_row_bytes<8>(rowp, qoff, lo ? a.x2nb : a.xnb, w);
          st.q[c] = make_uint2(w[0], w[1]);
        } else {
          uint32_t w[1];
          ld_row_bytes<4>(rowp, qoff, a.xnb, w);
          st.q[c] = make_uint2(w[0], 0u);
        }
      }
    }
  };

  // the exponentials of K-step ks (logits loaded with st) into Ash[ks & 1]
  auto publish_p = [&](const PVWStage<NTW>& st, int ks) {
    const int buf = ks & 1;
    const int sp = s_begin + ks * KSTEP + 8 * eh + ee;
    // computed for every thread and selected (logits past s_end are other
    // chunks' or unwritten workspace)
    const float ex = __builtin_amdgcn_exp2f(fmaf(st.p, 1.4426950408889634f, MqL));
    const float pv = (eok && sp < s_end) ? ex : 0.f;
    psum += pv;
    if constexpr (BF) {
      const __bf16 hi = (__bf16)pv;
      Ash[buf][0][tid] = __builtin_bit_cast(uint16_t, hi);
      Ash[buf][NA - 1][tid] = __builtin_bit_cast(uint16_t, (__bf16)(pv - (float)hi));
    } else {
      Ash[buf][0][tid] = __builtin_bit_cast(uint16_t, (_Float16)pv);
    }
  };
  // the scale / zero items of K-step ks (loaded with st) into Ssh[ks & 1]
  auto publish_sz = [&](const PVWStage<NTW>& st, int ks) {
    const int buf = ks & 1;
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (zok[u]) Ssh[buf][(2 * zg[u] + (zrow[u] & 1)) * 20 + (zrow[u] >> 1) * 2 + zsel[u]] = (uint32_t)st.sz[u] * 0x10001u;
  };
  // the (scale, zero) words of this lane's chunks of K-step ks, from Ssh[ks & 1]
  auto read_scales = [&](int ks, uint4 (&sz)[4]) {
    const uint32_t* p = &Ssh[ks & 1][(2 * qsel + hh) * 20];
#pragma unroll
    for (int k = 0; k < 4; ++k) sz[k] = *(const uint4*)(p + 4 * k);
  };
  // K-step ks's packed bytes (in st) dequantised with its scale words into
  // the wave's slab ks & 1
  auto dequant = [&](const PVWStage<NTW>& st, int ks, const uint4 (&sz)[4]) {
    const int buf = ks & 1;
    uint16_t* sbuf = &stage[wave][buf][0];
    uint32_t s2[NCH], z2[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      s2[c] = (c & 1) ? sz[c >> 1].z : sz[c >> 1].x;
      z2[c] = VQ == VQ_G64 ? ((c & 1) ? sz[c >> 1].w : sz[c >> 1].y) : 0u;
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      uint4 h = dequant8<VQ>(st.q[c], q8, s2[c], z2[c]);
      if constexpr (BF) h = f16x8_to_bf16x8(h);
      *(uint4*)&sbuf[soff0 + 2 * c * PITCH] = h;
    }
  };

  // transposed-read addressing: group g = lane/16, rho = lane%16
  const int g = lane >> 4, rho = lane & 15;
  const int tr_off = (8 * hh + (rho >> 2)) * PITCH + 16 * (g & 1) + 4 * (rho & 3);

  // the MFMAs of K-step ks: A from Ash[ks & 1], B from the slab ks & 1.
  // Every tile of the slab is multiplied (tiles past nvt hold finite data and
  // are never stored), so the iteration is one basic block and the compiler
  // can interleave these MFMAs with the next K-step's dequantisation.
  auto mfmas = [&](int ks) {
    const int buf = ks & 1;
    uint4 Araw[NA];
#pragma unroll
    for (int k = 0; k < NA; ++k) Araw[k] = *(const uint4*)&Ash[buf][k][8 * lane];
    const uint16_t* sb = &stage[wave][buf][0] + tr_off;
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      const uint2 lo = lds_read_tr16(sb + 32 * j);
      const uint2 hi = lds_read_tr16(sb + 32 * j + 4 * PITCH);
      const uint4 bv = make_uint4(lo.x, lo.y, hi.x, hi.y);
      if constexpr (BF) {
        acc[j] = mfma_bf16(__builtin_bit_cast(bf16x8, Araw[0]), __builtin_bit_cast(bf16x8, bv), acc[j]);
        acc[j] = mfma_bf16(__builtin_bit_cast(bf16x8, Araw[NA - 1]), __builtin_bit_cast(bf16x8, bv), acc[j]);
      } else {
        acc[j] = mfma_f16(__builtin_bit_cast(half8, Araw[0]), __builtin_bit_cast(half8, bv), acc[j]);
      }
    }
  };

  // Software pipeline over K-steps, DEPTH register stages (stage k in
  // st[k % DEPTH]).  Iteration k multiplies K-step k (its slab written by
  // this wave in iteration k-1) while the wave dequantises K-step k+1, forms
  // its exponentials and publishes the scale rows of K-step k+2; then it
  // loads K-step k+1+DEPTH into the registers K-step k+1 freed and barriers.
  // The last group runs up to DEPTH - 1 iterations past the chunk with P = 0
  // (clamped loads, no branch in the loop body).
  if (nks > 0) {                             // uniform: every wave takes part in the barriers
    PVWStage<NTW> st[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load(st[d], d);
    publish_p(st[0], 0);
    publish_sz(st[0], 0);
    __syncthreads();
    {
      uint4 sz[4];
      read_scales(0, sz);
      dequant(st[0], 0, sz);
    }
    publish_sz(st[1], 1);
    load(st[0], DEPTH);
    __syncthreads();                         // Ssh[1] published; Ssh[0] consumed
    for (int ks = 0; ks < nks; ks += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int k = ks + d;
        PVWStage<NTW>& cur = st[(d + 1) % DEPTH];          // K-step k+1
        uint4 sz[4];
        read_scales(k + 1, sz);                            // first: the dequantisation waits for them
        mfmas(k);
        dequant(cur, k + 1, sz);
        publish_p(cur, k + 1);
        publish_sz(st[(d + 2) % DEPTH], k + 2);            // K-step k+2's items
        load(cur, k + 1 + DEPTH);
        __syncthreads();
      }
    }
  }

  // ---- the chunk's softmax sums per head, then its partial sums (as in
  // pv_kernel's fused mode)
  psum += __shfl_xor(psum, 1, 64);
  psum += __shfl_xor(psum, 2, 64);
  psum += __shfl_xor(psum, 4, 64);
  if (ee == 0) Ps2[eh][en] = psum;
  __syncthreads();
  if (tid < 32) a.psum[((int64_t)bq * a.n_c2 + c2) * 32 + tid] = Ps2[0][tid] + Ps2[1][tid];
  const int Rvp = a.Rvp;
  if (a.part16) {
    _Float16* part = (_Float16*)a.part + (((int64_t)bq * a.n_c2 + c2) * 32) * Rvp;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int q = 8 * (v >> 2) + 4 * hh + (v & 3);
      const float sq = Ps2[0][q] + Ps2[1][q];
      const float inv = sq > 0.f ? 1.0f / sq : 0.f;
#pragma unroll
      for (int j = 0; j < NTW; ++j)
        if (j < nvt)
          part[(int64_t)q * Rvp + col0 + 32 * j + (VQ == VQ_G64 ? pv_g64_rank(n) : n)] = (_Float16)(acc[j][v] * inv);
    }
    return;
  }
  float* part = a.part + (((int64_t)bq * a.n_c2 + c2) * 32) * Rvp;
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    if (j < nvt) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int q = 8 * (v >> 2) + 4 * hh + (v & 3);
        part[(int64_t)q * Rvp + col0 + 32 * j + (VQ == VQ_G64 ? pv_g64_rank(n) : n)] = acc[j][v];
      }
    }
  }
}

// Fused group-64 int4 P.V over all columns, with the V latent staged raw.
//
// As pv_wide_kernel (one workgroup over all column tiles of one position
// chunk, each K-step's exponentials formed once and shared through LDS), but
// the packed rows go to LDS as they are and are dequantised after a
// transposed read, so LDS carries 1 byte per latent element instead of 4
// (the fp16 value written and read back).  8 waves serve 33..64 column tiles,
// 4 waves up to 16.
// * a K-step is 32 positions; the workgroup copies their rows (ranks padded
//   to whole 64-rank groups) into a ring of four LDS stages with
//   buffer_load_dword ... lds, or buffer_load_dwordx4 ... lds for rows of
//   whole aligned 16-byte pieces, one descriptor per K-step whose range ends
//   at the chunk's last row, so the copy needs no registers and no address
//   arithmetic per K-step;
// * wave w owns whole groups (two 32-column tiles each, the groups shared out
//   so that the two waves of a SIMD hold 14 or fewer tiles at Rv 1640) and
//   reads a tile with one ds_read_b64_tr_b4, the gfx950 transposed 4-bit
//   read: within a 16-lane group, lane j receives nibble j of the 8 bytes
//   each of the 16 lanes addresses (element i from lane i).  Lane (n, hh)
//   addresses row 16 hh + n % 16, ranks 16 (n / 16) .. +15 of the tile, so it
//   receives column n at rows 16 hh + 0..15: the B operands of two 32x32x16
//   MFMAs (rows 16 hh + 0..7, then 16 hh + 8..15);
// * the nibbles are dequantised there to the exact fp16(n * s + z) of the
//   other kernels: masked into bytes (the even rows' nibbles, then the odd
//   rows'), two bytes at a time go through v_cvt_scalef32_pk_f16_fp8 with
//   scale 512 -- a byte n <= 15 read as fp8 e4m3 is exactly n / 512 (n < 8
//   subnormal, 8..15 normal), so each pair becomes the exact fp16 pair (n_a,
//   n_b) -- and one packed FMA applies the pair's scales and zero points,
//   rounding once.  The pairs come out as rows 0 2 4 6 1 3 5 7 of each 8, the
//   K order of the MFMA, which the A operand (P) and the staged scale / zero
//   pairs follow.
// Logits and scale / zero items go through registers two K-steps ahead and
// are published (exponentials, transposed scale pairs) one K-step ahead;
// one barrier per K-step.
constexpr int PVN_KS = 32;                       // positions per K-step

__device__ inline uint2 lds_read_tr4(const uint8_t* p) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  const v2i r = __builtin_amdgcn_ds_read_tr4_b64_v2i32((__attribute__((address_space(3))) v2i*)(p));
  return make_uint2((uint32_t)r.x, (uint32_t)r.y);
}

// the LDS row pitch of the raw stage for ngp 64-rank groups: whole groups
// plus 8 bytes, an odd multiple of 8, so the 16 rows of one transposed read
// fall on distinct banks; with 16-byte copies (D16) whole groups plus 16
// bytes, an odd multiple of 16 (distinct banks over 256 bytes)
__host__ __device__ constexpr int pvn_pitch(int ngp, bool d16 = false) { return 32 * ngp + (d16 ? 16 : 8); }

// Workgroup shapes: NWV waves of up to NGW groups each -- 8 x 4 for 33..64
// column tiles (one workgroup per CU), 4 x 2 for up to 16 tiles (three per
// CU).  NJ copy instructions per wave and K-step (CB bytes per lane: 4, or 16
// for 16-byte aligned rows of whole 16-byte chunks, D16, at most 31 groups)
// fill a stage of 32 rows (padded to whole instructions); a thread forms PPT
// exponentials and loads ZS scale items per K-step.
template <int NWV, int NGW, bool D16 = false> struct PVNGeom {
  static constexpr int GMAX = NWV * NGW;
  static constexpr int CB = D16 ? 16 : 4;
  static constexpr int NJ = (32 * pvn_pitch(D16 ? GMAX - 1 : GMAX, D16) + 64 * CB * NWV - 1) / (64 * CB * NWV);
  static constexpr int STAGE = NJ * NWV * 64 * CB;
  static constexpr int PPT = 1024 / (64 * NWV);
  static constexpr int TPH = 32 / PPT;             // threads per head
  static constexpr int ZS = (32 * GMAX + 64 * NWV - 1) / (64 * NWV);
  static constexpr int WGS = NWV == 8 ? 1 : 3;     // workgroups per CU (LDS)
};

template <typename VT, int NWV, int NGW, bool D16>
__global__ __launch_bounds__(NWV * 64, (PVNGeom<NWV, NGW, D16>::WGS)) void pv_nib_kernel(const PVArgs a) {
  typedef PVNGeom<NWV, NGW, D16> G;
  constexpr int CB = G::CB;
  constexpr bool BF = __is_same(VT, __bf16);
  constexpr int NA = BF ? 2 : 1;
  constexpr int NJ = G::NJ, PPT = G::PPT, TPH = G::TPH, ZS = G::ZS, GMAX = G::GMAX;
  typedef __attribute__((address_space(3))) void lds_void;
  // four raw stages, separate arrays so that the compiler sees a stage's
  // reads apart from the copies in flight into the others
  __shared__ __attribute__((aligned(16))) uint8_t V0[G::STAGE], V1[G::STAGE], V2[G::STAGE], V3[G::STAGE];
  // A operands: [buf][piece][mfma m][lane * 8 + e], e the K order 0 2 4 6 1 3 5 7
  __shared__ __attribute__((aligned(16))) uint16_t Ash[2 * NA * 1024];
  // scale / zero pairs per (buf, group, row half hh): 16 words, word
  // 8 m + 4 z + k holding the scales (z = 0) or zero points (z = 1) of the
  // two rows of pair k of MFMA m (rows 16 hh + 8 m + {0,2}, {4,6}, {1,3}, {5,7})
  __shared__ __attribute__((aligned(16))) uint16_t Ssh[2 * GMAX * 2 * 32];
  __shared__ float Ms[32];
  __shared__ float Ps[32];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  const int c2 = blockIdx.x, bq = blockIdx.y;
  const int b = bq / a.n_hg, h0 = (bq - b * a.n_hg) * 32;
  const int H = a.H;

  if (tid < 256) {
    const int q = tid >> 3, j = tid & 7;
    float m = -INFINITY;
    if (h0 + q < H) m = chunk_max_part(a.chunkmax + ((int64_t)b * H + h0 + q) * a.n_chunk1, a.n_chunk1, j);
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    if (j == 0) Ms[q] = h0 + q < H ? m : 0.f;
  }
  __syncthreads();

  const int s_begin = c2 * a.c2_len;
  const int s_end = min(a.S, s_begin + a.c2_len);
  const int len = s_end - s_begin;
  const int nks = (len + PVN_KS - 1) / PVN_KS;
  const int ngp = (a.Rvp + 63) / 64;             // 64-rank groups (the last may be half a group)
  const int PB = pvn_pitch(ngp, D16);
  // CB-byte pieces of a packed row (Rv a multiple of 8; D16: the host checked
  // that the row pitch holds whole 16-byte pieces)
  const int ndw = (a.Rv / 2 + CB - 1) / CB;

  // ---- this wave's groups: ngp / NWV each, one more for the first
  // ngp % NWV waves (with 8 waves, waves w and w + 4 share a SIMD)
  const int gbase = ngp / NWV, grem = ngp % NWV;
  const int ngw = gbase + (wave < grem ? 1 : 0);
  const int g0 = wave * gbase + min(wave, grem);
  const int ntile = a.Rvp / 32;

  // ---- copy plan: a stage is 32 rows of PB bytes plus padding to whole
  // instructions (NJ of 64 CB bytes per wave); instruction m = wave + NWV j
  // writes stage bytes [64 CB m, 64 CB (m + 1)), lane i's piece D = 64 m + i
  // being row D / (PB / CB), piece D % (PB / CB) of the row (pad pieces
  // re-read the row's last piece).  A K-step's descriptor ends at its last
  // row, so rows past the chunk and the slots past row 31 read zeros (out of
  // range: no memory access) -- every wave issues the same NJ copies.
  const int PBd = PB / CB;
  uint32_t voff[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int D = 64 * (wave + NWV * j) + lane;
    const int r = D / PBd;
    voff[j] = (uint32_t)r * (uint32_t)a.x_ss + (uint32_t)CB * (uint32_t)min(D - r * PBd, ndw - 1);
  }
  const uint8_t* xq = (const uint8_t*)a.x + b * a.x_sb + (int64_t)s_begin * a.x_ss;
  const uint32_t xp = (uint32_t)a.x_ss;
  auto copy = [&](uint8_t* st, int ks) {
    const int rows = max(0, min(PVN_KS, len - ks * PVN_KS));
    // (uniform; readfirstlane keeps the descriptor in scalar registers)
    const uint64_t base = (uint64_t)(xq + (int64_t)min(ks, nks - 1) * PVN_KS * a.x_ss);
    const uint64_t bu = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)bu, (short)0, __builtin_amdgcn_readfirstlane((int)((uint32_t)rows * xp)), 0x00020000);
    // (the device pass only: the host pass rejects the 16-byte form, a gfx950
    // feature, and would then drop this instantiation's launch stub)
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(st + 64 * CB * (wave + NWV * j)), CB, voff[j], 0, 0, 0);
#endif
  };

  // ---- logits: thread (head eh, ej) takes positions PPT ej .. PPT ej + PPT - 1
  const int eh = tid / TPH, ej = tid % TPH;
  const bool hok = h0 + eh < H;
  const float MqL = -Ms[eh] * 1.4426950408889634f;
  // uniform bases with 32-bit lane offsets (the loads take the scalar-base form)
  const char* lbase = (const char*)(a.logits + b * a.l_sb + (int64_t)h0 * a.l_sh);
  const uint32_t loff = 4u * (uint32_t)(min(eh, H - 1 - h0) * (int)a.l_sh + PPT * ej);
  const uint32_t lst = 4u * (uint32_t)a.l_st;    // bytes per logit tile (32 positions of every head)
  const int tile_s0 = s_begin >> 5;              // c2_len is a multiple of 32
  // Ash slots (fp16 units, without buf / piece) of the thread's positions
  int aslot[PPT];
#pragma unroll
  for (int u = 0; u < PPT; ++u) {
    const int p = PPT * ej + u, q = p & 15, q8 = q & 7;
    aslot[u] = (q >> 3) * 512 + (eh + 32 * (p >> 4)) * 8 + (q8 >> 1) + 4 * (q8 & 1);
  }
  // ---- scale / zero items: slot u < ZS of the thread is item f = tid +
  // 64 NWV u of [row][g] (32 x ng items), whose scale and zero point it loads
  const int ng = (a.Rv + 63) / 64;
  const char* sbase = (const char*)a.xs + 2 * (b * a.xs_sb + (int64_t)s_begin * a.xs_ss);
  const char* zbase = (const char*)a.xz + 2 * (b * a.xs_sb + (int64_t)s_begin * a.xs_ss);
  const uint32_t zp = 2u * (uint32_t)a.xs_ss;
  int zrg[ZS], zdst[ZS];                         // row * 64 + g; the scale's u16 index within a buffer (-1: none)
#pragma unroll
  for (int u = 0; u < ZS; ++u) {
    const int f0 = tid + 64 * NWV * u;
    const int f = min(f0, 32 * ng - 1);
    const int row = f / ng, g = f - row * ng;
    zrg[u] = row * 64 + g;
    const int q = row & 15, q8 = q & 7;
    const int word = 8 * (q >> 3) + 2 * (q8 & 1) + (q8 >> 2);     // the zero point: word + 4
    zdst[u] = f0 < 32 * ng ? ((g * 2 + (row >> 4)) * 16 + word) * 2 + ((q8 >> 1) & 1) : -1;
  }

  typedef float lvec __attribute__((ext_vector_type(PPT)));
  struct Regs { lvec l; uint16_t z[2 * ZS]; };   // z: the slots' scales, then their zero points
  auto load = [&](Regs& R, int ks) {
    const int kc = min(ks, nks - 1);
    R.l = *(const lvec*)(lbase + ((uint32_t)(tile_s0 + kc) * lst + loff));
#pragma unroll
    for (int u = 0; u < ZS; ++u) {
      const uint32_t o = (uint32_t)min(kc * PVN_KS + (zrg[u] >> 6), len - 1) * zp + 2u * (uint32_t)(zrg[u] & 63);
      R.z[u] = *(const uint16_t*)(sbase + o);
      R.z[ZS + u] = *(const uint16_t*)(zbase + o);
    }
  };
  float psum = 0.f;
  auto publish = [&](const Regs& R, int ks) {
    const int buf = ks & 1;
    uint16_t* ab = &Ash[buf * NA * 1024];
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      const float ex = __builtin_amdgcn_exp2f(fmaf(R.l[u], 1.4426950408889634f, MqL));
      const float pv = (hok && ks * PVN_KS + PPT * ej + u < len) ? ex : 0.f;
      psum += pv;
      if constexpr (BF) {
        const __bf16 hi = (__bf16)pv;
        ab[aslot[u]] = __builtin_bit_cast(uint16_t, hi);
        ab[1024 + aslot[u]] = __builtin_bit_cast(uint16_t, (__bf16)(pv - (float)hi));
      } else {
        ab[aslot[u]] = __builtin_bit_cast(uint16_t, (_Float16)pv);
      }
    }
    uint16_t* sd = &Ssh[buf * GMAX * 64];
#pragma unroll
    for (int u = 0; u < ZS; ++u)
      if (zdst[u] >= 0) {
        sd[zdst[u]] = R.z[u];
        sd[zdst[u] + 8] = R.z[ZS + u];
      }
  };

  floatx16 acc[2 * NGW];
#pragma unroll
  for (int j = 0; j < 2 * NGW; ++j) acc[j] = floatx16{};

  // transposed-read address of the lane within a stage (tile 0)
  const int tr_off = (16 * hh + (lane & 15)) * PB + 8 * ((lane >> 4) & 1);

  auto compute = [&](const uint8_t* st, int ks) {
    const int buf = ks & 1;
    uint4 A[2][NA];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int p = 0; p < NA; ++p) A[m][p] = *(const uint4*)&Ash[(buf * NA + p) * 1024 + m * 512 + 8 * lane];
    const uint8_t* sb = st + tr_off;
#pragma unroll
    for (int gi = 0; gi < NGW; ++gi) {
      if (gi < ngw) {
        const int g = g0 + gi;
        const uint4* sp = (const uint4*)&Ssh[((buf * GMAX + g) * 2 + hh) * 32];
        const uint4 S0 = sp[0], Z0 = sp[1], S1 = sp[2], Z1 = sp[3];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const uint2 w = lds_read_tr4(sb + 32 * g + 16 * t);
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            const uint32_t wm = m ? w.y : w.x;
            const uint4 S = m ? S1 : S0, Z = m ? Z1 : Z0;
            const uint32_t lo = wm & 0x0F0F0F0Fu, hi = (wm >> 4) & 0x0F0F0F0Fu;
            const h2v nv[4] = {__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, false),
                               __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, true),
                               __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, false),
                               __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, true)};
            const uint32_t sk[4] = {S.x, S.y, S.z, S.w}, zk[4] = {Z.x, Z.y, Z.z, Z.w};
            uint32_t o[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
              o[k] = as_u32(__builtin_elementwise_fma(nv[k], as_h2(sk[k]), as_h2(zk[k])));
            uint4 bv = make_uint4(o[0], o[1], o[2], o[3]);
            if constexpr (BF) {
              bv = f16x8_to_bf16x8(bv);
              acc[2 * gi + t] = mfma_bf16(__builtin_bit_cast(bf16x8, A[m][0]), __builtin_bit_cast(bf16x8, bv), acc[2 * gi + t]);
              acc[2 * gi + t] = mfma_bf16(__builtin_bit_cast(bf16x8, A[m][NA - 1]), __builtin_bit_cast(bf16x8, bv), acc[2 * gi + t]);
            } else {
              acc[2 * gi + t] = mfma_f16(__builtin_bit_cast(half8, A[m][0]), __builtin_bit_cast(half8, bv), acc[2 * gi + t]);
            }
          }
        }
      }
    }
  };

  // ---- software pipeline: copies three K-steps ahead (stage k % 4),
  // register loads two ahead (set k & 1), publication one ahead.  Iteration
  // k: barrier (stage k and the A / scale buffers k & 1 visible; stage k - 1
  // and buffers (k + 1) & 1 free), load k + 2, copy k + 3, compute k, wait for
  // the loads of k + 1 (issued before the copies of k + 2 and k + 3 and the
  // loads of k + 2, and after the copy of k + 1), publish k + 1.  The loop is
  // unrolled by the four stages.
  uint8_t* const VS[4] = {V0, V1, V2, V3};
  if (nks > 0) {                                 // uniform
    Regs R[2];
    copy(V0, 0);
    copy(V1, 1);
    copy(V2, 2);
    load(R[0], 0);
    load(R[1], 1);
    __builtin_amdgcn_s_waitcnt(0);               // vmcnt(0) expcnt(0) lgkmcnt(0)
    publish(R[0], 0);
    for (int ks = 0; ks < nks; ks += 4) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int k = ks + d;
        if (d > 0 && k >= nks) break;            // uniform
        __builtin_amdgcn_s_waitcnt(0xC07F);      // this wave's LDS accesses are done
        __builtin_amdgcn_s_barrier();
        load(R[d & 1], k + 2);
        copy(VS[(d + 3) & 3], k + 3);
        compute(VS[d], k);
        constexpr int VM = 2 * NJ + 1 + 2 * ZS;  // 1 + 2 ZS: the register loads of one K-step
        __builtin_amdgcn_s_waitcnt(0x0F70 | (VM & 15) | ((VM >> 4) << 14));
        publish(R[(d & 1) ^ 1], k + 1);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);               // no copy may land after the wave ends
  }

  // ---- softmax sums per head (the TPH threads of a head are one wave's lanes)
#pragma unroll
  for (int d = 1; d < TPH; d *= 2) psum += __shfl_xor(psum, d, 64);
  if (ej == 0) Ps[eh] = psum;
  __syncthreads();
  if (tid < 32) a.psum[((int64_t)bq * a.n_c2 + c2) * 32 + tid] = Ps[tid];
  const int Rvp = a.Rvp;
#pragma unroll
  for (int gi = 0; gi < NGW; ++gi) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int T = 2 * (g0 + gi) + t;
      if (gi >= ngw || T >= ntile) continue;
      const int col = 32 * T + n;
      if (a.part16) {
        _Float16* part = (_Float16*)a.part + (((int64_t)bq * a.n_c2 + c2) * 32) * Rvp;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int q = 8 * (v >> 2) + 4 * hh + (v & 3);
          const float sq = Ps[q];
          part[(int64_t)q * Rvp + col] = (_Float16)(acc[2 * gi + t][v] * (sq > 0.f ? 1.0f / sq : 0.f));
        }
      } else {
        float* part = a.part + (((int64_t)bq * a.n_c2 + c2) * 32) * Rvp;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int q = 8 * (v >> 2) + 4 * hh + (v & 3);
          part[(int64_t)q * Rvp + col] = acc[2 * gi + t][v];
        }
      }
    }
  }
}

// Drop-in path (bx): sum of the chunk partials in fixed chunk order into the
// act-dtype output.  Each thread sums four columns of a 32x32 output tile;
// the partial loads are issued eight chunks at a time (32 loads in flight per
// thread) and added in chunk order.  More than PV_RG chunks are summed in two
// levels (deterministic, fixed grouping): MODE 1 sums each group of PV_RG
// chunks into part2 (grid z = group), MODE 2 sums the groups; MODE 0 sums the
// chunks directly.  blockIdx.y = (batch, group of 32 heads), as in pv_kernel.
// (The fused decode path reduces inside its up-projection, up_proj.hip.)
template <typename VT, int MODE>
__global__ __launch_bounds__(256) void pv_reduce_kernel(const PVArgs a) {
  const int tile = blockIdx.x, bq = blockIdx.y, grp = blockIdx.z;
  const int b = bq / a.n_hg, h0 = (bq - b * a.n_hg) * 32;
  const int Rvp = a.Rvp;
  const int q0 = threadIdx.x >> 5, col = tile * 32 + (threadIdx.x & 31);
  const int n_src = MODE == 2 ? a.n_grp : a.n_c2;
  const int c_begin = MODE == 1 ? grp * PV_RG : 0;
  const int c_end = MODE == 1 ? min(n_src, c_begin + PV_RG) : n_src;
  const float* part = MODE == 2 ? a.part2 : a.part;
  const float* pb = part + ((int64_t)bq * n_src * 32 + q0) * Rvp + col;
  const int64_t cstride = (int64_t)32 * Rvp, ustride = (int64_t)8 * Rvp;   // next chunk / next row group
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  int c = c_begin;
  for (; c + 8 <= c_end; c += 8) {
    float v[8][4];
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int u = 0; u < 4; ++u) v[k][u] = pb[(c + k) * cstride + u * ustride];
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u] += v[k][u];
  }
  for (; c < c_end; ++c)
#pragma unroll
    for (int u = 0; u < 4; ++u) s[u] += pb[c * cstride + u * ustride];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int q = q0 + 8 * u;
    if constexpr (MODE == 1) {
      a.part2[(((int64_t)bq * a.n_grp + grp) * 32 + q) * Rvp + col] = s[u];
    } else {
      if (h0 + q < a.H && col < a.Rv) ((VT*)a.out)[b * a.o_sb + (h0 + q) * a.o_sh + col] = (VT)s[u];
    }
  }
}

int pv_wide_tiles(int Rvp, bool fused, int vq) {
  const int tiles = Rvp / 32;
  // fused quantised latents past 32 tiles: the all-columns kernel, 8 waves
  // of ceil(tiles / 8) tiles (B16 S32768 int4-g64, 52 tiles: two column
  // blocks of 4 x 8 tiles fetch the logits and scale rows twice)
  if (!fused || vq == VQ_DENSE || tiles <= 32 || tiles > 64) return 0;
  return (tiles + 7) / 8;
}

int pv_tiles_per_wave(int Rvp, bool fused, int vq) {
  const int tiles = Rvp / 32;
  // Quantised formats: 8 tiles per wave, two workgroups per CU.  A quantised
  // K-step carries a quarter (int4) of the bytes of a dense one; its cost is
  // the VALU work (dequantisation, and the exponentials every wave forms for
  // its own A operand), so wider waves share it over more columns, while two
  // workgroups per CU keep 8 waves covering the memory latency (B16 S32768
  // int4-g64: 4 tiles 285 us, 8 tiles 244 us; 4 tiles x 3 workgroups 325 us).
  if (tiles <= 16) return 4;
  if (vq != VQ_DENSE) return 8;
  // the drop-in P-input variant stays at 8 (register budget)
  if (tiles <= 32 || !fused) return 8;
  return 13;
}

// fast: dense rows 16-byte aligned (ranks a multiple of 8); quantised rows
// aligned for 4-byte (int4) / 8-byte (int8) chunk loads, else the
// unaligned-row loads
template <typename VT, bool FUSED, int NTW>
static void launch_pv_n(const PVArgs& a, int vq, bool fast, int B, hipStream_t st) {
  dim3 grid(a.n_cb * a.n_c2, B), block(256);
  if (vq == VQ_BLOCK && fast) hipLaunchKernelGGL((pv_kernel<VT, NTW, FUSED, true, VQ_BLOCK>), grid, block, 0, st, a);
  else if (vq == VQ_BLOCK) hipLaunchKernelGGL((pv_kernel<VT, NTW, FUSED, false, VQ_BLOCK>), grid, block, 0, st, a);
  else if (vq == VQ_G64 && fast) hipLaunchKernelGGL((pv_kernel<VT, NTW, FUSED, true, VQ_G64>), grid, block, 0, st, a);
  else if (vq == VQ_G64) hipLaunchKernelGGL((pv_kernel<VT, NTW, FUSED, false, VQ_G64>), grid, block, 0, st, a);
  else if (fast) hipLaunchKernelGGL((pv_kernel<VT, NTW, FUSED, true, VQ_DENSE>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((pv_kernel<VT, NTW, FUSED, false, VQ_DENSE>), grid, block, 0, st, a);
}

template <typename VT>
static void launch_pv_n13(const PVArgs& a, bool fast, int B, hipStream_t st) {
  dim3 grid(a.n_cb * a.n_c2, B), block(256);
  if (fast) hipLaunchKernelGGL((pv_kernel<VT, 13, true, true, VQ_DENSE>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((pv_kernel<VT, 13, true, false, VQ_DENSE>), grid, block, 0, st, a);
}

template <typename VT, int NTW>
static void launch_pv_wide_n(const PVArgs& a, int vq, bool fast, int B, hipStream_t st) {
  dim3 grid(a.n_c2, B), block(512);
  if (vq == VQ_BLOCK && fast) hipLaunchKernelGGL((pv_wide_kernel<VT, NTW, true, VQ_BLOCK>), grid, block, 0, st, a);
  else if (vq == VQ_BLOCK) hipLaunchKernelGGL((pv_wide_kernel<VT, NTW, false, VQ_BLOCK>), grid, block, 0, st, a);
  else if (fast) hipLaunchKernelGGL((pv_wide_kernel<VT, NTW, true, VQ_G64>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((pv_wide_kernel<VT, NTW, false, VQ_G64>), grid, block, 0, st, a);
}

template <typename VT, bool FUSED>
static int launch_pv_t(const PVArgs& a, int vq, bool fast, int B, hipStream_t st) {
  const int ntw = pv_tiles_per_wave(a.Rvp, FUSED, vq);
  const int BQ = B * a.n_hg;
  if constexpr (FUSED) {
    // the host's geometry chose the all-columns kernel (one column block)
    if (const int w = pv_wide_tiles(a.Rvp, FUSED, vq); w && a.n_cb == 1) {
      if (vq == VQ_G64 && fast) {
        // rows of whole, aligned 16-byte pieces (the latent cache pads them): 16-byte copies
        const bool d16 = ((uintptr_t)a.x & 15) == 0 && a.x_ss % 16 == 0 && a.x_sb % 16 == 0 &&
                         a.x_ss >= 16 * ((a.Rv + 31) / 32) && a.Rvp <= 31 * 64;
        if (d16) hipLaunchKernelGGL((pv_nib_kernel<VT, 8, 4, true>), dim3(a.n_c2, BQ), dim3(512), 0, st, a);
        else hipLaunchKernelGGL((pv_nib_kernel<VT, 8, 4, false>), dim3(a.n_c2, BQ), dim3(512), 0, st, a);
        return (int)hipGetLastError();
      }
      if (w == 5) launch_pv_wide_n<VT, 5>(a, vq, fast, BQ, st);
      else if (w == 6) launch_pv_wide_n<VT, 6>(a, vq, fast, BQ, st);
      else if (w == 7) launch_pv_wide_n<VT, 7>(a, vq, fast, BQ, st);
      else launch_pv_wide_n<VT, 8>(a, vq, fast, BQ, st);
      return (int)hipGetLastError();
    }
  }
  if (FUSED && vq == VQ_G64 && fast && a.Rvp <= 512) {
    // group-64 V of up to 16 tiles: the raw-nibble kernel, 4 waves of up to two groups
    hipLaunchKernelGGL((pv_nib_kernel<VT, 4, 2, false>), dim3(a.n_c2, BQ), dim3(256), 0, st, a);
    return (int)hipGetLastError();
  }
  if (ntw == 4) launch_pv_n<VT, FUSED, 4>(a, vq, fast, BQ, st);
  else if (ntw == 8) launch_pv_n<VT, FUSED, 8>(a, vq, fast, BQ, st);
  else if constexpr (FUSED) launch_pv_n13<VT>(a, fast, BQ, st);
  int e = (int)hipGetLastError();
  if (e || FUSED) return e;
  if (a.n_grp > 1) {
    hipLaunchKernelGGL((pv_reduce_kernel<VT, 1>), dim3(a.Rvp / 32, BQ, a.n_grp), dim3(256), 0, st, a);
    hipLaunchKernelGGL((pv_reduce_kernel<VT, 2>), dim3(a.Rvp / 32, BQ), dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL((pv_reduce_kernel<VT, 0>), dim3(a.Rvp / 32, BQ), dim3(256), 0, st, a);
  }
  return (int)hipGetLastError();
}

// fast: the aligned-row variant (the C ABI decides which rows qualify).
// Fused: the P.V kernel alone (its partials are reduced by the up-projection
// kernel); drop-in: P.V and the partial reduction.
int launch_pv(const PVArgs& a, int dtype, int vq, bool fused, bool fast, int B, hipStream_t st) {
  if (dtype == STARKV_F16)
    return fused ? launch_pv_t<_Float16, true>(a, vq, fast, B, st) : launch_pv_t<_Float16, false>(a, vq, fast, B, st);
  return fused ? launch_pv_t<__bf16, true>(a, vq, fast, B, st) : launch_pv_t<__bf16, false>(a, vq, fast, B, st);
}

__global__ void fill_i32_kernel(int* p, int n, int v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

int launch_fill_i32(int* p, int n, int v, hipStream_t st) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, st, p, n, v);
  return (int)hipGetLastError();
}

}  // namespace starkv
