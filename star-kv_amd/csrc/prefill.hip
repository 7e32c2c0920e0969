// Prefill from the latent caches on gfx950: the counterpart of the
// reference's prefill branch (model.py:429-449), which materialises K and V
// from the latents and runs SDPA -- without a causal mask (the defect the
// build fixes: query t sees keys <= pos0 + t).
//
// 1. kv_recon_kernel: per (b, KV head, 64 positions) one MFMA GEMM tile,
//    K = RoPE(X_k[s] . B_k) (RoPE applied in the epilogue from the decode's
//    RoPE table) and V = X_v[s] . U_v[h]^T, into [B][Hkv][S_pad][128] act-dtype
//    buffers.  Quantised latents are dequantised on the way in, bit-exactly
//    as everywhere else (int8: fp16(q s); group-64 int4: fp16(n s + z)), then
//    rounded once more to bf16 for bf16 activations.  Rows in [S, S_pad) are
//    written as zeros.
// 2. fa_causal_kernel: flash attention over those buffers, one workgroup per
//    (b, query head, 128 queries), 4 waves of 32 queries.  Per 32-key block
//    it forms S^T = K . Q^T (so each lane holds 16 keys of one query and the
//    online softmax needs one cross-half exchange), with the K rows taken in
//    the order that makes the lane's probabilities the B operand of
//    O^T += V^T . P^T directly; V^T is read from LDS with the transpose load.
//    bf16 splits P into hi + lo so P.V keeps fp32-class accuracy.
#include "common.hpp"

namespace starkv {

namespace {

constexpr int WT_PITCH = 136;   // LDS row pitch (halves) of B_k^T and of the K / V blocks
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 pf_fp16x4;

__device__ inline uint2 pf_read_tr16(const uint16_t* p) {
  auto r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) pf_fp16x4*)(p));
  return __builtin_bit_cast(uint2, r);
}

template <typename XT> __device__ inline floatx16 pf_mfma(uint4 a, uint4 b, floatx16 c) {
  if constexpr (__is_same(XT, _Float16))
    return mfma_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c);
  else
    return mfma_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c);
}

template <typename XT> __device__ inline uint16_t pf_bits(float x) {
  return __builtin_bit_cast(uint16_t, (XT)x);
}

// fp16 pairs -> bf16 pairs (one rounding), for bf16 activations over
// dequantised (fp16) latents
__device__ inline uint4 pf_f16_to_bf16(uint4 h) {
  const uint32_t w[4] = {h.x, h.y, h.z, h.w};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const kh2 v = __builtin_bit_cast(kh2, w[k]);
    o[k] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(float)v[0]) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(float)v[1]) << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// 8 int8 (n) -> fp16(n * s), ranks in order, bit-exact (1152 + n is exact in fp16)
__device__ inline uint4 pf_dq_int8(uint2 q, uint16_t s16) {
  const uint32_t x = q.x ^ 0x80808080u, y = q.y ^ 0x80808080u;
  const uint32_t pr[4] = {__builtin_amdgcn_perm(0x64646464u, x, 0x04010400u),
                          __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u),
                          __builtin_amdgcn_perm(0x64646464u, y, 0x04010400u),
                          __builtin_amdgcn_perm(0x64646464u, y, 0x04030402u)};
  const kh2 s = __builtin_bit_cast(kh2, (uint32_t)s16 * 0x10001u);
  const kh2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(kh2, pr[k]) + bias) * s);
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// 8 int4 nibbles (rank 2k in the low nibble of byte k) -> fp16(n * s + z), ranks in order
__device__ inline uint4 pf_dq_g64(uint32_t w, uint16_t s16, uint16_t z16) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  const kh2 s = __builtin_bit_cast(kh2, (uint32_t)s16 * 0x10001u);
  const kh2 z = __builtin_bit_cast(kh2, (uint32_t)z16 * 0x10001u);
  const kh2 bias = {(_Float16)-1024.0f, (_Float16)-1024.0f};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t p = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u + 0x00010001u * k) | 0x64006400u;
    o[k] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(kh2, p) + bias, s, z));
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace

// KIND 0: K (dense or int8 latents), 1: V (dense or group-64 int4 latents)
template <typename XT, int KIND>
__global__ __launch_bounds__(256) void kv_recon_kernel(const PFArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t wT[KIND == 0 ? 128 * WT_PITCH : 8];   // K: B_k^T [d][j]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  const int p0 = blockIdx.x * 64, h = blockIdx.y, b = blockIdx.z;
  const int S = a.S;
  const int R = KIND == 0 ? a.krank[h] : a.Rv;            // multiple of 8 (host-checked)
  const int Rp = (R + 15) & ~15;
  if constexpr (KIND == 0) {
    const XT* bk = (const XT*)a.bk + a.bkoff[h];
    for (int e = tid; e < Rp * 128; e += 256) {
      const int j = e >> 7, d = e & 127;
      wT[d * WT_PITCH + j] = j < R ? __builtin_bit_cast(uint16_t, bk[(int64_t)j * a.bk_rs + d]) : (uint16_t)0;
    }
    __syncthreads();
  }
  const int pr = min(p0 + 32 * (wave & 1) + n, S - 1);      // A-operand row (position), clamped
  const int dc0 = 32 * (wave >> 1), dc1 = dc0 + 64;          // output dims dc + n (RoPE pairs in one lane)
  floatx16 acc0 = floatx16{}, acc1 = floatx16{};
  for (int j0 = 0; j0 < Rp; j0 += 16) {
    const int jj = j0 + 8 * hh;                               // this lane's 8 K indices
    const bool jok = jj < R;
    uint4 A = make_uint4(0, 0, 0, 0), B0 = A, B1 = A;
    if constexpr (KIND == 0) {
      if (a.k_i8) {
        const uint8_t* x = (const uint8_t*)a.kx + b * a.kx_sb + a.kxoff[h] + (int64_t)pr * a.kxpitch[h];
        const uint16_t s = ((const uint16_t*)a.kscale)[b * a.ks_sb + h * a.ks_sh + pr];
        if (jok) {
          A = pf_dq_int8(*(const uint2*)(x + jj), s);
          if constexpr (!__is_same(XT, _Float16)) A = pf_f16_to_bf16(A);
        }
      } else {
        const XT* x = (const XT*)a.kx + b * a.kx_sb + a.kxoff[h] + (int64_t)pr * a.kxpitch[h];
        if (jok) A = *(const uint4*)(x + jj);
      }
      B0 = *(const uint4*)&wT[(dc0 + n) * WT_PITCH + jj];
      B1 = *(const uint4*)&wT[(dc1 + n) * WT_PITCH + jj];
    } else {
      if (a.v_g64) {
        const uint8_t* x = (const uint8_t*)a.vx + b * a.vx_sb + (int64_t)pr * a.vx_ss;
        const int64_t so = b * a.vs_sb + (int64_t)pr * a.vs_ss + (jok ? jj / 64 : 0);
        if (jok) {
          A = pf_dq_g64(*(const uint32_t*)(x + jj / 2), ((const uint16_t*)a.vscale)[so], ((const uint16_t*)a.vzero)[so]);
          if constexpr (!__is_same(XT, _Float16)) A = pf_f16_to_bf16(A);
        }
      } else {
        const XT* x = (const XT*)a.vx + b * a.vx_sb + (int64_t)pr * a.vx_ss;
        if (jok) A = *(const uint4*)(x + jj);
      }
      const XT* u = (const XT*)a.uv + (int64_t)h * HEAD_DIM * a.uv_rs;
      if (jok) {
        B0 = *(const uint4*)(u + (int64_t)(dc0 + n) * a.uv_rs + jj);
        B1 = *(const uint4*)(u + (int64_t)(dc1 + n) * a.uv_rs + jj);
      }
    }
    acc0 = pf_mfma<XT>(A, B0, acc0);
    acc1 = pf_mfma<XT>(A, B1, acc1);
  }
  // epilogue: lane holds rows (positions) 8(v/4) + 4hh + v%4 of dims dc0 + n and dc1 + n
  XT* dst = (XT*)(KIND == 0 ? a.kbuf : a.vbuf) + (((int64_t)b * a.Hkv + h) * a.S_pad) * HEAD_DIM;
  const int i = dc0 + n;                                      // RoPE frequency of this lane (< 64)
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int p = p0 + 32 * (wave & 1) + 8 * (v >> 2) + 4 * hh + (v & 3);
    float y0 = acc0[v], y1 = acc1[v];
    if (p >= S) {
      y0 = y1 = 0.f;
    } else if constexpr (KIND == 0) {
      // RoPE table: (cos, sin) of position p and frequency i, times the attention scaling
      const int64_t te = ((int64_t)((p >> 5) * 8 + (i >> 3)) * 64 + ((i & 7) >> 2) * 32 + (p & 31)) * 8 + 2 * (i & 3);
      const uint32_t cs = ((const uint32_t*)a.rope)[te >> 1];
      const kh2 c2 = __builtin_bit_cast(kh2, cs);
      const float c = (float)c2[0], s = (float)c2[1];
      const float k0 = y0, k1 = y1;
      y0 = k0 * c - k1 * s;
      y1 = k1 * c + k0 * s;
    }
    if (p < a.S_pad) {
      dst[(int64_t)p * HEAD_DIM + dc0 + n] = (XT)y0;
      dst[(int64_t)p * HEAD_DIM + dc1 + n] = (XT)y1;
    }
  }
}

template <typename XT>
__global__ __launch_bounds__(256) void fa_causal_kernel(const PFArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[32 * WT_PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[32 * WT_PITCH];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  const int qb = blockIdx.x, qh = blockIdx.y, b = blockIdx.z;
  const int kv = qh / a.gs, T = a.T, pos0 = a.pos0;
  const int t = qb * 128 + 32 * wave + n;                     // this lane's query
  const int tc = min(t, T - 1);
  const int P = pos0 + tc;                                    // its position: sees keys <= P
  const XT* qrow = (const XT*)a.q + b * a.q_sb + qh * a.q_sh + (int64_t)tc * a.q_st;
  uint4 Qb[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) Qb[k] = *(const uint4*)(qrow + 16 * k + 8 * hh);
  floatx16 o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = floatx16{};
  float m = -INFINITY, l = 0.f;
  const int last_t = min(T, qb * 128 + 128) - 1;
  const int nkb = (pos0 + last_t) / 32 + 1;                   // 32-key blocks the workgroup needs
  const size_t hbase = (((size_t)b * a.Hkv + kv) * a.S_pad) * HEAD_DIM;
  const XT* kg = (const XT*)a.kbuf + hbase;
  const XT* vg = (const XT*)a.vbuf + hbase;
  // S^T A operand: MFMA row r = n takes key pi(r) (see the file comment)
  const int ra = n >> 3, rh = (n >> 2) & 1, rc = n & 3;
  const int key_r = 16 * (ra >> 1) + 8 * rh + 4 * (ra & 1) + rc;
  // V^T A operand: transposed reads (lane group g = lane/16, rho = lane%16)
  const int g = lane >> 4, rho = lane & 15;
  const int tr_off = (8 * hh + (rho >> 2)) * WT_PITCH + 16 * (g & 1) + 4 * (rho & 3);
  for (int kb = 0; kb < nkb; ++kb) {
    // stage the block's 32 keys of K and V (rows < S_pad: nkb * 32 <= S_pad)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int e = c * 256 + tid, key = e >> 4, d8 = (e & 15) * 8;
      const size_t go = (size_t)(kb * 32 + key) * HEAD_DIM + d8;
      *(uint4*)&Ks[key * WT_PITCH + d8] = *(const uint4*)(kg + go);
      *(uint4*)&Vs[key * WT_PITCH + d8] = *(const uint4*)(vg + go);
    }
    __syncthreads();
    floatx16 s = floatx16{};
#pragma unroll
    for (int k = 0; k < 8; ++k)
      s = pf_mfma<XT>(*(const uint4*)&Ks[key_r * WT_PITCH + 16 * k + 8 * hh], Qb[k], s);
    // lane: keys kb*32 + 16(v/8) + 8hh + v%8 of query t
    float x[16];
    float mb = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = kb * 32 + 16 * (v >> 3) + 8 * hh + (v & 7);
      x[v] = key <= P ? s[v] * a.scale_log2 : -INFINITY;
      mb = fmaxf(mb, x[v]);
    }
    mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
    const float mn = fmaxf(m, mb);                            // finite: key 0 <= P in block 0
    const float alpha = __builtin_amdgcn_exp2f(m - mn);
    float ps = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      x[v] = __builtin_amdgcn_exp2f(x[v] - mn);
      ps += x[v];
    }
    ps += __shfl_xor(ps, 32, 64);
    l = l * alpha + ps;
    m = mn;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[j][v] *= alpha;
    // O^T += V^T . P^T over the block's two 16-key halves
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const uint16_t* sb = Vs + 16 * kk * WT_PITCH + tr_off;
      if constexpr (__is_same(XT, _Float16)) {
        half8 ph;
#pragma unroll
        for (int e = 0; e < 8; ++e) ph[e] = (_Float16)x[8 * kk + e];
        const uint4 pb = __builtin_bit_cast(uint4, ph);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint2 lo = pf_read_tr16(sb + 32 * j), hi = pf_read_tr16(sb + 32 * j + 4 * WT_PITCH);
          o[j] = pf_mfma<XT>(make_uint4(lo.x, lo.y, hi.x, hi.y), pb, o[j]);
        }
      } else {
        bf16x8 ph, pl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const __bf16 hv = (__bf16)x[8 * kk + e];
          ph[e] = hv;
          pl[e] = (__bf16)(x[8 * kk + e] - (float)hv);
        }
        const uint4 pbh = __builtin_bit_cast(uint4, ph), pbl = __builtin_bit_cast(uint4, pl);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint2 lo = pf_read_tr16(sb + 32 * j), hi = pf_read_tr16(sb + 32 * j + 4 * WT_PITCH);
          const uint4 va = make_uint4(lo.x, lo.y, hi.x, hi.y);
          o[j] = pf_mfma<XT>(va, pbh, o[j]);
          o[j] = pf_mfma<XT>(va, pbl, o[j]);
        }
      }
    }
    __syncthreads();                                          // before the next block overwrites Ks / Vs
  }
  if (t < T) {
    const float inv = 1.0f / l;
    XT* orow = (XT*)a.out + b * a.o_sb + qh * a.o_sh + (int64_t)t * a.o_st;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) orow[32 * j + 8 * (v >> 2) + 4 * hh + (v & 3)] = (XT)(o[j][v] * inv);
  }
}

template <typename XT>
static int launch_prefill_t(const PFArgs& a, int B, hipStream_t st) {
  const dim3 rg((unsigned)ceil_div(a.S, 64), a.Hkv, B);
  hipLaunchKernelGGL((kv_recon_kernel<XT, 0>), rg, dim3(256), 0, st, a);
  hipLaunchKernelGGL((kv_recon_kernel<XT, 1>), rg, dim3(256), 0, st, a);
  hipLaunchKernelGGL((fa_causal_kernel<XT>), dim3((unsigned)ceil_div(a.T, 128), a.Hq, B), dim3(256), 0, st, a);
  return (int)hipGetLastError();
}

int launch_prefill(const PFArgs& a, int dtype, int B, hipStream_t st) {
  return dtype == STARKV_F16 ? launch_prefill_t<_Float16>(a, B, st) : launch_prefill_t<__bf16>(a, B, st);
}

}  // namespace starkv
