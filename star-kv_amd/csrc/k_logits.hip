// K1: latent-K decode logits on gfx950.
//
// Replaces the Triton _abx_fwd kernel (abx_rope_batched.py:55-132): for every
// cached position s and query head q,
//     logit[b,q,s] = scale * q_rot[b,q] . RoPE_s(X_k[b,kv,s,:] @ B_k[kv])   (kv = q // gs)
//
// Formulation.  With c = 2i+tau interleaving the 64 RoPE frequencies i with
// cos (tau=0) and sin (tau=1), the rotate_half RoPE and the dot with q fold
// into a per-(b,q) matrix W[j][c] (rank j x 128):
//     W[j][2i]   = scale * (B_k[j][i] q[i]    + B_k[j][i+64] q[i+64])
//     W[j][2i+1] = scale * (B_k[j][i] q[i+64] - B_k[j][i+64] q[i])
//     logit[s]   = sum_j X_k[s][j] * V[j][s],   V = W . T,  T[c][s] = (cos|sin)(s*theta_i)
// V for a 32-position tile is one 32x32x16 f16 MFMA chain per 32 ranks
// (K = the 128 rotation coefficients), with the position-dependent rotation
// table T as the B operand shared by every head and batch, and the latent X
// enters only through one FMA per element in the epilogue.  The MFMA output
// rows are permuted so that each lane holds 16 consecutive ranks of one
// position: the epilogue reads X with two 16-byte loads per lane and needs no
// shuffles except one half-wave swap per head.
//
// Work decomposition: grid (chunk of positions, workgroup plan, batch); the
// 4 waves of a workgroup each own up to K_MAXI items (query head, 32-rank
// M-tile) packed by the host so that ragged head-wise ranks are balanced.
// The T tile (32 positions x 128 coefficients, fp16, 8 KB) is produced once
// per workgroup and tile into LDS by a per-thread rotation recurrence seeded
// from the RoPE tables.
#include "common.hpp"

namespace starkv {

template <typename XT, int XFMT>
struct XBuf {
  uint4 v[K_MAXI][2];
  float sc[K_MAXI];
};

template <typename XT>
__device__ inline void load4(const XT* p, float* out) {
  // four consecutive elements (8 bytes, 8-byte aligned)
  uint2 u = *(const uint2*)p;
  if constexpr (sizeof(XT) == 2 && __is_same(XT, _Float16)) {
    half4 h = __builtin_bit_cast(half4, u);
    out[0] = (float)h[0]; out[1] = (float)h[1]; out[2] = (float)h[2]; out[3] = (float)h[3];
  } else {
    out[0] = __uint_as_float(u.x << 16); out[1] = __uint_as_float(u.x & 0xffff0000u);
    out[2] = __uint_as_float(u.y << 16); out[3] = __uint_as_float(u.y & 0xffff0000u);
  }
}

template <typename XT>
__device__ inline void load4_any(const XT* p, float* out) {
  for (int e = 0; e < 4; ++e) out[e] = to_f32(p[e]);
}

// dot of 8 packed 16-bit elements with 8 accumulators
template <typename XT>
__device__ inline float dot8(uint4 u, const float* acc, float part) {
  if constexpr (__is_same(XT, _Float16)) {
    half8 h = __builtin_bit_cast(half8, u);
#pragma unroll
    for (int v = 0; v < 8; ++v) part = fmaf((float)h[v], acc[v], part);
  } else {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      part = fmaf(__uint_as_float(w[v] << 16), acc[2 * v], part);
      part = fmaf(__uint_as_float(w[v] & 0xffff0000u), acc[2 * v + 1], part);
    }
  }
  return part;
}

__device__ inline float dot_i8x4(uint32_t w, const float* acc, float part) {
  part = fmaf((float)(int)(int8_t)(w & 0xff), acc[0], part);
  part = fmaf((float)(int)(int8_t)((w >> 8) & 0xff), acc[1], part);
  part = fmaf((float)(int)(int8_t)((w >> 16) & 0xff), acc[2], part);
  part = fmaf((float)(int)(int8_t)(w >> 24), acc[3], part);
  return part;
}

// XFMT: 0 = dense act dtype, 2 = int8 symmetric with per-(b,kv,s) fp16 scale
// OUTK: 0 = fp32 logits + chunk maxima, 1 = fp16 logits, 2 = bf16 logits
template <typename XT, int XFMT, int OUTK, bool FAST>
__global__ __launch_bounds__(256, 1) void k_logits_kernel(const KArgs a) {
  __shared__ half8 Tl[2][8][64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = lane & 31, hh = lane >> 5;
  const int chunk = blockIdx.x, wgp = blockIdx.y, b = blockIdx.z;

  if (a.zero_ptr != nullptr && chunk == 0 && wgp == 0 && b == 0)
    for (int i = tid; i < a.zero_count; i += 256) a.zero_ptr[i] = 0;

  const int S = a.S;
  const int n_tiles = (S + TILE - 1) / TILE;
  const int tile0 = chunk * a.tiles_per_chunk;
  const int tile1 = min(tile0 + a.tiles_per_chunk, n_tiles);
  if (tile0 >= tile1) return;   // uniform over the workgroup

  // ---- RoPE recurrence state: thread -> frequency quad fq, positions tt0, tt0+16
  const int fq = tid & 15, tt0 = tid >> 4;
  const int ti0 = 8 * (fq >> 1) + 4 * (fq & 1);
  const float* T0 = a.rope;
  const float* RT = a.rope + TILE * 128;
  float rc[2][4], rs[2][4], stc[4], sts[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int i = ti0 + e;
    stc[e] = RT[128 + 2 * i];
    sts[e] = RT[128 + 2 * i + 1];
    const float c0 = RT[(int64_t)tile0 * 128 + 2 * i], s0 = RT[(int64_t)tile0 * 128 + 2 * i + 1];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float ct = T0[(tt0 + 16 * u) * 128 + 2 * i], st = T0[(tt0 + 16 * u) * 128 + 2 * i + 1];
      rc[u][e] = c0 * ct - s0 * st;
      rs[u][e] = s0 * ct + c0 * st;
    }
  }

  // ---- items of this wave and their folded query matrices W (MFMA A operand)
  uint32_t it[K_MAXI];
#pragma unroll
  for (int i = 0; i < K_MAXI; ++i) it[i] = a.items[wgp][wave][i];

  half8 W[K_MAXI][8];
  const int rho = lane & 31;
  const int jrow = 16 * ((rho >> 2) & 1) + 4 * (rho >> 3) + (rho & 3);   // rank of A-row rho within the M-tile
#pragma unroll
  for (int i = 0; i < K_MAXI; ++i) {
#pragma unroll
    for (int k = 0; k < 8; ++k) W[i][k] = half8{};
    if (!item_valid(it[i])) continue;
    const int qh = item_qh(it[i]), kv = item_kv(it[i]), mt = item_mt(it[i]), nv = item_nv(it[i]);
    if (jrow >= nv) continue;
    const XT* qrow = (const XT*)a.q + b * a.q_sb + qh * a.q_sh;
    const XT* brow = (const XT*)a.bk + a.bkoff[kv] + (int64_t)(mt * 32 + jrow) * a.bk_rs;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i0 = 8 * k + 4 * hh;
      float ql[4], qu[4], bl[4], bu[4];
      if (FAST) {
        load4<XT>(qrow + i0, ql); load4<XT>(qrow + i0 + 64, qu);
        load4<XT>(brow + i0, bl); load4<XT>(brow + i0 + 64, bu);
      } else {
        load4_any<XT>(qrow + i0, ql); load4_any<XT>(qrow + i0 + 64, qu);
        load4_any<XT>(brow + i0, bl); load4_any<XT>(brow + i0 + 64, bu);
      }
      half8 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        w[2 * e] = (_Float16)(a.wscale * (bl[e] * ql[e] + bu[e] * qu[e]));
        w[2 * e + 1] = (_Float16)(a.wscale * (bl[e] * qu[e] - bu[e] * ql[e]));
      }
      W[i][k] = w;
    }
  }

  float mx[K_MAXI];
#pragma unroll
  for (int i = 0; i < K_MAXI; ++i) mx[i] = -INFINITY;

  // ---- latent loads for one tile
  auto load_x = [&](XBuf<XT, XFMT>& xb, int tile) {
    const int s = tile * TILE + t;
#pragma unroll
    for (int i = 0; i < K_MAXI; ++i) {
      xb.v[i][0] = make_uint4(0, 0, 0, 0);
      xb.v[i][1] = make_uint4(0, 0, 0, 0);
      xb.sc[i] = 0.f;
      if (!item_valid(it[i])) continue;
      const int kv = item_kv(it[i]), mt = item_mt(it[i]);
      const int nvh = item_nv(it[i]) - 16 * hh;
      if (s >= S || nvh <= 0) continue;
      const int64_t off = b * a.x_sb + a.xoff[kv] + (int64_t)s * a.xpitch[kv] + mt * 32 + 16 * hh;
      if constexpr (XFMT == 0) {
        const XT* p = (const XT*)a.x + off;
        if (FAST) {
          xb.v[i][0] = *(const uint4*)p;
          if (nvh >= 16) xb.v[i][1] = *(const uint4*)(p + 8);
        } else {
          uint16_t tmp[16];
#pragma unroll
          for (int v = 0; v < 16; ++v) tmp[v] = v < nvh ? ((const uint16_t*)p)[v] : (uint16_t)0;
          xb.v[i][0] = make_uint4(tmp[0] | (tmp[1] << 16), tmp[2] | (tmp[3] << 16), tmp[4] | (tmp[5] << 16), tmp[6] | (tmp[7] << 16));
          xb.v[i][1] = make_uint4(tmp[8] | (tmp[9] << 16), tmp[10] | (tmp[11] << 16), tmp[12] | (tmp[13] << 16), tmp[14] | (tmp[15] << 16));
        }
      } else {
        const uint8_t* p = (const uint8_t*)a.x + off;
        if (FAST) {
          if (nvh >= 16) xb.v[i][0] = *(const uint4*)p;
          else { uint2 u = *(const uint2*)p; xb.v[i][0] = make_uint4(u.x, u.y, 0, 0); }
        } else {
          uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
          for (int v = 0; v < 16; ++v) if (v < nvh) w[v >> 2] |= (uint32_t)p[v] << (8 * (v & 3));
          xb.v[i][0] = make_uint4(w[0], w[1], w[2], w[3]);
        }
        if (item_last(it[i]))
          xb.sc[i] = (float)((const _Float16*)a.xscale)[b * a.xs_sb + kv * a.xs_sh + s];
      }
    }
  };

  auto compute = [&](const XBuf<XT, XFMT>& xb, int tile, int buf) {
    // produce this tile's rotation operand
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      half8 h;
#pragma unroll
      for (int e = 0; e < 4; ++e) { h[2 * e] = (_Float16)rc[u][e]; h[2 * e + 1] = (_Float16)rs[u][e]; }
      Tl[buf][fq >> 1][(tt0 + 16 * u) * 2 + (fq & 1)] = h;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float c = rc[u][e], s_ = rs[u][e];
        rc[u][e] = c * stc[e] - s_ * sts[e];
        rs[u][e] = s_ * stc[e] + c * sts[e];
      }
    __syncthreads();
    half8 T[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) T[k] = Tl[buf][k][t * 2 + hh];

    floatx16 acc[K_MAXI];
#pragma unroll
    for (int i = 0; i < K_MAXI; ++i) acc[i] = floatx16{};
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int i = 0; i < K_MAXI; ++i)
        if (item_valid(it[i])) acc[i] = mfma_f16(W[i][k], T[k], acc[i]);

    const int s = tile * TILE + t;
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < K_MAXI; ++i) {
      if (!item_valid(it[i])) continue;
      float av[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) av[v] = acc[i][v];
      if constexpr (XFMT == 0) {
        part = dot8<XT>(xb.v[i][0], av, part);
        part = dot8<XT>(xb.v[i][1], av + 8, part);
      } else {
        part = dot_i8x4(xb.v[i][0].x, av, part);
        part = dot_i8x4(xb.v[i][0].y, av + 4, part);
        part = dot_i8x4(xb.v[i][0].z, av + 8, part);
        part = dot_i8x4(xb.v[i][0].w, av + 12, part);
      }
      if (item_last(it[i])) {
        float tot = add_halves(part);
        part = 0.f;
        if constexpr (XFMT == 2) tot *= xb.sc[i];
        const int qh = item_qh(it[i]);
        if (s < S) {
          if (a.mask != nullptr) tot += load_elem_f32(a.mask, a.mask_dtype, b * a.m_sb + qh * a.m_sh + s);
          if (hh == 0) {
            const int64_t o = b * a.o_sb + qh * a.o_sh + s;
            if constexpr (OUTK == 0) ((float*)a.out)[o] = tot;
            else if constexpr (OUTK == 1) ((_Float16*)a.out)[o] = (_Float16)tot;
            else ((__bf16*)a.out)[o] = (__bf16)tot;
          }
          mx[i] = fmaxf(mx[i], tot);
        }
      }
    }
  };

  XBuf<XT, XFMT> xa, xn;
  load_x(xa, tile0);
  for (int tile = tile0; tile < tile1; tile += 2) {
    if (tile + 1 < tile1) load_x(xn, tile + 1);
    compute(xa, tile, 0);
    if (tile + 1 >= tile1) break;
    if (tile + 2 < tile1) load_x(xa, tile + 2);
    compute(xn, tile + 1, 1);
  }

  if constexpr (OUTK == 0) {
    if (a.chunkmax != nullptr) {
#pragma unroll
      for (int i = 0; i < K_MAXI; ++i) {
        if (!item_valid(it[i]) || !item_last(it[i])) continue;
        const float m = wave_max32(mx[i]);
        if (lane == 0) a.chunkmax[((int64_t)b * a.Hq + item_qh(it[i])) * a.n_chunks + chunk] = m;
      }
    }
  }
}

template <typename XT, int XFMT, int OUTK>
static int launch_t(const KArgs& a, bool fast, int B, hipStream_t st) {
  dim3 grid(a.n_chunks, a.n_wg, B), block(256);
  if (fast) hipLaunchKernelGGL((k_logits_kernel<XT, XFMT, OUTK, true>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((k_logits_kernel<XT, XFMT, OUTK, false>), grid, block, 0, st, a);
  return (int)hipGetLastError();
}

template <typename XT, int XFMT>
static int launch_o(const KArgs& a, int outk, bool fast, int B, hipStream_t st) {
  if (outk == 0) return launch_t<XT, XFMT, 0>(a, fast, B, st);
  if (outk == 1) return launch_t<XT, XFMT, 1>(a, fast, B, st);
  return launch_t<XT, XFMT, 2>(a, fast, B, st);
}

int launch_k_logits(const KArgs& a, int dtype, int fmt, bool out_f32, int out_dtype, bool fast, int B, hipStream_t st) {
  const int outk = out_f32 ? 0 : (out_dtype == STARKV_F16 ? 1 : 2);
  const bool i8 = fmt == STARKV_FMT_INT8_SYM;
  if (dtype == STARKV_F16) return i8 ? launch_o<_Float16, 2>(a, outk, fast, B, st) : launch_o<_Float16, 0>(a, outk, fast, B, st);
  return i8 ? launch_o<__bf16, 2>(a, outk, fast, B, st) : launch_o<__bf16, 0>(a, outk, fast, B, st);
}

}  // namespace starkv
