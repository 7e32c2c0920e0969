// K2: probabilities x V-latent on gfx950.
//
// Replaces the reference's P @ X_v (model.py:484) and the Triton _bx_fwd
// kernel (bx_quant.py:37-114):   o[b, q, j] = sum_s P[b, q, s] * X_v[b, s, j].
//
// X_v is one latent shared by every head, so a workgroup streams a
// (position chunk x column block) slab of X_v once for all 32 heads: the MFMA
// 32x32x16 A operand is P (32 heads x 16 positions), the B operand is X_v
// (16 positions x 32 ranks).  X_v rows arrive with coalesced 16-byte loads,
// are staged in LDS (wave-private, double buffered) and are read back
// transposed with ds_read_b64_tr_b16, the gfx950 LDS transpose load: within
// each 16-lane group, lane j receives column j%4 of the rows addressed by
// lanes {j/4, 4+j/4, 8+j/4, 12+j/4}.
//
// Fused mode: P = exp(logit - M) is formed in registers from the fp32 logits
// of K1 with M the global row max (from K1's chunk maxima), so no softmax
// pass and no normalisation happen here; the denominators are summed on the
// side.  Drop-in mode (bx): P is read as given.
//
// Split-S: the 4 waves of a workgroup take interleaved 16-position K-steps of
// the chunk and are summed through LDS; the n_c2 chunk partials of each
// (batch, column block) are summed in fixed chunk order by whichever
// workgroup finishes last (atomic ticket), so the result is deterministic
// (no float atomics; the reference accumulates fp16 atomics into an
// uninitialised tensor, bx_quant.py:113-114, 147).
#include "common.hpp"

namespace starkv {

typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 lds_fp16x4;

__device__ inline uint2 lds_read_tr16(const uint16_t* p) {
  auto r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) lds_fp16x4*)(p));
  return __builtin_bit_cast(uint2, r);
}

template <typename VT>
__device__ inline void load8_f32(const float* p, float* out) {
  const float4 u = *(const float4*)p, v = *(const float4*)(p + 4);
  out[0] = u.x; out[1] = u.y; out[2] = u.z; out[3] = u.w; out[4] = v.x; out[5] = v.y; out[6] = v.z; out[7] = v.w;
}

template <typename VT, int NT, bool FUSED, bool FAST>
__global__ __launch_bounds__(256, 2) void pv_kernel(const PVArgs a) {
  constexpr int PITCH = NT * 32 + 8;            // elements per staged row (16-byte pad)
  constexpr int STAGE = 16 * PITCH;             // elements per staged K-step
  constexpr int NTP = 2;                        // N-tiles per LDS reduction pass
  __shared__ __attribute__((aligned(16))) uint16_t stage[4][2][STAGE];
  __shared__ float Ms[32];
  __shared__ float Ps[4][32];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  const int cb = blockIdx.x % a.n_cb, c2 = blockIdx.x / a.n_cb, b = blockIdx.y;
  const int col0 = cb * NT * 32;
  const int H = a.H;

  if constexpr (FUSED) {
    const int q = tid >> 3, j = tid & 7;
    float m = -INFINITY;
    if (q < H)
      for (int c = j; c < a.n_chunk1; c += 8) m = fmaxf(m, a.chunkmax[((int64_t)b * H + q) * a.n_chunk1 + c]);
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    if (j == 0) Ms[q] = q < H ? m : 0.f;
    __syncthreads();
  }
  const float Mq = FUSED ? Ms[n] : 0.f;
  const bool qok = n < H;

  const int s_begin = c2 * a.c2_len;
  const int s_end = min(a.S, s_begin + a.c2_len);
  const int nks = s_begin < s_end ? (s_end - s_begin + KSTEP - 1) / KSTEP : 0;

  floatx16 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = floatx16{};
  float psum = 0.f;

  // ---- staging map: lane, chunk c -> (row, 16-byte column chunk)
  uint4 R[NT];
  auto gload = [&](int ks) {
    const int s0 = s_begin + ks * KSTEP;
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      const int f = c * 64 + lane;
      const int row = f / (NT * 4), c16 = f % (NT * 4);
      const int s = s0 + row, col = col0 + c16 * 8;
      R[c] = make_uint4(0, 0, 0, 0);
      if (s < s_end && col < a.Rv) {
        const VT* p = (const VT*)a.x + b * a.x_sb + (int64_t)s * a.x_ss + col;
        if (FAST) {
          R[c] = *(const uint4*)p;
        } else {
          uint16_t tmp[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) tmp[e] = (col + e < a.Rv) ? ((const uint16_t*)p)[e] : (uint16_t)0;
          R[c] = make_uint4(tmp[0] | (tmp[1] << 16), tmp[2] | (tmp[3] << 16), tmp[4] | (tmp[5] << 16), tmp[6] | (tmp[7] << 16));
        }
      }
    }
  };
  auto swrite = [&](int buf) {
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      const int f = c * 64 + lane;
      const int row = f / (NT * 4), c16 = f % (NT * 4);
      *(uint4*)&stage[wave][buf][row * PITCH + c16 * 8] = R[c];
    }
  };

  // transposed-read addressing (see header): group g = lane/16, rho = lane%16
  const int g = lane >> 4, rho = lane & 15;
  const int tr_off = (8 * hh + (rho >> 2)) * PITCH + 16 * (g & 1) + 4 * (rho & 3);

  // P-operand source for one K-step (prefetched together with the X_v rows)
  float pn[8];
  auto pload = [&](int ks) {
    const int sa = s_begin + ks * KSTEP + 8 * hh;
    if constexpr (FUSED) {
      if (qok) {
        load8_f32<VT>(a.logits + b * a.l_sb + n * a.l_sh + sa, pn);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) pn[e] = 0.f;
      }
    } else {
      const VT* pp = (const VT*)a.p + b * a.p_sb + n * a.p_sh;
#pragma unroll
      for (int e = 0; e < 8; ++e) pn[e] = (qok && sa + e < s_end) ? to_f32(pp[sa + e]) : 0.f;
    }
  };

  int buf = 0;
  int ks = wave;
  if (ks < nks) { pload(ks); gload(ks); }
  for (; ks < nks; ks += 4) {
    swrite(buf);
    float pc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) pc[e] = pn[e];
    if (ks + 4 < nks) { pload(ks + 4); gload(ks + 4); }

    // A operand: P[q = n][s0 + 8hh + e]
    const int sa = s_begin + ks * KSTEP + 8 * hh;
    float pv[8];
    if constexpr (FUSED) {
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = (qok && sa + e < s_end) ? __builtin_amdgcn_exp2f((pc[e] - Mq) * 1.4426950408889634f) : 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) psum += pv[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = pc[e];
    }

    const uint16_t* sb = &stage[wave][buf][tr_off];
    if constexpr (__is_same(VT, _Float16)) {
      half8 A;
#pragma unroll
      for (int e = 0; e < 8; ++e) A[e] = (_Float16)pv[e];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const uint2 lo = lds_read_tr16(sb + 32 * j);
        const uint2 hi = lds_read_tr16(sb + 32 * j + 4 * PITCH);
        const half8 Bv = __builtin_bit_cast(half8, make_uint4(lo.x, lo.y, hi.x, hi.y));
        acc[j] = mfma_f16(A, Bv, acc[j]);
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
      for (int j = 0; j < NT; ++j) {
        const uint2 lo = lds_read_tr16(sb + 32 * j);
        const uint2 hi = lds_read_tr16(sb + 32 * j + 4 * PITCH);
        const bf16x8 Bv = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
        acc[j] = mfma_bf16(Ah, Bv, acc[j]);
        acc[j] = mfma_bf16(Al, Bv, acc[j]);
      }
    }
    buf ^= 1;
  }

  // ---- cross-wave reduction through LDS (reuses the staging buffers)
  float* red = (float*)&stage[0][0][0];    // [4 waves][NTP][64 lanes][17]
  static_assert(4 * NTP * 64 * 17 * 4 <= (int)sizeof(stage), "reduction buffer");
  const int Rvp = a.Rvp;
  float* part = a.part + (((int64_t)b * a.n_c2 + c2) * 32) * Rvp;
#pragma unroll
  for (int p0 = 0; p0 < NT; p0 += NTP) {
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < NTP; ++jj) {
      if (p0 + jj < NT) {
#pragma unroll
        for (int v = 0; v < 16; ++v) red[((wave * NTP + jj) * 64 + lane) * 17 + v] = acc[p0 + jj][v];
      }
    }
    __syncthreads();
    for (int e = tid; e < NTP * 1024; e += 256) {
      const int jj = e >> 10, q = (e >> 5) & 31, nn = e & 31;
      const int col = col0 + 32 * (p0 + jj) + nn;
      if (p0 + jj >= NT || col >= Rvp) continue;
      const int ln = nn + 32 * ((q >> 2) & 1), v = 4 * (q >> 3) + (q & 3);
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) s += red[((w * NTP + jj) * 64 + ln) * 17 + v];
      part[(int64_t)q * Rvp + col] = s;
    }
  }
  if constexpr (FUSED) {
    const float ps = add_halves(psum);
    if (hh == 0) Ps[wave][n] = ps;
    __syncthreads();
    if (cb == 0 && tid < 32) a.psum[((int64_t)b * a.n_c2 + c2) * 32 + tid] = Ps[0][tid] + Ps[1][tid] + Ps[2][tid] + Ps[3][tid];
  }

  // ---- fixed-order reduction of the chunk partials by the last workgroup
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = (atomicAdd(&a.counters[b * a.n_cb + cb], 1) == a.n_c2 - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const float* pb = a.part + ((int64_t)b * a.n_c2 * 32) * Rvp;
  for (int e = tid; e < 32 * NT * 32; e += 256) {
    const int q = e / (NT * 32), col = col0 + e % (NT * 32);
    if (col >= Rvp) continue;
    float s = 0.f;
    for (int c = 0; c < a.n_c2; ++c) s += pb[((int64_t)c * 32 + q) * Rvp + col];
    if constexpr (FUSED) {
      a.olat[((int64_t)b * 32 + q) * Rvp + col] = s;
    } else {
      if (q < H && col < a.Rv) ((VT*)a.out)[b * a.o_sb + q * a.o_sh + col] = (VT)s;
    }
  }
  if constexpr (FUSED) {
    if (cb == 0 && tid < 32) {
      float L = 0.f;
      for (int c = 0; c < a.n_c2; ++c) L += a.psum[((int64_t)b * a.n_c2 + c) * 32 + tid];
      a.lsum[b * 32 + tid] = L;
    }
  }
  if (tid == 0) a.counters[b * a.n_cb + cb] = 0;
}

constexpr int PV_NT = 8;

template <typename VT, bool FUSED>
static int launch_pv_t(const PVArgs& a, bool fast, int B, hipStream_t st) {
  dim3 grid(a.n_cb * a.n_c2, B), block(256);
  if (fast) hipLaunchKernelGGL((pv_kernel<VT, PV_NT, FUSED, true>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((pv_kernel<VT, PV_NT, FUSED, false>), grid, block, 0, st, a);
  return (int)hipGetLastError();
}

int launch_pv(const PVArgs& a, int dtype, bool fused, bool fast, int B, hipStream_t st) {
  if (dtype == STARKV_F16) return fused ? launch_pv_t<_Float16, true>(a, fast, B, st) : launch_pv_t<_Float16, false>(a, fast, B, st);
  return fused ? launch_pv_t<__bf16, true>(a, fast, B, st) : launch_pv_t<__bf16, false>(a, fast, B, st);
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
