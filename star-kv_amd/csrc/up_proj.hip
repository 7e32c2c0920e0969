// K3: split-S reduction, softmax normalisation and per-head up-projection on
// gfx950, in one launch.
//
// Replaces model.py:485-487 (v_u.weight viewed [Hkv, 128, Rv], repeated per
// query-head group, out = prob_v @ U^T) together with the sum over the P.V
// kernel's position chunks:
//     out[b, q, d] = (1 / L[b,q]) * sum_j U_v[kv*128 + d][j] * sum_c part_c[b, q, j]
//     L[b, q] = sum_c psum_c[b, q]
// Workgroup = (slice of UP_SW V-rank columns, KV head kv).  Its rows are the
// M = B * gs (batch, query head of kv's group) pairs.  It sums the chunk
// partials of its columns in fixed chunk order into LDS, multiplies them by
// its U_v columns (fp32, the weights converted exactly) and writes the
// [M][128] partial up-projection of its slice.  The workgroup that completes
// a KV head last (an arrival counter per KV head, zeroed by the P.V kernel
// that runs before) adds the slices in slice order and divides by L, so the
// result does not depend on which workgroup arrives last: the output is
// deterministic, with no float atomics and no second launch.  Nothing waits
// on another workgroup.
#include "common.hpp"

namespace starkv {

constexpr int UP_MB = 64;          // rows per LDS block

template <typename WT, typename OT, bool FAST>
__global__ __launch_bounds__(256) void up_proj_kernel(const UPArgs a) {
  __shared__ float os[UP_MB][UP_SW + 4];
  __shared__ float Ls[UP_MB];
  __shared__ int is_last;
  const int tid = threadIdx.x;
  const int sl = blockIdx.x, kv = blockIdx.y;
  const int gs = a.gs, M = a.B * gs;
  const int j0 = sl * UP_SW, nj = min(UP_SW, a.Rv - j0);   // valid columns of the slice
  const int64_t cstr = (int64_t)32 * a.Rvp;               // next chunk's partials

  // this thread's U_v row (d) over the slice, in fp32
  const int d = tid & (HEAD_DIM - 1), mh = tid >> 7;
  float u[UP_SW];
  const WT* urow = (const WT*)a.uv + (int64_t)(kv * HEAD_DIM + d) * a.uv_rs + j0;
  if (FAST && nj == UP_SW) {
#pragma unroll
    for (int k = 0; k < UP_SW / 8; ++k) {
      const uint4 w = *(const uint4*)(urow + 8 * k);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        u[8 * k + 2 * e] = to_f32(__builtin_bit_cast(WT, (uint16_t)(ww[e] & 0xffffu)));
        u[8 * k + 2 * e + 1] = to_f32(__builtin_bit_cast(WT, (uint16_t)(ww[e] >> 16)));
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < UP_SW; ++j) u[j] = j < nj ? to_f32(urow[j]) : 0.f;
  }

  float* yp = a.ypart + ((int64_t)kv * a.n_sl + sl) * M * HEAD_DIM;
  for (int m0 = 0; m0 < M; m0 += UP_MB) {
    const int mb = min(UP_MB, M - m0);
    // chunk sums of rows m0 .. m0+mb over the slice's columns
    for (int e = tid; e < mb * UP_SW; e += 256) {
      const int mm = e / UP_SW, jj = e % UP_SW;
      const int m = m0 + mm, q = kv * gs + m % gs;
      const int bq = (m / gs) * a.n_hg + (q >> 5);
      float s = 0.f;
      if (jj < nj) {
        const float* p = a.part + ((int64_t)bq * a.n_c2 * 32 + (q & 31)) * a.Rvp + j0 + jj;
        int c = 0;
        for (; c + 8 <= a.n_c2; c += 8) {
          float v[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) v[k] = p[(c + k) * cstr];
#pragma unroll
          for (int k = 0; k < 8; ++k) s += v[k];
        }
        for (; c < a.n_c2; ++c) s += p[c * cstr];
      }
      os[mm][jj] = s;
    }
    __syncthreads();
    // partial up-projection of the slice: two rows per pass (one per half block)
    for (int mm = mh; mm < mb; mm += 2) {
      float y[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < UP_SW; j += 4) {
        const float4 o4 = *(const float4*)&os[mm][j];
        y[0] = fmaf(u[j], o4.x, y[0]);
        y[1] = fmaf(u[j + 1], o4.y, y[1]);
        y[2] = fmaf(u[j + 2], o4.z, y[2]);
        y[3] = fmaf(u[j + 3], o4.w, y[3]);
      }
      yp[(int64_t)(m0 + mm) * HEAD_DIM + d] = (y[0] + y[1]) + (y[2] + y[3]);
    }
    __syncthreads();
  }

  // arrival: the last slice of this KV head finishes the head
  __threadfence();
  __syncthreads();
  if (tid == 0) is_last = atomicAdd(&a.ctr[kv], 1) == a.n_sl - 1;
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  const float* y0 = a.ypart + (int64_t)kv * a.n_sl * M * HEAD_DIM;
  const int64_t sstr = (int64_t)M * HEAD_DIM;             // next slice
  for (int m0 = 0; m0 < M; m0 += UP_MB) {
    const int mb = min(UP_MB, M - m0);
    if (tid < mb) {
      const int m = m0 + tid, q = kv * gs + m % gs;
      const int bq = (m / gs) * a.n_hg + (q >> 5);
      const float* ps = a.psum + (int64_t)bq * a.n_c2 * 32 + (q & 31);
      float L = 0.f;
      for (int c = 0; c < a.n_c2; ++c) L += ps[c * 32];
      Ls[tid] = 1.0f / L;
    }
    __syncthreads();
    for (int mm = mh; mm < mb; mm += 2) {
      const float* yr = y0 + (int64_t)(m0 + mm) * HEAD_DIM + d;
      float s = 0.f;
      int k = 0;
      for (; k + 8 <= a.n_sl; k += 8) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = yr[(k + e) * sstr];
#pragma unroll
        for (int e = 0; e < 8; ++e) s += v[e];
      }
      for (; k < a.n_sl; ++k) s += yr[k * sstr];
      const int m = m0 + mm, b = m / gs, q = kv * gs + m % gs;
      ((OT*)a.out)[b * a.o_sb + q * a.o_sh + d] = (OT)(s * Ls[mm]);
    }
    __syncthreads();
  }
  if (tid == 0) a.ctr[kv] = 0;
}

template <typename WT, typename OT>
static void launch_up_t(const UPArgs& a, bool fast, dim3 grid, hipStream_t st) {
  if (fast) hipLaunchKernelGGL((up_proj_kernel<WT, OT, true>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((up_proj_kernel<WT, OT, false>), grid, dim3(256), 0, st, a);
}

int launch_up_proj(const UPArgs& a, int dtype, bool fast, hipStream_t st) {
  const dim3 grid(a.n_sl, a.Hq / a.gs);
  if (dtype == STARKV_F16) {
    if (a.out_f32) launch_up_t<_Float16, float>(a, fast, grid, st);
    else launch_up_t<_Float16, _Float16>(a, fast, grid, st);
  } else {
    if (a.out_f32) launch_up_t<__bf16, float>(a, fast, grid, st);
    else launch_up_t<__bf16, __bf16>(a, fast, grid, st);
  }
  return (int)hipGetLastError();
}

}  // namespace starkv
