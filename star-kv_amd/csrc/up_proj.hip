// K3: split-S reduction, softmax normalisation and per-head up-projection on
// gfx950.
//
// Replaces model.py:485-487 (v_u.weight viewed [Hkv, 128, Rv], repeated per
// query-head group, out = prob_v @ U^T) together with the sum over the P.V
// kernel's position chunks:
//     out[b, q, d] = (1 / L[b,q]) * sum_j U_v[kv*128 + d][j] * sum_c part_c[b, q, j]
//     L[b, q] = sum_c psum_c[b, q]
// up_proj_kernel: workgroup = (slice of SW V-rank columns, KV head kv); its
// rows are the M = B * gs (batch, query head of kv's group) pairs.  It sums
// the chunk partials of its columns in fixed chunk order into LDS, multiplies
// them by its U_v columns (fp32; the weights convert exactly) and writes the
// [M][128] partial up-projection of its slice.  When a row block has fewer
// rows than the workgroup has thread rows (small batch), the chunk range is
// cut into P contiguous parts summed side by side and added in part order.
// With few workgroups (small batch, few KV heads) the chunks are also cut
// into n_cs contiguous sets, one workgroup each (grid z): the up-projection
// is linear, so each set's projection is a partial of its own.
// up_finish_kernel adds the n_sl * n_cs partials in order and divides by L,
// one thread per output element; the 128 threads of a row share L's chunk
// sum.
// Every sum runs in a fixed order: the output is deterministic, with no
// atomics.
//
// Both kernels move a few MB and are latency-bound, so each thread issues
// its loads in batches of up to 64 independent addresses and adds them
// afterwards in their fixed order.
#include <algorithm>
#include <type_traits>

#include "common.hpp"

namespace starkv {

constexpr int UP_MB = 32;          // rows per LDS block
constexpr int UP_CB = 16;          // chunk partials loaded per row and batch

// sum of n values p[0], p[stride], ... in index order, UP_CB loads in flight
__device__ inline float sum_strided(const float* p, int64_t stride, int n) {
  float s = 0.f;
  for (int c = 0; c < n; c += UP_CB) {
    float v[UP_CB];
#pragma unroll
    for (int k = 0; k < UP_CB; ++k) v[k] = p[min(c + k, n - 1) * stride];
#pragma unroll
    for (int k = 0; k < UP_CB; ++k)
      if (c + k < n) s += v[k];
  }
  return s;
}

// U_v element e of a row held as packed 16-bit words, in fp32
__device__ inline float uv_elem(const uint4* w, int e, _Float16*) {
  const uint4 q = w[e >> 3];
  const uint32_t x = (e & 7) < 2 ? q.x : (e & 7) < 4 ? q.y : (e & 7) < 6 ? q.z : q.w;
  return (float)__builtin_bit_cast(kh2, x)[e & 1];
}
__device__ inline float uv_elem(const uint4* w, int e, __bf16*) {
  const uint4 q = w[e >> 3];
  const uint32_t x = (e & 7) < 2 ? q.x : (e & 7) < 4 ? q.y : (e & 7) < 6 ? q.z : q.w;
  return __uint_as_float((e & 1) ? (x & 0xffff0000u) : (x << 16));
}

// RB: rows per thread and batch of the chunk sums (the row block's rows over
// the JT thread rows, rounded up: 2 or 4).  P16: the partials are fp16,
// each divided by its chunk's softmax sum, which multiplies it back here
// (the sum's address is the same for every column of a row).
template <typename WT, int SW, bool FAST, int RB, bool P16>
__global__ __launch_bounds__(256) void up_proj_kernel(const UPArgs a) {
  typedef typename std::conditional<P16, _Float16, float>::type PT;
  constexpr int JT = 256 / SW;                     // rows summed side by side
  __shared__ float os[UP_MB][SW + 4];
  __shared__ float osp[JT][SW + 4];                // chunk-part sums (P > 1)
  const int tid = threadIdx.x;
  const int sl = blockIdx.x, kv = blockIdx.y, cs = blockIdx.z;
  const int cb0 = (int)((int64_t)cs * a.n_c2 / a.n_cs), cb1 = (int)((int64_t)(cs + 1) * a.n_c2 / a.n_cs);
  const int nc = cb1 - cb0;                               // this workgroup's chunks
  const int gs = a.gs, M = a.B * gs;
  const int j0 = sl * SW, nj = min(SW, a.Rv - j0);        // valid columns of the slice
  const int64_t cstr = (int64_t)32 * a.Rvp;               // next chunk's partials

  // this thread's U_v row (d) over the slice, kept as packed 16-bit words
  // (converted inside the multiply-adds); columns past the slice are zero
  const int d = tid & (HEAD_DIM - 1), mh = tid >> 7;
  const WT* urow = (const WT*)a.uv + (int64_t)(kv * HEAD_DIM + d) * a.uv_rs + j0;
  uint4 uraw[SW / 8];
  if (FAST && nj == SW) {
#pragma unroll
    for (int k = 0; k < SW / 8; ++k) uraw[k] = *(const uint4*)(urow + 8 * k);
  } else {
#pragma unroll
    for (int k = 0; k < SW / 8; ++k) {
      uint32_t w4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = 8 * k + 2 * e;
        const uint32_t lo = j < nj ? __builtin_bit_cast(uint16_t, urow[j]) : 0u;
        const uint32_t hi = j + 1 < nj ? __builtin_bit_cast(uint16_t, urow[j + 1]) : 0u;
        w4[e] = lo | (hi << 16);
      }
      uraw[k] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }
  }

  // P16: softmax sum of row m's chunk c (c relative to cb0)
  auto psum_of = [&](int m, int c) -> float {
    const int q = kv * gs + m % gs, bq = (m / gs) * a.n_hg + (q >> 5);
    return a.psum[((int64_t)bq * a.n_c2 + cb0 + c) * 32 + (q & 31)];
  };

  float* yp = a.ypart + (((int64_t)kv * a.n_sl + sl) * a.n_cs + cs) * M * HEAD_DIM;
  const int jj = tid % SW, mr = tid / SW;
  const int jc = j0 + min(jj, nj - 1);                    // columns past the slice re-read its last
  for (int m0 = 0; m0 < M; m0 += UP_MB) {
    const int mb = min(UP_MB, M - m0);
    const int P = mb < JT ? JT / mb : 1;           // chunk parts per row
    if (P > 1) {
      // thread row mr = part * mb + row sums chunks [c_lo, c_hi) of its row
      if (mr < P * mb) {
        const int part = mr / mb, m = m0 + mr % mb, q = kv * gs + m % gs;
        const int bq = (m / gs) * a.n_hg + (q >> 5);
        const int c_lo = cb0 + (int)((int64_t)part * nc / P), c_hi = cb0 + (int)((int64_t)(part + 1) * nc / P);
        const PT* p = (const PT*)a.part + ((int64_t)bq * a.n_c2 * 32 + (q & 31)) * a.Rvp + jc;
        float sp = 0.f;
        for (int c = c_lo; c < c_hi; c += UP_CB) {
          float v[UP_CB];
#pragma unroll
          for (int k = 0; k < UP_CB; ++k) {
            const int cc = min(c + k, c_hi - 1);
            v[k] = (float)p[cc * cstr];
            if constexpr (P16) v[k] *= psum_of(m, cc - cb0);
          }
#pragma unroll
          for (int k = 0; k < UP_CB; ++k)
            if (c + k < c_hi) sp += v[k];
        }
        osp[mr][jj] = sp;
      }
      __syncthreads();
      if (tid < mb * SW) {
        const int row = tid / SW, col = tid % SW;
        float sr = 0.f;
        for (int part = 0; part < P; ++part) sr += osp[part * mb + row][col];
        os[row][col] = col < nj ? sr : 0.f;
      }
    }
    // chunk sums of rows m0 .. m0+mb over the slice's columns: UP_RB rows
    // per thread at a time, UP_CB chunks each (rows past mb re-read row mb-1)
    for (int mm0 = mr; P == 1 && mm0 < mb; mm0 += JT * RB) {
      const PT* p[RB];
      int mrow[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int m = m0 + min(mm0 + JT * r, mb - 1), q = kv * gs + m % gs;
        const int bq = (m / gs) * a.n_hg + (q >> 5);
        p[r] = (const PT*)a.part + (((int64_t)bq * a.n_c2 + cb0) * 32 + (q & 31)) * a.Rvp + jc;
        mrow[r] = m;
      }
      float s[RB] = {};
      for (int c = 0; c < nc; c += UP_CB) {
        float v[RB][UP_CB];
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
          for (int k = 0; k < UP_CB; ++k) {
            const int cc = min(c + k, nc - 1);
            v[r][k] = (float)p[r][cc * cstr];
            if constexpr (P16) v[r][k] *= psum_of(mrow[r], cc);
          }
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
          for (int k = 0; k < UP_CB; ++k)
            if (c + k < nc) s[r] += v[r][k];
      }
#pragma unroll
      for (int r = 0; r < RB; ++r)
        if (mm0 + JT * r < mb) os[mm0 + JT * r][jj] = jj < nj ? s[r] : 0.f;
    }
    __syncthreads();
    // partial up-projection of the slice: two rows per pass (one per half block)
    for (int mm = mh; mm < mb; mm += 2) {
      float y[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < SW; j += 4) {
        const float4 o4 = *(const float4*)&os[mm][j];
        y[0] = fmaf(uv_elem(uraw, j, (WT*)nullptr), o4.x, y[0]);
        y[1] = fmaf(uv_elem(uraw, j + 1, (WT*)nullptr), o4.y, y[1]);
        y[2] = fmaf(uv_elem(uraw, j + 2, (WT*)nullptr), o4.z, y[2]);
        y[3] = fmaf(uv_elem(uraw, j + 3, (WT*)nullptr), o4.w, y[3]);
      }
      yp[(int64_t)(m0 + mm) * HEAD_DIM + d] = (y[0] + y[1]) + (y[2] + y[3]);
    }
    __syncthreads();
  }
}

// Sum of the slices' partial up-projections in slice order, times 1 / L.
// One thread per output element (row m of KV head kv, dim d); a workgroup
// holds two whole rows, and the 128 threads of a row sum L's chunk partials
// in contiguous parts, added in a fixed tree.
template <typename OT>
__global__ __launch_bounds__(256) void up_finish_kernel(const UPArgs a) {
  __shared__ float red[256];
  const int gs = a.gs, M = a.B * gs;
  const int tid = threadIdx.x;
  const int64_t e = (int64_t)blockIdx.x * 256 + tid;
  const int n_kv = a.Hq / gs;
  const bool valid = e < (int64_t)n_kv * M * HEAD_DIM;   // whole rows: a row is valid or not as a whole
  const int d = (int)(e % HEAD_DIM), m = (int)((e / HEAD_DIM) % M), kv = (int)(e / ((int64_t)HEAD_DIM * M));
  const int q = kv * gs + m % gs, b = m / gs;
  const int bq = b * a.n_hg + (q >> 5);
  float lp = 0.f;
  if (valid) {
    const int c_lo = (int)((int64_t)d * a.n_c2 / HEAD_DIM), c_hi = (int)((int64_t)(d + 1) * a.n_c2 / HEAD_DIM);
    if (c_hi > c_lo) lp = sum_strided(a.psum + ((int64_t)bq * a.n_c2 + c_lo) * 32 + (q & 31), 32, c_hi - c_lo);
  }
  red[tid] = lp;
  __syncthreads();
#pragma unroll
  for (int w = HEAD_DIM / 2; w >= 1; w >>= 1) {
    if (d < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  if (!valid) return;
  const float L = red[tid - d];
  const int np = a.n_sl * a.n_cs;                         // partial up-projections of the row
  const float s = sum_strided(a.ypart + ((int64_t)kv * np * M + m) * HEAD_DIM + d, (int64_t)M * HEAD_DIM, np);
  ((OT*)a.out)[b * a.o_sb + q * a.o_sh + d] = (OT)(s / L);
}

template <typename WT, int SW, int RB>
static void launch_up_rb(const UPArgs& a, bool fast, dim3 grid, hipStream_t st) {
  if (a.part16) {
    if (fast) hipLaunchKernelGGL((up_proj_kernel<WT, SW, true, RB, true>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((up_proj_kernel<WT, SW, false, RB, true>), grid, dim3(256), 0, st, a);
  } else {
    if (fast) hipLaunchKernelGGL((up_proj_kernel<WT, SW, true, RB, false>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((up_proj_kernel<WT, SW, false, RB, false>), grid, dim3(256), 0, st, a);
  }
}

template <typename WT, int SW>
static void launch_up_sw(const UPArgs& a, bool fast, dim3 grid, hipStream_t st) {
  // rows of the largest row block per thread row: two per batch suffice up to 2 * JT
  const int mb = std::min(UP_MB, a.B * a.gs);
  if (mb > 2 * (256 / SW)) launch_up_rb<WT, SW, 4>(a, fast, grid, st);
  else launch_up_rb<WT, SW, 2>(a, fast, grid, st);
}

template <typename WT>
static void launch_up_t(const UPArgs& a, bool fast, hipStream_t st) {
  const dim3 grid(a.n_sl, a.Hq / a.gs, a.n_cs);
  if (a.sw == 64) launch_up_sw<WT, 64>(a, fast, grid, st);
  else launch_up_sw<WT, 32>(a, fast, grid, st);
}

// slice width: 64 columns when that still gives a workgroup per CU, else 32
// (whole 128-byte lines of the partials either way)
int up_slice_width(int n_kv, int Rv, int cus) { return (int64_t)n_kv * ceil_div(Rv, 64) >= cus ? 64 : 32; }

// chunk sets: enough workgroups for two per CU, with at least 16 chunks each
int up_chunk_sets(int n_kv, int n_sl, int n_c2, int cus) {
  const int64_t wg = (int64_t)n_kv * n_sl;
  return (int)std::max<int64_t>(1, std::min<int64_t>(ceil_div(2 * cus, wg), n_c2 / 16));
}

int launch_up_proj(const UPArgs& a, int dtype, bool fast, hipStream_t st) {
  if (dtype == STARKV_F16) launch_up_t<_Float16>(a, fast, st);
  else launch_up_t<__bf16>(a, fast, st);
  int e = (int)hipGetLastError();
  if (e) return e;
  const int64_t n = (int64_t)(a.Hq / a.gs) * a.B * a.gs * HEAD_DIM;
  const dim3 grid((unsigned)ceil_div(n, 256));
  if (a.out_f32) hipLaunchKernelGGL(up_finish_kernel<float>, grid, dim3(256), 0, st, a);
  else if (dtype == STARKV_F16) hipLaunchKernelGGL(up_finish_kernel<_Float16>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(up_finish_kernel<__bf16>, grid, dim3(256), 0, st, a);
  return (int)hipGetLastError();
}

}  // namespace starkv
