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
// up_finish_kernel adds the n_sl * n_cs partials and divides by L, one
// workgroup per output row: each half of it sums half of the partials in
// order, all 256 threads sum L's chunk partials in contiguous parts, added in
// a fixed tree.
// Every sum runs in a fixed order: the output is deterministic, with no
// atomics.
//
// Both kernels move a few MB and are latency-bound, so each thread issues
// its loads in batches of up to 64 independent addresses and adds them
// afterwards in their fixed order.  The U_v slice is read in whole 16-byte
// pieces by consecutive lanes (each wave instruction covers 8 rows of 128
// bytes) into registers before the chunk partials, and reaches each thread's
// row through LDS after the chunk sums, so the two loads overlap.
#include <algorithm>
#include <type_traits>

#include "common.hpp"

namespace starkv {

constexpr int UP_MB = 32;          // rows per LDS block
constexpr int UP_CB = 16;          // chunk partials loaded per row and batch
constexpr int UP_CB1 = 32;         // the same with one row per thread (chunk parts)

// sum of n values p[0], p[stride], ... in index order, CB loads in flight
template <int CB = UP_CB>
__device__ inline float sum_strided(const float* p, int64_t stride, int n) {
  float s = 0.f;
  for (int c = 0; c < n; c += CB) {
    float v[CB];
#pragma unroll
    for (int k = 0; k < CB; ++k) v[k] = p[min(c + k, n - 1) * stride];
#pragma unroll
    for (int k = 0; k < CB; ++k)
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
// Register budget: four waves per SIMD (at most 128 VGPRs), so that the
// workgroups of a decode-sized grid are resident in one round (bf16 weights
// with 64-column slices stay at three: their conversions would spill).
template <typename WT, int SW>
constexpr int up_waves() { return std::is_same<WT, __bf16>::value && SW == 64 ? 3 : 4; }
template <typename WT, int SW, bool FAST, int RB, bool P16>
__global__ __launch_bounds__(256, (up_waves<WT, SW>())) void up_proj_kernel(const UPArgs a) {
  typedef typename std::conditional<P16, _Float16, float>::type PT;
  constexpr int JT = 256 / SW;                     // rows summed side by side
  constexpr int PR = SW / 8, UL = HEAD_DIM * PR / 256;    // U_v pieces per slice row; per thread
  constexpr int HW = SW / 2;                       // columns per projection half
  constexpr int USH = std::max(HEAD_DIM * (PR + 1), UP_MB * HEAD_DIM / 4);
  __shared__ float os[UP_MB][SW + 4];
  __shared__ float osp[JT][SW + 4];                // chunk-part sums (P > 1)
  // U_v slice rows as 16-bit words (one 16-byte piece of padding per row);
  // once every thread holds its half row, the second half's projections
  __shared__ uint4 ush[USH];
  const int tid = threadIdx.x;
  const int sl = blockIdx.x, kv = blockIdx.y, cs = blockIdx.z;
  const int cb0 = (int)((int64_t)cs * a.n_c2 / a.n_cs), cb1 = (int)((int64_t)(cs + 1) * a.n_c2 / a.n_cs);
  const int nc = cb1 - cb0;                               // this workgroup's chunks
  const int gs = a.gs, M = a.B * gs;
  const int j0 = sl * SW, nj = min(SW, a.Rv - j0);        // valid columns of the slice
  const int64_t cstr = (int64_t)32 * a.Rvp;               // next chunk's partials

  // the U_v slice, piece e = tid + 256 i (row e / PR, columns 8 (e % PR) ..
  // + 7): whole 16-byte loads by consecutive lanes, or element loads with
  // zeros past the slice; stored to LDS after the chunk sums
  uint4 ust[UL];
#pragma unroll
  for (int i = 0; i < UL; ++i) {
    const int e = tid + 256 * i, r = e / PR, k = e % PR;
    const WT* src = (const WT*)a.uv + (int64_t)(kv * HEAD_DIM + r) * a.uv_rs + j0 + 8 * k;
    if (FAST && nj == SW) {
      ust[i] = *(const uint4*)src;
    } else {
      // (loads at clamped indices, all issued before the selects)
      const WT* row = src - 8 * k;
      uint16_t e8[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) e8[t] = __builtin_bit_cast(uint16_t, row[min(8 * k + t, nj - 1)]);
      uint32_t w4[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int j = 8 * k + 2 * t;
        w4[t] = (j < nj ? (uint32_t)e8[2 * t] : 0u) | ((j + 1 < nj ? (uint32_t)e8[2 * t + 1] : 0u) << 16);
      }
      ust[i] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }
  }

  // P16: softmax sum of row m's chunk c (c relative to cb0)
  auto psum_of = [&](int m, int c) -> float {
    const int q = kv * gs + m % gs, bq = (m / gs) * a.n_hg + (q >> 5);
    return a.psum[((int64_t)bq * a.n_c2 + cb0 + c) * 32 + (q & 31)];
  };

  // projection: thread (half h, dim d) holds U_v row d over columns
  // [h * HW, (h + 1) * HW) of the slice
  const int d = tid & (HEAD_DIM - 1), h = tid >> 7;
  uint4 ureg[PR / 2];
  float* yp = a.ypart + (((int64_t)kv * a.n_sl + sl) * a.n_cs + cs) * M * HEAD_DIM;
  const int jj = tid % SW;
  // thread row (wave-uniform with 64-column slices: scalar row addresses)
  const int mr = SW == 64 ? __builtin_amdgcn_readfirstlane(tid / SW) : tid / SW;
  const int jc = j0 + min(jj, nj - 1);                    // columns past the slice re-read its last
  // P16 with 64-column slices: a wave's lanes share their rows, so lane l
  // loads the softmax sum of chunk c + l % (chunks per batch) and each
  // multiply takes it from that lane as a scalar (one register per row and
  // batch instead of one per chunk)
  constexpr bool PLANE = P16 && SW == 64;
  const int lane = tid & 63;
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
        for (int c = c_lo; c < c_hi; c += UP_CB1) {
          float v[UP_CB1];
          float pl = 0.f;                          // PLANE: lane l holds chunk c + l % UP_CB1's sum
          if constexpr (PLANE) pl = psum_of(m, min(c + lane % UP_CB1, c_hi - 1) - cb0);
#pragma unroll
          for (int k = 0; k < UP_CB1; ++k) {
            const int cc = min(c + k, c_hi - 1);
            v[k] = (float)p[cc * cstr];
            if constexpr (P16 && !PLANE) v[k] *= psum_of(m, cc - cb0);
          }
#pragma unroll
          for (int k = 0; k < UP_CB1; ++k) {
            if constexpr (PLANE) v[k] *= __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pl), k));
            if (c + k < c_hi) sp += v[k];
          }
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
    // chunk sums of rows m0 .. m0+mb over the slice's columns: RB rows per
    // thread at a time, CB chunks each, 32 loads in flight; rows past mb
    // re-read row mb-1
    constexpr int CB = 32 / RB;
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
      for (int c = 0; c < nc; c += CB) {
        float v[RB][CB];
        float pl[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          if constexpr (PLANE) pl[r] = psum_of(mrow[r], min(c + lane % CB, nc - 1));
#pragma unroll
          for (int k = 0; k < CB; ++k) {
            const int cc = min(c + k, nc - 1);
            v[r][k] = (float)p[r][cc * cstr];
            if constexpr (P16 && !PLANE) v[r][k] *= psum_of(mrow[r], cc);
          }
        }
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
          for (int k = 0; k < CB; ++k) {
            if constexpr (PLANE)
              v[r][k] *= __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pl[r]), k));
            if (c + k < nc) s[r] += v[r][k];
          }
      }
#pragma unroll
      for (int r = 0; r < RB; ++r)
        if (mm0 + JT * r < mb) os[mm0 + JT * r][jj] = jj < nj ? s[r] : 0.f;
    }
    if (m0 == 0) {
#pragma unroll
      for (int i = 0; i < UL; ++i) {
        const int e = tid + 256 * i;
        ush[(e / PR) * (PR + 1) + e % PR] = ust[i];
      }
    }
    __syncthreads();
    if (m0 == 0) {
#pragma unroll
      for (int k = 0; k < PR / 2; ++k) ureg[k] = ush[d * (PR + 1) + h * (PR / 2) + k];
    }
    // partial up-projection of the slice's half h for every row of the block
    float acc[UP_MB];
#pragma unroll
    for (int r = 0; r < UP_MB; ++r) {
      acc[r] = 0.f;
      if (r < mb) {
#pragma unroll
        for (int j = 0; j < HW; j += 4) {
          const float4 o4 = *(const float4*)&os[r][h * HW + j];
          acc[r] = fmaf(uv_elem(ureg, j, (WT*)nullptr), o4.x, acc[r]);
          acc[r] = fmaf(uv_elem(ureg, j + 1, (WT*)nullptr), o4.y, acc[r]);
          acc[r] = fmaf(uv_elem(ureg, j + 2, (WT*)nullptr), o4.z, acc[r]);
          acc[r] = fmaf(uv_elem(ureg, j + 3, (WT*)nullptr), o4.w, acc[r]);
        }
      }
    }
    __syncthreads();                               // every half row read from ush
    float* yx = (float*)ush;
    if (h) {
#pragma unroll
      for (int r = 0; r < UP_MB; ++r)
        if (r < mb) yx[r * HEAD_DIM + d] = acc[r];
    }
    __syncthreads();
    if (!h) {
#pragma unroll
      for (int r = 0; r < UP_MB; ++r)
        if (r < mb) yp[(int64_t)(m0 + r) * HEAD_DIM + d] = acc[r] + yx[r * HEAD_DIM + d];
    }
    __syncthreads();
  }
}

// Sum of the slices' partial up-projections, times 1 / L.  Workgroup = one
// output row (row m of KV head kv): thread (half h, dim d) sums partials
// [h * np / 2, (h + 1) * np / 2) in order and half 0 adds half 1's sum; the
// 256 threads sum L's chunk partials in contiguous parts, added in a fixed
// tree.
template <typename OT>
__global__ __launch_bounds__(256) void up_finish_kernel(const UPArgs a) {
  __shared__ float red[256];
  __shared__ float ys[HEAD_DIM];
  const int gs = a.gs, M = a.B * gs;
  const int tid = threadIdx.x, d = tid & (HEAD_DIM - 1), h = tid >> 7;
  const int kv = blockIdx.x / M, m = blockIdx.x % M;
  const int q = kv * gs + m % gs, b = m / gs;
  const int bq = b * a.n_hg + (q >> 5);
  const int c_lo = (int)((int64_t)tid * a.n_c2 / 256), c_hi = (int)((int64_t)(tid + 1) * a.n_c2 / 256);
  const float lp = c_hi > c_lo ? sum_strided(a.psum + ((int64_t)bq * a.n_c2 + c_lo) * 32 + (q & 31), 32, c_hi - c_lo) : 0.f;
  const int np = a.n_sl * a.n_cs;                         // partial up-projections of the row
  const int p_lo = h * np / 2, p_hi = (h + 1) * np / 2;
  const float s = p_hi > p_lo ? sum_strided<UP_CB1>(a.ypart + (((int64_t)kv * np + p_lo) * M + m) * HEAD_DIM + d,
                                                    (int64_t)M * HEAD_DIM, p_hi - p_lo) : 0.f;
  red[tid] = lp;
  if (h) ys[d] = s;
  __syncthreads();
#pragma unroll
  for (int w = 128; w >= 1; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  if (h) return;
  ((OT*)a.out)[b * a.o_sb + q * a.o_sh + d] = (OT)((s + ys[d]) / red[0]);
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
  const dim3 grid((unsigned)((a.Hq / a.gs) * a.B * a.gs));
  if (a.out_f32) hipLaunchKernelGGL(up_finish_kernel<float>, grid, dim3(256), 0, st, a);
  else if (dtype == STARKV_F16) hipLaunchKernelGGL(up_finish_kernel<_Float16>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(up_finish_kernel<__bf16>, grid, dim3(256), 0, st, a);
  return (int)hipGetLastError();
}

}  // namespace starkv
