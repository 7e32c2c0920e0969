// Skinny GEMM for decode batches (M <= 16 activation rows) on gfx950:
//   out[m][n] (=|+=) sum_k x[m][k] W[n][k]      (nn.Linear: y = x W^T)
//
// The weight is read once, so the kernel is an HBM weight stream with 8-16
// flops per weight byte; the design keeps as many weight bytes in flight as
// the CU's LDS holds, in whole 128-byte lines:
//
// * A workgroup owns one tile of 16 output columns = 16 weight rows (two
//   tiles for GEMM_SILU_MUL: the gate rows n and the up rows n + half_rows).
//   The weight is row-major or packed [N/16][K/64][16][64]: packed, each
//   wave's range of a tile is one contiguous, linearly streamed region (a
//   row-major tile is 16 streams one row pitch apart, which HBM serves
//   measurably slower);
//   its waves split the K range in pairs of 32-k MFMA steps and run
//   independently until the final reduction.
// * Each wave streams its range through its own LDS ring of `nst` stages
//   with global_load_lds (16 bytes per lane straight into LDS, no VGPRs held
//   by loads in flight).  A stage covers 64 k = 128 bytes of every row: per
//   weight tile two DMA instructions of 8 rows x one full 128-byte line, and
//   the activation rows (8 per instruction).  The count of DMA instructions
//   per stage is fixed (the tail re-issues a valid clamped pair into the
//   stage just consumed), so s_waitcnt vmcnt tells exactly when a stage has
//   landed.
// * In LDS, 16-byte chunk k of row r in 8-row block i sits at slot
//   k ^ ((r >> 1) + 4 i) of its 128-byte row: the MFMA operand reads below
//   (16 lanes = rows 0..15 of one chunk per ds_read_b128 cycle) then touch 16
//   distinct 16-byte bank groups.
// * v_mfma_f32_16x16x32 per step: B = 16 weight rows x 32 k (lane (c, g)
//   reads row c, chunk 4h + g of the stage), A = activation rows (lane (c, g)
//   reads row c; for M <= 8 rows c and c - 8 share a slot row, and output
//   rows >= M are never stored).  fp32 accumulation; the waves' partials meet
//   in LDS (reusing the rings) and wave 0 applies the epilogue:
//     GEMM_STORE     out = act(acc)
//     GEMM_ADD       out = act(acc + out)           (the residual add, in place)
//     GEMM_SILU_MUL  out = act(act(silu(act(acc_g))) * act(acc_u))
//                    (LlamaMLP's act_fn(gate_proj(x)) * up_proj(x) with torch's roundings)
//   act() rounds to the activation dtype.  With `rms`, x is the raw input of
//   an RMSNorm whose weight the caller folded into W: every wave also sums
//   x^2 over its range (from the A operands it reads anyway), and acc is
//   scaled by rsqrt(sum / K + eps) per row before the epilogue -- the norm
//   without a launch of its own.
#include <algorithm>

#include "common.hpp"

namespace starkv {

namespace {

typedef __attribute__((address_space(3))) void lds_void;

template <int N> __device__ inline void vm_wait() {
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 63]
__device__ inline void vm_wait_n(int n) {
  switch (n) {
#define SG_CASE(N) case N: vm_wait<N>(); break;
#define SG_CASE8(B) SG_CASE(B) SG_CASE(B + 1) SG_CASE(B + 2) SG_CASE(B + 3) SG_CASE(B + 4) SG_CASE(B + 5) \
                    SG_CASE(B + 6) SG_CASE(B + 7)
    SG_CASE8(0) SG_CASE8(8) SG_CASE8(16) SG_CASE8(24) SG_CASE8(32) SG_CASE8(40) SG_CASE8(48) SG_CASE8(56)
#undef SG_CASE8
#undef SG_CASE
    default: vm_wait<0>(); break;
  }
}

__device__ inline floatx4 mfma16(uint4 a, uint4 b, floatx4 c, _Float16*) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
}
__device__ inline floatx4 mfma16(uint4 a, uint4 b, floatx4 c, __bf16*) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                 0);
}

template <typename T> __device__ inline float round_act(float f) { return (float)(T)f; }

// element e of 8 packed activation values, in fp32
__device__ inline float act_elem(uint4 v, int e, _Float16*) { return (float)__builtin_bit_cast(half8, v)[e]; }
__device__ inline float act_elem(uint4 v, int e, __bf16*) {
  const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
  return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
}

// LDS byte offset, within an 8-row block, of 16-byte chunk k of row r (block i)
__device__ inline int sg_slot(int r, int k, int i) { return r * 128 + ((k ^ ((r >> 1) + 4 * i)) << 4); }

}  // namespace

template <typename T, int NT, int EPI>
__global__ __launch_bounds__(64 * GEMM_MAX_WAVES) void skinny_gemm_kernel(const GemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int nst = a.nst, pps = a.pps, xr = a.M > 8 ? 2 : 1;  // ring stages, pairs per stage, activation DMAs
  const int pb = NT * 2048 + xr * 1024;                     // bytes of one pair (64 k) in a stage
  const int sb = pps * pb;                                  // stage bytes
  const int cnt = pps * (NT * 2 + xr);                      // DMA instructions per stage
  uint8_t* ring = lds + w * nst * sb;
  const int pairs = a.K >> 6;
  const int p0 = (int)((int64_t)pairs * w / nw), np = (int)((int64_t)pairs * (w + 1) / nw) - p0;
  const int ns = (np + pps - 1) / pps;                      // stages of this wave
  const int64_t n0 = (int64_t)blockIdx.x * 16;

  // DMA lane mapping: slot row rs = lane / 8 of the instruction's 8 rows,
  // slot q = lane % 8 receives chunk q ^ ((rs >> 1) + 4 i) of its row
  const int rs = lane >> 3, q = lane & 7;
  const uint8_t* wsrc[NT][2];
  const uint8_t* xsrc[2];
  // weight rows: row-major [N][ws] (pairs 128 bytes apart), or packed
  // [N / 16][K / 64][16 rows][64 k] (a tile's pair = one contiguous 2 KB block)
  const int64_t pstep = a.wpk ? 2048 : 128;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t row = EPI == GEMM_SILU_MUL ? n0 + 8 * i + rs + t * (int64_t)a.half_rows
                                               : std::min(n0 + 8 * i + rs, (int64_t)a.N - 1);
      const int64_t chunk = (q ^ ((rs >> 1) + 4 * i)) << 4;
      wsrc[t][i] = a.wpk ? (const uint8_t*)a.w + ((row >> 4) * pairs + p0) * 2048 + (row & 15) * 128 + chunk
                         : (const uint8_t*)a.w + row * a.ws * 2 + chunk + (int64_t)p0 * 128;
    }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t row = std::min(8 * i + rs, a.M - 1);
    xsrc[i] = (const uint8_t*)a.x + row * a.xs * 2 + ((q ^ ((rs >> 1) + 4 * i)) << 4) + (int64_t)p0 * 128;
  }
  // stage j holds pairs j*pps .. j*pps + pps - 1 of the wave's range: the
  // rows' consecutive 128-byte blocks back to back (pairs past the range
  // re-read the last one and are not used)
  auto issue = [&](int j) __attribute__((always_inline)) {
    uint8_t* st = ring + (j % nst) * sb;
    for (int sp = 0; sp < pps; ++sp) {
      const int64_t pj = std::min(j * pps + sp, np - 1);
      uint8_t* sq = st + sp * pb;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 2; ++i)
          __builtin_amdgcn_global_load_lds((const void*)(wsrc[t][i] + pj * pstep), (lds_void*)(sq + (t * 2 + i) * 1024),
                                           16, 0, 0);
      for (int i = 0; i < xr; ++i)
        __builtin_amdgcn_global_load_lds((const void*)(xsrc[i] + pj * 128), (lds_void*)(sq + NT * 2048 + i * 1024), 16,
                                         0, 0);
    }
  };

  floatx4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  float ss = 0.f;                              // RMS-normalised input: this lane's sum of x^2 (row c)
  const bool rms = a.rms != 0;
  if (np > 0) {
    for (int j = 0; j < nst - 1; ++j) issue(j);
    const int xrow = xr == 2 ? c : (c & 7);
    for (int j = 0; j < ns; ++j) {
      vm_wait_n((nst - 2) * cnt);              // stage j landed; stages j+1 .. j+nst-2 may be in flight
      issue(j + nst - 1);                      // into the stage consumed at j - 1
      const uint8_t* st = ring + (j % nst) * sb;
      const int nsp = std::min(pps, np - j * pps);
      for (int sp = 0; sp < nsp; ++sp) {
        const uint8_t* sq = st + sp * pb;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint4 av = *(const uint4*)(sq + NT * 2048 + (xrow >> 3) * 1024 + sg_slot(xrow & 7, 4 * h + g, xrow >> 3));
          if (rms) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float v = act_elem(av, e, (T*)nullptr);
              ss = fmaf(v, v, ss);
            }
          }
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            const uint4 bv = *(const uint4*)(sq + (t * 2 + (c >> 3)) * 1024 + sg_slot(c & 7, 4 * h + g, c >> 3));
            acc[t] = mfma16(av, bv, acc[t], (T*)nullptr);
          }
        }
      }
    }
    vm_wait<0>();                              // the tail's re-issued stages, before the rings are reused
  }
  __syncthreads();
  floatx4* red = (floatx4*)lds;
  float* red_ss = (float*)(red + (nw - 1) * NT * 64);    // [wave][16 rows]
  if (rms) {
    // the four k-chunk lanes of row c, then the waves through LDS
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    if (g == 0) red_ss[w * 16 + c] = ss;
  }
  if (w > 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t) red[((w - 1) * NT + t) * 64 + lane] = acc[t];
  }
  __syncthreads();
  if (w > 0) return;
  for (int v = 0; v < nw - 1; ++v)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] += red[(v * NT + t) * 64 + lane];
  // per-row scale of the RMS-normalised input: rsqrt(mean(x^2) + eps)
  float rscale[4] = {1.f, 1.f, 1.f, 1.f};
  if (rms) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float tot = 0.f;
      for (int v = 0; v < nw; ++v) tot += red_ss[v * 16 + 4 * g + e];
      rscale[e] = rsqrtf(tot * (1.0f / (float)a.K) + a.rms_eps);
    }
  }
  // lane (c, g) holds rows 4g .. 4g+3 of column n0 + c
  const int64_t col = n0 + c;
  if (EPI != GEMM_SILU_MUL && col >= a.N) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = 4 * g + e;
    if (m >= a.M) break;
    T* o = (T*)a.out + m * a.os + col;
    if constexpr (EPI == GEMM_SILU_MUL) {
      const float gt = round_act<T>(rscale[e] * acc[0][e]), up = round_act<T>(rscale[e] * acc[1][e]);
      *o = (T)(round_act<T>(gt / (1.0f + expf(-gt))) * up);
    } else {
      float v = rscale[e] * acc[0][e];
      if constexpr (EPI == GEMM_ADD) v += (float)*o;
      *o = (T)v;
    }
  }
}

template <typename T, int NT, int EPI>
static int launch_gemm_t(const GemmArgs& a, int n_wg, int nw, size_t lds, hipStream_t st) {
  static bool attr = false;                    // dynamic LDS beyond 64 KB, once per instantiation
  if (!attr) {
    const int e = (int)hipFuncSetAttribute((const void*)skinny_gemm_kernel<T, NT, EPI>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
    if (e) return e;
    attr = true;
  }
  hipLaunchKernelGGL((skinny_gemm_kernel<T, NT, EPI>), dim3(n_wg), dim3(64 * nw), lds, st, a);
  return (int)hipGetLastError();
}

template <typename T>
static int launch_gemm_epi(const GemmArgs& a, int epi, int n_wg, int nw, size_t lds, hipStream_t st) {
  if (epi == GEMM_SILU_MUL) return launch_gemm_t<T, 2, GEMM_SILU_MUL>(a, n_wg, nw, lds, st);
  if (epi == GEMM_ADD) return launch_gemm_t<T, 1, GEMM_ADD>(a, n_wg, nw, lds, st);
  return launch_gemm_t<T, 1, GEMM_STORE>(a, n_wg, nw, lds, st);
}

int launch_skinny_gemm(const GemmArgs& a0, int dtype, int epi, hipStream_t st) {
  if (a0.M == 0) return 0;
  GemmArgs a = a0;
  const int nt = epi == GEMM_SILU_MUL ? 2 : 1;
  const int n_wg = epi == GEMM_SILU_MUL ? a.half_rows / 16 : (a.N + 15) / 16;
  const int xr = a.M > 8 ? 2 : 1;
  // Every tile resident at once: the workgroups that must share a CU split
  // its 160 KB of LDS.  Within that budget: as many waves as leave room for
  // three stages (at most one per pair of k steps), then longer stages (a
  // row's consecutive 128-byte blocks fetched back to back), then a deeper
  // ring, with at most 63 DMA instructions in flight (what vmcnt counts).
  const int pb = nt * 2048 + xr * 1024;
  const int per_cu = std::min(8, std::max(1, (n_wg + 255) / 256));
  const int budget = 163840 / per_cu;
  const int pairs = a.K >> 6;
  auto fits = [&](int nw, int nst, int pps) {
    return nw * nst * pps * pb <= budget && (nst - 2) * pps * (2 * nt + xr) <= 63;
  };
  int nw = GEMM_MAX_WAVES;
  while (nw > 1 && (!fits(nw, 3, 1) || nw > pairs)) nw /= 2;
  int pps = std::min(GEMM_PAIRS_PER_STAGE, std::max(1, pairs / nw));
  while (pps > 1 && !fits(nw, 3, pps)) --pps;
  int nst = GEMM_MAX_STAGES;
  while (nst > 3 && !fits(nw, nst, pps)) --nst;
  a.pps = pps;
  a.nst = nst;
  const int sbf = pps * pb;
  const size_t lds = std::max((size_t)nw * a.nst * sbf, (size_t)(nw - 1) * nt * 1024 + nw * 16 * 4);
  return dtype == STARKV_F16 ? launch_gemm_epi<_Float16>(a, epi, n_wg, nw, lds, st)
                             : launch_gemm_epi<__bf16>(a, epi, n_wg, nw, lds, st);
}

}  // namespace starkv
