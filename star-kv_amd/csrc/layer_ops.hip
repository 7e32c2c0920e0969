// The e2e decoder layer's own elementwise work, one launch each (the
// attention path itself is in the other files):
//
// * rms_norm_kernel: HF LlamaRMSNorm (transformers models/llama/
//   modeling_llama.py, LlamaRMSNorm.forward), optionally after the residual
//   add that precedes it in LlamaDecoderLayer.forward:
//     x'  = act(x + residual)                       (when a residual is given; written out)
//     out = act(w * act(x' * rsqrt(mean(x'^2) + eps)))   mean and rsqrt in fp32
//   where act() rounds to the activation dtype, as torch does after each of
//   HF's fp16 / bf16 operations.  torch runs this as six or seven launches
//   (casts, pow, mean, rsqrt-multiply, weight multiply; the add).
//   One workgroup per row: the row stays in registers between the sum of
//   squares and the scaling (hidden <= 16384: at most 8 chunks of 8 values
//   per thread), the four waves' partial sums meet in LDS.
// * silu_mul_kernel: LlamaMLP's act_fn(gate_proj(x)) * up_proj(x) with
//   act_fn = SiLU: out = act(act(g / (1 + exp(-g))) * u), fp32 inside, over
//   the gate and up halves of one merged projection (or two tensors).
//
// Both are HBM-bound (2-3 bytes moved per element and a handful of VALU
// operations); at decode batch sizes they are latency-bound single waves of
// small workgroups, which is the point: one launch instead of several.
#include <algorithm>

#include "common.hpp"

namespace starkv {

namespace {

constexpr int NORM_THREADS = 256;
constexpr int NORM_MAXC = NORM_MAX_HIDDEN / 8 / NORM_THREADS;      // 16-byte chunks per thread

template <typename T> __device__ inline float elem_f32(uint4 v, int e);
template <> __device__ inline float elem_f32<_Float16>(uint4 v, int e) {
  return (float)__builtin_bit_cast(half8, v)[e];
}
template <> __device__ inline float elem_f32<__bf16>(uint4 v, int e) {
  const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
  return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
}

// eight fp32 values rounded to T (round to nearest even), packed
template <typename T> __device__ inline uint4 pack8(const float* f);
template <> __device__ inline uint4 pack8<_Float16>(const float* f) {
  half8 h;
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = (_Float16)f[e];
  return __builtin_bit_cast(uint4, h);
}
template <> __device__ inline uint4 pack8<__bf16>(const float* f) {
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const __bf16 lo = (__bf16)f[2 * k], hi = (__bf16)f[2 * k + 1];
    w[k] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// value of T nearest to f, back in fp32
template <typename T> __device__ inline float round_act(float f) { return (float)(T)f; }

}  // namespace

template <typename T, bool RES>
__global__ __launch_bounds__(NORM_THREADS) void rms_norm_kernel(const NormArgs a) {
  __shared__ float part[NORM_THREADS / 64];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int n8 = a.H >> 3;
  const uint8_t* x = (const uint8_t*)a.x + row * a.xs * 2;
  const uint8_t* r = RES ? (const uint8_t*)a.res + row * a.rs * 2 : nullptr;

  float v[NORM_MAXC][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NORM_MAXC; ++k) {
    const int c = tid + k * NORM_THREADS;
    if (c < n8) {
      const uint4 xv = *(const uint4*)(x + (int64_t)c * 16);
      if constexpr (RES) {
        const uint4 rv = *(const uint4*)(r + (int64_t)c * 16);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[k][e] = round_act<T>(elem_f32<T>(xv, e) + elem_f32<T>(rv, e));
        if (a.res_out) *(uint4*)((uint8_t*)a.res_out + (row * a.ros + (int64_t)c * 8) * 2) = pack8<T>(v[k]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[k][e] = elem_f32<T>(xv, e);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[k][e], v[k][e], ss);
    }
  }
  // row sum of squares: the wave by butterfly, the four waves through LDS
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  const float tot = (part[0] + part[1]) + (part[2] + part[3]);
  const float inv = rsqrtf(tot * (1.0f / (float)a.H) + a.eps);

  const uint8_t* w = (const uint8_t*)a.w;
#pragma unroll
  for (int k = 0; k < NORM_MAXC; ++k) {
    const int c = tid + k * NORM_THREADS;
    if (c < n8) {
      const uint4 wv = *(const uint4*)(w + (int64_t)c * 16);
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = elem_f32<T>(wv, e) * round_act<T>(v[k][e] * inv);
      *(uint4*)((uint8_t*)a.out + (row * a.os + (int64_t)c * 8) * 2) = pack8<T>(o);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(const SiluMulArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;     // (row, 8-value chunk)
  const int n8 = a.W >> 3;
  if (idx >= (int64_t)a.rows * n8) return;
  const int64_t row = idx / n8;
  const int c = (int)(idx - row * n8);
  const uint4 g = *(const uint4*)((const uint8_t*)a.g + (row * a.gs + (int64_t)c * 8) * 2);
  const uint4 u = *(const uint4*)((const uint8_t*)a.u + (row * a.us + (int64_t)c * 8) * 2);
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float gf = elem_f32<T>(g, e);
    const float s = round_act<T>(gf / (1.0f + expf(-gf)));
    o[e] = s * elem_f32<T>(u, e);
  }
  *(uint4*)((uint8_t*)a.out + (row * a.os + (int64_t)c * 8) * 2) = pack8<T>(o);
}

// ---------------------------------------------------------------------------
// Skinny GEMM for decode batches (M <= 16 activation rows):
//   out[m][n] (=|+=) sum_k x[m][k] W[n][k]      (nn.Linear: y = x W^T)
// The weight is streamed once, so the kernel is an HBM weight stream with
// 8-16 flops per weight byte.  A workgroup owns NT tiles of 16 output columns
// (16 weight rows each) and its waves split the K range; wave w runs
// v_mfma_f32_16x16x32 over its steps of 32 k: B operand = 16 weight rows x
// 32 k (lane (c, g) holds row c, k 8g..8g+7: one 16-byte load; cached, as a
// non-temporal load of half a 128-byte line measured 10-25 % slower),
// A operand = the activation rows (lane (c, g) holds row min(c, M-1), same k;
// rows >= M are never stored), eight steps of loads in flight per wave.  The
// waves' 16x16 fp32 partials meet in LDS and wave 0 applies the epilogue:
//   GEMM_STORE     out = act(acc)
//   GEMM_ADD       out = act(acc + out)        (the residual add, in place)
//   GEMM_SILU_MUL  tile 0 = gate rows n, tile 1 = up rows n + half_rows:
//                  out = act(act(silu(act(acc_g))) * act(acc_u))   (LlamaMLP's
//                  act_fn(gate_proj(x)) * up_proj(x) with torch's roundings)
// ---------------------------------------------------------------------------
constexpr int GEMM_UNROLL = 8;

__device__ inline floatx4 mfma16(uint4 a, uint4 b, floatx4 c, _Float16*) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
}
__device__ inline floatx4 mfma16(uint4 a, uint4 b, floatx4 c, __bf16*) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                 0);
}


template <typename T, int NT, int EPI>
__global__ __launch_bounds__(64 * GEMM_MAX_WAVES) void skinny_gemm_kernel(const GemmArgs a) {
  __shared__ floatx4 red[GEMM_MAX_WAVES - 1][NT][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * 16 * (EPI == GEMM_SILU_MUL ? 1 : NT);
  const int steps = a.K >> 5;
  const int s0 = (int)((int64_t)steps * w / nw), s1 = (int)((int64_t)steps * (w + 1) / nw);
  const uint8_t* xr = (const uint8_t*)a.x + ((int64_t)min(c, a.M - 1) * a.xs + 8 * g) * 2;
  const uint8_t* wr[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t row = n0 + c + (EPI == GEMM_SILU_MUL ? t * (int64_t)a.half_rows : 16 * t);
    wr[t] = (const uint8_t*)a.w + (row * a.ws + 8 * g) * 2;
  }
  floatx4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};

  int s = s0;
  for (; s + GEMM_UNROLL <= s1; s += GEMM_UNROLL) {
    uint4 xa[GEMM_UNROLL], wb[GEMM_UNROLL][NT];
#pragma unroll
    for (int u = 0; u < GEMM_UNROLL; ++u) {
#pragma unroll
      for (int t = 0; t < NT; ++t) wb[u][t] = *(const uint4*)(wr[t] + (int64_t)(s + u) * 64);
      xa[u] = *(const uint4*)(xr + (int64_t)(s + u) * 64);
    }
#pragma unroll
    for (int u = 0; u < GEMM_UNROLL; ++u)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = mfma16(xa[u], wb[u][t], acc[t], (T*)nullptr);
  }
  for (; s < s1; ++s) {
    const uint4 xa = *(const uint4*)(xr + (int64_t)s * 64);
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = mfma16(xa, *(const uint4*)(wr[t] + (int64_t)s * 64), acc[t], (T*)nullptr);
  }

  if (w > 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t) red[w - 1][t][lane] = acc[t];
  }
  __syncthreads();
  if (w > 0) return;
  for (int v = 0; v < nw - 1; ++v)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] += red[v][t][lane];
  // lane (c, g) holds rows 4g .. 4g+3 of column c
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = 4 * g + e;
    if (m >= a.M) break;
    if constexpr (EPI == GEMM_SILU_MUL) {
      const float gt = round_act<T>(acc[0][e]), up = round_act<T>(acc[1][e]);
      const float sl = round_act<T>(gt / (1.0f + expf(-gt)));
      ((T*)a.out)[m * a.os + n0 + c] = (T)(sl * up);
    } else {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        T* o = (T*)a.out + m * a.os + n0 + 16 * t + c;
        float v = acc[t][e];
        if constexpr (EPI == GEMM_ADD) v += (float)*o;
        *o = (T)v;
      }
    }
  }
}

template <typename T>
static int launch_gemm_t(const GemmArgs& a, int epi, int nw, hipStream_t st) {
  const dim3 block(64 * nw);
  if (epi == GEMM_SILU_MUL) {
    hipLaunchKernelGGL((skinny_gemm_kernel<T, 2, GEMM_SILU_MUL>), dim3(a.half_rows / 16), block, 0, st, a);
  } else if (epi == GEMM_ADD) {
    hipLaunchKernelGGL((skinny_gemm_kernel<T, 1, GEMM_ADD>), dim3(a.N / 16), block, 0, st, a);
  } else {
    hipLaunchKernelGGL((skinny_gemm_kernel<T, 1, GEMM_STORE>), dim3(a.N / 16), block, 0, st, a);
  }
  return (int)hipGetLastError();
}

int launch_skinny_gemm(const GemmArgs& a, int dtype, int epi, hipStream_t st) {
  if (a.M == 0) return 0;
  // waves per workgroup: split K so that about GEMM_TARGET_WAVES stream the weight
  const int n_wg = epi == GEMM_SILU_MUL ? a.half_rows / 16 : a.N / 16;
  const int nw = std::max(1, std::min({GEMM_MAX_WAVES, GEMM_TARGET_WAVES / n_wg, a.K / 32}));
  return dtype == STARKV_F16 ? launch_gemm_t<_Float16>(a, epi, nw, st) : launch_gemm_t<__bf16>(a, epi, nw, st);
}

int launch_rms_norm(const NormArgs& a, int dtype, hipStream_t st) {
  if (a.rows == 0) return 0;
  const dim3 grid((unsigned)a.rows), block(NORM_THREADS);
  const bool res = a.res != nullptr;
  if (dtype == STARKV_F16) {
    if (res) hipLaunchKernelGGL((rms_norm_kernel<_Float16, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((rms_norm_kernel<_Float16, false>), grid, block, 0, st, a);
  } else {
    if (res) hipLaunchKernelGGL((rms_norm_kernel<__bf16, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((rms_norm_kernel<__bf16, false>), grid, block, 0, st, a);
  }
  return (int)hipGetLastError();
}

int launch_silu_mul(const SiluMulArgs& a, int dtype, hipStream_t st) {
  const int64_t n = (int64_t)a.rows * (a.W >> 3);
  if (n == 0) return 0;
  const dim3 grid((unsigned)ceil_div(n, 256));
  if (dtype == STARKV_F16) hipLaunchKernelGGL(silu_mul_kernel<_Float16>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(silu_mul_kernel<__bf16>, grid, dim3(256), 0, st, a);
  return (int)hipGetLastError();
}

}  // namespace starkv
