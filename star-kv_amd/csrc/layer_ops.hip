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
