// Latent-cache writer on gfx950: quantise (or copy) new latent rows in place
// into a preallocated cache.
//
// Replaces the per-step cache growth of the reference -- HF DynamicLayer.update
// (HF:cache_utils.py:127-146, a torch.cat of the whole cache per token, reached
// from model.py:411-419) -- and the quantise-on-write of the quantised module
// (LlamaLoRaAttention_headwise_quant.py:107-127, whose quantize_r_split_int8_
// int4_packed the reference does not ship).  A "row" is one K latent vector
// (b, h, s) of rank r_h or one V latent vector (b, s) of rank Rv; one wave
// quantises one row:
//   int8 block:  s = fp16(amax / 127), q = clip(rint(x / s), -127, 127)
//   int4 block:  s = fp16(amax / 7),   n = clip(rint(x / s), -8, 7), nibble n + 8
//                (rank 2k in the low nibble of byte k)
//   group-64:    z = fp16(min), s = fp16((max - z) / 15), n = clip(rint((x - z) / s), 0, 15)
// with s = 1 when it would be 0, divisions correctly rounded and rint
// rounding half to even -- the rounding steps of the CPU oracle's quantisers.
// The cache is described by the same starkv_klatent / starkv_vlatent structs
// the attention entry points read.
#include "common.hpp"

namespace starkv {

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ inline float wave_min(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
  return v;
}

template <typename T>
__device__ inline float ldx(const T* p, int j) { return to_f32(p[j]); }

__device__ inline _Float16 fp16_scale(float amax, float qmax) {
  _Float16 s = (_Float16)__fdiv_rn(amax, qmax);
  return (float)s == 0.f ? (_Float16)1.0f : s;
}

// Quantise ranks [j0, j1) of the row at x (act dtype) as one symmetric block:
// int8 bytes into q8 (j - j0) or int4 nibbles into q4 ((j - j0) / 2); scale to *sp.
template <typename T>
__device__ void quant_block(const T* x, int j0, int j1, bool int8, uint8_t* q, uint16_t* sp, int lane) {
  float amax = 0.f;
  for (int j = j0 + lane; j < j1; j += 64) amax = fmaxf(amax, fabsf(ldx(x, j)));
  amax = wave_max(amax);
  const _Float16 s16 = fp16_scale(amax, int8 ? 127.f : 7.f);
  const float s = (float)s16;
  if (lane == 0) *sp = __builtin_bit_cast(uint16_t, s16);
  if (int8) {
    for (int j = j0 + lane; j < j1; j += 64) {
      const float n = fminf(fmaxf(rintf(__fdiv_rn(ldx(x, j), s)), -127.f), 127.f);
      q[j - j0] = (uint8_t)(int8_t)(int)n;
    }
  } else {
    for (int k = j0 + 2 * lane; k < j1; k += 128) {       // one byte = ranks k, k+1
      const float n0 = fminf(fmaxf(rintf(__fdiv_rn(ldx(x, k), s)), -8.f), 7.f);
      const float n1 = k + 1 < j1 ? fminf(fmaxf(rintf(__fdiv_rn(ldx(x, k + 1), s)), -8.f), 7.f) : 0.f;
      q[(k - j0) >> 1] = (uint8_t)(((int)n0 + 8) | (((int)n1 + 8) << 4));
    }
  }
}

// Group-64 asymmetric int4 of the row: nibbles into q, scale / zero of group g at sp[g] / zp[g].
// one group of 64 ranks (ranks g0 .. g0 + 63 of the row)
template <typename T>
__device__ void quant_g64(const T* x, int R, int g0, uint8_t* q, uint16_t* sp, uint16_t* zp, int lane) {
  {
    const int j = g0 + lane;
    const bool ok = j < R;
    const float v = ok ? ldx(x, j) : 0.f;
    const float lo = wave_min(ok ? v : INFINITY), hi = wave_max(ok ? v : -INFINITY);
    const _Float16 z16 = (_Float16)lo;
    const float z = (float)z16;
    _Float16 s16 = (_Float16)__fdiv_rn(hi - z, 15.f);
    if ((float)s16 == 0.f) s16 = (_Float16)1.0f;
    const float s = (float)s16;
    if (lane == 0) {
      sp[g0 / 64] = __builtin_bit_cast(uint16_t, s16);
      zp[g0 / 64] = __builtin_bit_cast(uint16_t, z16);
    }
    const int n = ok ? (int)fminf(fmaxf(rintf(__fdiv_rn(v - z, s)), 0.f), 15.f) : 0;
    const int n_odd = __shfl_xor(n, 1, 64);
    if (ok && !(lane & 1)) q[j >> 1] = (uint8_t)(n | (n_odd << 4));
  }
}

// one row per wave; 4 waves per workgroup (blk: the workgroup's index)
template <typename T>
__device__ inline void k_append_rows(const KAppendArgs& a, int64_t blk) {
  const int lane = threadIdx.x & 63;
  const int64_t row = blk * 4 + (threadIdx.x >> 6);
  if (row >= (int64_t)a.B * a.H * a.T) return;
  const int t = (int)(row % a.T), h = (int)((row / a.T) % a.H), b = (int)(row / ((int64_t)a.T * a.H));
  const int s = (a.pos0_dev ? *a.pos0_dev : a.pos0) + t, r = a.rank[h];
  if (s < 0 || s >= a.cap) {                        // only a run-time position can land here
    if (a.err != nullptr && lane == 0) *a.err = 1;
    return;
  }
  const T* x = (const T*)a.src + b * a.src_sb + a.src_off[h] + (int64_t)t * a.src_st;
  if (a.fmt == STARKV_FMT_DENSE) {
    T* d = (T*)a.data + b * a.stride_b + a.off[h] + (int64_t)s * a.pitch[h];
    for (int j = lane; j < r; j += 64) d[j] = x[j];
    return;
  }
  const int ra = min(r, a.split);
  uint8_t* qa = (uint8_t*)a.data + b * a.stride_b + a.off[h] + (int64_t)s * a.pitch[h];
  uint16_t* sa = (uint16_t*)a.scale + b * a.sc_sb + h * a.sc_sh + s;
  quant_block(x, 0, ra, a.a_int8, qa, sa, lane);
  if (r > a.split) {
    uint8_t* qb = (uint8_t*)a.data2 + b * a.stride2_b + a.off2[h] + (int64_t)s * a.pitch2[h];
    uint16_t* sb = (uint16_t*)a.scale2 + b * a.sc2_sb + h * a.sc2_sh + s;
    quant_block(x, a.split, r, false, qb, sb, lane);
  }
}

// one row per wave; group-64 int4: one (row, group) per wave
template <typename T>
__device__ inline void v_append_rows(const VAppendArgs& a, int64_t blk) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = blk * 4 + (threadIdx.x >> 6);
  const int64_t row = wid / a.gw;
  const int grp = (int)(wid - row * a.gw);
  if (row >= (int64_t)a.B * a.T) return;
  const int t = (int)(row % a.T), b = (int)(row / a.T);
  const int s = (a.pos0_dev ? *a.pos0_dev : a.pos0) + t, R = a.R;
  if (s < 0 || s >= a.cap) {                        // only a run-time position can land here
    if (a.err != nullptr && lane == 0) *a.err = 1;
    return;
  }
  const T* x = (const T*)a.src + b * a.src_sb + (int64_t)t * a.src_st;
  if (a.vq == VQ_DENSE) {
    T* d = (T*)a.data + b * a.stride_b + (int64_t)s * a.stride_s;
    for (int j = lane; j < R; j += 64) d[j] = x[j];
    return;
  }
  uint8_t* q = (uint8_t*)a.data + b * a.stride_b + (int64_t)s * a.stride_s;
  uint16_t* sp = (uint16_t*)a.scale + b * a.sc_sb + (int64_t)s * a.sc_ss;
  if (a.vq == VQ_G64) {
    quant_g64(x, R, 64 * grp, q, sp, (uint16_t*)a.zero + b * a.sc_sb + (int64_t)s * a.sc_ss, lane);
    return;
  }
  quant_block(x, 0, min(R, a.split), a.a_int8, q, sp, lane);
  if (R > a.split) {
    uint8_t* q2 = (uint8_t*)a.data2 + b * a.stride2_b + (int64_t)s * a.stride2_s;
    uint16_t* s2 = (uint16_t*)a.scale2 + b * a.sc2_sb + (int64_t)s * a.sc2_ss;
    quant_block(x, a.split, R, false, q2, s2, lane);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void k_append_kernel(const KAppendArgs a) {
  k_append_rows<T>(a, blockIdx.x);
}
template <typename T>
__global__ __launch_bounds__(256) void v_append_kernel(const VAppendArgs a) {
  v_append_rows<T>(a, blockIdx.x);
}

// A decode step's three small writes in one launch: workgroups [0, nbk) write
// the K rows, [nbk, nbk + nbv) the V rows, the rest rotate the query rows
// (64 threads per row, as rope_apply_kernel).
template <typename T>
__global__ __launch_bounds__(256) void step_append_kernel(const StepAppendArgs a) {
  int64_t blk = blockIdx.x;
  if (blk < a.nbk) {
    k_append_rows<T>(a.k, blk);
    return;
  }
  blk -= a.nbk;
  if (blk < a.nbv) {
    v_append_rows<T>(a.v, blk);
    return;
  }
  blk -= a.nbv;
  rope_apply_row<T>(a.r, blk * 256 + threadIdx.x);
}

int launch_step_append(const StepAppendArgs& a0, int dtype, hipStream_t st) {
  StepAppendArgs a = a0;
  a.v.gw = a.v.vq == VQ_G64 ? (int)ceil_div(a.v.R, 64) : 1;
  a.nbk = ceil_div((int64_t)a.k.B * a.k.H * a.k.T, 4);
  a.nbv = ceil_div((int64_t)a.v.B * a.v.T * a.v.gw, 4);
  const int64_t nbr = a.has_rope ? ceil_div((int64_t)a.r.B * a.r.H * a.r.T * 64, 256) : 0;
  const int64_t n = a.nbk + a.nbv + nbr;
  if (n == 0) return 0;
  if (dtype == STARKV_F16) hipLaunchKernelGGL(step_append_kernel<_Float16>, dim3((unsigned)n), dim3(256), 0, st, a);
  else hipLaunchKernelGGL(step_append_kernel<__bf16>, dim3((unsigned)n), dim3(256), 0, st, a);
  return (int)hipGetLastError();
}

int launch_k_append(const KAppendArgs& a, int dtype, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.H * a.T;
  if (rows == 0) return 0;
  const dim3 grid((unsigned)ceil_div(rows, 4));
  if (dtype == STARKV_F16) hipLaunchKernelGGL(k_append_kernel<_Float16>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(k_append_kernel<__bf16>, grid, dim3(256), 0, st, a);
  return (int)hipGetLastError();
}

int launch_v_append(const VAppendArgs& a, int dtype, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.T;
  if (rows == 0) return 0;
  VAppendArgs r = a;
  r.gw = a.vq == VQ_G64 ? (int)ceil_div(a.R, 64) : 1;
  const dim3 grid((unsigned)ceil_div(rows * r.gw, 4));
  if (dtype == STARKV_F16) hipLaunchKernelGGL(v_append_kernel<_Float16>, grid, dim3(256), 0, st, r);
  else hipLaunchKernelGGL(v_append_kernel<__bf16>, grid, dim3(256), 0, st, r);
  return (int)hipGetLastError();
}

}  // namespace starkv
