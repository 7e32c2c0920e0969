// RoPE operand table for the K-logit kernel.
//
// The reference recomputes cos/sin of 64 positions x 64 frequencies in every
// Triton program with NVIDIA fast intrinsics (abx_rope_batched.py:40-48) and
// hard-codes theta=10000 (184).  Here the rotation operand of the K-logit
// MFMA is tabulated once per (inv_freq, attention scaling, max positions),
// already in the register layout of the 32x32x16 f16 MFMA B operand, so the
// kernel fetches it with one coalesced 16-byte load per lane and K-step:
//
//   table[tile][k][lane][e]   (fp16; tile = 32 positions, k = 0..7, lane = 0..63, e = 0..7)
//     position s = 32*tile + (lane % 32)
//     frequency i = 8*k + 4*(lane / 32) + e/2
//     value = a * cos(s*inv_freq[i]) for even e, a * sin(s*inv_freq[i]) for odd e
//
// Angles are the fp32 product inv_freq*s as HF forms them
// (HF:models/llama/modeling_llama.py:113-126); sincosf is ROCm's device libm.
#include "common.hpp"

namespace starkv {

struct InvFreq { float v[64]; };

__global__ void rope_table_kernel(InvFreq f, float scaling, int n_tiles, uint4* table) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;   // (tile, k, lane)
  if (idx >= n_tiles * 512) return;
  const int tile = idx >> 9, k = (idx >> 6) & 7, lane = idx & 63;
  const float pos = (float)(tile * TILE + (lane & 31));
  half8 h;
#pragma unroll
  for (int f4 = 0; f4 < 4; ++f4) {
    const int i = 8 * k + 4 * (lane >> 5) + f4;
    const float ang = __fmul_rn(f.v[i], pos);
    float s, c;
    sincosf(ang, &s, &c);
    h[2 * f4] = (_Float16)(c * scaling);
    h[2 * f4 + 1] = (_Float16)(s * scaling);
  }
  table[idx] = __builtin_bit_cast(uint4, h);
}

// In-place rotation of [B][H][T][128] rows by the table (rope_apply_row):
// one thread per (row, frequency i < 64).
template <typename T>
__global__ void rope_apply_kernel(RopeApplyArgs a) {
  rope_apply_row<T>(a, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

int launch_rope_apply(const RopeApplyArgs& a, int dtype, hipStream_t st) {
  const int64_t n = (int64_t)a.B * a.H * a.T * 64;
  if (n == 0) return 0;
  const dim3 grid((unsigned)ceil_div(n, 256));
  if (dtype == STARKV_F16) hipLaunchKernelGGL(rope_apply_kernel<_Float16>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(rope_apply_kernel<__bf16>, grid, dim3(256), 0, st, a);
  return (int)hipGetLastError();
}

int rope_table_tiles(int max_positions) { return (int)ceil_div(max_positions, TILE); }

int launch_rope_table(const float* inv_freq_host, int max_positions, float scaling, void* table, hipStream_t st) {
  InvFreq f;
  for (int i = 0; i < 64; ++i) f.v[i] = inv_freq_host[i];
  const int n_tiles = rope_table_tiles(max_positions);
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)ceil_div((int64_t)n_tiles * 512, 256)), dim3(256), 0, st,
                     f, scaling, n_tiles, (uint4*)table);
  return (int)hipGetLastError();
}

}  // namespace starkv
