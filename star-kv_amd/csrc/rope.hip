// RoPE rotation tables for the K-logit kernel.
//
// The reference recomputes cos/sin of 64 positions x 64 frequencies in every
// Triton program with NVIDIA fast intrinsics (abx_rope_batched.py:40-48).
// Here two small fp32 tables are built once per (inv_freq, max_positions):
//   T0[t][i]  = a * (cos, sin)(t * inv_freq[i])      t in [0, 32), a = attention scaling
//   RT[u][i]  = (cos, sin)((32*u) * inv_freq[i])     u in [0, n_tiles]
// The K-logit kernel seeds each chunk with the angle-addition of RT and T0
// and advances tile by tile with the fixed rotation RT[1].  Angles are the
// fp32 product inv_freq*pos, as HF forms them
// (HF:models/llama/modeling_llama.py:113-122); sincosf is ROCm's device libm.
#include "common.hpp"

namespace starkv {

struct InvFreq { float v[64]; };

__global__ void rope_tables_kernel(InvFreq f, float scaling, int rows, float* table) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;   // (row, freq)
  const int row = idx >> 6, i = idx & 63;
  if (row >= rows) return;
  const float pos = row < TILE ? (float)row : (float)((row - TILE) * TILE);
  const float ang = __fmul_rn(f.v[i], pos);
  float s, c;
  sincosf(ang, &s, &c);
  // the attention scaling rides on T0 only, so RT stays a pure rotation
  const float m = row < TILE ? scaling : 1.0f;
  table[2 * idx] = c * m;
  table[2 * idx + 1] = s * m;
}

int launch_rope_tables(const float* inv_freq_host, int max_positions, float scaling, float* table, hipStream_t st) {
  InvFreq f;
  for (int i = 0; i < 64; ++i) f.v[i] = inv_freq_host[i];
  const int n_tiles = (int)ceil_div(max_positions, TILE) + 2;
  const int rows = TILE + n_tiles;
  hipLaunchKernelGGL(rope_tables_kernel, dim3((unsigned)ceil_div(rows * 64, 256)), dim3(256), 0, st, f, scaling, rows, table);
  return (int)hipGetLastError();
}

}  // namespace starkv
