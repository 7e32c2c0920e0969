// K3: softmax normalisation + per-head up-projection on gfx950.
//
// Replaces model.py:485-487 (v_u.weight viewed [Hkv, 128, Rv], repeated per
// query-head group, out = prob_v @ U^T):
//     out[b, q, d] = (1 / L[b,q]) * sum_j U_v[kv*128 + d][j] * o_lat[b, q, j]
// For KV head kv the rows (b, q in group(kv)) form one M x Rv matrix, so the
// product is a small GEMM per KV head on MFMA 32x32x16: A = o_lat rows split
// into hi + lo halves of the weight dtype (fp32-accurate), B = U_v rows read
// straight from the weight layout (the k-contiguous operand needs no
// transpose).  Workgroup = (32-column block of d, KV head, 32-row M-tile);
// its UP_WAVES waves split the Rv reduction (a handful of K-steps each, so the
// dependent load chains stay short) and are summed through LDS.
#include "common.hpp"

namespace starkv {

constexpr int UP_WAVES = 16;

template <typename WT, typename OT, bool FAST>
__global__ __launch_bounds__(UP_WAVES * 64) void up_proj_kernel(const UPArgs a) {
  __shared__ float red[UP_WAVES][64][17];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  const int db = blockIdx.x, kv = blockIdx.y, mt = blockIdx.z;
  const int gs = a.gs;

  // A row (lane n): M-row rho -> (b, g)
  const int rho = mt * 32 + n;
  const int rb = rho / gs, rg = rho % gs;
  const bool rok = rb < a.B;
  const int q = kv * gs + rg;
  const float invL = rok ? 1.0f / a.lsum[rb * 32 + q] : 0.f;
  const float* orow = a.olat + ((int64_t)(rok ? rb : 0) * 32 + q) * a.Rvp;
  const int d = db * 32 + n;
  const WT* urow = (const WT*)a.uv + (int64_t)(kv * HEAD_DIM + d) * a.uv_rs;

  const int nk = a.Rvp / KSTEP;
  const int per = (nk + UP_WAVES - 1) / UP_WAVES;
  const int k0 = wave * per, k1 = min(nk, k0 + per);

  floatx16 acc = floatx16{};
  for (int kk = k0; kk < k1; ++kk) {
    const int r0 = kk * KSTEP + 8 * hh;
    float o[8];
    if (rok) {
      const float4 u = *(const float4*)(orow + r0), v = *(const float4*)(orow + r0 + 4);
      o[0] = u.x; o[1] = u.y; o[2] = u.z; o[3] = u.w; o[4] = v.x; o[5] = v.y; o[6] = v.z; o[7] = v.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = 0.f;
    }
    uint4 bu = make_uint4(0, 0, 0, 0);
    if (FAST && r0 + 8 <= a.Rv) {
      bu = *(const uint4*)(urow + r0);
    } else {
      uint16_t tmp[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) tmp[e] = (r0 + e < a.Rv) ? ((const uint16_t*)urow)[r0 + e] : (uint16_t)0;
      bu = make_uint4(tmp[0] | (tmp[1] << 16), tmp[2] | (tmp[3] << 16), tmp[4] | (tmp[5] << 16), tmp[6] | (tmp[7] << 16));
    }
    if constexpr (__is_same(WT, _Float16)) {
      half8 ah, al;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = o[e] * invL;
        const _Float16 h = (_Float16)x;
        ah[e] = h;
        al[e] = (_Float16)(x - (float)h);
      }
      const half8 bv = __builtin_bit_cast(half8, bu);
      acc = mfma_f16(ah, bv, acc);
      acc = mfma_f16(al, bv, acc);
    } else {
      bf16x8 ah, al;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = o[e] * invL;
        const __bf16 h = (__bf16)x;
        ah[e] = h;
        al[e] = (__bf16)(x - (float)h);
      }
      const bf16x8 bv = __builtin_bit_cast(bf16x8, bu);
      acc = mfma_bf16(ah, bv, acc);
      acc = mfma_bf16(al, bv, acc);
    }
  }

#pragma unroll
  for (int v = 0; v < 16; ++v) red[wave][lane][v] = acc[v];
  __syncthreads();
  for (int e = tid; e < 1024; e += UP_WAVES * 64) {
    const int row = e >> 5, col = e & 31;          // D[row][col]
    const int ln = col + 32 * ((row >> 2) & 1), v = 4 * (row >> 3) + (row & 3);
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < UP_WAVES; ++w) s += red[w][ln][v];
    const int rr = mt * 32 + row;
    const int ob = rr / gs, og = rr % gs;
    if (ob < a.B) ((OT*)a.out)[ob * a.o_sb + (kv * gs + og) * a.o_sh + db * 32 + col] = (OT)s;
  }
}

template <typename WT, typename OT>
static void launch_up_t(const UPArgs& a, bool fast, dim3 grid, dim3 block, hipStream_t st) {
  if (fast) hipLaunchKernelGGL((up_proj_kernel<WT, OT, true>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((up_proj_kernel<WT, OT, false>), grid, block, 0, st, a);
}

int launch_up_proj(const UPArgs& a, int dtype, bool fast, hipStream_t st) {
  const int n_kv = a.Hq / a.gs;
  dim3 grid(HEAD_DIM / 32, n_kv, (unsigned)ceil_div((int64_t)a.B * a.gs, 32)), block(UP_WAVES * 64);
  if (dtype == STARKV_F16) {
    if (a.out_f32) launch_up_t<_Float16, float>(a, fast, grid, block, st);
    else launch_up_t<_Float16, _Float16>(a, fast, grid, block, st);
  } else {
    if (a.out_f32) launch_up_t<__bf16, float>(a, fast, grid, block, st);
    else launch_up_t<__bf16, __bf16>(a, fast, grid, block, st);
  }
  return (int)hipGetLastError();
}

}  // namespace starkv
