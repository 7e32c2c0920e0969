// K1: latent-K decode logits on gfx950.
//
// Replaces the Triton _abx_fwd kernel (abx_rope_batched.py:55-132): for every
// cached position s and query head q,
//     logit[b,q,s] = scale * q_rot[b,q] . RoPE_s(X_k[b,kv,s,:] @ B_k[kv])   (kv = q // gs)
//
// Formulation.  With c = 2i+tau interleaving the 64 RoPE frequencies i with
// cos (tau=0) and sin (tau=1), the rotate_half RoPE and the dot with q fold
// into a per-(b,q) matrix W[j][c] (rank j x 128):
//     W[j][2i]   = scale * (B_k[j][i] q[i]    + B_k[j][i+64] q[i+64])
//     W[j][2i+1] = scale * (B_k[j][i] q[i+64] - B_k[j][i+64] q[i])
//     logit[s]   = sum_j X_k[s][j] * V[j][s],   V = W . T,  T[c][s] = (cos|sin)(s*theta_i)
// V for a 32-position tile is one chain of eight 32x32x16 f16 MFMAs per 32
// ranks (K = the 128 rotation coefficients).  The rotation operand T comes
// from a table already laid out as the MFMA B operand (rope.hip), shared by
// every head and batch through L2 and by the waves of a workgroup through LDS.
// The MFMA output rows are permuted so that each lane holds 16 consecutive
// ranks of one position: the latent X enters only through one fused
// multiply-add per element, read with two 16-byte loads per lane, and a
// head's logit needs one half-wave swap.
//
// Work decomposition: grid (chunk of positions, workgroup plan, batch).
// Each wave owns whole query heads: up to 2 items (query head, 32-rank
// M-tile) in 8-wave workgroups, or up to 4 in 4-wave workgroups when a head
// has rank > 64, packed on the host so ragged head-wise ranks are balanced.
// A wave streams its latent rows two tiles ahead in registers; the MFMA
// result of each item is consumed before the next item's MFMAs.
#include <climits>

#include "common.hpp"

namespace starkv {

template <typename XT>
__device__ inline void load4(const XT* p, float* out) {
  // four consecutive elements (8 bytes, 8-byte aligned)
  uint2 u = *(const uint2*)p;
  if constexpr (__is_same(XT, _Float16)) {
    half4 h = __builtin_bit_cast(half4, u);
    out[0] = (float)h[0]; out[1] = (float)h[1]; out[2] = (float)h[2]; out[3] = (float)h[3];
  } else {
    out[0] = __uint_as_float(u.x << 16); out[1] = __uint_as_float(u.x & 0xffff0000u);
    out[2] = __uint_as_float(u.y << 16); out[3] = __uint_as_float(u.y & 0xffff0000u);
  }
}

template <typename XT>
__device__ inline void load4_any(const XT* p, float* out) {
  for (int e = 0; e < 4; ++e) out[e] = to_f32(p[e]);
}

// dot of 8 packed 16-bit latent elements with 8 fp32 accumulators
template <typename XT>
__device__ inline float dot8(uint4 u, const floatx16& acc, int v0, float part) {
  if constexpr (__is_same(XT, _Float16)) {
    const half8 h = __builtin_bit_cast(half8, u);
#pragma unroll
    for (int v = 0; v < 8; ++v) part = fmaf((float)h[v], acc[v0 + v], part);
  } else {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      part = fmaf(__uint_as_float(w[v] << 16), acc[v0 + 2 * v], part);
      part = fmaf(__uint_as_float(w[v] & 0xffff0000u), acc[v0 + 2 * v + 1], part);
    }
  }
  return part;
}

// Latent loads are cached: one instruction reads 16 bytes of each of 32
// position rows, so the other pieces of each cache line are picked up by the
// item's next load from L1/L2 (non-temporal loads would refetch the line).
__device__ inline uint4 ld_stream(const void* p) { return *(const uint4*)p; }
__device__ inline uint2 ld_stream8(const void* p) { return *(const uint2*)p; }

// native vector type: a HIP uint4 assignment between address spaces lowers to
// a memcpy that keeps the staging registers in scratch memory
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int G, int TPT>
struct TStage {
  u32x4 v[G][TPT];       // rotation pieces of one staging group (this thread's share)
};

template <int XFMT, int MAXI>
struct KBuf {
  uint4 x[MAXI][XFMT == 0 ? 2 : 1];   // latent: 16 ranks of one position per lane (quantised: packed)
  uint16_t sq[XFMT == 0 ? 1 : MAXI];  // quantised: fp16 scale bits of the lane's block at that position
};

// XFMT: 0 = dense act dtype, 1 = quantised blocks (int8 / int4 with per-(b,kv,s)
//       fp16 scales, dequantised to fp16 before the dot)
// OUTK: 0 = fp32 logits + chunk maxima, 1 = fp16 logits, 2 = bf16 logits
// NW waves x MAXI items.  The folded query matrices W stay in registers (the
// MFMA A operand, 32 VGPRs per item).  The rotation operand (8 KB per
// 32-position tile) is staged once per workgroup, three tiles at a time, into
// a two-slot LDS ring and read by every wave from there: read per wave from
// global memory it triples the L2 traffic of the latent stream and caps the
// kernel near 3.5 TB/s.
template <typename XT, int XFMT, int OUTK, bool FAST, int MAXI, int NW, int G>
__global__ __launch_bounds__(NW * 64, 1) void k_logits_kernel(const KArgs a) {
  constexpr int XE = 2;   // dense latent element size
  constexpr int NT = NW * 64;
  constexpr int TPT = 512 / NT;   // 16-byte rotation pieces staged per thread per tile
  static_assert(512 % NT == 0, "workgroup must divide the rotation tile");
  static_assert(G % 3 == 0, "groups are whole cycles of the 3-tile latent ring");
  __shared__ u32x4 Ts[2][G][512];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = lane & 31, hh = lane >> 5;
  const int chunk = blockIdx.x, wgp = blockIdx.y, b = blockIdx.z;

  const int S = a.S;
  const int n_tiles = (S + TILE - 1) / TILE;
  const int tile0 = chunk * a.tiles_per_chunk;
  const int tile1 = min(tile0 + a.tiles_per_chunk, n_tiles);
  if (tile0 >= tile1) return;

  uint32_t it[MAXI];
#pragma unroll
  for (int i = 0; i < MAXI; ++i) it[i] = a.items[wgp * NW + wave][i];

  // ---- W of this wave's items (rows at or beyond the valid ranks are zero)
  const int rho = lane & 31;
  const int jrow = 16 * ((rho >> 2) & 1) + 4 * (rho >> 3) + (rho & 3);
  half8 wr[MAXI][8];
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    const bool ok = item_valid(it[i]) && jrow < item_nv(it[i]);
    const int qh = item_qh(it[i]), kv = item_kv(it[i]), mt = item_mt(it[i]);
    const XT* qrow = (const XT*)a.q + b * a.q_sb + qh * a.q_sh;
    const XT* brow = (const XT*)a.bk + a.bkoff[kv] + (int64_t)(mt * 32 + jrow) * a.bk_rs;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      half8 w = half8{};
      if (ok) {
        const int i0 = 8 * k + 4 * hh;
        float ql[4], qu[4], bl[4], bu[4];
        if (FAST) {
          load4<XT>(qrow + i0, ql); load4<XT>(qrow + i0 + 64, qu);
          load4<XT>(brow + i0, bl); load4<XT>(brow + i0 + 64, bu);
        } else {
          load4_any<XT>(qrow + i0, ql); load4_any<XT>(qrow + i0 + 64, qu);
          load4_any<XT>(brow + i0, bl); load4_any<XT>(brow + i0 + 64, bu);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          w[2 * e] = (_Float16)(a.wscale * (bl[e] * ql[e] + bu[e] * qu[e]));
          w[2 * e + 1] = (_Float16)(a.wscale * (bl[e] * qu[e] - bu[e] * ql[e]));
        }
      }
      wr[i][k] = w;
    }
  }
  // idle waves (plan padding) load and compute nothing but take part in the
  // rotation staging and its barriers
  const bool active = item_valid(it[0]);

  // ---- per-item latent row bases (bytes).  Lanes whose ranks lie beyond the
  // item's valid ranks re-read the item's first chunk of the same row (in
  // bounds; multiplied by the zero rows of W).
  const char* xb[MAXI];
  int off1[MAXI], off2[MAXI];
  int64_t xpitch[MAXI];
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    const int kv = item_kv(it[i]), mt = item_mt(it[i]);
    const int nvh = item_valid(it[i]) ? item_nv(it[i]) - 16 * hh : 0;
    xpitch[i] = (int64_t)a.xpitch[kv] * XE;
    xb[i] = (const char*)a.x + (b * a.x_sb + a.xoff[kv] + mt * 32) * XE;
    off1[i] = nvh > 0 ? 16 * hh * XE : 0;
    off2[i] = nvh >= 16 ? (16 * hh + 8) * XE : off1[i];
  }
  // quantised: each lane's 16 ranks sit in one block (split is a multiple of 16)
  // Unaligned rows (!FAST): each lane reads its 16 ranks' bytes from any
  // address (qnb: the bytes its block's row holds) and zeroes the ranks past
  // the head's rank after dequantisation (qnl: ranks valid from its first).
  const uint8_t* qb[MAXI];
  const uint16_t* qs[MAXI];
  int64_t qpitch[MAXI];
  int qoff[MAXI], qnb[MAXI], qnl[MAXI];
  bool qk8[MAXI], q16[MAXI];
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    if constexpr (XFMT != 1) break;
    const int kv = item_kv(it[i]), mt = item_mt(it[i]);
    const int nv = item_valid(it[i]) ? item_nv(it[i]) : 0;
    const int nvh = nv - 16 * hh;
    const int jl = nvh > 0 ? mt * 32 + 16 * hh : mt * 32;     // lanes past the valid ranks re-read the first 16
    const bool inA = jl < a.ksplit;
    qk8[i] = inA && a.k_a_int8;
    q16[i] = (nvh > 0 ? nvh : nv) >= 16;
    qnl[i] = nvh > 0 ? nvh : nv;
    const int r = a.krank[kv], ra = min(r, a.ksplit);
    qnb[i] = inA ? (qk8[i] ? ra : (ra + 1) / 2) : (r - a.ksplit + 1) / 2;
    qb[i] = inA ? (const uint8_t*)a.x + b * a.x_sb + a.xoff[kv] : (const uint8_t*)a.x2 + b * a.x2_sb + a.xoff2[kv];
    qpitch[i] = inA ? a.xpitch[kv] : a.xpitch2[kv];
    qoff[i] = qk8[i] ? jl : (inA ? jl / 2 : (jl - a.ksplit) / 2);
    qs[i] = inA ? (const uint16_t*)a.xscale + b * a.xs_sb + (int64_t)kv * a.xs_sh
                : (const uint16_t*)a.xscale2 + b * a.xs2_sb + (int64_t)kv * a.xs2_sh;
  }

  float mx[MAXI];
#pragma unroll
  for (int i = 0; i < MAXI; ++i) mx[i] = -INFINITY;

  // Tiles are processed in groups of G (a multiple of the 3-tile latent
  // register ring) per staging barrier.  Every
  // index is clamped to the chunk's last tile, so a group past the end
  // re-reads that tile (cached) and only its stores are predicated off: the
  // group body has no data-dependent branches and the compiler keeps the
  // latent loads two tiles ahead of their use.
  const int last = tile1 - 1;
  const int n_groups = (tile1 - tile0 + G - 1) / G;

  auto load = [&](KBuf<XFMT, MAXI>& kb, int tile) __attribute__((always_inline)) {
    const int pos = min(min(tile, last) * TILE + t, S - 1);
#pragma unroll
    for (int i = 0; i < MAXI; ++i) {
      if (!item_valid(it[i])) continue;
      if constexpr (XFMT == 0) {
        const char* p = xb[i] + (int64_t)pos * xpitch[i];
        if (FAST) {
          kb.x[i][0] = ld_stream(p + off1[i]);
          kb.x[i][1] = ld_stream(p + off2[i]);
        } else {
          const int nvh = item_nv(it[i]) - 16 * hh;
          uint16_t tmp[16];
#pragma unroll
          for (int v = 0; v < 16; ++v) tmp[v] = v < nvh ? ((const uint16_t*)(p + 16 * hh * XE))[v] : (uint16_t)0;
          kb.x[i][0] = make_uint4(tmp[0] | (tmp[1] << 16), tmp[2] | (tmp[3] << 16), tmp[4] | (tmp[5] << 16), tmp[6] | (tmp[7] << 16));
          kb.x[i][1] = make_uint4(tmp[8] | (tmp[9] << 16), tmp[10] | (tmp[11] << 16), tmp[12] | (tmp[13] << 16), tmp[14] | (tmp[15] << 16));
        }
      } else {
        const uint8_t* q = qb[i] + (int64_t)pos * qpitch[i] + qoff[i];
        uint4 r = make_uint4(0, 0, 0, 0);
        if (!FAST) {
          const uint8_t* row = qb[i] + (int64_t)pos * qpitch[i];
          if (qk8[i]) {
            uint32_t w[4];
            ld_row_bytes<16>(row, qoff[i], qnb[i], w);
            r = make_uint4(w[0], w[1], w[2], w[3]);
          } else {
            uint32_t w[2];
            ld_row_bytes<8>(row, qoff[i], qnb[i], w);
            r.x = w[0]; r.y = w[1];
          }
        } else if (qk8[i]) {
          const uint2 lo = *(const uint2*)q;
          r.x = lo.x; r.y = lo.y;
          if (q16[i]) {
            const uint2 hi = *(const uint2*)(q + 8);
            r.z = hi.x; r.w = hi.y;
          }
        } else {
          r.x = *(const uint32_t*)q;
          if (q16[i]) r.y = *(const uint32_t*)(q + 4);
        }
        kb.x[i][0] = r;
        kb.sq[i] = qs[i][pos];
      }
    }
  };

  // rotation operand of group g (tiles tile0 + G*g + j) -> Ts[slot][j]
  const u32x4* rt = (const u32x4*)a.rope + tid;
  TStage<G, TPT> tst;
  auto tload = [&](TStage<G, TPT>& ts, int g) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const u32x4* q = rt + (int64_t)min(tile0 + G * g + j, last) * 512;
#pragma unroll
      for (int p = 0; p < TPT; ++p) ts.v[j][p] = q[p * NT];
    }
  };
  auto twrite = [&](const TStage<G, TPT>& ts, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int p = 0; p < TPT; ++p) Ts[slot][j][tid + p * NT] = ts.v[j][p];
  };

  // positions past a device-held last position take -1e30 (read once)
  const int lastp = a.last_pos != nullptr ? *a.last_pos : INT_MAX;
  // this batch's logits: a uniform base and 32-bit element offsets (kept
  // below 2^32 by the host)
  char* const obase = (char*)a.out + b * a.o_sb * (OUTK == 0 ? 4 : 2);
  const uint32_t ost = (uint32_t)a.o_st, osh = (uint32_t)a.o_sh;
  auto compute = [&](const KBuf<XFMT, MAXI>& kb, int tile, int slot, int j) __attribute__((always_inline)) {
    const int s = tile * TILE + t;
    const bool store = tile < tile1 && s < S;
    float part = 0.f;
    half8 T[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) T[k] = __builtin_bit_cast(half8, Ts[slot][j][k * 64 + lane]);
#pragma unroll
    for (int i = 0; i < MAXI; ++i) {
      if (!item_valid(it[i])) break;
      floatx16 acc = mfma_f16(wr[i][0], T[0], floatx16{});
#pragma unroll
      for (int k = 1; k < 8; ++k) acc = mfma_f16(wr[i][k], T[k], acc);
      if constexpr (XFMT == 0) {
        part = dot8<XT>(kb.x[i][0], acc, 0, part);
        part = dot8<XT>(kb.x[i][1], acc, 8, part);
      } else {
        uint4 h0, h1;
        dequant16(kb.x[i][0], qk8[i], kb.sq[i], h0, h1);
        if (!FAST) {
          h0 = mask_h8(h0, qnl[i]);
          h1 = mask_h8(h1, qnl[i] - 8);
        }
        part = dot8<_Float16>(h0, acc, 0, part);
        part = dot8<_Float16>(h1, acc, 8, part);
      }
      if (item_last(it[i])) {
        float tot = add_halves(part);
        part = 0.f;
        const int qh = item_qh(it[i]);
        if (store) {
          if (a.mask != nullptr) tot += load_elem_f32(a.mask, a.mask_dtype, b * a.m_sb + qh * a.m_sh + s);
          if (s > lastp) tot = -1e30f;
          const uint32_t o = (uint32_t)(s >> 5) * ost + (uint32_t)qh * osh + (uint32_t)(s & 31);
          if constexpr (OUTK == 0) ((float*)obase)[o] = tot;
          else if constexpr (OUTK == 1) ((_Float16*)obase)[o] = (_Float16)tot;
          else ((__bf16*)obase)[o] = (__bf16)tot;
          mx[i] = fmaxf(mx[i], tot);
        }
      }
    }
  };

  // Staging: slot g&1 holds group g from the barrier at the start of group g;
  // behind that barrier group g+1 is written into the other slot (last read
  // in group g-1) and group g+2 is fetched into registers.
  tload(tst, 0);
  twrite(tst, 0);
  tload(tst, 1);
  if (!active) {
    for (int g = 0; g < n_groups; ++g) {
      __syncthreads();
      twrite(tst, (g + 1) & 1);
      tload(tst, g + 2);
    }
    return;
  }
  KBuf<XFMT, MAXI> b0, b1, b2;
  load(b0, tile0);
  load(b1, tile0 + 1);
  for (int g = 0; g < n_groups; ++g) {
    __syncthreads();
    twrite(tst, (g + 1) & 1);
    tload(tst, g + 2);
    const int tb = tile0 + G * g, slot = g & 1;
#pragma unroll
    for (int j = 0; j < G; j += 3) {
      load(b2, tb + j + 2);
      compute(b0, tb + j, slot, j);
      load(b0, tb + j + 3);
      compute(b1, tb + j + 1, slot, j + 1);
      load(b1, tb + j + 4);
      compute(b2, tb + j + 2, slot, j + 2);
    }
  }

  if constexpr (OUTK == 0) {
    if (a.chunkmax != nullptr) {
#pragma unroll
      for (int i = 0; i < MAXI; ++i) {
        if (!item_valid(it[i]) || !item_last(it[i])) continue;
        const float m = wave_max32(mx[i]);
        if (lane == 0) a.chunkmax[((int64_t)b * a.Hq + item_qh(it[i])) * a.n_chunks + chunk] = m;
      }
    }
  }
}

template <typename XT, int XFMT, int OUTK, int MAXI, int NW, int G>
static void launch_v(const KArgs& a, bool fast, dim3 grid, hipStream_t st) {
  if (fast) hipLaunchKernelGGL((k_logits_kernel<XT, XFMT, OUTK, true, MAXI, NW, G>), grid, dim3(NW * 64), 0, st, a);
  else hipLaunchKernelGGL((k_logits_kernel<XT, XFMT, OUTK, false, MAXI, NW, G>), grid, dim3(NW * 64), 0, st, a);
}

// items per wave -> workgroup shape: up to 2 items in 8-wave workgroups (two
// waves per SIMD), else up to 4 items in 4-wave workgroups.  (Measured on
// MI355X with ragged ranks up to 96: four independent item chains per wave
// beat a 3-item, 8-wave shape, which spills at 256 registers.)
template <typename XT, int XFMT, int OUTK>
static int launch_t(const KArgs& a, bool fast, int B, hipStream_t st) {
  dim3 grid(a.n_chunks, a.n_wg, B);
  if (a.maxi <= 2) launch_v<XT, XFMT, OUTK, 2, 8, 3>(a, fast, grid, st);
  else launch_v<XT, XFMT, OUTK, 4, 4, 3>(a, fast, grid, st);
  return (int)hipGetLastError();
}

template <typename XT, int XFMT>
static int launch_o(const KArgs& a, int outk, bool fast, int B, hipStream_t st) {
  if (outk == 0) return launch_t<XT, XFMT, 0>(a, fast, B, st);
  if (outk == 1) return launch_t<XT, XFMT, 1>(a, fast, B, st);
  return launch_t<XT, XFMT, 2>(a, fast, B, st);
}

int launch_k_logits(const KArgs& a, int dtype, int fmt, bool out_f32, int out_dtype, bool fast, int B, hipStream_t st) {
  if (a.gqa) return launch_k_logits_gqa(a, dtype, out_f32, out_dtype, B, st);
  if (a.ws) return launch_k_logits_ws(a, dtype, out_f32, out_dtype, B, st);
  const int outk = out_f32 ? 0 : (out_dtype == STARKV_F16 ? 1 : 2);
  const bool q = fmt != STARKV_FMT_DENSE;
  if (dtype == STARKV_F16) return q ? launch_o<_Float16, 1>(a, outk, fast, B, st) : launch_o<_Float16, 0>(a, outk, fast, B, st);
  return q ? launch_o<__bf16, 1>(a, outk, fast, B, st) : launch_o<__bf16, 0>(a, outk, fast, B, st);
}

}  // namespace starkv
