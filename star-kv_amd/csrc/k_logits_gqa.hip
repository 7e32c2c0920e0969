// K1 for grouped-query attention on gfx950: the key of every position is
// reconstructed once per KV head and then dotted with the group's queries.
//
// The reference forms K = RoPE(B_k X) inside each query head's program
// (abx_rope_batched.py:81, 101-131, grid over query heads at :170), so a
// group of gs query heads rebuilds the same keys gs times.  The folded form
// of k_logits_ws.hip costs gs * r * 128 MACs per position and KV head; here
// it is r * 128 (reconstruction) + 32 * 128 (the group's dots, gs <= 8 query
// rows of one MFMA tile), per 32-position tile:
//
//   K^T[d][s]   = sum_j B_k[j][d] X[s][j]                    (MFMA, act dtype)
//   K_rot       = a * (K cos - rotate_half(K) sin)            (VALU, fp32)
//   logit[h][s] = scale * sum_d q_h[d] K_rot[d][s]            (MFMA, fp16)
//
// Layout facts the kernel leans on (32x32x16 MFMA: lane l holds A row l%32,
// B column l%32, the K elements 8*(l/32)..+8; accumulator v of lane l is row
// 8*(v/4) + 4*(l/32) + v%4, column l%32):
// * With dims as accumulator rows, dims d and d+64 (a RoPE pair) sit in the
//   same lane and accumulator index of M-tiles m and m+2, and lane half hh
//   holds exactly the frequencies whose (cos, sin) the RoPE operand table
//   gives that lane half (rope.hip: frequency 8k + 4*(lane/32) + e/2).
// * The q.K contraction may visit dims in any order.  Visiting d in the order
//   kappa = d with bits 2 and 3 swapped turns accumulator entries 8j..8j+7
//   of M-tile m into the B operand of K-step 2m + j as they are.
//
// Workgroup: 4 producer waves (the warp-specialised DMA ring of
// k_logits_ws.hip: each tile's latent rows of the workgroup's KV heads, rows
// rotated for conflict-free reads, plus the 8 KB RoPE operand) and 4
// consumer waves, two per KV head: wave (slot, p) reconstructs M-tiles p and
// p+2 (dims 32p..32p+31 and their RoPE partners), so its B_k^T operands (r/2
// registers per lane) stay resident.  The p = 0 wave leaves its partial
// logits of tile i in LDS; the p = 1 wave adds its own one tile later (after
// the next barrier) and stores.
#include "common.hpp"

namespace starkv {

namespace {

constexpr int GQ_PRODUCERS = 4;
constexpr int GQ_CONSUMERS = 4;                  // 2 KV heads x 2 dim halves
constexpr int GQ_MAXH = 2;                       // KV heads per workgroup
constexpr int GQ_RING = K1_GQ_RING_BYTES;
constexpr int GQ_MAXK = (GQ_MAXH * 32 * 16 / 64 + 8 + GQ_PRODUCERS - 1) / GQ_PRODUCERS;   // DMA instructions per producer
typedef __attribute__((address_space(3))) void lds_void;

// 16-byte chunk rotation of staged rows (see k_logits_ws.hip: conflict-free
// ds_read_b128 of one chunk of 8 consecutive rows)
__device__ inline int gq_shift(int row, int n16) {
  const int g = min(n16 & -n16, 8);
  return row / (8 / g);
}

template <int N> __device__ inline void gq_wait_vm() {
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
__device__ inline void gq_wait_vm_n(int n) {
  switch (n) {
#define GQ_CASE(N) case N: gq_wait_vm<N>(); break;
    GQ_CASE(0) GQ_CASE(1) GQ_CASE(2) GQ_CASE(3) GQ_CASE(4) GQ_CASE(5) GQ_CASE(6) GQ_CASE(7)
    GQ_CASE(8) GQ_CASE(9) GQ_CASE(10) GQ_CASE(11) GQ_CASE(12) GQ_CASE(13) GQ_CASE(14) GQ_CASE(15)
    GQ_CASE(16) GQ_CASE(17) GQ_CASE(18) GQ_CASE(19) GQ_CASE(20)
#undef GQ_CASE
    default: gq_wait_vm<0>(); break;
  }
}

template <typename XT> struct GqVec;
template <> struct GqVec<_Float16> { typedef half8 T; };
template <> struct GqVec<__bf16> { typedef bf16x8 T; };

template <typename XT>
__device__ inline floatx16 gq_mfma(typename GqVec<XT>::T a, typename GqVec<XT>::T b, floatx16 c) {
  if constexpr (__is_same(XT, _Float16)) return mfma_f16(a, b, c);
  else return mfma_bf16(a, b, c);
}

}  // namespace

// OUTK: 0 = fp32 logits + chunk maxima, 1 = fp16 logits, 2 = bf16 logits
template <typename XT, int OUTK>
__global__ __launch_bounds__((GQ_CONSUMERS + GQ_PRODUCERS) * 64, 1) void k_logits_gqa_kernel(const KArgs a) {
  typedef typename GqVec<XT>::T XV;
  __shared__ __attribute__((aligned(16))) char ring[GQ_RING];          // a.ws_nst stages of a.ws_stage bytes
  __shared__ float carry[2][GQ_MAXH][64][4];                           // p = 0 partial logits, by tile parity

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = lane & 31, hh = lane >> 5;
  const int chunk = blockIdx.x, wgp = blockIdx.y, b = blockIdx.z;
  const int S = a.S;
  const int n_tiles = (S + TILE - 1) / TILE;
  const int tile0 = chunk * a.tiles_per_chunk;
  const int tile1 = min(tile0 + a.tiles_per_chunk, n_tiles);
  if (tile0 >= tile1) return;
  const int last = tile1 - 1;
  const int ntl = tile1 - tile0;

  // ---- the workgroup's KV heads (items of consumer waves 0 and 2), their
  // ranks and chunk offsets in a stage
  int hkv[GQ_MAXH], hrank[GQ_MAXH], hoff[GQ_MAXH];
  int tot = 0;
#pragma unroll
  for (int k = 0; k < GQ_MAXH; ++k) {
    const uint32_t itm = a.items[wgp * GQ_CONSUMERS + 2 * k][0];
    hkv[k] = 0; hrank[k] = 8; hoff[k] = 1 << 30;
    if (!item_valid(itm)) continue;
    hkv[k] = item_kv(itm);
    hrank[k] = a.krank[hkv[k]];
    hoff[k] = tot;
    tot += 32 * (hrank[k] >> 3);
  }
  // stage: latent chunks [0, 64 * nX), the RoPE operand in the last 8 KB
  const int nX = (tot + 63) / 64, stage = a.ws_stage, nst = a.ws_nst;
  if (tot == 0 || nX * 1024 + 8192 > stage || nst < 2 || nst * stage > GQ_RING) return;   // uniform

  if (wave >= GQ_CONSUMERS) {
    // ================= producer (as in k_logits_ws.hip) =================
    const int pw = wave - GQ_CONSUMERS;
    const int nI = nX + 8, ahead = nst - 1;
    const char* src[GQ_MAXK];
    int64_t adv[GQ_MAXK];
    int rowpos[GQ_MAXK], tmul[GQ_MAXK], pmax[GQ_MAXK], dst[GQ_MAXK];
    int cnt = 0;
#pragma unroll
    for (int k = 0; k < GQ_MAXK; ++k) {
      const int m = pw + GQ_PRODUCERS * k;
      src[k] = (const char*)a.rope; adv[k] = 8192; rowpos[k] = 0; tmul[k] = 1; pmax[k] = 1 << 30; dst[k] = 0;
      if (m >= nI) continue;
      ++cnt;
      if (m >= nX) {
        const int j = m - nX;
        src[k] = (const char*)a.rope + (j * 64 + lane) * 16;
        dst[k] = stage - 8192 + j * 1024;
        continue;
      }
      int q = m * 64 + lane;
      if (q >= tot) q = tot - 1;            // lanes past the last chunk re-read it into an unused slot
      int hb = hoff[0], hr = hrank[0], hk = hkv[0];
#pragma unroll
      for (int j = 1; j < GQ_MAXH; ++j)
        if (hoff[j] <= q) { hb = hoff[j]; hr = hrank[j]; hk = hkv[j]; }
      const int n16 = hr >> 3, loc = q - hb;
      const int row = loc / n16, cr = loc % n16;
      const int c = (cr - gq_shift(row, n16) % n16 + n16) % n16;
      src[k] = (const char*)a.x + (b * a.x_sb + a.xoff[hk]) * 2 + (int64_t)c * 16;
      adv[k] = (int64_t)a.xpitch[hk] * 2;
      rowpos[k] = row;
      tmul[k] = TILE;
      pmax[k] = S - 1;
      dst[k] = m * 1024;
    }
    // full tiles (all 32 positions below S): first-tile address plus
    // (tile - tile0) times a fixed per-lane step; the tail tile is clamped
    const char* base[GQ_MAXK];     // lane address at tile0
    uint32_t lstep[GQ_MAXK];       // bytes per tile (< 2^31, checked on the host)
#pragma unroll
    for (int k = 0; k < GQ_MAXK; ++k) {
      base[k] = src[k] + (int64_t)(tile0 * tmul[k] + rowpos[k]) * adv[k];
      lstep[k] = (uint32_t)(tmul[k] * adv[k]);
    }
    auto issue = [&](int i) __attribute__((always_inline)) {
      const int tl = min(tile0 + i, last);
      char* st = ring + (i % nst) * stage;
      if ((tl + 1) * TILE <= S) {
        const uint32_t ti = (uint32_t)(tl - tile0);
#pragma unroll
        for (int k = 0; k < GQ_MAXK; ++k) {
          const int m = pw + GQ_PRODUCERS * k;
          if (m >= nI) break;
          __builtin_amdgcn_global_load_lds((const void*)(base[k] + (uint64_t)ti * lstep[k]), (lds_void*)(st + dst[k]), 16, 0, 0);
        }
      } else {
#pragma unroll
        for (int k = 0; k < GQ_MAXK; ++k) {
          const int m = pw + GQ_PRODUCERS * k;
          if (m >= nI) break;
          const int64_t pos = min(tl * tmul[k] + rowpos[k], pmax[k]);
          __builtin_amdgcn_global_load_lds((const void*)(src[k] + pos * adv[k]), (lds_void*)(st + dst[k]), 16, 0, 0);
        }
      }
    };
    for (int i = 0; i < ahead; ++i) issue(i);
    for (int i = 0; i < ntl; ++i) {
      gq_wait_vm_n((ahead - 1) * cnt);
      __builtin_amdgcn_s_barrier();
      issue(i + ahead);
    }
    __builtin_amdgcn_s_barrier();           // the consumers' extra barrier
    gq_wait_vm<0>();
    return;
  }

  // ================= consumer: KV head slot, dim half p =================
  const int slot = wave >> 1, p = wave & 1;
  const uint32_t itm = a.items[wgp * GQ_CONSUMERS + wave][0];
  if (!item_valid(itm)) {                    // keep the workgroup's barrier count
    for (int i = 0; i <= ntl; ++i) {
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_s_barrier();
    }
    return;
  }
  const int kv = item_kv(itm), gs = a.gs;
  const int r = hrank[slot], hb = hoff[slot], n16 = r >> 3, nk = (r + 15) >> 4;

  // B_k^T operands of M-tiles p and p+2: lane l holds dim 32m + l%32, ranks
  // 16kk + 8hh + 0..7 (zero past r)
  XV bt[2][8];
  {
    const XT* bk = (const XT*)a.bk + a.bkoff[kv];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
      const int dim = 32 * (p + 2 * mi) + t;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        XV v;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int rk = 16 * kk + 8 * hh + i;
          v[i] = rk < r ? bk[(int64_t)rk * a.bk_rs + dim] : (XT)0.f;
        }
        bt[mi][kk] = v;
      }
    }
  }
  // query operands of K-steps 2p, 2p+1, 2p+4, 2p+5: lane l holds query row
  // h = l%32 of the group (zero for h >= gs) at dims d(kappa), kappa =
  // 16 kk2 + 8hh + i, d = kappa with bits 2 and 3 swapped
  half8 qa[4];
  {
    const int h = t;
    const XT* qrow = (const XT*)a.q + b * a.q_sb + (int64_t)(kv * gs + min(h, gs - 1)) * a.q_sh;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int kk2 = 2 * p + (n & 1) + 4 * (n >> 1);
      half8 v;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int d = 32 * (kk2 >> 1) + 8 * (2 * (kk2 & 1) + (i >> 2)) + 4 * hh + (i & 3);
        v[i] = h < gs ? (_Float16)to_f32(qrow[d]) : (_Float16)0.f;
      }
      qa[n] = v;
    }
  }
  // LDS offsets of this lane's latent chunk per rank K-step: row t, chunk
  // 2kk + hh (past the rank: chunk 2kk, against zero B_k^T rows)
  int xo[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    const int c = min(2 * kk + hh < n16 ? 2 * kk + hh : 2 * kk, n16 - 1);
    xo[kk] = (hb + t * n16 + (c + gq_shift(t, n16)) % n16) * 16;
  }
  // query rows h < gs <= 8 are accumulator entries v = h % 4 of lane half h / 4
  float mx[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) mx[v] = -INFINITY;
  float prev[4] = {0.f, 0.f, 0.f, 0.f};      // p = 1: own partial logits of the previous tile

  // epilogue of tile `ti` (absolute tile index): scale, mask, store, maxima
  auto emit = [&](const float* sum, int ti) __attribute__((always_inline)) {
    const int s = ti * TILE + t;
    if (s >= S) return;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int h = 4 * hh + v;
      if (h >= gs) continue;
      const int qh = kv * gs + h;
      float val = a.wscale * sum[v];
      if (a.mask != nullptr) val += load_elem_f32(a.mask, a.mask_dtype, b * a.m_sb + qh * a.m_sh + s);
      const int64_t o = b * a.o_sb + (int64_t)ti * a.o_st + qh * a.o_sh + t;
      if constexpr (OUTK == 0) ((float*)a.out)[o] = val;
      else if constexpr (OUTK == 1) ((_Float16*)a.out)[o] = (_Float16)val;
      else ((__bf16*)a.out)[o] = (__bf16)val;
      mx[v] = fmaxf(mx[v], val);
    }
  };

  for (int i = 0; i < ntl; ++i) {
    __builtin_amdgcn_s_waitcnt(0xC07F);      // this wave's LDS reads and writes are done
    __builtin_amdgcn_s_barrier();
    if (p == 1 && i > 0) {
      float sum[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) sum[v] = prev[v] + carry[(i - 1) & 1][slot][lane][v];
      emit(sum, tile0 + i - 1);
    }
    const char* st = ring + (i % nst) * stage;
    XV xb[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      if (kk < nk) xb[kk] = *(const XV*)(st + xo[kk]);
    half8 T4[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) T4[g] = *(const half8*)(st + stage - 8192 + ((4 * p + g) * 64 + lane) * 16);
    // K^T of M-tiles p (k0) and p+2 (k1)
    floatx16 k0 = floatx16{}, k1 = floatx16{};
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      if (kk < nk) {
        k0 = gq_mfma<XT>(bt[0][kk], xb[kk], k0);
        k1 = gq_mfma<XT>(bt[1][kk], xb[kk], k1);
      }
    }
    // rotate: accumulator v is dim d = 32m + 8g + 4hh + e (g = v/4, e = v%4)
    // and its partner d + 64; (a cos, a sin) of frequency 32p + 8g + 4hh + e
    // are elements 2e, 2e+1 of table K-step 4p + g
    half8 bop[4];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float c = (float)T4[v >> 2][2 * (v & 3)], s = (float)T4[v >> 2][2 * (v & 3) + 1];
      const float lo = k0[v] * c - k1[v] * s;
      const float hi = k1[v] * c + k0[v] * s;
      bop[v >> 3][v & 7] = (_Float16)lo;
      bop[2 + (v >> 3)][v & 7] = (_Float16)hi;
    }
    floatx16 la = mfma_f16(qa[0], bop[0], floatx16{});
    la = mfma_f16(qa[1], bop[1], la);
    la = mfma_f16(qa[2], bop[2], la);
    la = mfma_f16(qa[3], bop[3], la);
    if (p == 0) {
#pragma unroll
      for (int v = 0; v < 4; ++v) carry[i & 1][slot][lane][v] = la[v];
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) prev[v] = la[v];
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();              // publishes the last tile's partials
  if (p == 0) return;
  {
    float sum[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) sum[v] = prev[v] + carry[(ntl - 1) & 1][slot][lane][v];
    emit(sum, tile0 + ntl - 1);
  }
  if constexpr (OUTK == 0) {
    if (a.chunkmax != nullptr) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float m = wave_max32(mx[v]);
        const int h = 4 * hh + v;
        if (t == 0 && h < gs) a.chunkmax[((int64_t)b * a.Hq + kv * gs + h) * a.n_chunks + chunk] = m;
      }
    }
  }
}

template <typename XT>
static int launch_gqa_t(const KArgs& a, int outk, int B, hipStream_t st) {
  dim3 grid(a.n_chunks, a.n_wg, B), block((GQ_CONSUMERS + GQ_PRODUCERS) * 64);
  if (outk == 0) hipLaunchKernelGGL((k_logits_gqa_kernel<XT, 0>), grid, block, 0, st, a);
  else if (outk == 1) hipLaunchKernelGGL((k_logits_gqa_kernel<XT, 1>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((k_logits_gqa_kernel<XT, 2>), grid, block, 0, st, a);
  return (int)hipGetLastError();
}

int launch_k_logits_gqa(const KArgs& a, int dtype, bool out_f32, int out_dtype, int B, hipStream_t st) {
  const int outk = out_f32 ? 0 : (out_dtype == STARKV_F16 ? 1 : 2);
  return dtype == STARKV_F16 ? launch_gqa_t<_Float16>(a, outk, B, st) : launch_gqa_t<__bf16>(a, outk, B, st);
}

}  // namespace starkv
