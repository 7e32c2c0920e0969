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
// Workgroup: 4 waves, two per KV head: wave (slot, p) reconstructs M-tiles
// p and p+2 (dims 32p..32p+31 and their RoPE partners), so its B_k^T
// operands (r/2 registers per lane) stay resident.  Every wave also issues
// its share of each tile's DMA into an LDS ring (the tile's latent rows of
// the workgroup's KV heads, rows rotated for conflict-free reads, plus the
// 8 KB RoPE operand), `ahead` = stages - 1 tiles ahead, and waits for its
// own share with an explicit vmcnt before the tile's barrier.  Two
// workgroups share a CU (80 KB of LDS and <= 256 registers each), so each
// SIMD interleaves two waves' per-tile chains (reconstruction MFMAs ->
// rotation -> q.K MFMAs).  The p = 0 wave hands its partial logits of a
// tile to the p = 1 wave through LDS one tile later; the p = 1 wave adds
// its own and stores.
#include <climits>

#include "common.hpp"

namespace starkv {

namespace {

constexpr int GQ_WAVES = 4;                      // 2 KV heads x 2 dim halves
constexpr int GQ_MAXH = 2;                       // KV heads per workgroup
constexpr int GQ_RING = K1_GQ_RING_BYTES;
constexpr int GQ_MAXK = (GQ_MAXH * 32 * 16 / 64 + 8 + GQ_WAVES - 1) / GQ_WAVES;   // DMA instructions per wave and tile

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
#define GQ_CASE8(N) GQ_CASE(N) GQ_CASE(N + 1) GQ_CASE(N + 2) GQ_CASE(N + 3) GQ_CASE(N + 4) GQ_CASE(N + 5) \
    GQ_CASE(N + 6) GQ_CASE(N + 7)
    GQ_CASE8(0) GQ_CASE8(8) GQ_CASE8(16) GQ_CASE8(24) GQ_CASE8(32) GQ_CASE8(40) GQ_CASE8(48) GQ_CASE8(56)
#undef GQ_CASE8
#undef GQ_CASE
    default: gq_wait_vm<0>(); break;
  }
}

// One 1 KB global -> LDS DMA (16 bytes per lane, to LDS byte address `lds` +
// 16 * lane).  Written as inline assembly so that the compiler, which does
// not see it write LDS, adds no waits of its own before the reads of other
// stages; the kernel orders it with explicit vmcnt waits and barriers.
// Each statement sets m0 itself (the compiler treats m0 as reserved and
// ignores it as a clobber; its code for this kernel holds nothing in m0,
// which tests/test_gqa_m0.py checks on the compiled gfx950 assembly).
__device__ inline void gq_dma(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}

template <typename XT> struct GqVec;
template <> struct GqVec<_Float16> { typedef half8 T; };
template <> struct GqVec<__bf16> { typedef bf16x8 T; };

template <typename XT>
__device__ inline floatx16 gq_mfma(typename GqVec<XT>::T a, typename GqVec<XT>::T b, floatx16 c) {
  if constexpr (__is_same(XT, _Float16)) return mfma_f16(a, b, c);
  else return mfma_bf16(a, b, c);
}

// this wave's share of every tile's DMA: instructions m = wave + 4k
struct GqDma {
  const char* base[GQ_MAXK];   // lane address at tile0
  uint32_t lstep[GQ_MAXK];     // bytes per tile (< 2^31, checked on the host)
  int rowp[GQ_MAXK];           // latent: the lane's row in a tile; RoPE operand: -2^30 (never clamped)
  int adv[GQ_MAXK];            // latent row pitch in bytes
  int dst[GQ_MAXK];            // byte offset in a stage
  int cnt;                     // instructions per tile
  uint32_t ring;               // LDS byte address of the ring
  int stage, nst, tile0, S;

  // tile tile0 + i into stage i % nst; rows past S re-read row S - 1 (only
  // the last tile has any: the others take one address add per instruction)
  __device__ inline void issue(int i) const {
    const int tl = tile0 + i;
    const uint32_t lb = ring + (uint32_t)((i % nst) * stage);
    if ((tl + 1) * TILE <= S) {
#pragma unroll
      for (int k = 0; k < GQ_MAXK; ++k) {
        if (k >= cnt) break;
        gq_dma(base[k] + (uint64_t)(uint32_t)i * lstep[k], lb + (uint32_t)dst[k]);
      }
      return;
    }
#pragma unroll
    for (int k = 0; k < GQ_MAXK; ++k) {
      if (k >= cnt) break;
      const int over = max(tl * TILE + rowp[k] - (S - 1), 0);
      gq_dma(base[k] + (uint64_t)(uint32_t)i * lstep[k] - (int64_t)over * adv[k], lb + (uint32_t)dst[k]);
    }
  }
};

// the workgroup's KV heads and where their rows sit in a stage
struct GqHeads {
  int hkv[GQ_MAXH], hrank[GQ_MAXH], hoff[GQ_MAXH];
  int tot;                     // 16-byte chunks of one tile
};

}  // namespace

// One consumer wave (KV head slot, dim half p) over its tiles; NK = rank
// K-steps (16 ranks each) rounded up to even, the B_k^T rows past the rank
// being zero.  MASKED: an additive mask is read in the epilogue (its loads,
// which the compiler waits for with counts that do not see the DMA, drain
// the ring once per tile; the unmasked kernel issues no waited-for load in
// its loop).
template <typename XT, int OUTK, int NK, bool MASKED>
__device__ __attribute__((always_inline)) inline void gq_consume(const KArgs& a, const GqHeads& H, const GqDma& d,
                                                                  char* ring, float (*carry)[GQ_MAXH][64][4],
                                                                  int slot, int p, int kv, int b, int chunk, int ntl,
                                                                  int ahead) {
  typedef typename GqVec<XT>::T XV;
  const int lane = threadIdx.x & 63, t = lane & 31, hh = lane >> 5;
  const int gs = a.gs, S = a.S, tile0 = d.tile0, stage = d.stage, nst = d.nst;
  const int r = H.hrank[slot], hb = H.hoff[slot], n16 = (r + 7) >> 3;   // chunks of a row (padded rows past r)

  // The q.K step runs on fp16 MFMA.  bf16 models hold keys and queries in
  // bf16 (the reference too, abx_rope_batched.py:114-125), whose range fp16
  // lacks.  Their queries enter scaled by 2^-8 (exact: |q| up to 1.6e7;
  // those below 0.016 among fp16's subnormals, with an absolute error under
  // 7.6e-6) and the logits leave scaled by 2^8.  A tile one of whose rotated
  // keys passed fp16's range (found from its logits: inf or NaN) runs again
  // with its keys scaled by 2^-16 (exact; up to ~4e9).  Keys are not scaled on
  // every tile: that puts the small ones among fp16's subnormals, measured
  // 1.6x slower; checking the rotated keys' range before the conversion cost
  // ~50 VALU instructions per tile and wave.
  constexpr bool BF = !__is_same(XT, _Float16);
  constexpr float IN_SCALE = BF ? 0x1p-8f : 1.f;
  constexpr float F32_FINITE = 3.4028235e38f;         // largest finite float
  const float wscale = a.wscale * (BF ? 0x1p8f : 1.f);
  // B_k^T operands of M-tiles p and p+2: lane l holds dim 32m + l%32, ranks
  // 16kk + 8hh + 0..7 (zero past r)
  XV bt[2][NK];
  {
    const XT* bk = (const XT*)a.bk + a.bkoff[kv];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
      const int dim = 32 * (p + 2 * mi) + t;
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
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
        const int dd = 32 * (kk2 >> 1) + 8 * (2 * (kk2 & 1) + (i >> 2)) + 4 * hh + (i & 3);
        // scaled in the act dtype first (exact): converted to fp16 before
        // the multiply, which the compiler may otherwise do, it would overflow
        const XT qs = (XT)(to_f32(qrow[dd]) * IN_SCALE);
        v[i] = h < gs ? (_Float16)to_f32(qs) : (_Float16)0.f;
      }
      qa[n] = v;
    }
  }
  // LDS offsets of this lane's latent chunk per rank K-step: row t, chunk
  // 2kk + hh (past the rank: a chunk of the same row, against zero B_k^T rows)
  int xo[NK];
#pragma unroll
  for (int kk = 0; kk < NK; ++kk) {
    const int c = min(2 * kk + hh < n16 ? 2 * kk + hh : 2 * kk, n16 - 1);
    xo[kk] = (hb + t * n16 + (c + gq_shift(t, n16)) % n16) * 16;
  }
  // query rows h < gs <= 8 are accumulator entries v = h % 4 of lane half h / 4
  // operands in before the ring fills: the compiler's waits for them, which
  // do not see the DMA, then hold none
  gq_wait_vm<0>();
  for (int i = 0; i < min(ahead, ntl); ++i) d.issue(i);

  float mx[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) mx[v] = -INFINITY;
  float prev[4] = {0.f, 0.f, 0.f, 0.f};      // this wave's partial logits of the tile before the current one

  // positions past a device-held last position take -1e30 (read once)
  const int lastp = a.last_pos != nullptr ? *a.last_pos : INT_MAX;
  // epilogue of tile `ti` (absolute tile index): scale, mask, store, maxima
  // (one store instruction per v < min(gs, 4): lane t = 0 of lane half 0
  // always stores, so none is skipped; the DMA waits count them)
  // this batch's logits: a uniform base and 32-bit element offsets (kept
  // below 2^32 by the host)
  char* const obase = (char*)a.out + b * a.o_sb * (OUTK == 0 ? 4 : 2);
  const uint32_t ost = (uint32_t)a.o_st, osh = (uint32_t)a.o_sh;
  auto emit = [&](const float* sum, int ti) __attribute__((always_inline)) {
    const int s = ti * TILE + t;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if (v >= gs) break;
      const int h = 4 * hh + v;
      if (h >= gs || s >= S) continue;
      const int qh = kv * gs + h;
      float val = wscale * sum[v];
      if constexpr (MASKED) val += load_elem_f32(a.mask, a.mask_dtype, b * a.m_sb + qh * a.m_sh + s);
      if (s > lastp) val = -1e30f;
      const uint32_t o = (uint32_t)ti * ost + (uint32_t)qh * osh + (uint32_t)t;
      if constexpr (OUTK == 0) ((float*)obase)[o] = val;
      else if constexpr (OUTK == 1) ((_Float16*)obase)[o] = (_Float16)val;
      else ((__bf16*)obase)[o] = (__bf16)val;
      mx[v] = fmaxf(mx[v], val);
    }
  };

  // the start of step i: tile i - 1 handed over and stored, tile i's stage
  // complete for every wave, the DMA of tile i + ahead issued.  The wait
  // leaves outstanding exactly what this wave issued after its DMA of tile i:
  // the DMA of tiles i + 1 .. i + ahead - 1 and (p = 1) the ns logit stores
  // of each step from i - ahead (after that step's DMA) to i - 1 that
  // emitted (steps >= 1).  The counter retires in issue order.
  const int ns = p == 1 ? min(gs, 4) : 0;
  for (int i = 0; i < ntl; ++i) {
    if (p == 0 && i >= 1) {
#pragma unroll
      for (int v = 0; v < 4; ++v) carry[i & 1][slot][lane][v] = prev[v];
    }
    gq_wait_vm_n(min(ahead - 1, ntl - 1 - i) * d.cnt + ns * min(ahead, max(i - 1, 0)));
    __builtin_amdgcn_s_waitcnt(0xC07F);      // this wave's LDS reads and writes are done
    asm volatile("s_barrier" ::: "memory");
    if (i + ahead < ntl) d.issue(i + ahead);  // into the stage of tile i - 1, read before this barrier
    if (p == 1 && i >= 1) {
      float sum[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) sum[v] = prev[v] + carry[i & 1][slot][lane][v];
      emit(sum, tile0 + i - 1);
    }
    const char* st = ring + (i % nst) * stage;
    // the tile's group logits (rows v < 4 of this lane's column), keys
    // scaled by ks before their rotation
    auto tile_logits = [&](float ks, float sum[4]) __attribute__((always_inline)) {
      XV xb[NK];
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) xb[kk] = *(const XV*)(st + xo[kk]);
      half8 T4[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) T4[g] = *(const half8*)(st + stage - 8192 + ((4 * p + g) * 64 + lane) * 16);
      // K^T of M-tiles p (k0) and p+2 (k1)
      floatx16 k0 = floatx16{}, k1 = floatx16{};
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        k0 = gq_mfma<XT>(bt[0][kk], xb[kk], k0);
        k1 = gq_mfma<XT>(bt[1][kk], xb[kk], k1);
      }
      if (ks != 1.f) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          k0[v] *= ks;
          k1[v] *= ks;
        }
      }
      // rotate: accumulator v is dim d = 32m + 8g + 4hh + e (g = v/4, e = v%4)
      // and its partner d + 64; (a cos, a sin) of frequency 32p + 8g + 4hh + e
      // are elements 2e, 2e+1 of table K-step 4p + g
      half8 bop[4];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        // every product takes the table's fp16 (cos, sin) as it is (mixed-
        // precision FMAs, no conversions): k1 s and k0 s rounded to fp32, then
        // k0 c - k1 s and k1 c + k0 s rounded to fp16
        const _Float16 c = T4[v >> 2][2 * (v & 3)], s = T4[v >> 2][2 * (v & 3) + 1];
        const float t1 = __builtin_fmaf(k1[v], (float)s, 0.f), t2 = __builtin_fmaf(k0[v], (float)s, 0.f);
        bop[v >> 3][v & 7] = (_Float16)__builtin_fmaf(k0[v], (float)c, -t1);
        bop[2 + (v >> 3)][v & 7] = (_Float16)__builtin_fmaf(k1[v], (float)c, t2);
      }
      // two chains of two K-steps each (dims 0-63 and their partners)
      floatx16 la = mfma_f16(qa[0], bop[0], floatx16{});
      floatx16 lb = mfma_f16(qa[2], bop[2], floatx16{});
      la = mfma_f16(qa[1], bop[1], la);
      lb = mfma_f16(qa[3], bop[3], lb);
#pragma unroll
      for (int v = 0; v < 4; ++v) sum[v] = la[v] + lb[v];
    };
    float sum[4];
    tile_logits(1.f, sum);
    if constexpr (BF) {
      // a rotated key past fp16's range became inf, which makes every logit
      // of its position inf or NaN (a zero query row gives 0 * inf = NaN):
      // then the wave runs the tile again with its keys scaled by 2^-16
      const float chk = (sum[0] + sum[1]) + (sum[2] + sum[3]);
      if (__builtin_amdgcn_ballot_w64(!(fabsf(chk) <= F32_FINITE)) != 0) {
        // (operands read from LDS again rather than kept in registers)
        asm volatile("" ::: "memory");
        tile_logits(0x1p-16f, sum);
#pragma unroll
        for (int v = 0; v < 4; ++v) sum[v] *= 0x1p16f;
      }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) prev[v] = sum[v];
  }
  // the last tile: handed over after one more barrier
  if (p == 0) {
#pragma unroll
    for (int v = 0; v < 4; ++v) carry[ntl & 1][slot][lane][v] = prev[v];
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("s_barrier" ::: "memory");
  if (p == 0) return;
  {
    float sum[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) sum[v] = prev[v] + carry[ntl & 1][slot][lane][v];
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

// OUTK: 0 = fp32 logits + chunk maxima, 1 = fp16 logits, 2 = bf16 logits
template <typename XT, int OUTK, bool MASKED>
__global__ __launch_bounds__(GQ_WAVES * 64, 2) void k_logits_gqa_kernel(const KArgs a) {
  __shared__ __attribute__((aligned(16))) char ring[GQ_RING];          // a.ws_nst stages of a.ws_stage bytes
  __shared__ float carry[2][GQ_MAXH][64][4];                           // p = 0 partial logits, by tile parity

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int chunk = blockIdx.x, wgp = blockIdx.y, b = blockIdx.z;
  const int S = a.S;
  const int n_tiles = (S + TILE - 1) / TILE;
  const int tile0 = chunk * a.tiles_per_chunk;
  const int tile1 = min(tile0 + a.tiles_per_chunk, n_tiles);
  if (tile0 >= tile1) return;
  const int ntl = tile1 - tile0;

  // ---- the workgroup's KV heads (items of waves 0 and 2), their ranks and
  // chunk offsets in a stage
  GqHeads H;
  H.tot = 0;
#pragma unroll
  for (int k = 0; k < GQ_MAXH; ++k) {
    const uint32_t itm = a.items[wgp * GQ_WAVES + 2 * k][0];
    H.hkv[k] = 0; H.hrank[k] = 8; H.hoff[k] = 1 << 30;
    if (!item_valid(itm)) continue;
    H.hkv[k] = item_kv(itm);
    H.hrank[k] = a.krank[H.hkv[k]];
    H.hoff[k] = H.tot;
    H.tot += 32 * ((H.hrank[k] + 7) >> 3);
  }
  // stage: latent chunks [0, 64 * nX), the RoPE operand in the last 8 KB
  const int nX = (H.tot + 63) / 64, stage = a.ws_stage, nst = a.ws_nst;
  if (H.tot == 0 || nX * 1024 + 8192 > stage || nst < 2 || nst * stage > GQ_RING) return;   // uniform
  const int ahead = nst - 1;     // stage of tile i - 1 (its reads ended at barrier i) takes tile i + ahead

  // ---- this wave's DMA share
  GqDma d;
  {
    const int nI = nX + 8;
    d.cnt = 0;
#pragma unroll
    for (int k = 0; k < GQ_MAXK; ++k) {
      const int m = wave + GQ_WAVES * k;
      d.base[k] = (const char*)a.rope; d.lstep[k] = 0; d.rowp[k] = -(1 << 30); d.adv[k] = 0; d.dst[k] = 0;
      if (m >= nI) continue;
      ++d.cnt;
      if (m >= nX) {
        const int j = m - nX;
        d.base[k] = (const char*)a.rope + (int64_t)tile0 * 8192 + (j * 64 + lane) * 16;
        d.lstep[k] = 8192;
        d.dst[k] = stage - 8192 + j * 1024;
        continue;
      }
      int q = m * 64 + lane;
      if (q >= H.tot) q = H.tot - 1;        // lanes past the last chunk re-read it into an unused slot
      int hb = H.hoff[0], hr = H.hrank[0], hk = H.hkv[0];
#pragma unroll
      for (int j = 1; j < GQ_MAXH; ++j)
        if (H.hoff[j] <= q) { hb = H.hoff[j]; hr = H.hrank[j]; hk = H.hkv[j]; }
      const int n16 = (hr + 7) >> 3, loc = q - hb;
      const int row = loc / n16, cr = loc % n16;
      const int c = (cr - gq_shift(row, n16) % n16 + n16) % n16;
      const int pitch = a.xpitch[hk] * 2;
      d.base[k] = (const char*)a.x + (b * a.x_sb + a.xoff[hk]) * 2 + (int64_t)c * 16 +
                  (int64_t)(tile0 * TILE + row) * pitch;
      d.lstep[k] = (uint32_t)(TILE * pitch);
      d.rowp[k] = row;
      d.adv[k] = pitch;
      d.dst[k] = m * 1024;
    }
    d.ring = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)ring;
    d.stage = stage; d.nst = nst; d.tile0 = tile0; d.S = S;
  }
  const int slot = wave >> 1, p = wave & 1;
  const uint32_t itm = a.items[wgp * GQ_WAVES + wave][0];
  if (!item_valid(itm)) {
    // no head: this wave's DMA share and the workgroup's barriers only
    for (int i = 0; i < min(ahead, ntl); ++i) d.issue(i);
    for (int i = 0; i < ntl; ++i) {
      gq_wait_vm_n(min(ahead - 1, ntl - 1 - i) * d.cnt);
      __builtin_amdgcn_s_waitcnt(0xC07F);
      asm volatile("s_barrier" ::: "memory");
      if (i + ahead < ntl) d.issue(i + ahead);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("s_barrier" ::: "memory");
    return;
  }
  const int kv = item_kv(itm);
  const int nk = (H.hrank[slot] + 15) >> 4;
  if (nk <= 2) gq_consume<XT, OUTK, 2, MASKED>(a, H, d, ring, carry, slot, p, kv, b, chunk, ntl, ahead);
  else if (nk <= 4) gq_consume<XT, OUTK, 4, MASKED>(a, H, d, ring, carry, slot, p, kv, b, chunk, ntl, ahead);
  else if (nk <= 6) gq_consume<XT, OUTK, 6, MASKED>(a, H, d, ring, carry, slot, p, kv, b, chunk, ntl, ahead);
  else gq_consume<XT, OUTK, 8, MASKED>(a, H, d, ring, carry, slot, p, kv, b, chunk, ntl, ahead);
}

template <typename XT, int OUTK>
static void launch_gqa_o(const KArgs& a, dim3 grid, dim3 block, hipStream_t st) {
  if (a.mask != nullptr) hipLaunchKernelGGL((k_logits_gqa_kernel<XT, OUTK, true>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((k_logits_gqa_kernel<XT, OUTK, false>), grid, block, 0, st, a);
}

template <typename XT>
static int launch_gqa_t(const KArgs& a, int outk, int B, hipStream_t st) {
  dim3 grid(a.n_chunks, a.n_wg, B), block(GQ_WAVES * 64);
  if (outk == 0) launch_gqa_o<XT, 0>(a, grid, block, st);
  else if (outk == 1) launch_gqa_o<XT, 1>(a, grid, block, st);
  else launch_gqa_o<XT, 2>(a, grid, block, st);
  return (int)hipGetLastError();
}

int launch_k_logits_gqa(const KArgs& a, int dtype, bool out_f32, int out_dtype, int B, hipStream_t st) {
  const int outk = out_f32 ? 0 : (out_dtype == STARKV_F16 ? 1 : 2);
  return dtype == STARKV_F16 ? launch_gqa_t<_Float16>(a, outk, B, st) : launch_gqa_t<__bf16>(a, outk, B, st);
}

}  // namespace starkv
