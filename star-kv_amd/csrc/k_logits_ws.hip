// K1, warp-specialised: latent-K decode logits for 16-byte aligned fp16/bf16
// latents on gfx950.
//
// Same arithmetic as k_logits.hip (the folded query matrix W times the RoPE
// operand T per 32-position tile, one FMA per latent element; see there), with
// the work of a workgroup split by role:
//
// * 4 producer waves stream, per 32-position tile, the latent rows of every
//   KV head the workgroup serves (each head's tile is 32 rows of 2*r_h bytes)
//   and the tile's RoPE operand (8 KB) into an LDS ring of 3 or 4 stages
//   (as many as fit; the stage is sized on the host for the largest
//   workgroup) with global_load_lds: 16 bytes per lane, 1 KB per
//   instruction, only as many instructions as the workgroup's chunks need.
//   Rows are stored with their 16-byte chunks rotated (ws_shift) so the
//   consumers' row-wise reads are free of LDS bank conflicts.
// * Consumer waves.  The plan packs whole heads into bins of up to 4 items
//   (query head, 32-rank M-tile), 4 bins per workgroup.
//   - Dense latents: 4 consumer waves, one per SIMD, wave c runs bin c.  Its
//     four MFMA chains run one after another and chain j+1's MFMAs carry
//     chain j's dot products, in an order fixed by scheduling fences, so the
//     VALU work runs under the MFMA pipe.  One wave per SIMD also halves the
//     RoPE-operand LDS reads (every consumer wave reads the whole 8 KB tile).
//   - int8 latents: 8 consumer waves, two per SIMD, wave c runs items
//     2*(c/4) and 2*(c/4)+1 of bin c%4, so one wave's dequantisation and dot
//     products overlap the other's MFMA chains.  A head whose items straddle
//     the two halves of a bin is combined through LDS: the first wave leaves
//     its partial logits for the tile, the second adds them one tile later
//     (after the next barrier) and stores.
//
// Measured on MI355X (B16, S32768, ragged ranks summing to 1640): with the
// consumers idle the producers alone stream 5.6 TB/s at 2.4 GHz; the full
// kernel needs only ~5 % more shader cycles than that, but the decode layer
// runs at the board's 1400 W limit and the shader clock settles near
// 2.0-2.2 GHz while the consumers run, so the time is set by the energy per
// tile (MFMA work, LDS traffic, VALU work) as much as by the byte stream.
//
// Stage protocol (one s_barrier per tile, no fence): at tile i the producers
// wait for their own DMA of tile i (vmcnt counts exactly: every lane of an
// issued instruction is in bounds and the per-wave count is fixed), the
// workgroup barriers, the producers issue the DMA of tile i+nst-1 into the
// stage consumed at tile i-1, and the consumers compute tile i.  One extra
// barrier after the last tile publishes the last straddle partials.
#include <climits>

#include "common.hpp"

namespace starkv {

namespace {

constexpr int WS_PRODUCERS = 4;
// consumer waves: dense latents 4 (one per SIMD, a whole bin of up to 4
// items each); int8 latents 8 (two per SIMD, two items each), whose
// dequantisation is better hidden by the second wave
template <bool XI8> constexpr int ws_consumers() { return XI8 ? 8 : 4; }
constexpr int WS_BINS = 4;                          // item bins (of up to 4 items) per workgroup
constexpr int WS_RING = K1_WS_RING_BYTES;           // LDS ring (the straddle carry takes the rest of the 160 KB)
constexpr int WS_MAXK = (2048 / 64 + 9 + WS_PRODUCERS - 1) / WS_PRODUCERS;   // DMA instructions per producer per tile
constexpr int WS_MAXH = 16;                        // KV heads staged by one workgroup
typedef __attribute__((address_space(3))) void lds_void;

// Latent rows sit in LDS with their 16-byte chunks rotated by ws_shift(row):
// ds_read_b128 serves 8 lanes (128 bytes, 32 banks) per cycle, and the lanes
// of a group read the same logical chunk of 8 consecutive rows.  Rows of n16
// chunks repeat their bank offset every p = 8 / gcd(n16, 8) rows; rotating
// by row / p separates the rows that collide, so every group is conflict-free
// for every rank (checked exhaustively for n16 = 1..16).
__device__ inline int ws_shift(int row, int n16) {
  const int g = min(n16 & -n16, 8);
  return row / (8 / g);
}

// 16-byte chunks of one staged row: fp16/bf16 2r bytes, int8 r bytes, each
// rounded up (rows are padded to 16 bytes past the rank)
template <bool XI8> __device__ inline int ws_n16(int r) { return XI8 ? (r + 15) >> 4 : (r + 7) >> 3; }

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 31]
template <int N> __device__ inline void wait_vm() {
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
__device__ inline void wait_vm_n(int n) {
  switch (n) {
#define WS_CASE(N) case N: wait_vm<N>(); break;
    WS_CASE(0) WS_CASE(1) WS_CASE(2) WS_CASE(3) WS_CASE(4) WS_CASE(5) WS_CASE(6) WS_CASE(7)
    WS_CASE(8) WS_CASE(9) WS_CASE(10) WS_CASE(11) WS_CASE(12) WS_CASE(13) WS_CASE(14) WS_CASE(15)
    WS_CASE(16) WS_CASE(17) WS_CASE(18) WS_CASE(19) WS_CASE(20) WS_CASE(21) WS_CASE(22) WS_CASE(23)
    WS_CASE(24) WS_CASE(25) WS_CASE(26) WS_CASE(27) WS_CASE(28) WS_CASE(29) WS_CASE(30)
#undef WS_CASE
    default: wait_vm<0>(); break;
  }
}

// 16 latent values (two 16-byte LDS chunks) . 16 accumulator rows, four partial sums
__device__ inline float dot16h(uint4 u0, uint4 u1, const floatx16& acc) {
  const half8 h0 = __builtin_bit_cast(half8, u0), h1 = __builtin_bit_cast(half8, u1);
  float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int v = 0; v < 8; ++v) p[v & 3] = fmaf((float)h0[v], acc[v], p[v & 3]);
#pragma unroll
  for (int v = 0; v < 8; ++v) p[v & 3] = fmaf((float)h1[v], acc[8 + v], p[v & 3]);
  return (p[0] + p[1]) + (p[2] + p[3]);
}
__device__ inline float dot16b(uint4 u0, uint4 u1, const floatx16& acc) {
  const uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
  float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    p[(2 * v) & 3] = fmaf(__uint_as_float(w[v] << 16), acc[2 * v], p[(2 * v) & 3]);
    p[(2 * v + 1) & 3] = fmaf(__uint_as_float(w[v] & 0xffff0000u), acc[2 * v + 1], p[(2 * v + 1) & 3]);
  }
  return (p[0] + p[1]) + (p[2] + p[3]);
}

// values 2k, 2k+1 of a 16-value dot (word k % 4 of u0 for k < 4, else of
// u1) into the partial sums p[(2k) & 3], p[(2k+1) & 3]: the order of
// dot16h / dot16b, split so the pieces can sit between MFMAs
template <bool BF>
__device__ inline void dot_piece(const uint4& u0, const uint4& u1, const floatx16& acc, int k, float p[4]) {
  const uint4& u = k < 4 ? u0 : u1;
  const uint32_t w = (k & 3) == 0 ? u.x : (k & 3) == 1 ? u.y : (k & 3) == 2 ? u.z : u.w;
  float a, c;
  if constexpr (BF) {
    a = __uint_as_float(w << 16);
    c = __uint_as_float(w & 0xffff0000u);
  } else {
    const kh2 h = __builtin_bit_cast(kh2, w);
    a = (float)h[0];
    c = (float)h[1];
  }
  p[(2 * k) & 3] = fmaf(a, acc[2 * k], p[(2 * k) & 3]);
  p[(2 * k + 1) & 3] = fmaf(c, acc[2 * k + 1], p[(2 * k + 1) & 3]);
}

#define WS_FENCE() __builtin_amdgcn_sched_barrier(0)

// int8 latents: the 16 bytes of a lane with the sign bit flipped (n + 128,
// unsigned) and the fp16 scale broadcast to both halves
__device__ inline uint4 i8_bias(uint4 r) {
  return make_uint4(r.x ^ 0x80808080u, r.y ^ 0x80808080u, r.z ^ 0x80808080u, r.w ^ 0x80808080u);
}
__device__ inline kh2 i8_scale(uint16_t s16) { return __builtin_bit_cast(kh2, (uint32_t)s16 * 0x10001u); }

// piece k of an int8 dot: ranks 2k, 2k+1 of the lane's 16 (bytes 2k, 2k+1 of
// w = i8_bias(latent)) dequantised bit-exactly, fp16(n * s) as in dequant16,
// times accumulator rows 2k, 2k+1 into p[(2k) & 3], p[(2k+1) & 3]: pieces
// 0..7 in order are the sums of dequant16 + dot16h
__device__ inline void i8_piece(const uint4& w, kh2 s, const floatx16& acc, int k, float p[4]) {
  const uint32_t u = (k >> 1) == 0 ? w.x : (k >> 1) == 1 ? w.y : (k >> 1) == 2 ? w.z : w.w;
  const uint32_t pr = __builtin_amdgcn_perm(0x64646464u, u, (k & 1) ? 0x04030402u : 0x04010400u);
  const kh2 b2 = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  const kh2 h = (__builtin_bit_cast(kh2, pr) + b2) * s;
  p[(2 * k) & 3] = fmaf((float)h[0], acc[2 * k], p[(2 * k) & 3]);
  p[(2 * k + 1) & 3] = fmaf((float)h[1], acc[2 * k + 1], p[(2 * k + 1) & 3]);
}

}  // namespace

// OUTK: 0 = fp32 logits + chunk maxima, 1 = fp16 logits, 2 = bf16 logits
// XI8: int8 latents (rows padded to 16 bytes) with one fp16 scale per (b, h, s),
//      dequantised bit-exactly to fp16 after the LDS read; the tile's scales
//      are staged with its rows (one more DMA instruction), so the consumers
//      issue no global loads
template <typename XT, int OUTK, bool XI8>
__global__ __launch_bounds__((ws_consumers<XI8>() + WS_PRODUCERS) * 64, 1) void k_logits_ws_kernel(const KArgs a) {
  constexpr int NCONS = ws_consumers<XI8>();
  constexpr int MAXI = XI8 ? 2 : 4;                  // items per consumer wave
  constexpr bool XB = !XI8 && !__is_same(XT, _Float16);   // bf16 latents
  constexpr int RING = XI8 ? K1_WS_RING_I8_BYTES : WS_RING;
  __shared__ __attribute__((aligned(16))) char ring[RING];   // a.ws_nst stages of a.ws_stage bytes
  __shared__ float carry[XI8 ? 3 : 2][WS_BINS][32];  // straddling heads: first half's partial logits

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

  // ---- the workgroup's KV heads (scalar, identical in every wave): distinct
  // KV heads of its items in first-use order, with rank and offset in a stage
  // in 16-byte chunks.  Loops are fully unrolled so the tables stay in
  // registers.
  int hkv[WS_MAXH], hrank[WS_MAXH], hoff[WS_MAXH];
#pragma unroll
  for (int k = 0; k < WS_MAXH; ++k) { hkv[k] = -1; hrank[k] = 8; hoff[k] = 1 << 30; }
  int nh = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < WS_BINS; ++w) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t itm = a.items[wgp * WS_BINS + w][i];
      if (!item_valid(itm) || !item_last(itm)) continue;
      const int kv = item_kv(itm), r = item_mt(itm) * 32 + item_nv(itm);
      bool found = false;
#pragma unroll
      for (int k = 0; k < WS_MAXH; ++k) found |= hkv[k] == kv;
      if (found) continue;
#pragma unroll
      for (int k = 0; k < WS_MAXH; ++k)
        if (k == nh) { hkv[k] = kv; hrank[k] = r; hoff[k] = tot; }
      tot += 32 * ws_n16<XI8>(r);           // 16-byte chunks per 32-row tile
      ++nh;
    }
  }
  // stage: latent chunks [0, 64 * nX), int8: the tile's scales in the 1 KB
  // before the RoPE operand (64 bytes per head slot), the RoPE operand in the
  // last 8 KB
  const int nX = (tot + 63) / 64, stage = a.ws_stage, nst = a.ws_nst;
  constexpr int SCB = XI8 ? 1024 : 0;
  const int sc_off = stage - 8192 - SCB;
  if (tot == 0 || nX * 1024 + SCB + 8192 > stage || nst < 2 || nst * stage > RING) return;   // uniform

  if (wave >= NCONS) {
    // ================= producer =================
    const int pw = wave - NCONS;
    // DMA instruction m (latent chunks [64m, 64m+64) for m < nX, then the
    // RoPE operand in 1 KB pieces, then (int8) the scales) belongs to
    // producer m % 4.  Per instruction k of this wave: the lane's source and
    // stage offset; it reads position min(tile * tmul + rowpos, pmax).
    const int nI = nX + 8 + (XI8 ? 1 : 0), ahead = nst - 1;
    const char* src[WS_MAXK];
    int64_t adv[WS_MAXK];   // latent / scales: bytes per position; RoPE: bytes per tile
    int rowpos[WS_MAXK];    // latent: row within the tile; scales: first of the lane's 8 positions
    int tmul[WS_MAXK];      // positions per tile (RoPE: 1, indexed by tile)
    int pmax[WS_MAXK];      // last position that may be read
    int dst[WS_MAXK];       // wave-uniform stage offset
    int cnt = 0;
#pragma unroll
    for (int k = 0; k < WS_MAXK; ++k) {
      const int m = pw + WS_PRODUCERS * k;
      src[k] = (const char*)a.rope; adv[k] = 8192; rowpos[k] = 0; tmul[k] = 1; pmax[k] = 1 << 30; dst[k] = 0;
      if (m >= nI) continue;
      ++cnt;
      if (XI8 && m == nX + 8) {
        // lane = 4 * head slot + piece: 16 bytes = the scales of 8 positions;
        // pieces past the tile's last position re-read the row's last piece
        // (the host checked that each row is readable through round_up(S, 8))
        const int hs = lane >> 2;
        int hk = hkv[0];
#pragma unroll
        for (int j = 1; j < WS_MAXH; ++j)
          if (j == hs && j < nh) hk = hkv[j];
        src[k] = (const char*)a.xscale + (b * a.xs_sb + hk * a.xs_sh) * 2;
        adv[k] = 2; rowpos[k] = 8 * (lane & 3); tmul[k] = TILE; pmax[k] = ((S - 1) >> 3) << 3;
        dst[k] = sc_off;
        continue;
      }
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
      for (int j = 1; j < WS_MAXH; ++j)
        if (hoff[j] <= q) { hb = hoff[j]; hr = hrank[j]; hk = hkv[j]; }
      const int n16 = ws_n16<XI8>(hr), loc = q - hb;
      const int row = loc / n16, cr = loc % n16;             // stored (rotated) chunk cr of row
      const int c = (cr - ws_shift(row, n16) % n16 + n16) % n16;   // the row's chunk that lives there
      constexpr int XE = XI8 ? 1 : 2;        // quantised offsets are in bytes
      src[k] = (const char*)a.x + (b * a.x_sb + a.xoff[hk]) * XE + (int64_t)c * 16;
      adv[k] = (int64_t)a.xpitch[hk] * XE;
      rowpos[k] = row;
      tmul[k] = TILE;
      pmax[k] = S - 1;
      dst[k] = m * 1024;
    }
    // A tile whose 32 positions all lie below S needs no clamping: there each
    // lane's address is its first tile's address plus (tile - tile0) times a
    // fixed per-lane step (latent rows and scales: 32 positions; RoPE operand:
    // 8 KB), one 32x32->64-bit multiply-add instead of the clamped form.  The
    // producers share their SIMDs with the consumers, so this VALU work is
    // taken from the consumers' issue slots.
    const char* base[WS_MAXK];     // lane address at tile0
    uint32_t lstep[WS_MAXK];       // bytes per tile (< 2^31, checked on the host)
#pragma unroll
    for (int k = 0; k < WS_MAXK; ++k) {
      base[k] = src[k] + (int64_t)(tile0 * tmul[k] + rowpos[k]) * adv[k];
      lstep[k] = (uint32_t)(tmul[k] * adv[k]);
    }
    auto issue = [&](int i) __attribute__((always_inline)) {
      const int tl = min(tile0 + i, last);
      char* st = ring + (i % nst) * stage;
      if ((tl + 1) * TILE <= S) {
        const uint32_t ti = (uint32_t)(tl - tile0);
#pragma unroll
        for (int k = 0; k < WS_MAXK; ++k) {
          const int m = pw + WS_PRODUCERS * k;
          if (m >= nI) break;
          __builtin_amdgcn_global_load_lds((const void*)(base[k] + (uint64_t)ti * lstep[k]), (lds_void*)(st + dst[k]), 16, 0, 0);
        }
      } else {
#pragma unroll
        for (int k = 0; k < WS_MAXK; ++k) {
          const int m = pw + WS_PRODUCERS * k;
          if (m >= nI) break;
          const int64_t pos = min(tl * tmul[k] + rowpos[k], pmax[k]);
          __builtin_amdgcn_global_load_lds((const void*)(src[k] + pos * adv[k]), (lds_void*)(st + dst[k]), 16, 0, 0);
        }
      }
    };
    for (int i = 0; i < ahead; ++i) issue(i);
    for (int i = 0; i < ntl; ++i) {
      // this producer's DMA of tile i complete: tiles i+1 .. i+ahead-1 may be in flight
      wait_vm_n((ahead - 1) * cnt);
      __builtin_amdgcn_s_barrier();
      issue(i + ahead);                      // into the stage consumed at tile i-1
    }
    __builtin_amdgcn_s_barrier();           // the consumers' extra barrier
    wait_vm<0>();                            // drain the trailing (clamped) DMA before the wave ends
    return;
  }

  // ================= consumer =================
  // int8: consumer wave c runs items 2*(c/4), 2*(c/4)+1 of bin c%4; dense:
  // wave c runs bin c
  const int bin = wave & (WS_BINS - 1), half = XI8 ? wave / WS_BINS : 0;
  uint32_t it[MAXI];
#pragma unroll
  for (int i = 0; i < MAXI; ++i) it[i] = a.items[wgp * WS_BINS + bin][MAXI * half + i];
  // int8: the bin's item 1 ends the first half; if it is not its head's last
  // item the head straddles the two waves
  const uint32_t i1 = a.items[wgp * WS_BINS + bin][1];
  const bool straddle = XI8 && item_valid(i1) && !item_last(i1);
  const bool send = straddle && half == 0;   // leaves the partial logits of its last head
  const bool recv = straddle && half == 1;   // completes its first head one tile later

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
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ql[e] = to_f32(qrow[i0 + e]); qu[e] = to_f32(qrow[i0 + 64 + e]);
          bl[e] = to_f32(brow[i0 + e]); bu[e] = to_f32(brow[i0 + 64 + e]);
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
  // LDS byte offsets (within a stage) of this lane's 16 ranks of each item's
  // row t: two 16-byte chunks (fp16/bf16) or one (int8); lanes past the valid
  // ranks re-read valid data (multiplied by the zero rows of W)
  int xo0[MAXI], xo1[MAXI];
  int sco[MAXI];                             // int8: this lane's scale (position t of the item's head)
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    xo0[i] = xo1[i] = 0;
    sco[i] = sc_off;
    if (!item_valid(it[i])) continue;
    const int kv = item_kv(it[i]), mt = item_mt(it[i]), nvh = item_nv(it[i]) - 16 * hh;
    int hb = 0, hr = 8, hs = 0;
#pragma unroll
    for (int j = 0; j < WS_MAXH; ++j)
      if (hkv[j] == kv) { hb = hoff[j]; hr = hrank[j]; hs = j; }
    sco[i] = sc_off + hs * 64 + t * 2;
    const int n16 = ws_n16<XI8>(hr);
    const int rowb = (hb + t * n16) * 16;
    const int sh = ws_shift(t, n16);
    if constexpr (XI8) {
      const int c0 = nvh > 0 ? mt * 2 + hh : mt * 2;
      xo0[i] = xo1[i] = rowb + ((c0 + sh) % n16) * 16;
    } else {
      const int c0 = nvh > 0 ? mt * 4 + 2 * hh : mt * 4;
      const int c1 = nvh > 8 ? c0 + 1 : c0;
      xo0[i] = rowb + ((c0 + sh) % n16) * 16;
      xo1[i] = rowb + ((c1 + sh) % n16) * 16;
    }
  }
  float mx[MAXI];
#pragma unroll
  for (int i = 0; i < MAXI; ++i) mx[i] = -INFINITY;

  // positions past a device-held last position take -1e30 (read once)
  const int lastp = a.last_pos != nullptr ? *a.last_pos : INT_MAX;
  // logit epilogue of one head at position s: mask, store, running maximum
  // this batch's logits: a uniform base and 32-bit element offsets (the host
  // keeps a batch's offsets below 2^32; a 64-bit per-lane address held
  // across the tile loop had cost the int8 kernel a spill)
  char* const obase = (char*)a.out + b * a.o_sb * (OUTK == 0 ? 4 : 2);
  const uint32_t ost = (uint32_t)a.o_st, osh = (uint32_t)a.o_sh;
  auto emit = [&](float v, int qh, int s, float& m) __attribute__((always_inline)) {
    if (s < S) {
      if (a.mask != nullptr) v += load_elem_f32(a.mask, a.mask_dtype, b * a.m_sb + qh * a.m_sh + s);
      if (s > lastp) v = -1e30f;
      if (hh == 0) {                         // both halves hold the sum; one stores
        const uint32_t o = (uint32_t)(s >> 5) * ost + (uint32_t)qh * osh + (uint32_t)(s & 31);
        if constexpr (OUTK == 0) ((float*)obase)[o] = v;
        else if constexpr (OUTK == 1) ((_Float16*)obase)[o] = (_Float16)v;
        else ((__bf16*)obase)[o] = (__bf16)v;
      }
      m = fmaxf(m, v);
    }
  };
  // the first head of a receiving wave ends at its item j0
  const int j0 = item_last(it[0]) ? 0 : 1;

  if constexpr (!XI8) {
  for (int i = 0; i < ntl; ++i) {
    __builtin_amdgcn_s_waitcnt(0xC07F);      // this wave's LDS reads are done
    __builtin_amdgcn_s_barrier();
    if (!item_valid(it[0])) continue;
    const char* st = ring + (i % nst) * stage;
    const int s = (tile0 + i) * TILE + t;
    uint4 x0[MAXI], x1[MAXI];
#pragma unroll
    for (int j = 0; j < MAXI; ++j) {
      x0[j] = *(const uint4*)(st + xo0[j]);
      x1[j] = *(const uint4*)(st + xo1[j]);
    }
    half8 T[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) T[k] = *(const half8*)(st + stage - 8192 + (k * 64 + lane) * 16);
    // every item's chain (an unused item has zero W rows and reads valid LDS
    // data); chain j+1's MFMAs carry chain j's dot products, in an order fixed
    // by scheduling fences (the empty asm keeps each piece where it is), so
    // the VALU work runs while the MFMA pipe is busy
    float d[MAXI];
    floatx16 accp, accc;
#pragma unroll
    for (int j = 0; j < MAXI; ++j) {
      float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        accc = mfma_f16(wr[j][k], T[k], k == 0 ? floatx16{} : accc);
        if (j > 0) {
          WS_FENCE();
          dot_piece<XB>(x0[j - 1], x1[j - 1], accp, k, p);
          asm volatile("" :: "v"(p[(2 * k) & 3]), "v"(p[(2 * k + 1) & 3]));
          WS_FENCE();
        }
      }
      if (j > 0) d[j - 1] = (p[0] + p[1]) + (p[2] + p[3]);
      accp = accc;
    }
    {
      float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 8; ++k) dot_piece<XB>(x0[MAXI - 1], x1[MAXI - 1], accp, k, p);
      d[MAXI - 1] = (p[0] + p[1]) + (p[2] + p[3]);
    }
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < MAXI; ++j) {
      part += d[j];
      if (item_last(it[j])) {
        const float v = add_halves(part);
        part = 0.f;
        emit(v, item_qh(it[j]), s, mx[j]);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();              // the producers' extra barrier
  } else {
    // int8: the MFMA chains of tile i carry the dequantisation and dot
    // products of the item before in (tile, item) order,
    //     chain (i, 0) || pieces of (i-1, 1),   chain (i, 1) || pieces of (i, 0),
    // so each chain's VALU work runs under the MFMA pipe of the same wave (the
    // per-tile barrier keeps the two consumer waves of a SIMD in phase: one
    // wave's VALU work does not hide under the other's MFMAs).  Item 1 of the
    // last tile is finished after the loop.  Straddling heads: the sending
    // wave writes tile k's partials during tile k+1 (after the loop for the
    // last tile) into carry slot k % 3; the receiving wave adds them to its
    // own part after the barrier of tile k+2 (after the final barrier for the
    // last two tiles), holding its parts in a two-tile shift register (qn
    // newest, qo older).  Three slots: within one barrier interval the
    // receiver reads tile k's slot while the sender writes tile k+1's and,
    // after the loop, tile k+2's.
    const bool v0 = item_valid(it[0]);
    if (a.mask != nullptr) {
      // With an additive mask, each emission's mask load waits for the
      // logit stores issued before it (the memory counter retires in order),
      // and the pipelined order below leaves one more of those waits exposed
      // per tile: 70.5 against 67.8 us at the e2e shape.  Masked launches
      // keep both chains before both dot products (carry slot k & 1, read one
      // tile later).
      float pend = 0.f;                      // receiving wave: own part of the tile before
      for (int i = 0; i < ntl; ++i) {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS reads and writes are done
        __builtin_amdgcn_s_barrier();
        if (!v0) continue;
        if (recv && i > 0)
          emit(pend + carry[(i - 1) & 1][bin][t], item_qh(it[j0]), (tile0 + i - 1) * TILE + t, mx[j0]);
        const char* st = ring + (i % nst) * stage;
        const int s = (tile0 + i) * TILE + t;
        half8 T[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) T[k] = *(const half8*)(st + stage - 8192 + (k * 64 + lane) * 16);
        uint4 x0[MAXI];
        uint16_t sc[MAXI];
#pragma unroll
        for (int j = 0; j < MAXI; ++j) {
          x0[j] = *(const uint4*)(st + xo0[j]);
          sc[j] = *(const uint16_t*)(st + sco[j]);
        }
        floatx16 acc[MAXI];
#pragma unroll
        for (int j = 0; j < MAXI; ++j) acc[j] = mfma_f16(wr[j][0], T[0], floatx16{});
#pragma unroll
        for (int k = 1; k < 8; ++k)
#pragma unroll
          for (int j = 0; j < MAXI; ++j) acc[j] = mfma_f16(wr[j][k], T[k], acc[j]);
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < MAXI; ++j) {
          uint4 lo, hi;
          dequant16(x0[j], true, sc[j], lo, hi);
          part += dot16h(lo, hi, acc[j]);
          if (item_last(it[j])) {
            const float v = add_halves(part);
            part = 0.f;
            if (recv && j == j0) pend = v;
            else emit(v, item_qh(it[j]), s, mx[j]);
          }
        }
        if (send) {
          const float v = add_halves(part);
          if (hh == 0) carry[i & 1][bin][t] = v;
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_s_barrier();          // publishes the last tile's partials
      if (recv && v0)
        emit(pend + carry[(ntl - 1) & 1][bin][t], item_qh(it[j0]), (tile0 + ntl - 1) * TILE + t, mx[j0]);
    } else {
    floatx16 accp = floatx16{};              // accumulators of item (i-1, 1)
    uint4 wp = make_uint4(0, 0, 0, 0);       // its latent bytes ^ 0x80 and scale
    kh2 sp = kh2{};
    float hold = 0.f;                        // item 0's part of a head that continues into item 1
    float qn = 0.f, qo = 0.f;
    auto fin0 = [&](float d, int s) __attribute__((always_inline)) {
      if (item_last(it[0])) {
        const float v = add_halves(d);
        if (recv && j0 == 0) qn = v;
        else emit(v, item_qh(it[0]), s, mx[0]);
      } else {
        hold = d;
      }
    };
    auto fin1 = [&](float d, int s, int slot) __attribute__((always_inline)) {
      if (!item_valid(it[1])) return;
      const float v = add_halves((item_last(it[0]) ? 0.f : hold) + d);
      if (item_last(it[1])) {
        if (recv && j0 == 1) qn = v;
        else emit(v, item_qh(it[1]), s, mx[1]);
      } else if (send && hh == 0) {
        carry[slot][bin][t] = v;
      }
    };
    for (int i = 0; i < ntl; ++i) {
      __builtin_amdgcn_s_waitcnt(0xC07F);    // this wave's LDS reads and writes are done
      __builtin_amdgcn_s_barrier();
      if (!v0) continue;
      if (recv) {
        if (i >= 2) emit((j0 ? qn : qo) + carry[(i - 2) % 3][bin][t], item_qh(it[j0]), (tile0 + i - 2) * TILE + t, mx[j0]);
        qo = qn;
      }
      const char* st = ring + (i % nst) * stage;
      const int s = (tile0 + i) * TILE + t;
      half8 T[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) T[k] = *(const half8*)(st + stage - 8192 + (k * 64 + lane) * 16);
      uint4 xn[MAXI];
      uint16_t scn[MAXI];
#pragma unroll
      for (int j = 0; j < MAXI; ++j) {
        xn[j] = *(const uint4*)(st + xo0[j]);
        scn[j] = *(const uint16_t*)(st + sco[j]);
      }
      // an unused item has zero W rows and reads valid LDS data; at i = 0 the
      // pieces of chain 0 work on zeros and are discarded
      float p[4] = {0.f, 0.f, 0.f, 0.f};
      floatx16 acc0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        acc0 = mfma_f16(wr[0][k], T[k], k == 0 ? floatx16{} : acc0);
        WS_FENCE();
        i8_piece(wp, sp, accp, k, p);
        asm volatile("" :: "v"(p[(2 * k) & 3]), "v"(p[(2 * k + 1) & 3]));
        WS_FENCE();
      }
      if (i > 0) fin1((p[0] + p[1]) + (p[2] + p[3]), s - TILE, (i - 1) % 3);
      const uint4 w0 = i8_bias(xn[0]);
      const kh2 s0 = i8_scale(scn[0]);
#pragma unroll
      for (int e = 0; e < 4; ++e) p[e] = 0.f;
      floatx16 acc1;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        acc1 = mfma_f16(wr[1][k], T[k], k == 0 ? floatx16{} : acc1);
        WS_FENCE();
        i8_piece(w0, s0, acc0, k, p);
        asm volatile("" :: "v"(p[(2 * k) & 3]), "v"(p[(2 * k + 1) & 3]));
        WS_FENCE();
      }
      fin0((p[0] + p[1]) + (p[2] + p[3]), s);
      accp = acc1;
      wp = i8_bias(xn[1]);
      sp = i8_scale(scn[1]);
    }
    if (v0) {
      float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 8; ++k) i8_piece(wp, sp, accp, k, p);
      if (recv && j0 == 1) qo = qn;
      fin1((p[0] + p[1]) + (p[2] + p[3]), (tile0 + ntl - 1) * TILE + t, (ntl - 1) % 3);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();            // publishes the last two tiles' partials
    if (recv && v0) {
      if (ntl >= 2) emit(qo + carry[(ntl - 2) % 3][bin][t], item_qh(it[j0]), (tile0 + ntl - 2) * TILE + t, mx[j0]);
      emit(qn + carry[(ntl - 1) % 3][bin][t], item_qh(it[j0]), (tile0 + ntl - 1) * TILE + t, mx[j0]);
    }
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

template <typename XT, bool XI8>
static int launch_ws_t(const KArgs& a, int outk, int B, hipStream_t st) {
  dim3 grid(a.n_chunks, a.n_wg, B), block((ws_consumers<XI8>() + WS_PRODUCERS) * 64);
  if (outk == 0) hipLaunchKernelGGL((k_logits_ws_kernel<XT, 0, XI8>), grid, block, 0, st, a);
  else if (outk == 1) hipLaunchKernelGGL((k_logits_ws_kernel<XT, 1, XI8>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((k_logits_ws_kernel<XT, 2, XI8>), grid, block, 0, st, a);
  return (int)hipGetLastError();
}

int launch_k_logits_ws(const KArgs& a, int dtype, bool out_f32, int out_dtype, int B, hipStream_t st) {
  const int outk = out_f32 ? 0 : (out_dtype == STARKV_F16 ? 1 : 2);
  if (a.ws_i8) return dtype == STARKV_F16 ? launch_ws_t<_Float16, true>(a, outk, B, st) : launch_ws_t<__bf16, true>(a, outk, B, st);
  return dtype == STARKV_F16 ? launch_ws_t<_Float16, false>(a, outk, B, st) : launch_ws_t<__bf16, false>(a, outk, B, st);
}

}  // namespace starkv
