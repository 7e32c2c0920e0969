// Prefill from the latent caches on gfx950: the counterpart of the
// reference's prefill branch (model.py:429-449), which materialises K and V
// from the latents and runs SDPA -- without a causal mask (the defect the
// build fixes: query t sees keys <= pos0 + t).
//
// 1. recon_kernel / recon_v_kernel: MFMA GEMM tiles computing
//    K = RoPE(X_k[s] . B_k) (RoPE applied in the epilogue from the decode's
//    RoPE table; per (KV head, b, 256 positions)) and V = X_v[s] . U_v[h]^T
//    (per (KV-head pair, b, 256 positions)), into [B][Hkv][S_pad][128]
//    fp16 buffers (for either activation dtype: the reference materialises
//    K and V in the activation dtype, model.py:431-442; fp16 holds bf16
//    models' K and V with 2^-12 instead of 2^-9 unit roundoff).  Quantised
//    latents are dequantised on the way in, bit-exactly as everywhere else
//    (int8: fp16(q s); the reference int4 format: fp16((nibble - 8) s);
//    group-64 int4: fp16(n s + z)), then rounded once more to bf16 for bf16
//    activations.  Rows in [S, S_pad) are written as zeros.
// 2. fa_causal_kernel: flash attention over those buffers, one workgroup per
//    (b, query head, 256 queries), 8 waves of 32 queries, fp16 MFMAs (bf16
//    queries converted to fp16 on load).  Per 64-key block it forms
//    S^T = K . Q^T (so each lane holds 32 keys of one query and the online
//    softmax needs one cross-half exchange); the lane's probabilities are the
//    B operand of O^T += V^T . P^T as they stand, V^T read from LDS with the
//    transpose load in the matching key order.
#include "common.hpp"

namespace starkv {

namespace {

constexpr int WT_PITCH = 136;   // LDS row pitch (halves) of B_k^T and of the K / V blocks
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 pf_fp16x4;

__device__ inline uint2 pf_read_tr16(const uint16_t* p) {
  auto r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) pf_fp16x4*)(p));
  return __builtin_bit_cast(uint2, r);
}

template <typename XT> __device__ inline floatx16 pf_mfma(uint4 a, uint4 b, floatx16 c) {
  if constexpr (__is_same(XT, _Float16))
    return mfma_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c);
  else
    return mfma_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c);
}

template <typename XT> __device__ inline uint16_t pf_bits(float x) {
  return __builtin_bit_cast(uint16_t, (XT)x);
}

// The reconstructed K and V are held in fp16 for both activation dtypes: for
// bf16 activations fp16 keeps 3 more significand bits (unit roundoff 2^-12
// instead of 2^-9), so the attention over them stays within the decode path's
// accuracy.  Values beyond +-65504 are not representable (far outside what
// attention keys and values reach).
typedef _Float16 KVT;

// bf16 pairs -> fp16 pairs (exact for values inside fp16's normal range)
__device__ inline uint4 pf_bf16_to_f16(uint4 h) {
  const uint32_t w[4] = {h.x, h.y, h.z, h.w};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    o[k] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(w[k] << 16)) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(w[k] & 0xffff0000u)) << 16);
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// fp16 pairs -> bf16 pairs (one rounding), for bf16 activations over
// dequantised (fp16) latents
__device__ inline uint4 pf_f16_to_bf16(uint4 h) {
  const uint32_t w[4] = {h.x, h.y, h.z, h.w};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const kh2 v = __builtin_bit_cast(kh2, w[k]);
    o[k] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(float)v[0]) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(float)v[1]) << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// 8 int8 (n) -> fp16(n * s), ranks in order, bit-exact (1152 + n is exact in fp16)
__device__ inline uint4 pf_dq_int8(uint2 q, uint16_t s16) {
  const uint32_t x = q.x ^ 0x80808080u, y = q.y ^ 0x80808080u;
  const uint32_t pr[4] = {__builtin_amdgcn_perm(0x64646464u, x, 0x04010400u),
                          __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u),
                          __builtin_amdgcn_perm(0x64646464u, y, 0x04010400u),
                          __builtin_amdgcn_perm(0x64646464u, y, 0x04030402u)};
  const kh2 s = __builtin_bit_cast(kh2, (uint32_t)s16 * 0x10001u);
  const kh2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(kh2, pr[k]) + bias) * s);
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// 8 int4 nibbles of the reference format (rank 2k in the low nibble of byte k,
// value nibble - 8) -> fp16((nibble - 8) * s), ranks in order, bit-exact
// (1024 + nibble - 1032 is exact in fp16; one rounding in the multiply)
__device__ inline uint4 pf_dq_int4ref(uint32_t w, uint16_t s16) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  const kh2 s = __builtin_bit_cast(kh2, (uint32_t)s16 * 0x10001u);
  const kh2 bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t p = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u + 0x00010001u * k) | 0x64006400u;
    o[k] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(kh2, p) + bias) * s);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// 8 ranks of a per-token block latent (the reference split format): the chunk
// of ranks j .. j+7 lies wholly in the upper block (j < split; int8 or int4)
// or the lower one (int4); the raw words hold 8 bytes (int8) or 4 (int4, .x)
__device__ inline uint2 pf_ld_block(const uint8_t* up, const uint8_t* lo, int j, int split, bool a8) {
  if (j < split) {
    if (a8) return *(const uint2*)(up + j);
    return make_uint2(*(const uint32_t*)(up + j / 2), 0u);
  }
  return make_uint2(*(const uint32_t*)(lo + (j - split) / 2), 0u);
}
__device__ inline uint4 pf_dq_block(uint2 w, int j, int split, bool a8, uint16_t s_up, uint16_t s_lo) {
  if (j < split) return a8 ? pf_dq_int8(w, s_up) : pf_dq_int4ref(w.x, s_up);
  return pf_dq_int4ref(w.x, s_lo);
}

// 8 int4 nibbles (rank 2k in the low nibble of byte k) -> fp16(n * s + z), ranks in order
__device__ inline uint4 pf_dq_g64(uint32_t w, uint16_t s16, uint16_t z16) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  const kh2 s = __builtin_bit_cast(kh2, (uint32_t)s16 * 0x10001u);
  const kh2 z = __builtin_bit_cast(kh2, (uint32_t)z16 * 0x10001u);
  const kh2 bias = {(_Float16)-1024.0f, (_Float16)-1024.0f};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t p = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u + 0x00010001u * k) | 0x64006400u;
    o[k] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(kh2, p) + bias, s, z));
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace

// ---------------------------------------------------------------------------
// K reconstruction: per (KV head h, b, 256 positions) one workgroup of 4
// waves; wave w computes C^T[d][p] for all 128 dims d and its 64 positions
// p as 4 x 2 MFMA tiles (128 accumulators: two workgroups share a CU, so one's
// stores overlap the other's loads and MFMAs) (A = B_k[h], dims as rows, staged whole in LDS as
// [j][d] and read with the transposed LDS load; B = latent rows, positions as
// columns, loaded from global straight into registers one K-step ahead).  A
// K-step is 64 ranks; within it lane half hh takes ranks [32 hh, 32 hh + 32)
// (MFMA K-chunk kk: ranks 32 hh + 8 kk .. + 7) in both operands, so each lane
// reads one contiguous 32-rank run of a latent row.  RoPE pairs (d, d + 64)
// sit in M-tiles mt and mt + 2 of the same lane.  The epilogue stages each
// wave's 64 x 128 tile in LDS and writes whole 256-byte rows.
// ---------------------------------------------------------------------------
constexpr int RC_WAVE_POS = 64;                  // positions per wave
constexpr int RC_NT = RC_WAVE_POS / 32;          // N-tiles per wave
constexpr int RC_POS = 4 * RC_WAVE_POS;          // positions per workgroup
static_assert(RC_POS == PF_K_POS, "host grid sizing");
constexpr int RC_KS = 64;                        // ranks per K-step
constexpr int BK_PITCH = 136;                    // halves per staged B_k row (128 dims + 8)
constexpr int C_PITCH = 136;                     // halves per epilogue row
constexpr int RC_LDS = 4 * RC_WAVE_POS * C_PITCH;

// raw K latent data of one K-step for this lane: [N-tile][K-chunk]
template <int Q> struct RkRaw { uint2 d[RC_NT][4]; };                         // int8 / reference split: <= 8 bytes per chunk
template <> struct RkRaw<0> { uint4 d[RC_NT][4]; };                          // dense: 8 ranks per chunk

// Q: 0 dense act dtype, 1 int8 with one scale per (b, h, s), 2 the reference
// split format (ranks below ksplit int8 or int4, the rest int4, each block
// with its scale per (b, h, s))
template <typename XT, int Q>
__global__ __launch_bounds__(256, 2) void recon_kernel(const PFArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[RC_LDS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  // XCD-aware order: workgroup L runs on XCD L % 8, and the Hkv heads of one
  // (batch, 256-position block) all land on one XCD
  const int L = blockIdx.x, t8 = L >> 3;
  const int h = t8 % a.Hkv, blk = (t8 / a.Hkv) * 8 + (L & 7);
  if (blk >= a.rc_blocks) return;
  const int b = blk / a.rc_nb;
  const int pw = (blk - b * a.rc_nb) * RC_POS + wave * RC_WAVE_POS;
  const int S = a.S;
  // latent rows hold Rl = round_up(R, 8) ranks (rows of other ranks are
  // repacked by the host into padded copies whose extra ranks are zero)
  const int R = a.krank[h], Rl = (R + 7) & ~7;
  const int nks = (Rl + RC_KS - 1) / RC_KS;

  // per N-tile latent row (clamped position) and scales
  const uint8_t* xrow[RC_NT];
  const uint8_t* xrow2[RC_NT];                           // reference split: the lower (int4) block
  uint16_t ksc[RC_NT] = {}, ksc2[RC_NT] = {};
  const bool klo = Q == 2 && R > a.ksplit;           // this head has a lower block
#pragma unroll
  for (int nt = 0; nt < RC_NT; ++nt) {
    const int pc = min(pw + nt * 32 + n, S - 1);
    constexpr int64_t es = Q ? 1 : 2;                // latent offsets: bytes (quantised) or elements
    xrow[nt] = (const uint8_t*)a.kx + (b * a.kx_sb + a.kxoff[h] + (int64_t)pc * a.kxpitch[h]) * es;
    xrow2[nt] = xrow[nt];
    if constexpr (Q) ksc[nt] = ((const uint16_t*)a.kscale)[b * a.ks_sb + h * a.ks_sh + pc];
    if (klo) {
      xrow2[nt] = (const uint8_t*)a.kx2 + b * a.kx2_sb + a.kxoff2[h] + (int64_t)pc * a.kxpitch2[h];
      ksc2[nt] = ((const uint16_t*)a.kscale2)[b * a.ks2_sb + h * a.ks2_sh + pc];
    }
  }

  // Ranks past Rl (the last step only) read a valid chunk instead (address
  // clamped to rank Rl - 8): the A rows of those ranks are zero, so any finite
  // value adds nothing, and no load is conditional (a conditional load would
  // zero its register first and wait for the previous load into it).
  auto load = [&](int ks, RkRaw<Q>& r) {
    const int j0 = ks * RC_KS + 32 * hh;             // this lane's first rank of the step
#pragma unroll
    for (int nt = 0; nt < RC_NT; ++nt)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int j = min(j0 + 8 * kk, Rl - 8);
        if constexpr (Q == 0) r.d[nt][kk] = *(const uint4*)(xrow[nt] + 2 * j);
        else if constexpr (Q == 1) r.d[nt][kk] = *(const uint2*)(xrow[nt] + j);
        else r.d[nt][kk] = pf_ld_block(xrow[nt], xrow2[nt], j, a.ksplit, a.k_a8);
      }
  };
  // raw -> B fragment (act dtype) of K-step ks
  auto frag = [&](const RkRaw<Q>& r, int ks, int nt, int kk) -> uint4 {
    if constexpr (Q == 0) {
      return r.d[nt][kk];
    } else {
      uint4 f;
      if constexpr (Q == 1) {
        f = pf_dq_int8(r.d[nt][kk], ksc[nt]);
      } else {
        const int j = min(ks * RC_KS + 32 * hh + 8 * kk, Rl - 8);
        f = pf_dq_block(r.d[nt][kk], j, a.ksplit, a.k_a8, ksc[nt], ksc2[nt]);
      }
      if constexpr (!__is_same(XT, _Float16)) f = pf_f16_to_bf16(f);
      return f;
    }
  };

  // B_k[h] rows [0, nks * 64) in LDS as [j][d] (rows past R zero)
  const int g4 = lane >> 4, rho = lane & 15;
  const int tr_off = (32 * hh + (rho >> 2)) * BK_PITCH + 16 * (g4 & 1) + 4 * (rho & 3);
  {
    const XT* bk = (const XT*)a.bk + a.bkoff[h];
    const int Rp = nks * RC_KS;
    for (int e = tid; e < Rp * 16; e += 256) {        // 16-byte pieces of rows [0, Rp)
      const int j = e >> 4, d8 = (e & 15) * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (j < R) {
        const XT* src = bk + (int64_t)j * a.bk_rs + d8;
        half8 t;
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = __builtin_bit_cast(_Float16, __builtin_bit_cast(uint16_t, src[i]));
        v = __builtin_bit_cast(uint4, t);
      }
      *(uint4*)&lds[j * BK_PITCH + d8] = v;
    }
  }
  floatx16 acc[4][RC_NT];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < RC_NT; ++nt) acc[mt][nt] = floatx16{};

  RkRaw<Q> cur, nxt;
  load(0, cur);
  __syncthreads();
  for (int ks = 0; ks < nks; ++ks) {
    const bool more = ks + 1 < nks;
    if (more) load(ks + 1, nxt);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint4 bf[RC_NT];
#pragma unroll
      for (int nt = 0; nt < RC_NT; ++nt) bf[nt] = frag(cur, ks, nt, kk);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const uint16_t* sb = lds + (ks * RC_KS + 8 * kk) * BK_PITCH + tr_off + 32 * mt;
        const uint2 lo = pf_read_tr16(sb), hi = pf_read_tr16(sb + 4 * BK_PITCH);
        const uint4 af = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
        for (int nt = 0; nt < RC_NT; ++nt) acc[mt][nt] = pf_mfma<XT>(af, bf[nt], acc[mt][nt]);
      }
    }
    if (more) cur = nxt;
  }
  __syncthreads();                                   // B_k reads done before the epilogue reuses LDS

  // epilogue: lane holds positions pw + 32 nt + n, dims 32 mt + 8 q + 4 hh + c in acc[mt][nt][4q + c]
  uint16_t* cw = lds + wave * RC_WAVE_POS * C_PITCH;
#pragma unroll
  for (int nt = 0; nt < RC_NT; ++nt) {
    const int p = pw + nt * 32 + n;
    const bool live = p < S;
    uint16_t* crow = cw + (nt * 32 + n) * C_PITCH + 4 * hh;
    const uint4* rt = (const uint4*)a.rope + ((int64_t)(min(p, S - 1) >> 5) * 8) * 64 + hh * 32 + (p & 31);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 cs4 = rt[(mt * 4 + q) * 64];       // (cos, sin) of frequencies 32 mt + 8 q + 4 hh + 0..3
        const uint32_t cw4[4] = {cs4.x, cs4.y, cs4.z, cs4.w};
        uint32_t y0w[2], y1w[2];
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
          float y0[2], y1[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int c = 2 * c2 + e;
            const kh2 t = __builtin_bit_cast(kh2, cw4[c]);
            const float co = (float)t[0], si = (float)t[1];
            const float k0 = acc[mt][nt][4 * q + c], k1 = acc[mt + 2][nt][4 * q + c];
            y0[e] = live ? k0 * co - k1 * si : 0.f;
            y1[e] = live ? k1 * co + k0 * si : 0.f;
          }
          y0w[c2] = (uint32_t)pf_bits<KVT>(y0[0]) | ((uint32_t)pf_bits<KVT>(y0[1]) << 16);
          y1w[c2] = (uint32_t)pf_bits<KVT>(y1[0]) | ((uint32_t)pf_bits<KVT>(y1[1]) << 16);
        }
        *(uint2*)(crow + mt * 32 + 8 * q) = make_uint2(y0w[0], y0w[1]);
        *(uint2*)(crow + (mt + 2) * 32 + 8 * q) = make_uint2(y1w[0], y1w[1]);
      }
  }
  __syncthreads();
  KVT* dst = (KVT*)a.kbuf + (((int64_t)b * a.Hkv + h) * a.S_pad) * HEAD_DIM;
#pragma unroll 4
  for (int it = 0; it < RC_WAVE_POS * 16 / 64; ++it) {
    const int idx = it * 64 + lane, row = idx >> 4, ch = idx & 15;
    const int p = pw + row;
    if (p < a.S_pad) *(uint4*)(dst + (int64_t)p * HEAD_DIM + ch * 8) = *(const uint4*)&cw[row * C_PITCH + ch * 8];
  }
}

// ---------------------------------------------------------------------------
// V reconstruction, two KV heads per workgroup of 4 waves: 256 positions x
// 256 dims (both heads), wave w computing all 256 dims of positions
// 64 w .. + 63 as 8 x 2 MFMA tiles (256 fp32 accumulators, one wave per
// SIMD), so each dequantised latent fragment feeds eight MFMAs.
// * U_v rows of both heads stream through an LDS ring of NST stages of 64
//   ranks with global_load_lds (no VGPRs held by loads in flight); each wave
//   DMAs 64 of a stage's 256 rows.  In LDS, 16-byte chunk c of stage row r
//   sits at slot c ^ ((r >> 1) & 7) of its 128-byte row, so an operand read
//   (16 lanes = rows r .. r + 15 of one chunk per ds_read_b128 cycle)
//   touches 16 distinct (bank half, slot) pairs.
// * Each stage is an LDS array of its own and the step loop is unrolled by
//   NST, so every access names its stage at compile time: the compiler then
//   sees that an operand read of one stage cannot alias the DMA in flight
//   into another, and waits only where the code says so.
// * Latent words (and group-64 scale / zero) are loaded NST - 1 steps ahead
//   into NST rotating register sets.  Per step the DMA of stage ks + NST - 1
//   and the latents of step ks + NST - 1 are issued in that order, so fixed
//   s_waitcnt vmcnt counts tell when this step's latents (top of the step)
//   and the next stage (before the barrier) have landed.
// * One barrier per step, before the step's last K-chunk: the next stage's
//   first operand reads are then in flight while that chunk's MFMAs run, and
//   the stage consumed in the previous step is refilled right after it.
// * Ranks past Rv (the last stage only): the DMA copies a 16-byte zero line
//   for those U_v chunks, against clamped valid latent chunks.
// Same lane / K-chunk layout as recon_kernel; the epilogue stages each
// wave's 64 x 256 tile in one stage array (16-byte chunks XOR-swizzled by
// row) and writes whole 256-byte rows per head.
// ---------------------------------------------------------------------------
constexpr int RV_POS = PF_V_POS;                     // positions per workgroup
constexpr int RV_WAVE_POS = 64;                      // positions per wave (2 N-tiles)
static_assert(4 * RV_WAVE_POS == RV_POS, "V reconstruction: 4 waves");
constexpr int RV_STAGE = 2 * HEAD_DIM * 128;         // bytes per stage: 256 rows x 64 ranks x 2 bytes
static_assert(RV_WAVE_POS * 2 * HEAD_DIM * 2 == RV_STAGE, "epilogue tile = one stage array");

template <int Q> struct RvRaw { uint4 d[2][4]; };                        // dense: [N-tile][K-chunk]
template <> struct RvRaw<1> { uint4 d[2]; uint16_t sz[2]; };              // group-64 int4: word kk = chunk kk; scale (lanes
                                                                         // 0-31) / zero (lanes 32-63) of the two positions
template <> struct RvRaw<2> { uint2 d[2][4]; };                          // per-token blocks: <= 8 bytes per chunk
// ring depth (= latent register sets): dense latents take 32 registers per
// step, so they get one set less
template <int Q> constexpr int rv_nst() { return Q == 0 ? 3 : 4; }
// fewest vector-memory instructions one step's latent loads issue (the wait
// counts assume no fewer; a step that issues more only waits longer)
template <int Q> constexpr int rv_lat_ops() { return Q == 1 ? 4 : 8; }

template <int N> __device__ inline void rv_vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

typedef __attribute__((address_space(3))) void pf_lds_void;

// 16 zero bytes in global memory: the DMA source of U_v chunks past Rv
__device__ __attribute__((aligned(16))) uint4 pf_zero_line = {0u, 0u, 0u, 0u};

// Q: 0 dense act dtype, 1 group-64 int4 (scale and zero per (b, s, group)),
// 2 per-token blocks (the reference int4 format with an optional int8 / int4
// upper block, or int8; one scale per (b, s) and block)
// NARROW (group-64 only): round_up(Rv, 8) < 32, rows shorter than one 16-byte load
template <typename XT, int Q, bool NARROW>
__global__ __launch_bounds__(256, 1) void recon_v_kernel(const PFArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t st0[RV_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t st1[RV_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t st2[RV_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t st3[RV_STAGE];
  constexpr int NST = rv_nst<Q>();
  constexpr int D = NST - 1;                         // prefetch distance (steps)
  constexpr int NL = rv_lat_ops<Q>();
  // where a step's refill and latent loads are issued: packed formats (ring
  // depth 4) in the first two regions of the next step, dense (depth 3, one
  // step less lead) at the end of the step itself; either way the next
  // stage's wait before the barrier counts one step's DMA + latent loads
  constexpr bool EARLY = D == 3;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  // XCD-aware order (workgroup L runs on XCD L % 8).  With 8 or more head
  // pairs each XCD owns rv_hpx of them and walks all position blocks, so its
  // L2 holds those heads' U_v (2 x 128 x Rv x 2 bytes each) and only the
  // latents are read by several XCDs; with fewer, the head pairs of one
  // (b, 256 positions) share an XCD as in recon_kernel.
  const int L = blockIdx.x, t8 = L >> 3;
  const int nhp = (a.Hkv + 1) >> 1;
  int hp, blk;
  if (a.rv_hpx) {
    hp = (L & 7) * a.rv_hpx + t8 % a.rv_hpx;
    blk = t8 / a.rv_hpx;
    if (hp >= nhp) return;
  } else {
    hp = t8 % nhp;
    blk = (t8 / nhp) * 8 + (L & 7);
  }
  if (blk >= a.rv_blocks) return;
  const int b = blk / a.rv_nb;
  const int pw = (blk - b * a.rv_nb) * RV_POS + RV_WAVE_POS * wave;   // this wave's first position
  // latent rows hold Rl = round_up(Rv, 8) ranks (see recon_kernel); U_v
  // columns at or past Rv are zero in LDS
  const int S = a.S, R = a.Rv, Rl = (R + 7) & ~7;
  const int nks = (Rl + 63) >> 6;

  auto stage = [&](auto ic) __attribute__((always_inline)) -> uint8_t* {
    constexpr int i = decltype(ic)::value % 4;
    if constexpr (i == 0) return st0;
    else if constexpr (i == 1) return st1;
    else if constexpr (i == 2) return st2;
    else return st3;
  };

  const uint8_t* xrow[2];
  const uint8_t* xrow2[2];                           // per-token blocks: the lower (int4) block
  uint16_t vsc[2] = {0, 0}, vsc2[2] = {0, 0};
  const bool vlo = Q == 2 && R > a.vsplit;
  const uint16_t* srow[2];                           // per-token blocks: scale rows of the two positions
  const uint16_t* szrow[2];                          // group-64: scale (lane half 0) or zero (half 1) rows
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int pc = min(pw + nt * 32 + n, S - 1);
    constexpr int64_t es = Q ? 1 : 2;
    xrow[nt] = (const uint8_t*)a.vx + (b * a.vx_sb + (int64_t)pc * a.vx_ss) * es;
    xrow2[nt] = xrow[nt];
    srow[nt] = (const uint16_t*)a.vscale + b * a.vs_sb + (int64_t)pc * a.vs_ss;
    szrow[nt] = (const uint16_t*)(hh ? a.vzero : a.vscale) + b * a.vs_sb + (int64_t)pc * a.vs_ss;
    if constexpr (Q == 2) vsc[nt] = *srow[nt];
    if (vlo) {
      xrow2[nt] = (const uint8_t*)a.vx2 + b * a.vx2_sb + (int64_t)pc * a.vx2_ss;
      vsc2[nt] = ((const uint16_t*)a.vscale2)[b * a.vs2_sb + (int64_t)pc * a.vs2_ss];
    }
  }

  // latent loads of step ks (clamped to the last step; ranks past Rl read the
  // chunk at rank Rl - 8, which meets zero U_v chunks)
  typedef RvRaw<Q> Raw;
  auto load = [&](int ks_, Raw& r) __attribute__((always_inline)) {
    const int ks = min(ks_, nks - 1);
    const int j0 = ks * 64 + 32 * hh;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      if constexpr (Q == 2) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          r.d[nt][kk] = pf_ld_block(xrow[nt], xrow2[nt], min(j0 + 8 * kk, Rl - 8), a.vsplit, a.v_a8);
      } else if constexpr (Q == 1) {
        // one 16-byte load per N-tile in every step (an equal instruction
        // count keeps the compiler's own wait counts exact).  Where the lane's
        // 32 ranks pass the row end (last step), it loads the row's last 16
        // bytes and moves chunk kk + sh down to kk (the chunks left over are
        // past R and meet zero U_v).  Rows shorter than 16 bytes take 4-byte
        // loads (NARROW: more instructions, so the waits only wait longer).
        if constexpr (!NARROW) {
          r.d[nt] = *(const uint4*)(xrow[nt] + min(j0, Rl - 32) / 2);   // shifted by tail_fix
        } else {
          uint32_t w[4];
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) w[kk] = *(const uint32_t*)(xrow[nt] + min(j0 + 8 * kk, Rl - 8) / 2);
          r.d[nt] = make_uint4(w[0], w[1], w[2], w[3]);
        }
        r.sz[nt] = szrow[nt][ks];
      } else {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) r.d[nt][kk] = *(const uint4*)(xrow[nt] + 2 * min(j0 + 8 * kk, Rl - 8));
      }
    }
  };
  // the last step's 16-byte latent loads (group-64): a lane whose 32 ranks
  // pass the row end loaded the row's last 16 bytes; move chunk kk + sh down
  // to kk (the chunks left over are past R and meet zero U_v)
  auto tail_fix = [&](Raw& r, int ks) __attribute__((always_inline)) {
    if constexpr (Q == 1 && !NARROW) {
      const int j0 = ks * 64 + 32 * hh;
      const int sh = (j0 - min(j0, Rl - 32)) >> 3;   // 0 .. 3
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const uint4 w = r.d[nt];
        r.d[nt] = make_uint4(sh == 0 ? w.x : sh == 1 ? w.y : sh == 2 ? w.z : w.w,
                             sh == 0 ? w.y : sh == 1 ? w.z : w.w, sh == 0 ? w.z : w.w, w.w);
      }
    }
  };
  // raw -> B fragment (act dtype) of N-tile nt, K-chunk kk of step ks
  auto frag = [&](const Raw& r, int ks, int nt, int kk) __attribute__((always_inline)) -> uint4 {
    uint4 f;
    if constexpr (Q == 1) {
      const uint32_t w = kk == 0 ? r.d[nt].x : kk == 1 ? r.d[nt].y : kk == 2 ? r.d[nt].z : r.d[nt].w;
      // the lane halves swap: every lane then holds the scale (first) and
      // the zero (second) of its position
      const auto sz = __builtin_amdgcn_permlane32_swap((uint32_t)r.sz[nt], (uint32_t)r.sz[nt], false, false);
      f = pf_dq_g64(w, (uint16_t)sz[0], (uint16_t)sz[1]);
    } else if constexpr (Q == 2) {
      const int j = min(ks * 64 + 32 * hh + 8 * kk, Rl - 8);
      f = pf_dq_block(r.d[nt][kk], j, a.vsplit, a.v_a8, vsc[nt], vsc2[nt]);
    } else {
      f = r.d[nt][kk];
    }
    if constexpr (Q != 0 && !__is_same(XT, _Float16)) f = pf_f16_to_bf16(f);
    return f;
  };

  // U_v DMA: this wave fills stage rows 64 wave .. + 63 (head 2 hp + wave / 2,
  // dims 64 (wave % 2) .. + 63); instruction i covers rows 8 i + rs, and lane
  // slot q receives chunk q ^ ((rs >> 1) + 4 (i & 1)) of its row
  const int rs = lane >> 3, q = lane & 7;
  const int uh = min(2 * hp + (wave >> 1), a.Hkv - 1);
  const uint8_t* ug = (const uint8_t*)a.uv + ((int64_t)uh * HEAD_DIM + 64 * (wave & 1) + rs) * a.uv_rs * 2;
  const int64_t urow8 = a.uv_rs * 16;                // bytes between rows 8 apart
  const int uc0 = (q ^ (rs >> 1)) * 8, uc1 = (q ^ ((rs >> 1) + 4)) * 8;   // the lane's chunk (ranks), even / odd i
  const int wrow = wave * 64 * 128;                  // this wave's rows within a stage
  auto issue = [&](auto ic, int j) __attribute__((always_inline)) {   // stage j into array ic
    const int r0 = min(j, nks - 1) * 64;
    uint8_t* dst = stage(ic) + wrow;
    // chunks of ranks >= Rv (the last stage when Rv is not a multiple of 64)
    // copy a zero line, so those U_v rows are zero in LDS
    const int c0 = r0 + uc0, c1 = r0 + uc1;
    const uint8_t* src0 = c0 < R ? ug + c0 * 2 : (const uint8_t*)&pf_zero_line;
    const uint8_t* src1 = c1 < R ? ug + c1 * 2 : (const uint8_t*)&pf_zero_line;
    const int64_t st0 = c0 < R ? urow8 : 0, st1 = c1 < R ? urow8 : 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      __builtin_amdgcn_global_load_lds((const void*)((i & 1) ? src1 + i * st1 : src0 + i * st0),
                                       (pf_lds_void*)(dst + i * 1024), 16, 0, 0);
  };
  // operand reads: lane (n, hh) reads row 32 mt + n, chunk 4 hh + kk
  int rd[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) rd[kk] = n * 128 + (((4 * hh + kk) ^ ((n >> 1) & 7)) << 4);
  auto read_a = [&](auto ic, int kk, uint4* af) __attribute__((always_inline)) {
    const uint8_t* base = stage(ic) + rd[kk];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) af[mt] = *(const uint4*)(base + mt * 4096);
  };

  floatx16 acc[8][2];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = floatx16{};

  uint4 afA[8], afB[8];                              // A fragments: chunks 0, 2 in afA, chunks 1, 3 in afB
  uint4 bfA[2], bfB[2];                              // B fragments, alternating the same way
  Raw raw[NST];
  // One step: stage ks in array ic, its latents in raw[ic]; on entry the
  // chunk-0 A fragments are in afA and (packed formats) the chunk-0 B
  // fragments in bfA.  Each chunk is one scheduling region: the next chunk's
  // operand reads are issued first, then this chunk's MFMAs interleave with
  // the next chunk's dequantisation.  The last chunk also refills the array
  // of stage ks - 1 with stage ks + D and loads the latents of ks + D.
  auto step = [&](auto ic, int ks) __attribute__((always_inline)) {
    constexpr int i = decltype(ic)::value;
    const std::integral_constant<int, (i + 1) % NST> inext;
    const std::integral_constant<int, (i + NST - 1) % NST> iprev;
    const std::integral_constant<int, (i + NST - 2) % NST> ipre2;
    if constexpr (Q == 0) rv_vm_wait<8 + NL>();      // this step's latents landed (issued two steps back)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint4* afc = (kk & 1) ? afB : afA;
      uint4* afn = (kk & 1) ? afA : afB;
      uint4* bfc = (kk & 1) ? bfB : bfA;
      uint4* bfn = (kk & 1) ? bfA : bfB;
      if (kk < 3) {
        // this chunk's operands (read a region ago) are in; with them retired
        // the next chunk's 8 reads keep the LDS counter within its 15
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_sched_barrier(0);
        read_a(ic, kk + 1, afn);
      } else {
        __builtin_amdgcn_s_waitcnt(0xC07F);           // chunk 3's operands in (as above)
        // this wave's part of stage ks + 1 landed (packed formats: and the
        // latents of ks + 1, issued just after it)
        if constexpr (Q == 0) rv_vm_wait<0>();
        else rv_vm_wait<8 + NL>();
        if (ks + 2 == nks && (Rl & 63)) tail_fix(raw[(i + 1) % NST], ks + 1);
        // stage ks + 1 complete for all waves; stage ks - 1 free.  A bare
        // barrier: each wave has waited for its own DMA above, and a fence
        // here would also wait for the refills still in flight into the
        // other stages.  The memory clobber keeps the compiler from moving
        // LDS accesses across it.
        asm volatile("s_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        read_a(inext, 0, afn);                       // the next step's chunk 0, in flight under this chunk's MFMAs
      }
      if constexpr (Q == 0) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) bfc[nt] = raw[i].d[nt][kk];
      }
#pragma unroll
      for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = pf_mfma<XT>(afc[mt], bfc[nt], acc[mt][nt]);
      if constexpr (Q != 0) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) bfn[nt] = kk < 3 ? frag(raw[i], ks, nt, kk + 1) : frag(raw[(i + 1) % NST], ks + 1, nt, 0);
        // an empty use here keeps the dequantisation in this region (under
        // this chunk's MFMAs) instead of sunk past the next region's branch
        asm volatile("" ::"v"(bfn[0].x), "v"(bfn[0].y), "v"(bfn[0].z), "v"(bfn[0].w), "v"(bfn[1].x), "v"(bfn[1].y),
                     "v"(bfn[1].z), "v"(bfn[1].w));
      }
      if constexpr (EARLY) {
        // packed formats: stage ks + D - 1 into the array freed by the last
        // barrier, and its latents, one region each
        if (kk == 0) issue(ipre2, ks + D - 1);
        if (kk == 1) load(ks + D - 1, raw[(i + D - 1) % NST]);
      } else {
        if (kk == 3) {
          issue(iprev, ks + D);
          load(ks + D, raw[(i + D) % NST]);
        }
      }
      // one wave per SIMD issues in program order: spread the operand reads,
      // loads and VALU work between the MFMAs so that they issue while the
      // previous MFMA runs
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);          // 1 LDS read
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);          // 3 VALU
      }
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // 1 MFMA
        if (EARLY ? kk < 2 : kk == 3) {
          __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);        // 2 global loads (DMA, latents)
          __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);        // 5 VALU
        } else {
          __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);        // 3 VALU
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  const std::integral_constant<int, 0> i0;
  const std::integral_constant<int, 1> i1;
  const std::integral_constant<int, 2> i2;
  const std::integral_constant<int, 3> i3;

  // prologue: stages 0 and 1 and their latents, in the steady state's order
  // (step 0 issues stage 2 with EARLY, and D = 2 needs no more)
  issue(i0, 0);
  load(0, raw[0]);
  issue(i1, 1);
  load(1, raw[1]);
  rv_vm_wait<8 + NL>();                              // this wave's part of stage 0 and the latents of step 0
  __builtin_amdgcn_s_waitcnt(0xC07F);                // lgkmcnt(0): no scalar loads pending into the loop
  __syncthreads();
  read_a(i0, 0, afA);
  if (nks == 1 && (Rl & 63)) tail_fix(raw[0], 0);
  if constexpr (Q != 0) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) bfA[nt] = frag(raw[0], 0, nt, 0);
  }
  int ks = 0;
  for (; ks + NST <= nks; ks += NST) {
    step(i0, ks);
    step(i1, ks + 1);
    step(i2, ks + 2);
    if constexpr (NST == 4) step(i3, ks + 3);
  }
  if (ks < nks) step(i0, ks);
  if (ks + 1 < nks) step(i1, ks + 1);
  if constexpr (NST == 4) {
    if (ks + 2 < nks) step(i2, ks + 2);
  }
  rv_vm_wait<0>();                                   // the clamped refills past the last step, before LDS is reused
  __syncthreads();

  // epilogue: lane holds positions pw + 32 nt + n, dims 32 mt + 8 q + 4 hh + c
  // (head mt / 4) in acc[mt][nt][4 q + c].  Wave w stages its 64 x 256 tile in
  // array w: row = local position (512 bytes), 16-byte chunk c at c ^ (row & 31).
  uint8_t* cw = wave == 0 ? st0 : wave == 1 ? st1 : wave == 2 ? st2 : st3;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int row = nt * 32 + n;
    const bool live = pw + row < S;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        uint32_t w[2];
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
          const float v0 = live ? acc[mt][nt][4 * q4 + 2 * c2] : 0.f;
          const float v1 = live ? acc[mt][nt][4 * q4 + 2 * c2 + 1] : 0.f;
          w[c2] = (uint32_t)pf_bits<KVT>(v0) | ((uint32_t)pf_bits<KVT>(v1) << 16);
        }
        const int c16 = (mt * 4 + q4) ^ (row & 31);
        *(uint2*)(cw + row * 512 + c16 * 16 + hh * 8) = make_uint2(w[0], w[1]);
      }
  }
  // each wave reads back only its own array: no barrier
#pragma unroll
  for (int hs = 0; hs < 2; ++hs) {
    const int hw = 2 * hp + hs;
    if (hw >= a.Hkv) break;                          // an odd Hkv leaves the last pair's second head empty
    KVT* dst = (KVT*)a.vbuf + (((int64_t)b * a.Hkv + hw) * a.S_pad) * HEAD_DIM;
#pragma unroll 4
    for (int it = 0; it < RV_WAVE_POS * 16 / 64; ++it) {
      const int idx = it * 64 + lane, row = idx >> 4, ch = idx & 15;
      const int p = pw + row;
      if (p < a.S_pad)
        *(uint4*)(dst + (int64_t)p * HEAD_DIM + ch * 8) = *(const uint4*)(cw + row * 512 + (((hs * 16 + ch) ^ (row & 31)) << 4));
    }
  }
}

// ---------------------------------------------------------------------------
// Causal flash attention over the reconstructed K / V.  Workgroup: 8 waves x
// 32 queries of one (b, query head); key blocks of 64 staged in LDS, the next
// block loaded into registers while the current one is computed.  Per block
// and wave: S^T = K . Q^T as two 32-key MFMA tiles, the online softmax (the
// causal mask only on blocks that reach past the wave's first query; blocks
// wholly in the wave's future skipped), then O^T += V^T . P^T.  The running
// maximum moves only when a block's maximum exceeds it by more than
// 2^FA_RESCALE_LOG2 in exp2 units, so the O rescale is rare and every
// probability stays <= 2^FA_RESCALE_LOG2 (exact in the final O / l).
// ---------------------------------------------------------------------------
constexpr int FA_KB = 64;                        // keys per block
constexpr int FA_VPITCH = 144;                   // halves per staged V row: rows 8 banks apart for the
                                                 // transposed reads (K keeps WT_PITCH for 16-byte reads)
constexpr int FA_WAVES = 8;                      // waves per workgroup, 32 queries each
constexpr int FA_QB = 32 * FA_WAVES;             // queries per workgroup
static_assert(FA_QB == PF_Q_POS, "host grid sizing");
constexpr float FA_RESCALE_LOG2 = 8.0f;

template <typename XT>
__global__ __launch_bounds__(FA_WAVES * 64, 1) void fa_causal_kernel(const PFArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][FA_KB * WT_PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][FA_KB * FA_VPITCH];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  // XCD-aware order: workgroup L runs on XCD L % 8; every query block of
  // every query head of one (b, KV head) runs on one XCD, consecutively, so
  // that XCD's L2 serves their shared K / V.  Within it the latest (longest)
  // query blocks start first.
  const int L = blockIdx.x, t8 = L >> 3;
  const int per_kv = a.gs * a.fa_nqb;
  const int kvi = (t8 / per_kv) * 8 + (L & 7);      // b * Hkv + kv
  if (kvi >= a.fa_nkvi) return;
  const int rem = t8 % per_kv;
  const int qb = a.fa_nqb - 1 - rem % a.fa_nqb;
  const int b = kvi / a.Hkv, kv = kvi - b * a.Hkv;
  const int qh = kv * a.gs + rem / a.fa_nqb;
  const int T = a.T, pos0 = a.pos0;
  const int t = qb * FA_QB + 32 * wave + n;         // this lane's query
  const int tc = min(t, T - 1);
  const int P = pos0 + tc;                          // its position: sees keys <= P
  const int w_first = pos0 + min(qb * FA_QB + 32 * wave, T - 1);
  const int w_last = pos0 + min(qb * FA_QB + 32 * wave + 31, T - 1);
  const int last_t = min(T, qb * FA_QB + FA_QB) - 1;
  const int nkb = (pos0 + last_t) / FA_KB + 1;      // key blocks the workgroup needs
  const XT* qrow = (const XT*)a.q + b * a.q_sb + qh * a.q_sh + (int64_t)tc * a.q_st;
  uint4 Qb[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    Qb[k] = *(const uint4*)(qrow + 16 * k + 8 * hh);
    if constexpr (!__is_same(XT, _Float16)) Qb[k] = pf_bf16_to_f16(Qb[k]);   // exact in fp16's range
  }
  floatx16 o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = floatx16{};
  const float c = a.scale_log2;
  const float thr = FA_RESCALE_LOG2 / c;            // in raw logit units
  float m = -INFINITY, l = 0.f;
  const size_t hbase = (((size_t)b * a.Hkv + kv) * a.S_pad) * HEAD_DIM;
  const KVT* kg = (const KVT*)a.kbuf + hbase;
  const KVT* vg = (const KVT*)a.vbuf + hbase;
  // S^T = K . Q^T puts key 8 (v/4) + 4 hh + v%4 of its 32-key tile in
  // element v of lane (n, hh).  The P.V MFMA takes its 16-key chunk kk in that
  // order: lane half hh holds keys 16 kk + 4 hh + 0..3 and 16 kk + 8 + 4 hh +
  // 0..3 of both P^T (elements 8 kk .. 8 kk + 7) and V^T (transposed reads of
  // rows 4 hh + 0..3 and 8 + 4 hh + 0..3; lane group g = lane/16, rho = lane%16).
  const int g = lane >> 4, rho = lane & 15;
  const int tr_off = (4 * hh + (rho >> 2)) * FA_VPITCH + 16 * (g & 1) + 4 * (rho & 3);
  // staging: thread piece i (of 2) covers key 32 i + tid / 16, dims (tid % 16) * 8 .. + 7
  static_assert(FA_KB * 16 == 2 * FA_WAVES * 64, "two 16-byte pieces per thread and tensor");
  const int skey = tid >> 4, sd8 = (tid & 15) * 8;
  const size_t so0 = (size_t)skey * HEAD_DIM + sd8, so1 = so0 + (size_t)32 * HEAD_DIM;
  const int lo0 = skey * WT_PITCH + sd8, lo1 = lo0 + 32 * WT_PITCH;
  const int vo0 = skey * FA_VPITCH + sd8, vo1 = vo0 + 32 * FA_VPITCH;
  // K / V pieces in flight (plain variables: they stay in registers)
  uint4 k0 = *(const uint4*)(kg + so0), k1 = *(const uint4*)(kg + so1);
  uint4 v0 = *(const uint4*)(vg + so0), v1 = *(const uint4*)(vg + so1);
  *(uint4*)&Ks[0][lo0] = k0; *(uint4*)&Ks[0][lo1] = k1;
  *(uint4*)&Vs[0][vo0] = v0; *(uint4*)&Vs[0][vo1] = v1;
  // every load so far (Q included) complete: the loop's MFMAs then wait only
  // on LDS, never on the next block's loads in flight
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) {
      const size_t go = (size_t)(kb + 1) * FA_KB * HEAD_DIM;
      k0 = *(const uint4*)(kg + go + so0); k1 = *(const uint4*)(kg + go + so1);
      v0 = *(const uint4*)(vg + go + so0); v1 = *(const uint4*)(vg + go + so1);
    }
    if (kb * FA_KB <= w_last) {                     // wave-uniform: the block has keys this wave sees
      // the two key tiles' MFMA chains interleaved, all 16 K fragments read up front
      floatx16 s[2] = {floatx16{}, floatx16{}};
      const uint16_t* kbase = &Ks[buf][n * WT_PITCH + 8 * hh];
      uint4 kf[2][8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) kf[kt][k] = *(const uint4*)(kbase + kt * 32 * WT_PITCH + 16 * k);
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) s[kt] = pf_mfma<KVT>(kf[kt][k], Qb[k], s[kt]);
      // lane: keys kb*64 + 32 kt + 8 (v/4) + 4 hh + v%4 of query t
      if (kb * FA_KB + FA_KB - 1 > w_first) {         // the block reaches past some query of the wave
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int key = kb * FA_KB + 32 * kt + 8 * (v >> 2) + 4 * hh + (v & 3);
            if (key > P) s[kt][v] = -INFINITY;
          }
      }
      float mb = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) mb = fmaxf(mb, s[kt][v]);
      mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
      if (__ballot(mb > m + thr)) {                  // some query of the wave moves its maximum
        const float mn = fmaxf(m, mb);                // finite: key 0 <= P in block 0
        const float alpha = __builtin_amdgcn_exp2f((m - mn) * c);
        l *= alpha;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) o[j][v] *= alpha;
        m = mn;
      }
      const float mc = m * c;
      float ps = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          s[kt][v] = __builtin_amdgcn_exp2f(fmaf(s[kt][v], c, -mc));
          ps += s[kt][v];
        }
      l += ps;                                        // this half's keys; halves joined at the end
      // O^T += V^T . P^T over the block's four 16-key chunks
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const uint16_t* sb = &Vs[buf][(32 * kt + 16 * kk) * FA_VPITCH + tr_off];
          half8 ph;
#pragma unroll
          for (int e = 0; e < 8; ++e) ph[e] = (_Float16)s[kt][8 * kk + e];
          const uint4 pb = __builtin_bit_cast(uint4, ph);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint2 lo = pf_read_tr16(sb + 32 * j), hi = pf_read_tr16(sb + 32 * j + 8 * FA_VPITCH);
            o[j] = pf_mfma<KVT>(make_uint4(lo.x, lo.y, hi.x, hi.y), pb, o[j]);
          }
        }
    }
    if (more) {
      *(uint4*)&Ks[buf ^ 1][lo0] = k0; *(uint4*)&Ks[buf ^ 1][lo1] = k1;
      *(uint4*)&Vs[buf ^ 1][vo0] = v0; *(uint4*)&Vs[buf ^ 1][vo1] = v1;
    }
    __syncthreads();                                // next block staged; this one free to overwrite
  }
  l += __shfl_xor(l, 32, 64);
  if (t < T) {
    const float inv = 1.0f / l;
    XT* orow = (XT*)a.out + b * a.o_sb + qh * a.o_sh + (int64_t)t * a.o_st;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) orow[32 * j + 8 * (v >> 2) + 4 * hh + (v & 3)] = (XT)(o[j][v] * inv);
  }
}

// ---------------------------------------------------------------------------
// Row repack (see RepackArgs): one thread per 16-byte piece of a destination
// row (pitches are multiples of 16), so the reconstruction and K-logit kernels
// always see 16-byte aligned rows of a multiple of 8 ranks.  A piece of
// 16-bit elements whose source is 4-byte aligned and wholly inside the row is
// read as four words; any other piece byte by byte (any alignment, zero /
// nibble-8 fill past the row).  Grid (pieces of one head's S rows / 256,
// head, batch).
// ---------------------------------------------------------------------------
__device__ inline uint32_t repack_word(const RepackArgs& a, const uint8_t* row, int n, int o) {
  uint32_t w = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int by = o + k;
    uint32_t v;
    if (a.kind == RP_HALF) {
      v = (by >> 1) < n ? row[by] : 0u;
    } else if (a.kind == RP_BYTE) {
      v = by < n ? row[by] : 0u;
    } else {
      const uint32_t x = 2 * by < n ? row[by] : 0x88u;
      v = (2 * by < n ? (x & 0xFu) : 8u) | ((2 * by + 1 < n ? (x >> 4) : 8u) << 4);
    }
    w |= v << (8 * k);
  }
  return w;
}

__global__ __launch_bounds__(256) void repack_rows_kernel(const RepackArgs a) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int ppr = a.pitch >> 4;                      // 16-byte pieces per row
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)a.S * ppr) return;
  const int s = (int)(idx / ppr), o = (int)(idx - (int64_t)s * ppr) * 16;
  const uint8_t* row = a.src + b * a.src_sb + a.src_off[h] + (int64_t)s * a.src_pitch[h];
  const int n = a.nel[h];
  uint32_t w[4];
  if (a.kind == RP_HALF && o + 16 <= 2 * n && ((uintptr_t)(row + o) & 3) == 0) {
    const uint32_t* p = (const uint32_t*)(row + o);
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = p[k];
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = repack_word(a, row, n, o + 4 * k);
  }
  *(uint4*)(a.dst + b * a.dst_sb + ((int64_t)h * a.S + s) * a.pitch + o) = make_uint4(w[0], w[1], w[2], w[3]);
}

// 16-bit rows of at most RPB_MAXP source bytes each, a block of RPB_ROWS rows
// per workgroup: the block's source bytes (from its first row's first element
// to its last row's last element: the gaps between rows, none past the last
// row) are read with 16-byte loads where they are 16-byte aligned and bytewise
// at the two ends, staged in LDS at their address modulo 16, and written out
// as whole 16-byte pieces of the padded rows.  Rows of 2n bytes at any 4-byte
// alignment (rank 102: 204-byte rows) then take one 16-byte load per 16
// bytes instead of four 4-byte loads and a bytewise tail per row.
constexpr int RPB_ROWS = 64, RPB_MAXP = 512;
__global__ __launch_bounds__(256) void repack_block_kernel(const RepackArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t blk[RPB_ROWS * RPB_MAXP + 32];
  const int h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int s0 = blockIdx.x * RPB_ROWS, nr = min(RPB_ROWS, a.S - s0);
  const int n = a.nel[h];
  const int64_t P = a.src_pitch[h];
  const uint8_t* A = a.src + b * a.src_sb + a.src_off[h] + (int64_t)s0 * P;
  const int64_t T = (int64_t)(nr - 1) * P + 2 * n;                 // bytes of the block
  const int lead = (int)((uintptr_t)A & 15);
  const uint8_t* A0 = A - lead;
  const int64_t first = lead ? 16 : 0;                               // first whole aligned piece (offset from A0)
  const int64_t last = (lead + T) & ~(int64_t)15;                    // end of the last whole piece
  for (int64_t o = first + 16 * (int64_t)tid; o < last; o += 16 * 256)
    *(uint4*)(blk + o) = *(const uint4*)(A0 + o);
  // the partial pieces at both ends, bytewise
  if (tid < 16) {
    const int64_t o = lead + tid;                                    // head: [lead, min(16, lead + T))
    if (lead && o < 16 && o < lead + T) blk[o] = A0[o];
  } else if (tid < 32) {
    const int64_t o = last + (tid - 16);                             // tail: [last, lead + T)
    if (o >= first && o < lead + T) blk[o] = A0[o];
  }
  __syncthreads();
  const int ppr = a.pitch >> 4;
  uint8_t* dst = a.dst + b * a.dst_sb + ((int64_t)h * a.S + s0) * a.pitch;
  for (int i = tid; i < nr * ppr; i += 256) {
    const int r = i / ppr, o = (i - r * ppr) * 16;
    const int64_t so = lead + (int64_t)r * P + o;                    // the piece's first byte in blk
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = (o >> 1) + 2 * k;                                // first element of the word
      const uint32_t lo = e < n ? *(const uint16_t*)(blk + so + 4 * k) : 0u;
      const uint32_t hi = e + 1 < n ? *(const uint16_t*)(blk + so + 4 * k + 2) : 0u;
      w[k] = lo | (hi << 16);
    }
    *(uint4*)(dst + (int64_t)r * a.pitch + o) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

int launch_repack(const RepackArgs& a, int B, hipStream_t st) {
  const int64_t pieces = (int64_t)a.S * (a.pitch / 16);
  if (pieces == 0) return 0;
  bool blockwise = a.kind == RP_HALF;
  for (int h = 0; h < a.H && blockwise; ++h)
    blockwise = a.src_pitch[h] % 2 == 0 && a.src_pitch[h] >= 2 * a.nel[h] && a.src_pitch[h] <= RPB_MAXP;
  if (blockwise)
    hipLaunchKernelGGL(repack_block_kernel, dim3((unsigned)ceil_div(a.S, RPB_ROWS), a.H, B), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(repack_rows_kernel, dim3((unsigned)ceil_div(pieces, 256), a.H, B), dim3(256), 0, st, a);
  return (int)hipGetLastError();
}

template <typename XT>
static int launch_prefill_t(const PFArgs& a, int B, hipStream_t st, hipEvent_t mid) {
  PFArgs r = a;
  r.rc_nb = (int)ceil_div(a.S, RC_POS);
  r.rc_blocks = r.rc_nb * B;
  const dim3 rg((unsigned)(ceil_div(r.rc_blocks, 8) * 8 * a.Hkv));
  if (a.k_ref) hipLaunchKernelGGL((recon_kernel<XT, 2>), rg, dim3(256), 0, st, r);
  else if (a.k_i8) hipLaunchKernelGGL((recon_kernel<XT, 1>), rg, dim3(256), 0, st, r);
  else hipLaunchKernelGGL((recon_kernel<XT, 0>), rg, dim3(256), 0, st, r);
  r.rv_nb = (int)ceil_div(a.S, RV_POS);
  r.rv_blocks = r.rv_nb * B;
  const int nhp = (a.Hkv + 1) / 2;
  r.rv_hpx = nhp >= 8 ? (int)ceil_div(nhp, 8) : 0;
  const dim3 vg((unsigned)(r.rv_hpx ? 8 * r.rv_hpx * r.rv_blocks : ceil_div(r.rv_blocks, 8) * 8 * nhp));
  if (a.v_blk) hipLaunchKernelGGL((recon_v_kernel<XT, 2, false>), vg, dim3(256), 0, st, r);
  else if (a.v_g64 && ((a.Rv + 7) & ~7) < 32) hipLaunchKernelGGL((recon_v_kernel<XT, 1, true>), vg, dim3(256), 0, st, r);
  else if (a.v_g64) hipLaunchKernelGGL((recon_v_kernel<XT, 1, false>), vg, dim3(256), 0, st, r);
  else hipLaunchKernelGGL((recon_v_kernel<XT, 0, false>), vg, dim3(256), 0, st, r);
  int e = (int)hipGetLastError();
  if (e) return e;
  if (mid && (e = (int)hipEventRecord(mid, st))) return e;
  r.fa_nqb = (int)ceil_div(a.T, FA_QB);
  r.fa_nkvi = B * a.Hkv;
  const dim3 fg((unsigned)(ceil_div(r.fa_nkvi, 8) * 8 * a.gs * r.fa_nqb));
  hipLaunchKernelGGL((fa_causal_kernel<XT>), fg, dim3(FA_WAVES * 64), 0, st, r);
  return (int)hipGetLastError();
}

int launch_prefill(const PFArgs& a, int dtype, int B, hipStream_t st, hipEvent_t mid) {
  return dtype == STARKV_F16 ? launch_prefill_t<_Float16>(a, B, st, mid) : launch_prefill_t<__bf16>(a, B, st, mid);
}

}  // namespace starkv
