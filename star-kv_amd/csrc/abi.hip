// C ABI of libstarkv: argument validation, launch planning, workspace layout.
//
// Nothing here allocates device memory or synchronises; validation runs
// before any HIP call so that every argument error is reported without a GPU.
#include <algorithm>
#include <climits>
#include <mutex>
#include <vector>

#include "common.hpp"

using namespace starkv;

namespace {

constexpr int FULL_CHIP_CUS = 256;  // an MI355X: planning default when no device can be queried
constexpr int K1_WG_PER_CU = 1;     // k_logits_kernel: one 8-wave (or 4-wave) workgroup per CU
constexpr int MAX_S = 1 << 24;
constexpr int MAX_RV = 8192;
constexpr int64_t V_MAX_PITCH = 1 << 24;   // V row pitch (bytes) of the 24-bit offset multiply in P.V
constexpr int K2_MAX_H = 64;       // P.V: up to two 32-head groups
constexpr int64_t MAX_THREADS_1D = ((int64_t)1 << 32) - 256;   // one-dimensional grids: grid x block < 2^32

int esize(int dt) {
  switch (dt) {
    case STARKV_F16: case STARKV_BF16: return 2;
    case STARKV_F32: return 4;
    case STARKV_I8: case STARKV_U8: return 1;
    default: return 0;
  }
}
bool al(const void* p, int n) { return ((uintptr_t)p % (uintptr_t)n) == 0; }
bool al64(int64_t v, int n) { return v % n == 0; }

size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }

// Compute units of the current device, the unit of every launch plan below
// (rounds of resident workgroups), read once per device.  A partitioned GPU
// or another part reports fewer; with no device to ask (argument validation
// on a machine without a GPU) the plan assumes a whole MI355X.
int device_cus() {
  constexpr int MAXD = 64;
  static std::mutex mu;
  static int cus[MAXD] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXD) return FULL_CHIP_CUS;
  std::lock_guard<std::mutex> lk(mu);
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
      n = FULL_CHIP_CUS;
    cus[dev] = n;
  }
  return cus[dev];
}

// Choose how many position splits minimise the modelled time of a launch of
// `groups` independent (batch, plan) groups over `n_units` position units:
// rounds of `slots` concurrent workgroups, each costing its units plus a fixed
// `c0` units (setup, pipeline fill), times (1 + frac_per_split * splits) for
// split partials written and re-read.
int choose_splits(int64_t groups, int slots, int n_units, int max_n, double c0, double frac_per_split) {
  int best = 1;
  double best_t = 1e300;
  for (int n = 1; n <= std::max(1, std::min(max_n, n_units)); ++n) {
    const int len = (int)ceil_div(n_units, n);
    const int ne = (int)ceil_div(n_units, len);
    const int64_t rounds = ceil_div(groups * ne, slots);
    const double t = (double)rounds * (len + c0) * (1.0 + frac_per_split * ne);
    if (t < best_t * 0.9999) { best_t = t; best = ne; }
  }
  return best;
}

struct KPlan {
  int n_wg = 0;
  int per_cu = K1_WG_PER_CU;   // K1 workgroups resident per CU (the grouped-query kernel: two)
  bool fast = false;
};

int validate_klayout(const starkv_klatent& k, int dtype);

int validate_klatent(const starkv_klatent& k, int Hq, int dtype, int* gs_out) {
  if (k.n_kv_heads < 1 || k.n_kv_heads > K_MAX_KV) return k.n_kv_heads < 1 ? STARKV_ERR_SHAPE : STARKV_ERR_LIMIT;
  if (Hq < 1 || Hq % k.n_kv_heads) return STARKV_ERR_SHAPE;
  if (Hq > K_MAX_QH) return STARKV_ERR_LIMIT;
  if (!k.bk_head_offset || !k.bk) return STARKV_ERR_NULL;
  if (k.bk_row_stride < HEAD_DIM) return STARKV_ERR_SHAPE;
  const int st = validate_klayout(k, dtype);
  if (st) return st;
  *gs_out = Hq / k.n_kv_heads;
  return STARKV_OK;
}

// Where the K latent lives and how it is stored (shared by the attention
// entry points and the cache writer).
int validate_klayout(const starkv_klatent& k, int dtype) {
  if (k.n_kv_heads < 1 || k.n_kv_heads > K_MAX_KV) return k.n_kv_heads < 1 ? STARKV_ERR_SHAPE : STARKV_ERR_LIMIT;
  if (!k.rank || !k.head_offset || !k.pos_stride) return STARKV_ERR_NULL;
  if (!k.data) return STARKV_ERR_NULL;
  if (k.format != STARKV_FMT_DENSE && k.format != STARKV_FMT_INT8_SYM && k.format != STARKV_FMT_INT4_REF)
    return STARKV_ERR_FORMAT;
  if (dtype != STARKV_F16 && dtype != STARKV_BF16) return STARKV_ERR_DTYPE;
  for (int h = 0; h < k.n_kv_heads; ++h)
    if (k.rank[h] < 1 || k.rank[h] > 128) return STARKV_ERR_RANK;
  if (k.stride_b < 0) return STARKV_ERR_SHAPE;
  if (k.format == STARKV_FMT_DENSE) {
    for (int h = 0; h < k.n_kv_heads; ++h)
      if (k.pos_stride[h] < k.rank[h] || k.head_offset[h] < 0) return STARKV_ERR_SHAPE;
  } else {
    // quantised: any rank and any byte layout (rows that are not aligned for
    // whole 8-byte (int8) / 4-byte (int4) chunks, or ranks that are not a
    // multiple of 8, take the unaligned-row loads: k_quant_aligned)
    if (!k.scale) return STARKV_ERR_NULL;
    const bool two = k.format == STARKV_FMT_INT4_REF && k.split > 0;
    if (two && (k.split % 16 || k.split > 128)) return STARKV_ERR_SHAPE;
    if (two && k.split_format != STARKV_FMT_INT4_REF && k.split_format != STARKV_FMT_INT8_SYM) return STARKV_ERR_FORMAT;
    const int split = two ? k.split : 128;
    const bool a8 = two ? k.split_format == STARKV_FMT_INT8_SYM : k.format == STARKV_FMT_INT8_SYM;
    if (!al(k.scale, 2)) return STARKV_ERR_ALIGN;
    if (k.scale_stride_b < 0 || k.scale_stride_h < 0) return STARKV_ERR_SHAPE;
    bool any_lo = false;
    for (int h = 0; h < k.n_kv_heads; ++h) {
      const int r = k.rank[h];
      const int ra = std::min(r, split);
      if (k.head_offset[h] < 0 || k.pos_stride[h] < (a8 ? ra : (ra + 1) / 2)) return STARKV_ERR_SHAPE;
      any_lo |= r > split;
    }
    if (any_lo) {
      if (!k.data2 || !k.scale2 || !k.head_offset2 || !k.pos_stride2) return STARKV_ERR_NULL;
      if (!al(k.scale2, 2)) return STARKV_ERR_ALIGN;
      if (k.stride2_b < 0 || k.scale2_stride_b < 0 || k.scale2_stride_h < 0) return STARKV_ERR_SHAPE;
      for (int h = 0; h < k.n_kv_heads; ++h) {
        if (k.rank[h] <= split) continue;
        if (k.head_offset2[h] < 0 || k.pos_stride2[h] < (k.rank[h] - split + 1) / 2) return STARKV_ERR_SHAPE;
      }
    }
  }
  return STARKV_OK;
}

// Quantised K whose rows take whole 8-byte (int8) / 4-byte (int4) chunk loads:
// ranks multiples of 8 and every row start aligned to the chunk size.
bool k_quant_aligned(const starkv_klatent& k) {
  const bool two = k.format == STARKV_FMT_INT4_REF && k.split > 0;
  const int split = two ? k.split : 128;
  const bool a8 = two ? k.split_format == STARKV_FMT_INT8_SYM : k.format == STARKV_FMT_INT8_SYM;
  const int al_a = a8 ? 8 : 4;
  if (!al(k.data, al_a) || !al64(k.stride_b, al_a)) return false;
  bool any_lo = false;
  for (int h = 0; h < k.n_kv_heads; ++h) {
    if (k.rank[h] % 8) return false;
    if (!al64(k.head_offset[h], al_a) || !al64(k.pos_stride[h], al_a)) return false;
    any_lo |= k.rank[h] > split;
  }
  if (any_lo) {
    if (!al(k.data2, 4) || !al64(k.stride2_b, 4)) return false;
    for (int h = 0; h < k.n_kv_heads; ++h)
      if (k.rank[h] > split && (!al64(k.head_offset2[h], 4) || !al64(k.pos_stride2[h], 4))) return false;
  }
  return true;
}

// Warp-specialised K-logit kernel: dense latents with 16-byte aligned rows
// (ranks a multiple of 8), or int8 latents with one scale per (b, h, s) whose
// rows start on 16-byte boundaries (pitch a multiple of 16 bytes, so the 16-byte
// DMA pieces never straddle rows); q and B_k are read element-wise there.
// padded: dense rows hold round_up(r, 8) elements, zero past r (the K-logit
// entry's repacked copy), so a rank need not be a multiple of 8.
bool k_ws(const starkv_klatent& k, int dtype, int S, bool padded = false) {
  const bool i8 = k.format == STARKV_FMT_INT8_SYM;
  if (k.format != STARKV_FMT_DENSE && !i8) return false;
  const int xe = i8 ? 1 : esize(dtype);
  if (!al(k.data, 16) || !al64(k.stride_b * xe, 16)) return false;
  // int8: the scales of a tile are staged in 16-byte pieces (8 positions), so
  // each (b, h) scale row is read up to position round_up(S, 8) - 1, inside
  // its pitch
  if (i8 && (!al(k.scale, 16) || !al64(k.scale_stride_b * 2, 16) || !al64(k.scale_stride_h * 2, 16) ||
             k.scale_stride_h < round_up(S, 8)))
    return false;
  for (int h = 0; h < k.n_kv_heads; ++h) {
    if (k.rank[h] % 8 && !(padded && !i8)) return false;
    if (!al64(k.head_offset[h] * xe, 16) || !al64(k.pos_stride[h] * xe, 16)) return false;
    if ((int64_t)TILE * k.pos_stride[h] * xe >= ((int64_t)1 << 31)) return false;   // 32-bit per-tile DMA step
  }
  return true;
}

// 16-byte LDS chunks of one 32-position tile row of a head in that kernel
int ws_row_chunks(const starkv_klatent& k, int h) {
  return (int)ceil_div(k.rank[h], k.format == STARKV_FMT_INT8_SYM ? 16 : 8);
}

// First-fit decreasing of heads hs (u[h] units each) into at most nb bins of
// cap units; false if they do not fit.
static bool ffd_bins(std::vector<int> hs, const std::vector<int>& u, int nb, int cap,
                     std::vector<std::vector<int>>* out) {
  std::stable_sort(hs.begin(), hs.end(), [&](int x, int y) { return u[x] > u[y]; });
  std::vector<std::vector<int>> bins;
  std::vector<int> load;
  for (int h : hs) {
    size_t i = 0;
    while (i < bins.size() && load[i] + u[h] > cap) ++i;
    if (i == bins.size()) {
      if ((int)bins.size() == nb) return false;
      bins.emplace_back();
      load.push_back(0);
    }
    bins[i].push_back(h);
    load[i] += u[h];
  }
  if (out) *out = bins;
  return true;
}

// MHA query heads over workgroups of up to nw bins of cap units each, so that
// the largest workgroup stages as few 16-byte chunks per tile as possible (a
// single round of workgroups runs at the pace of the heaviest): longest first
// into the least loaded workgroup where its heads still pack, then single
// moves and pairwise swaps off the heaviest workgroup while they lower its
// load.  Starts from n_min workgroups, one more while the greedy pass does not
// fit.  Results are cached per (rank vector, geometry).
static bool ws_balance(const starkv_klatent& k, int Hq, int unit, int nw, int cap, int n_min,
                       std::vector<std::vector<int>>& parts) {
  std::vector<int> u(Hq), c(Hq), order(Hq);
  std::vector<int> key = {Hq, unit, nw, cap, n_min};
  for (int h = 0; h < Hq; ++h) {
    u[h] = (int)ceil_div(k.rank[h], unit);
    c[h] = ws_row_chunks(k, h);
    order[h] = h;
    key.push_back(c[h]);
    key.push_back(u[h]);
  }
  static std::mutex mu;
  static std::vector<std::pair<std::vector<int>, std::vector<std::vector<int>>>> cache;
  {
    std::lock_guard<std::mutex> lk(mu);
    for (const auto& e : cache)
      if (e.first == key) { parts = e.second; return true; }
  }
  std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return c[x] > c[y]; });
  auto fits = [&](const std::vector<int>& hs) { return ffd_bins(hs, u, nw, cap, nullptr); };
  for (int n = std::max(n_min, 1); n * nw <= K_MAX_WAVES; ++n) {
    parts.assign(n, {});
    std::vector<int> load(n, 0);
    bool ok = true;
    for (int h : order) {
      int best = -1;
      for (int g = 0; g < n; ++g) {
        if (best >= 0 && load[g] >= load[best]) continue;
        std::vector<int> t = parts[g];
        t.push_back(h);
        if (fits(t)) best = g;
      }
      if (best < 0) { ok = false; break; }
      parts[best].push_back(h);
      load[best] += c[h];
    }
    if (!ok) continue;
    for (int iter = 0; iter < 256; ++iter) {
      const int g = (int)(std::max_element(load.begin(), load.end()) - load.begin());
      bool moved = false;
      for (int o = 0; o < n && !moved; ++o) {
        if (o == g) continue;
        for (size_t i = 0; i < parts[g].size() && !moved; ++i) {
          const int h = parts[g][i];
          std::vector<int> rest = parts[g];
          rest.erase(rest.begin() + i);
          std::vector<int> grown = parts[o];
          grown.push_back(h);
          if (load[o] + c[h] < load[g] && fits(grown)) {           // move h to o
            parts[g] = rest; parts[o] = grown;
            load[g] -= c[h]; load[o] += c[h];
            moved = true;
            break;
          }
          for (size_t j = 0; j < parts[o].size(); ++j) {           // swap h with a lighter head of o
            const int h2 = parts[o][j], d = c[h] - c[h2];
            if (d <= 0 || load[o] + d >= load[g]) continue;
            std::vector<int> a2 = rest, b2 = parts[o];
            a2.push_back(h2);
            b2[j] = h;
            if (fits(a2) && fits(b2)) {
              parts[g] = a2; parts[o] = b2;
              load[g] -= d; load[o] += d;
              moved = true;
              break;
            }
          }
        }
      }
      if (!moved) break;
    }
    std::lock_guard<std::mutex> lk(mu);
    if (cache.size() >= 64) cache.erase(cache.begin());
    cache.emplace_back(key, parts);
    return true;
  }
  return false;
}

// Pack (query head, 32-rank M-tile) items into waves of up to 2 or 4 items
// (first fit decreasing, whole heads per wave; 4 once any head has rank > 64)
// and deal the waves round-robin over workgroups of 8 waves (2-item waves) or
// 4 waves (4-item waves).
int build_k_plan(const starkv_klatent& k, int Hq, int gs, int dtype, int S, KArgs& a, KPlan& plan,
                 bool padded = false) {
  const bool ws = k_ws(k, dtype, S, padded);
  const int unit = 32;                        // ranks per item
  struct QH { int qh, kv, ni; };              // ni: items of the head
  std::vector<QH> heads;
  int max_items = 1;
  for (int qh = 0; qh < Hq; ++qh) {
    const int kv = qh / gs;
    max_items = std::max(max_items, (int)ceil_div(k.rank[kv], 32));
    heads.push_back({qh, kv, (int)ceil_div(k.rank[kv], unit)});
  }
  const int maxi = ws || max_items > 2 ? 4 : 2;   // items per (consumer) wave
  const int nw = maxi == 2 ? 8 : 4;
  const int cap = maxi * 32 / unit;               // units per wave
  // Bins of up to cap units (whole query heads), first-fit decreasing.  With
  // GQA the query heads of one KV head are packed together (KV-major), so the
  // workgroup that stages or streams that head's latent serves all of them.
  std::vector<std::vector<QH>> bins;
  std::vector<int> load;
  auto pack = [&](const std::vector<QH>& hs) {
    const size_t first = bins.size();
    for (const QH& h : hs) {
      size_t i = first;
      for (; i < bins.size(); ++i) if (load[i] + h.ni <= cap) break;
      if (i == bins.size()) { bins.emplace_back(); load.push_back(0); }
      bins[i].push_back(h);
      load[i] += h.ni;
    }
  };
  if (gs == 1) {
    std::stable_sort(heads.begin(), heads.end(), [](const QH& x, const QH& y) { return x.ni > y.ni; });
    pack(heads);
  } else {
    for (int kv = 0; kv < k.n_kv_heads; ++kv) {
      std::vector<QH> grp;
      for (const QH& h : heads) if (h.kv == kv) grp.push_back(h);
      pack(grp);
    }
  }
  int n_waves = (int)bins.size();
  plan.n_wg = (int)ceil_div(n_waves, nw);
  if (plan.n_wg * nw > K_MAX_WAVES) return STARKV_ERR_LIMIT;
  // bin -> (workgroup, wave).  MHA: the heaviest bins (latent rank sum) first,
  // each into the least loaded workgroup with a free wave, so workgroups
  // stream similar byte counts.  GQA: consecutive bins share a workgroup.
  // Warp-specialised MHA: heads are partitioned over the workgroups first
  // (ws_balance), then packed into bins per workgroup.
  std::vector<int> wg_of(n_waves), wave_of(n_waves);
  std::vector<std::vector<int>> parts;
  if (ws && gs == 1 && ws_balance(k, Hq, unit, nw, cap, plan.n_wg, parts)) {
    bins.clear();
    wg_of.clear();
    wave_of.clear();
    for (int g = 0; g < (int)parts.size(); ++g) {
      std::vector<int> u(Hq, 0);
      for (int h : parts[g]) u[h] = (int)ceil_div(k.rank[h], unit);
      std::vector<std::vector<int>> wb;
      ffd_bins(parts[g], u, nw, cap, &wb);
      for (int w = 0; w < (int)wb.size(); ++w) {
        std::vector<QH> bin;
        for (int h : wb[w]) bin.push_back({h, h, u[h]});
        bins.push_back(bin);
        wg_of.push_back(g);
        wave_of.push_back(w);
      }
    }
    n_waves = (int)bins.size();
    plan.n_wg = (int)parts.size();
  } else if (gs == 1) {
    std::vector<int> order(n_waves), rsum(n_waves, 0);
    for (int bi = 0; bi < n_waves; ++bi) {
      order[bi] = bi;
      for (const QH& h : bins[bi]) rsum[bi] += k.rank[h.kv];
    }
    std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return rsum[x] > rsum[y]; });
    std::vector<int64_t> wload(plan.n_wg, 0);
    std::vector<int> used(plan.n_wg, 0);
    for (int bi : order) {
      int best = -1;
      for (int g = 0; g < plan.n_wg; ++g)
        if (used[g] < nw && (best < 0 || wload[g] < wload[best])) best = g;
      wg_of[bi] = best;
      wave_of[bi] = used[best]++;
      wload[best] += rsum[bi];
    }
  } else {
    for (int bi = 0; bi < n_waves; ++bi) { wg_of[bi] = bi / nw; wave_of[bi] = bi % nw; }
  }
  for (int w = 0; w < K_MAX_WAVES; ++w)
    for (int i = 0; i < K_MAXI; ++i) a.items[w][i] = 0;
  for (int bi = 0; bi < n_waves; ++bi) {
    std::vector<QH> v = bins[bi];
    std::sort(v.begin(), v.end(), [](const QH& x, const QH& y) { return x.qh < y.qh; });
    uint32_t* row = a.items[wg_of[bi] * nw + wave_of[bi]];
    int i = 0;
    for (const QH& h : v) {
      const int r = k.rank[h.kv];
      for (int mt = 0; mt < h.ni; ++mt) row[i++] = item_pack(h.qh, h.kv, mt, std::min(32, r - 32 * mt), mt == h.ni - 1);
    }
  }
  // grouped-query heads (k_logits_gqa.hip): K reconstructed once per KV
  // head; two KV heads per workgroup (the largest rank with the smallest),
  // each run by two consumer waves (dims halves p = 0, 1)
  const bool gqa = ws && gs > 1 && gs <= 8 && k.format == STARKV_FMT_DENSE;
  if (gqa) {
    const int n = k.n_kv_heads;
    std::vector<int> order(n);
    for (int h = 0; h < n; ++h) order[h] = h;
    std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return k.rank[x] > k.rank[y]; });
    plan.n_wg = (int)ceil_div(n, 2);
    plan.per_cu = 2;
    if (plan.n_wg * 4 > K_MAX_WAVES) return STARKV_ERR_LIMIT;
    for (int w = 0; w < K_MAX_WAVES; ++w)
      for (int i = 0; i < K_MAXI; ++i) a.items[w][i] = 0;
    for (int g = 0; g < plan.n_wg; ++g) {
      const int h0 = order[g], h1 = n - 1 - g > g ? order[n - 1 - g] : -1;
      for (int p = 0; p < 2; ++p) {
        a.items[g * 4 + p][0] = item_pack(h0 * gs, h0, p, 0, 1);
        if (h1 >= 0) a.items[g * 4 + 2 + p][0] = item_pack(h1 * gs, h1, p, 0, 1);
      }
    }
  }
  a.gqa = gqa;
  a.gs = gs;
  for (int h = 0; h < K_MAX_KV; ++h) a.krank[h] = (int16_t)(h < k.n_kv_heads ? k.rank[h] : 0);
  const bool two = k.format == STARKV_FMT_INT4_REF && k.split > 0;
  a.ksplit = two ? k.split : 128;
  a.k_a_int8 = two ? k.split_format == STARKV_FMT_INT8_SYM : k.format == STARKV_FMT_INT8_SYM;
  a.x2 = k.data2; a.x2_sb = k.stride2_b;
  a.xscale2 = k.scale2; a.xs2_sb = k.scale2_stride_b; a.xs2_sh = k.scale2_stride_h;
  for (int h = 0; h < k.n_kv_heads; ++h) {
    a.xoff[h] = k.head_offset[h];
    a.xpitch[h] = (int)k.pos_stride[h];
    a.bkoff[h] = k.bk_head_offset[h];
    const bool lo = two && k.rank[h] > k.split;
    a.xoff2[h] = lo ? k.head_offset2[h] : 0;
    a.xpitch2[h] = lo ? (int)k.pos_stride2[h] : 0;
  }
  a.n_wg = plan.n_wg;
  a.maxi = maxi;
  a.ws = ws;
  a.ws_i8 = ws && k.format == STARKV_FMT_INT8_SYM;
  a.ws_stage = a.ws_nst = 0;
  if (ws) {
    // stage = the largest workgroup's latent tile (16-byte chunks of its
    // distinct KV heads, whole 1 KB DMA pieces) [+ 1 KB of int8 scales:
    // 32 positions of up to 16 heads] + the 8 KB RoPE operand
    int max_chunks = 0;
    for (int g = 0; g < plan.n_wg; ++g) {
      bool seen[K_MAX_KV] = {};
      int chunks = 0;
      for (int w = 0; w < nw; ++w)
        for (int i = 0; i < K_MAXI; ++i) {
          const uint32_t it = a.items[g * nw + w][i];
          const int kv = (it >> 8) & 0xff;
          if (!((it >> 27) & 1) || seen[kv]) continue;
          seen[kv] = true;
          chunks += 32 * ws_row_chunks(k, kv);
        }
      max_chunks = std::max(max_chunks, chunks);
    }
    a.ws_stage = (int)round_up(max_chunks, 64) * 16 + 8192 + (a.ws_i8 ? 1024 : 0);
    a.ws_nst = gqa ? std::min(6, K1_GQ_RING_BYTES / a.ws_stage) : std::min(4, (a.ws_i8 ? K1_WS_RING_I8_BYTES : K1_WS_RING_BYTES) / a.ws_stage);
  }
  return STARKV_OK;
}

// Vector-load variant: B_k and q rows 8-byte aligned, and latent rows aligned
// for whole-chunk loads with ranks a multiple of 8 (dense: 16-byte rows;
// quantised: k_quant_aligned).
bool k_fast(const starkv_klatent& k, int dtype, const void* q, int64_t q_sb, int64_t q_sh) {
  const bool dense = k.format == STARKV_FMT_DENSE;
  const int xe = esize(dtype);
  if (!dense && !k_quant_aligned(k)) return false;
  if (dense && (!al(k.data, 16) || !al64(k.stride_b * xe, 16))) return false;
  for (int h = 0; h < k.n_kv_heads; ++h) {
    if (dense && k.rank[h] % 8) return false;
    if (dense && (!al64(k.head_offset[h] * xe, 16) || !al64(k.pos_stride[h] * xe, 16))) return false;
    if (!al64(k.bk_head_offset[h] * 2, 8)) return false;
  }
  if (!al(k.bk, 8) || !al64(k.bk_row_stride * 2, 8)) return false;
  if (!al(q, 8) || !al64(q_sb * 2, 8) || !al64(q_sh * 2, 8)) return false;
  return true;
}

int check_mask(const void* mask, int mask_dtype) {
  if (!mask) return STARKV_OK;
  if (mask_dtype != STARKV_F32 && mask_dtype != STARKV_F16 && mask_dtype != STARKV_BF16) return STARKV_ERR_DTYPE;
  return STARKV_OK;
}


// ---- P.V geometry: workgroup = 4 waves x NTW column tiles of one position chunk
struct PVGeom {
  int Rvp, n_cb, n_c2, c2_len, n_grp;   // n_grp > 1: two-level split reduction
};

// row_bytes: the largest row pitch (bytes) of the V latent's streams; the
// kernel addresses a chunk with 32-bit offsets, so a chunk stays below 2 GB
PVGeom pv_geometry(int B, int S, int Rv, bool fused, int vq, int64_t row_bytes) {
  PVGeom g;
  g.Rvp = (int)round_up(Rv, 32);
  const int ntw = pv_tiles_per_wave(g.Rvp, fused, vq);
  // one 8-wave workgroup for all columns (its 24-bit row offsets need
  // every pitch below 16 MB)
  const bool wide = pv_wide_tiles(g.Rvp, fused, vq) > 0 && row_bytes < V_MAX_PITCH;
  // fused group-64 V of up to 16 tiles: the 4-wave raw-nibble kernel, three per CU
  const bool nib4 = fused && vq == VQ_G64 && g.Rvp <= 512;
  g.n_cb = wide ? 1 : (int)ceil_div(g.Rvp / 32, 4 * ntw);
  const int wg_per_cu = wide ? 1 : nib4 ? 3 : pv_wg_per_cu(ntw, vq);
  const int n_ks = (int)ceil_div(S, KSTEP);
  // each extra split writes and re-reads one fp32 partial of 32 x Rvp per
  // column block, against the X_v bytes and logits the split streams
  const double vbytes = vq == VQ_DENSE ? 2.0 * Rv : Rv / 2.0 + 4.0 * ceil_div(Rv, 64);
  // (below ~8K positions the launch is latency-bound and partials are cheap)
  const double frac = 32.0 * g.Rvp * 8.0 / g.n_cb / ((double)std::max(S, 8192) * (vbytes / g.n_cb + 128.0));
  int n = choose_splits((int64_t)B * g.n_cb, device_cus() * wg_per_cu, n_ks, 512, 4.0, frac);
  const int64_t max_ks = std::max<int64_t>(1, ((int64_t)1 << 31) / std::max<int64_t>(row_bytes, 1) / KSTEP);
  n = std::max<int64_t>(n, ceil_div(n_ks, max_ks));
  g.c2_len = (int)ceil_div(n_ks, n) * KSTEP;
  // the all-columns and raw-nibble kernels take whole 32-position steps (a
  // chunk still below 2 GB)
  if (wide || nib4) g.c2_len = (int)std::min<int64_t>(round_up(g.c2_len, 2 * KSTEP), std::max<int64_t>(2 * KSTEP, max_ks * KSTEP / (2 * KSTEP) * (2 * KSTEP)));
  g.n_c2 = (int)ceil_div(S, g.c2_len);
  g.n_grp = g.n_c2 > PV_RG ? (int)ceil_div(g.n_c2, PV_RG) : 0;
  return g;
}

// ---- decode workspace layout (shared by the size query and the call)
int head_groups(int H) { return (int)ceil_div(H, 32); }   // P.V passes of 32 heads

struct DecodeLayout {
  int S_pad, n_c1, tiles_per_chunk, n_hg, sw, n_sl, n_cs;
  PVGeom pv;
  bool part16;
  size_t off_logits, off_cmax, off_part, off_psum, off_ypart, total;
};

// f16: fp16 model.  Short P.V chunks (<= 512 positions) then keep their
// partials in fp16, each divided by its chunk's softmax sum (a convex
// combination of V rows: bounded by max |V|): there the partials are a large
// share of the P.V traffic (at 272 positions about as many bytes as the
// int4 V latent) and halving them pays for the per-chunk rescale in the
// up-projection.  With long chunks the time comes out even (measured); group-64
// V keeps them in fp16 there too, halving the partials' share of its traffic
// (55 of 613 MB at B16 S32768), dense V in fp32.
DecodeLayout decode_layout(int B, int Hq, int Hkv, int S, int Rv, int n_wg, int k1pc, int vq, int64_t v_row_bytes,
                           bool f16) {
  DecodeLayout L;
  L.S_pad = (int)round_up(S, 64);
  const int n_tiles = (int)ceil_div(S, TILE);
  const int cus = device_cus();
  L.n_c1 = choose_splits((int64_t)B * n_wg, cus * k1pc, n_tiles, 256, 3.0, 0.0);
  L.tiles_per_chunk = (int)ceil_div(n_tiles, L.n_c1);
  L.n_c1 = (int)ceil_div(n_tiles, L.tiles_per_chunk);
  L.n_hg = head_groups(Hq);
  L.pv = pv_geometry(B * L.n_hg, S, Rv, true, vq, v_row_bytes);
  L.sw = up_slice_width(Hkv, Rv, cus);
  L.n_sl = (int)ceil_div(Rv, L.sw);
  L.n_cs = up_chunk_sets(Hkv, L.n_sl, L.pv.n_c2, cus);
  const int Rvp = L.pv.Rvp, n_c2 = L.pv.n_c2;
  const size_t BQ = (size_t)B * L.n_hg;
  size_t o = 0;
  L.off_logits = o; o = a256(o + (size_t)B * Hq * L.S_pad * 4);
  L.off_cmax = o; o = a256(o + (size_t)B * Hq * L.n_c1 * 4);
  const bool part16 = f16 && (L.pv.c2_len <= 512 || vq == VQ_G64);
  L.part16 = part16;
  L.off_part = o; o = a256(o + BQ * n_c2 * 32 * Rvp * (part16 ? 2 : 4));
  L.off_psum = o; o = a256(o + BQ * n_c2 * 32 * 4);
  L.off_ypart = o; o = a256(o + (size_t)Hkv * L.n_sl * L.n_cs * ((size_t)B * (Hq / Hkv)) * HEAD_DIM * 4);
  L.total = o;
  return L;
}

// V latent: validate the description and fill the P.V kernel's storage
// fields (x / x2 / scales / zero points, split, bytes per row); *vq = its
// storage kind.  Quantised formats take any rank and byte layout (the
// per-token block formats need a split that is a multiple of 8, so an 8-rank
// chunk never straddles it); pa.qfast tells whether every row is aligned for
// whole 4-byte (int4) / 8-byte (int8) chunk loads with ranks (and the lower
// block) a multiple of 8, else the P.V kernel reads unaligned rows.
int validate_v(const starkv_vlatent& v, PVArgs& pa, int* vq) {
  if (!v.data) return STARKV_ERR_NULL;
  if (v.rank < 1 || v.rank > MAX_RV) return STARKV_ERR_RANK;
  if (v.stride_b < 0 || v.stride_s < 0) return STARKV_ERR_SHAPE;
  pa.x = v.data; pa.x_sb = v.stride_b; pa.x_ss = v.stride_s;
  switch (v.format) {
    case STARKV_FMT_DENSE:
      if (v.stride_s < v.rank) return STARKV_ERR_SHAPE;
      *vq = VQ_DENSE;
      return STARKV_OK;
    case STARKV_FMT_INT4_REF:
    case STARKV_FMT_INT8_SYM: {
      if (!v.scale) return STARKV_ERR_NULL;
      const bool two = v.format == STARKV_FMT_INT4_REF && v.split > 0 && v.split < v.rank;
      if (two && v.split_format != STARKV_FMT_INT4_REF && v.split_format != STARKV_FMT_INT8_SYM)
        return STARKV_ERR_FORMAT;
      const int split = two ? v.split : v.rank;
      const bool a8 = two ? v.split_format == STARKV_FMT_INT8_SYM : v.format == STARKV_FMT_INT8_SYM;
      if (two && split % 8) return STARKV_ERR_SHAPE;
      const int al_a = a8 ? 8 : 4;
      const int nb = a8 ? split : (split + 1) / 2;
      if (v.stride_s < nb) return STARKV_ERR_SHAPE;
      if (!al(v.scale, 2)) return STARKV_ERR_ALIGN;
      if (v.scale_stride_b < 0 || v.scale_stride_s < 0) return STARKV_ERR_SHAPE;
      pa.split = split; pa.a_int8 = a8; pa.xnb = nb;
      pa.xs = v.scale; pa.xs_sb = v.scale_stride_b; pa.xs_ss = v.scale_stride_s;
      bool fast = split % 8 == 0 && al(v.data, al_a) && al64(v.stride_s, al_a) && al64(v.stride_b, al_a);
      if (two) {
        const int nb2 = (v.rank - split + 1) / 2;
        if (!v.data2 || !v.scale2) return STARKV_ERR_NULL;
        if (v.stride2_s < nb2 || v.stride2_b < 0 || v.scale2_stride_b < 0 || v.scale2_stride_s < 0)
          return STARKV_ERR_SHAPE;
        if (!al(v.scale2, 2)) return STARKV_ERR_ALIGN;
        pa.x2 = v.data2; pa.x2_sb = v.stride2_b; pa.x2_ss = v.stride2_s; pa.x2nb = nb2;
        pa.xs2 = v.scale2; pa.xs2_sb = v.scale2_stride_b; pa.xs2_ss = v.scale2_stride_s;
        fast = fast && (v.rank - split) % 8 == 0 && al(v.data2, 4) && al64(v.stride2_s, 4) && al64(v.stride2_b, 4);
      }
      pa.qfast = fast;
      *vq = VQ_BLOCK;
      return STARKV_OK;
    }
    case STARKV_FMT_INT4_G64: {
      if (!v.scale || !v.zero) return STARKV_ERR_NULL;
      const int nb = (v.rank + 1) / 2;
      if (v.stride_s < nb || v.scale_stride_s < (v.rank + 63) / 64 || v.scale_stride_b < 0)
        return STARKV_ERR_SHAPE;
      if (!al(v.scale, 2) || !al(v.zero, 2)) return STARKV_ERR_ALIGN;
      if (v.stride_s >= V_MAX_PITCH || v.scale_stride_s * 2 >= V_MAX_PITCH) return STARKV_ERR_LIMIT;
      pa.xs = v.scale; pa.xs_sb = v.scale_stride_b; pa.xs_ss = v.scale_stride_s;
      pa.xz = v.zero; pa.xnb = nb;
      pa.qfast = v.rank % 8 == 0 && al(v.data, 4) && al64(v.stride_s, 4) && al64(v.stride_b, 4);
      *vq = VQ_G64;
      return STARKV_OK;
    }
    default:
      return STARKV_ERR_FORMAT;
  }
}

// the P.V kernel's aligned-row variant: dense rows 16-byte aligned with the
// rank a multiple of 8; quantised rows as validate_v found them (pa.qfast)
bool v_fast(const starkv_vlatent& v, const PVArgs& pa) {
  if (v.format != STARKV_FMT_DENSE) return pa.qfast != 0;
  return al(v.data, 16) && al64(v.stride_s * 2, 16) && al64(v.stride_b * 2, 16) && v.rank % 8 == 0 &&
         v.stride_s * 2 < V_MAX_PITCH;
}

// largest row pitch in bytes over the V latent's streams (dense: 16-bit elements)
int64_t v_row_bytes(const starkv_vlatent& v) {
  if (v.format == STARKV_FMT_DENSE) return v.stride_s * 2;
  return std::max({v.stride_s, v.scale_stride_s * 2, v.stride2_s, v.scale2_stride_s * 2});
}

int validate_decode(const starkv_decode_desc* d, int* gs, int* n_wg, int* k1pc, int* vq) {
  if (!d) return STARKV_ERR_NULL;
  if (d->batch < 1 || d->seq_len < 1 || d->seq_len > MAX_S) return STARKV_ERR_SHAPE;
  if (d->head_dim != HEAD_DIM) return STARKV_ERR_SHAPE;
  if (d->dtype != STARKV_F16 && d->dtype != STARKV_BF16) return STARKV_ERR_DTYPE;
  if (d->n_q_heads > K2_MAX_H) return STARKV_ERR_LIMIT;
  int st = validate_klatent(d->k, d->n_q_heads, d->dtype, gs);
  if (st) return st;
  PVArgs vtmp = {};
  if ((st = validate_v(d->v, vtmp, vq))) return st;
  if (!d->q || !d->uv || !d->out || !d->rope_table) return STARKV_ERR_NULL;
  if (d->seq_len > d->rope_max_positions) return STARKV_ERR_SHAPE;
  if (d->uv_row_stride < d->v.rank) return STARKV_ERR_SHAPE;
  if ((st = check_mask(d->mask, d->mask_dtype))) return st;
  if (d->out_dtype != 0 && d->out_dtype != d->dtype && d->out_dtype != STARKV_F32) return STARKV_ERR_DTYPE;
  KArgs tmp;
  KPlan plan;
  if ((st = build_k_plan(d->k, d->n_q_heads, *gs, d->dtype, d->seq_len, tmp, plan))) return st;
  *n_wg = plan.n_wg;
  *k1pc = plan.per_cu;
  return STARKV_OK;
}

// Prefill inputs the reconstruction kernels cannot read in place -- latent
// ranks that are not a multiple of 8, latent rows not aligned for their chunk
// loads, or U_v rows that are not 16-byte aligned whole multiples of 8
// columns -- are repacked into aligned copies in the workspace first
// (RepackArgs).  The workspace holds the reconstructed K and V, then these
// copies.
struct PrefillPlan {
  int64_t S = 0, S_pad = 0;
  bool rk = false, rv = false, ru = false;          // repack the K latent, the V latent, U_v
  int k_kind1 = 0, k_kind2 = 0, v_kind1 = 0, v_kind2 = 0;
  int k_p1 = 0, k_p2 = 0, v_p1 = 0, v_p2 = 0, u_p = 0;   // repacked row pitches, bytes
  size_t kvb = 0, off_k1 = 0, off_k2 = 0, off_v1 = 0, off_v2 = 0, off_u = 0, total = 0;
};

int pitch16(int64_t bytes) { return (int)round_up(std::max<int64_t>(bytes, 1), 16); }
// bytes of n elements of a repack kind, n padded to 8
int64_t rp_bytes(int kind, int n) {
  const int64_t n8 = round_up(n, 8);
  return kind == RP_HALF ? 2 * n8 : kind == RP_BYTE ? n8 : n8 / 2;
}

// Prefill: any K latent format and rank (dense, int8 or the reference split
// format), any V latent format and rank (dense, group-64 int4 or per-token
// blocks), q 16-byte aligned.  Positions reconstructed: pos0 + n_tokens,
// padded to 64 in the workspace.
int validate_prefill(const starkv_prefill_desc* d, int* gs, PrefillPlan* P) {
  if (!d) return STARKV_ERR_NULL;
  if (d->batch < 1 || d->batch > 65535 || d->n_tokens < 1 || d->pos0 < 0) return STARKV_ERR_SHAPE;
  if ((int64_t)d->pos0 + d->n_tokens > MAX_S) return STARKV_ERR_LIMIT;
  if (d->head_dim != HEAD_DIM) return STARKV_ERR_SHAPE;
  if (d->dtype != STARKV_F16 && d->dtype != STARKV_BF16) return STARKV_ERR_DTYPE;
  int st = validate_klatent(d->k, d->n_q_heads, d->dtype, gs);
  if (st) return st;
  const starkv_klatent& k = d->k;
  PVArgs vb = {};
  int vq = 0;
  if ((st = validate_v(d->v, vb, &vq))) return st;
  if (!d->q || !d->uv || !d->out || !d->rope_table) return STARKV_ERR_NULL;
  if ((int64_t)d->pos0 + d->n_tokens > d->rope_max_positions) return STARKV_ERR_SHAPE;
  if (d->uv_row_stride < d->v.rank) return STARKV_ERR_SHAPE;
  if (d->q_stride_b < 0 || d->q_stride_h < 0 || d->q_stride_t < 0) return STARKV_ERR_SHAPE;
  if (!al(d->q, 16) || !al64(d->q_stride_b, 8) || !al64(d->q_stride_h, 8) || !al64(d->q_stride_t, 8))
    return STARKV_ERR_ALIGN;
  if (d->out_stride_b < 0 || d->out_stride_h < 0 || d->out_stride_t < 0) return STARKV_ERR_SHAPE;
  // one-dimensional grids of the three launches (workgroup counts, ints in the kernels)
  const int64_t S = (int64_t)d->pos0 + d->n_tokens, Hkv = d->k.n_kv_heads;
  const int64_t g_k = round_up((int64_t)d->batch * ceil_div(S, PF_K_POS), 8) * Hkv;
  const int64_t nhp = (Hkv + 1) / 2;
  const int64_t g_v = nhp >= 8 ? 8 * ceil_div(nhp, 8) * d->batch * ceil_div(S, PF_V_POS)
                               : round_up((int64_t)d->batch * ceil_div(S, PF_V_POS), 8) * nhp;
  const int64_t g_a = round_up((int64_t)d->batch * Hkv, 8) * *gs * ceil_div(d->n_tokens, PF_Q_POS);
  if (std::max({g_k, g_v, g_a}) > INT32_MAX) return STARKV_ERR_LIMIT;

  PrefillPlan& p = *P;
  p = PrefillPlan{};
  p.S = S;
  p.S_pad = round_up(S, 64);
  // K latent
  int rmax = 0;
  for (int h = 0; h < k.n_kv_heads; ++h) rmax = std::max(rmax, k.rank[h]);
  const int rmax8 = (int)round_up(rmax, 8);
  if (k.format == STARKV_FMT_DENSE) {
    p.rk = !al(k.data, 16) || !al64(k.stride_b, 8);
    for (int h = 0; h < k.n_kv_heads; ++h)
      p.rk |= k.rank[h] % 8 || !al64(k.head_offset[h], 8) || !al64(k.pos_stride[h], 8);
    p.k_kind1 = RP_HALF;
    p.k_p1 = pitch16(rp_bytes(RP_HALF, rmax8));
  } else {
    p.rk = !k_quant_aligned(k);
    const bool two = k.format == STARKV_FMT_INT4_REF && k.split > 0;
    const bool a8 = two ? k.split_format == STARKV_FMT_INT8_SYM : k.format == STARKV_FMT_INT8_SYM;
    const int split = two ? k.split : 128;
    p.k_kind1 = a8 ? RP_BYTE : RP_NIB;
    p.k_p1 = pitch16(rp_bytes(p.k_kind1, std::min(rmax8, split)));
    if (rmax > split) {
      p.k_kind2 = RP_NIB;
      p.k_p2 = pitch16(rp_bytes(RP_NIB, rmax8 - split));
    }
  }
  // V latent
  const int Rv = d->v.rank;
  if (vq == VQ_DENSE) {
    p.rv = !(al(d->v.data, 16) && al64(d->v.stride_s, 8) && al64(d->v.stride_b, 8) && Rv % 8 == 0);
    p.v_kind1 = RP_HALF;
    p.v_p1 = pitch16(rp_bytes(RP_HALF, Rv));
  } else if (vq == VQ_G64) {
    p.rv = !vb.qfast;
    p.v_kind1 = RP_NIB;
    p.v_p1 = pitch16(rp_bytes(RP_NIB, Rv));
  } else {
    p.rv = !vb.qfast;
    p.v_kind1 = vb.a_int8 ? RP_BYTE : RP_NIB;
    p.v_p1 = pitch16(rp_bytes(p.v_kind1, vb.split));
    if (Rv > vb.split) {
      p.v_kind2 = RP_NIB;
      p.v_p2 = pitch16(rp_bytes(RP_NIB, Rv - vb.split));
    }
  }
  // U_v: 16-byte rows of whole 8-column chunks (the DMA's 16-byte pieces)
  p.ru = !(al(d->uv, 16) && al64(d->uv_row_stride, 8) && Rv % 8 == 0);
  p.u_p = pitch16(rp_bytes(RP_HALF, Rv));

  const size_t B = d->batch;
  p.kvb = a256((size_t)B * Hkv * p.S_pad * HEAD_DIM * 2);
  size_t o = 2 * p.kvb;
  if (p.rk) {
    p.off_k1 = o; o += a256(B * Hkv * S * p.k_p1);
    p.off_k2 = o; o += a256(B * Hkv * S * p.k_p2);
  }
  if (p.rv) {
    p.off_v1 = o; o += a256(B * S * p.v_p1);
    p.off_v2 = o; o += a256(B * S * p.v_p2);
  }
  if (p.ru) {
    p.off_u = o; o += a256((size_t)Hkv * HEAD_DIM * p.u_p);
  }
  p.total = o;
  return STARKV_OK;
}

}  // namespace

extern "C" {

int starkv_abi_version(void) { return STARKV_ABI_VERSION; }

const char* starkv_status_string(int s) {
  switch (s) {
    case STARKV_OK: return "ok";
    case STARKV_ERR_NULL: return "a required pointer is NULL";
    case STARKV_ERR_SHAPE: return "inconsistent or unsupported sizes";
    case STARKV_ERR_DTYPE: return "unsupported element type";
    case STARKV_ERR_ALIGN: return "pointer or stride misaligned";
    case STARKV_ERR_RANK: return "latent rank out of range";
    case STARKV_ERR_WORKSPACE: return "workspace missing or too small";
    case STARKV_ERR_LIMIT: return "exceeds a compiled limit";
    case STARKV_ERR_FORMAT: return "unknown quantisation format";
    default: return s > 0 ? hipGetErrorString((hipError_t)s) : "unknown error";
  }
}

size_t starkv_rope_table_bytes(int max_positions) {
  if (max_positions < 1) return 0;
  return (size_t)rope_table_tiles(max_positions) * 512 * 16;
}

int starkv_rope_build(const float* inv_freq_host, float attention_scaling, int max_positions,
                      void* table, size_t table_bytes, void* stream) {
  if (!inv_freq_host || !table) return STARKV_ERR_NULL;
  if (max_positions < 1 || max_positions > MAX_S) return STARKV_ERR_SHAPE;
  if (table_bytes < starkv_rope_table_bytes(max_positions)) return STARKV_ERR_WORKSPACE;
  if (!al(table, 16)) return STARKV_ERR_ALIGN;
  float f[64];
  for (int i = 0; i < 64; ++i) f[i] = inv_freq_host[i];
  return launch_rope_table(f, max_positions, attention_scaling, table, (hipStream_t)stream);
}

// Dense K whose rows the warp-specialised and grouped-query K-logit kernels
// cannot stream (a rank not a multiple of 8, or rows not 16-byte aligned: the
// reference abx benchmark's 102 ranks per KV head, abx_rope_batched.py:274-280,
// leaves 204-byte rows) is first copied into the workspace as rows of
// round_up(r, 8) elements, zero past r, one 16-byte pitch for all heads
// ([B][Hkv][S][pitch]); the kernels then read that copy.
struct KRepack {
  bool on = false;
  int pitch = 0;              // bytes
  size_t bytes = 0;
};

KRepack k_repack_plan(const starkv_klatent& k, int dtype, int B, int S) {
  KRepack r;
  if (k.format != STARKV_FMT_DENSE || k_ws(k, dtype, S)) return r;
  int rmax = 8;
  for (int h = 0; h < k.n_kv_heads; ++h) rmax = std::max(rmax, k.rank[h]);
  r.pitch = (int)round_up((int64_t)round_up(rmax, 8) * esize(dtype), 16);
  if ((int64_t)TILE * r.pitch >= ((int64_t)1 << 31)) return r;
  r.bytes = a256((size_t)B * k.n_kv_heads * S * r.pitch);
  r.on = true;
  return r;
}

size_t starkv_k_logits_workspace_bytes(const starkv_klogits_desc* d) {
  int gs = 0;
  if (!d || d->batch < 1 || d->seq_len < 1 || d->seq_len > MAX_S || validate_klatent(d->k, d->n_q_heads, d->dtype, &gs))
    return 0;
  return k_repack_plan(d->k, d->dtype, d->batch, d->seq_len).bytes;
}

int starkv_k_logits(const starkv_klogits_desc* d, void* workspace, size_t workspace_bytes, void* stream) {
  if (!d) return STARKV_ERR_NULL;
  if (d->batch < 1 || d->seq_len < 1 || d->seq_len > MAX_S || d->head_dim != HEAD_DIM) return STARKV_ERR_SHAPE;
  int gs = 0, st;
  if ((st = validate_klatent(d->k, d->n_q_heads, d->dtype, &gs))) return st;
  if (!d->q || !d->out || !d->rope_table) return STARKV_ERR_NULL;
  if (d->seq_len > d->rope_max_positions) return STARKV_ERR_SHAPE;
  if (d->out_dtype != STARKV_F32 && d->out_dtype != STARKV_F16 && d->out_dtype != STARKV_BF16) return STARKV_ERR_DTYPE;
  if ((st = check_mask(d->mask, d->mask_dtype))) return st;
  const KRepack rp = k_repack_plan(d->k, d->dtype, d->batch, d->seq_len);
  starkv_klatent k = d->k;
  int64_t rp_hoff[K_MAX_KV], rp_pstr[K_MAX_KV];   // the repacked copy's head offsets and row pitches
  if (rp.on) {
    if (!workspace || workspace_bytes < rp.bytes) return STARKV_ERR_WORKSPACE;
    if (!al(workspace, 256)) return STARKV_ERR_ALIGN;
    const int H = k.n_kv_heads, S = d->seq_len, xe = esize(d->dtype);
    RepackArgs ra = {};
    ra.src = (const uint8_t*)k.data; ra.src_sb = k.stride_b * xe;
    for (int h = 0; h < H; ++h) {
      ra.src_off[h] = k.head_offset[h] * xe;
      ra.src_pitch[h] = k.pos_stride[h] * xe;
      ra.nel[h] = k.rank[h];
    }
    ra.dst = (uint8_t*)workspace; ra.dst_sb = (int64_t)H * S * rp.pitch; ra.pitch = rp.pitch;
    ra.kind = RP_HALF; ra.H = H; ra.S = S;
    if ((st = launch_repack(ra, d->batch, (hipStream_t)stream))) return st;
    k.data = workspace;
    k.stride_b = (int64_t)H * S * rp.pitch / xe;
    for (int h = 0; h < H; ++h) {
      rp_hoff[h] = (int64_t)h * S * rp.pitch / xe;
      rp_pstr[h] = rp.pitch / xe;
    }
    k.head_offset = rp_hoff;
    k.pos_stride = rp_pstr;
  }
  KArgs a;
  KPlan plan;
  if ((st = build_k_plan(k, d->n_q_heads, gs, d->dtype, d->seq_len, a, plan, rp.on))) return st;
  a.q = d->q; a.q_sb = d->q_stride_b; a.q_sh = d->q_stride_h;
  a.x = k.data; a.x_sb = k.stride_b;
  a.xscale = d->k.scale; a.xs_sb = d->k.scale_stride_b; a.xs_sh = d->k.scale_stride_h;
  a.bk = d->k.bk; a.bk_rs = d->k.bk_row_stride;
  a.rope = (const uint4*)d->rope_table;
  a.mask = d->mask; a.m_sb = d->mask_stride_b; a.m_sh = d->mask_stride_h; a.mask_dtype = d->mask_dtype;
  a.last_pos = nullptr;
  a.out = d->out; a.o_sb = d->out_stride_b; a.o_st = TILE; a.o_sh = d->out_stride_h;   // rows
  a.chunkmax = nullptr;
  a.S = d->seq_len; a.Hq = d->n_q_heads; a.wscale = d->scale;
  const int n_tiles = (int)ceil_div(d->seq_len, TILE);
  // the K-logit kernels address one batch's logits with 32-bit element offsets
  if ((int64_t)(d->n_q_heads - 1) * d->out_stride_h + (int64_t)n_tiles * TILE >= ((int64_t)1 << 32))
    return STARKV_ERR_LIMIT;
  int nc = choose_splits((int64_t)d->batch * plan.n_wg, device_cus() * plan.per_cu, n_tiles, 256, 3.0, 0.0);
  a.tiles_per_chunk = (int)ceil_div(n_tiles, nc);
  a.n_chunks = (int)ceil_div(n_tiles, a.tiles_per_chunk);
  const bool fast = k_fast(k, d->dtype, d->q, d->q_stride_b, d->q_stride_h);
  return launch_k_logits(a, d->dtype, k.format, d->out_dtype == STARKV_F32, d->out_dtype, fast, d->batch, (hipStream_t)stream);
}

size_t starkv_pv_latent_workspace_bytes(const starkv_pv_desc* d) {
  if (!d || d->batch < 1 || d->seq_len < 1 || d->v.rank < 1) return 0;
  PVArgs tmp = {};
  int vq = 0;
  if (validate_v(d->v, tmp, &vq)) return 0;
  const int BQ = d->batch * head_groups(d->n_heads);
  const PVGeom g = pv_geometry(BQ, d->seq_len, d->v.rank, false, vq, v_row_bytes(d->v));
  return a256((size_t)BQ * g.n_c2 * 32 * g.Rvp * 4) + a256((size_t)BQ * g.n_grp * 32 * g.Rvp * 4);
}

int starkv_pv_latent(const starkv_pv_desc* d, void* workspace, size_t workspace_bytes, void* stream) {
  if (!d) return STARKV_ERR_NULL;
  if (d->batch < 1 || d->seq_len < 1 || d->seq_len > MAX_S || d->n_heads < 1) return STARKV_ERR_SHAPE;
  if (d->n_heads > K2_MAX_H) return STARKV_ERR_LIMIT;
  if (d->dtype != STARKV_F16 && d->dtype != STARKV_BF16) return STARKV_ERR_DTYPE;
  int st, vq = 0;
  PVArgs a = {};
  if ((st = validate_v(d->v, a, &vq))) return st;
  if (!d->p || !d->out) return STARKV_ERR_NULL;
  const size_t need = starkv_pv_latent_workspace_bytes(d);
  if (!workspace || workspace_bytes < need) return STARKV_ERR_WORKSPACE;
  if (!al(workspace, 256)) return STARKV_ERR_ALIGN;
  const int n_hg = head_groups(d->n_heads), BQ = d->batch * n_hg;
  const PVGeom g = pv_geometry(BQ, d->seq_len, d->v.rank, false, vq, v_row_bytes(d->v));
  a.n_hg = n_hg;
  a.Rv = d->v.rank; a.Rvp = g.Rvp; a.n_cb = g.n_cb; a.n_c2 = g.n_c2; a.c2_len = g.c2_len; a.n_grp = g.n_grp;
  a.p = d->p; a.p_sb = d->p_stride_b; a.p_sh = d->p_stride_h;
  a.p_vec = al(d->p, 16) && al64(d->p_stride_b * 2, 16) && al64(d->p_stride_h * 2, 16);
  a.part = (float*)workspace;
  a.part2 = (float*)((char*)workspace + a256((size_t)BQ * g.n_c2 * 32 * g.Rvp * 4));
  a.out = d->out; a.o_sb = d->out_stride_b; a.o_sh = d->out_stride_h;
  a.S = d->seq_len; a.H = d->n_heads;
  return launch_pv(a, d->dtype, vq, false, v_fast(d->v, a), d->batch, (hipStream_t)stream);
}

size_t starkv_decode_workspace_bytes(const starkv_decode_desc* d) {
  int gs = 0, n_wg = 0, k1pc = 1, vq = 0;
  if (validate_decode(d, &gs, &n_wg, &k1pc, &vq)) return 0;
  return decode_layout(d->batch, d->n_q_heads, d->k.n_kv_heads, d->seq_len, d->v.rank, n_wg, k1pc, vq, v_row_bytes(d->v),
                    d->dtype == STARKV_F16).total;
}

static int decode_impl(const starkv_decode_desc* d, void* workspace, size_t workspace_bytes, void* stream,
                       void* const* events) {
  int gs = 0, n_wg = 0, k1pc = 1, vq = 0, st;
  if ((st = validate_decode(d, &gs, &n_wg, &k1pc, &vq))) return st;
  const DecodeLayout L =
      decode_layout(d->batch, d->n_q_heads, d->k.n_kv_heads, d->seq_len, d->v.rank, n_wg, k1pc, vq, v_row_bytes(d->v),
                    d->dtype == STARKV_F16);
  if (!workspace || workspace_bytes < L.total) return STARKV_ERR_WORKSPACE;
  if (!al(workspace, 256)) return STARKV_ERR_ALIGN;
  char* ws = (char*)workspace;
  hipStream_t s = (hipStream_t)stream;
  const int B = d->batch, Hq = d->n_q_heads;

  KArgs ka;
  KPlan plan;
  if ((st = build_k_plan(d->k, Hq, gs, d->dtype, d->seq_len, ka, plan))) return st;
  ka.q = d->q; ka.q_sb = d->q_stride_b; ka.q_sh = d->q_stride_h;
  ka.x = d->k.data; ka.x_sb = d->k.stride_b;
  ka.xscale = d->k.scale; ka.xs_sb = d->k.scale_stride_b; ka.xs_sh = d->k.scale_stride_h;
  ka.bk = d->k.bk; ka.bk_rs = d->k.bk_row_stride;
  ka.rope = (const uint4*)d->rope_table;
  ka.mask = d->mask; ka.m_sb = d->mask_stride_b; ka.m_sh = d->mask_stride_h; ka.mask_dtype = d->mask_dtype;
  ka.last_pos = d->last_pos_device;
  // logits in 32-position tiles of all heads: a tile's 4 KB is written together
  // by the workgroups of one chunk and read contiguously by P.V
  ka.out = ws + L.off_logits; ka.o_sb = (int64_t)Hq * L.S_pad; ka.o_st = (int64_t)Hq * TILE; ka.o_sh = TILE;
  ka.chunkmax = (float*)(ws + L.off_cmax);
  ka.S = d->seq_len; ka.Hq = Hq; ka.n_chunks = L.n_c1; ka.tiles_per_chunk = L.tiles_per_chunk;
  ka.wscale = d->scale;
  const bool kfast = k_fast(d->k, d->dtype, d->q, d->q_stride_b, d->q_stride_h);
  if (events && (st = (int)hipEventRecord((hipEvent_t)events[0], s))) return st;
  if ((st = launch_k_logits(ka, d->dtype, d->k.format, true, STARKV_F32, kfast, B, s))) return st;
  if (events && (st = (int)hipEventRecord((hipEvent_t)events[1], s))) return st;

  PVArgs pa = {};
  if ((st = validate_v(d->v, pa, &vq))) return st;
  pa.logits = (const float*)(ws + L.off_logits); pa.l_sb = ka.o_sb; pa.l_st = ka.o_st; pa.l_sh = ka.o_sh;
  pa.chunkmax = (const float*)(ws + L.off_cmax); pa.n_chunk1 = L.n_c1;
  pa.part = (float*)(ws + L.off_part); pa.psum = (float*)(ws + L.off_psum); pa.part16 = L.part16;
  pa.S = d->seq_len; pa.H = Hq; pa.n_hg = L.n_hg; pa.Rv = d->v.rank; pa.Rvp = L.pv.Rvp;
  pa.n_cb = L.pv.n_cb; pa.n_c2 = L.pv.n_c2; pa.c2_len = L.pv.c2_len;
  if ((st = launch_pv(pa, d->dtype, vq, true, v_fast(d->v, pa), B, s))) return st;
  if (events && (st = (int)hipEventRecord((hipEvent_t)events[2], s))) return st;

  UPArgs ua;
  ua.part = pa.part; ua.psum = pa.psum; ua.part16 = L.part16; ua.n_c2 = L.pv.n_c2; ua.Rvp = L.pv.Rvp;
  ua.n_hg = L.n_hg;
  ua.uv = d->uv; ua.uv_rs = d->uv_row_stride;
  ua.out = d->out; ua.o_sb = d->out_stride_b; ua.o_sh = d->out_stride_h;
  ua.B = B; ua.Hq = Hq; ua.gs = gs; ua.Rv = d->v.rank;
  ua.sw = L.sw; ua.n_sl = L.n_sl; ua.n_cs = L.n_cs; ua.ypart = (float*)(ws + L.off_ypart);
  ua.out_f32 = d->out_dtype == STARKV_F32;
  const bool ufast = al(d->uv, 16) && al64(d->uv_row_stride * 2, 16);
  if ((st = launch_up_proj(ua, d->dtype, ufast, s))) return st;
  if (events && (st = (int)hipEventRecord((hipEvent_t)events[3], s))) return st;
  return STARKV_OK;
}

int starkv_decode_attention(const starkv_decode_desc* d, void* workspace, size_t workspace_bytes, void* stream) {
  return decode_impl(d, workspace, workspace_bytes, stream, nullptr);
}

int starkv_decode_attention_timed(const starkv_decode_desc* d, void* workspace, size_t workspace_bytes,
                                  void* stream, void* const* events) {
  if (!events || !events[0] || !events[1] || !events[2] || !events[3]) return STARKV_ERR_NULL;
  return decode_impl(d, workspace, workspace_bytes, stream, events);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free decode: the workspace is a file-scope device array of
// STARKV_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds until
// the process ends.  Its device address is looked up once per device (the
// array's name is only a host-side stand-in) and kept; calls on one GPU share
// it, so calls that overlap on one GPU race.  The decode kernels write every
// workspace element they read (nothing needs clearing between calls).
// ---------------------------------------------------------------------------
namespace {

__device__ __align__(256) char scratch[STARKV_NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

// the current device's address of `scratch` (looked up on its first use)
int scratch_address(void** out) {
  int dev = 0;
  int st = (int)hipGetDevice(&dev);
  if (st) return st;
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return STARKV_ERR_LIMIT;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if ((st = (int)hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)))) return st;
    if (!p) return (int)hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return STARKV_OK;
}

}  // namespace

extern "C" {

int starkv_decode_attention_noalloc(const starkv_decode_desc* d, void* stream) {
  int gs = 0, n_wg = 0, k1pc = 1, vq = 0, st;
  if ((st = validate_decode(d, &gs, &n_wg, &k1pc, &vq))) return st;
  const size_t need =
      decode_layout(d->batch, d->n_q_heads, d->k.n_kv_heads, d->seq_len, d->v.rank, n_wg, k1pc, vq, v_row_bytes(d->v),
                    d->dtype == STARKV_F16).total;
  if (need > (size_t)STARKV_NOALLOC_SCRATCH_BYTES) return STARKV_ERR_LIMIT;
  void* ws = nullptr;
  if ((st = scratch_address(&ws))) return st;
  return decode_impl(d, ws, STARKV_NOALLOC_SCRATCH_BYTES, stream, nullptr);
}

static int build_rope_apply(const starkv_rope_apply_desc* d, RopeApplyArgs& a) {
  if (!d) return STARKV_ERR_NULL;
  if (d->batch < 1 || d->n_heads < 1 || d->n_tokens < 0 || d->pos0 < 0) return STARKV_ERR_SHAPE;
  if (d->dtype != STARKV_F16 && d->dtype != STARKV_BF16) return STARKV_ERR_DTYPE;
  if (!d->x || !d->rope_table) return STARKV_ERR_NULL;
  if (d->stride_b < 0 || d->stride_h < 0 || d->stride_t < 0) return STARKV_ERR_SHAPE;
  if (!d->pos0_device && (int64_t)d->pos0 + d->n_tokens > d->rope_max_positions) return STARKV_ERR_SHAPE;
  // one thread per (row, frequency); HIP keeps grid x block below 2^32
  if ((int64_t)d->batch * d->n_heads * d->n_tokens * 64 > MAX_THREADS_1D) return STARKV_ERR_LIMIT;
  a = RopeApplyArgs{};
  a.x = d->x; a.sb = d->stride_b; a.sh = d->stride_h; a.st = d->stride_t;
  a.B = d->batch; a.H = d->n_heads; a.T = d->n_tokens; a.pos0 = d->pos0; a.max_pos = d->rope_max_positions;
  a.pos0_dev = d->pos0_device; a.err = d->error_flag; a.table = d->rope_table;
  return STARKV_OK;
}

int starkv_rope_apply(const starkv_rope_apply_desc* d, void* stream) {
  RopeApplyArgs a;
  const int st = build_rope_apply(d, a);
  return st ? st : launch_rope_apply(a, d->dtype, (hipStream_t)stream);
}

static int build_k_append(const starkv_k_append_desc* d, KAppendArgs& a) {
  if (!d) return STARKV_ERR_NULL;
  if (d->batch < 1 || d->n_tokens < 0 || d->pos0 < 0 || d->capacity < 1 || d->capacity > MAX_S) return STARKV_ERR_SHAPE;
  if (!d->pos0_device && (int64_t)d->pos0 + d->n_tokens > d->capacity) return STARKV_ERR_SHAPE;
  if (d->dtype != STARKV_F16 && d->dtype != STARKV_BF16) return STARKV_ERR_DTYPE;
  const starkv_klatent& k = d->k;
  int st = validate_klayout(k, d->dtype);
  if (st) return st;
  if (!d->src) return STARKV_ERR_NULL;
  if (d->src_stride_b < 0 || d->src_stride_h < 0 || d->src_stride_t < 0) return STARKV_ERR_SHAPE;
  // one wave (64 threads) per row
  if ((int64_t)d->batch * k.n_kv_heads * d->n_tokens * 64 > MAX_THREADS_1D) return STARKV_ERR_LIMIT;
  a = KAppendArgs{};
  a.src = d->src; a.src_sb = d->src_stride_b; a.src_sh = d->src_stride_h; a.src_st = d->src_stride_t;
  a.B = d->batch; a.H = k.n_kv_heads; a.T = d->n_tokens; a.pos0 = d->pos0; a.cap = d->capacity;
  a.pos0_dev = d->pos0_device; a.err = d->error_flag;
  a.fmt = k.format;
  a.data = (void*)k.data; a.stride_b = k.stride_b;
  a.scale = (void*)k.scale; a.sc_sb = k.scale_stride_b; a.sc_sh = k.scale_stride_h;
  const bool two = k.format == STARKV_FMT_INT4_REF && k.split > 0;
  a.split = two ? k.split : 128;
  a.a_int8 = two ? k.split_format == STARKV_FMT_INT8_SYM : k.format == STARKV_FMT_INT8_SYM;
  a.data2 = (void*)k.data2; a.stride2_b = k.stride2_b;
  a.scale2 = (void*)k.scale2; a.sc2_sb = k.scale2_stride_b; a.sc2_sh = k.scale2_stride_h;
  for (int h = 0; h < k.n_kv_heads; ++h) {
    a.rank[h] = k.rank[h];
    a.off[h] = k.head_offset[h]; a.pitch[h] = k.pos_stride[h];
    const bool lo = two && k.rank[h] > k.split;
    a.off2[h] = lo ? k.head_offset2[h] : 0; a.pitch2[h] = lo ? k.pos_stride2[h] : 0;
    a.src_off[h] = d->src_head_offset ? d->src_head_offset[h] : h * d->src_stride_h;
    if (a.src_off[h] < 0) return STARKV_ERR_SHAPE;
  }
  return STARKV_OK;
}

int starkv_k_append(const starkv_k_append_desc* d, void* stream) {
  KAppendArgs a;
  const int st = build_k_append(d, a);
  return st ? st : launch_k_append(a, d->dtype, (hipStream_t)stream);
}

static int build_v_append(const starkv_v_append_desc* d, VAppendArgs& a) {
  if (!d) return STARKV_ERR_NULL;
  if (d->batch < 1 || d->n_tokens < 0 || d->pos0 < 0 || d->capacity < 1 || d->capacity > MAX_S) return STARKV_ERR_SHAPE;
  if (!d->pos0_device && (int64_t)d->pos0 + d->n_tokens > d->capacity) return STARKV_ERR_SHAPE;
  if (d->dtype != STARKV_F16 && d->dtype != STARKV_BF16) return STARKV_ERR_DTYPE;
  PVArgs pa = {};
  int vq = 0, st;
  if ((st = validate_v(d->v, pa, &vq))) return st;
  if (!d->src) return STARKV_ERR_NULL;
  if (d->src_stride_b < 0 || d->src_stride_t < 0) return STARKV_ERR_SHAPE;
  // one wave per row (group-64: per row and group of 64 ranks)
  const int64_t waves_per_row = vq == VQ_G64 ? ceil_div(d->v.rank, 64) : 1;
  if ((int64_t)d->batch * d->n_tokens * waves_per_row * 64 > MAX_THREADS_1D) return STARKV_ERR_LIMIT;
  a = VAppendArgs{};
  a.src = d->src; a.src_sb = d->src_stride_b; a.src_st = d->src_stride_t;
  a.B = d->batch; a.T = d->n_tokens; a.pos0 = d->pos0; a.cap = d->capacity; a.R = d->v.rank; a.vq = vq;
  a.pos0_dev = d->pos0_device; a.err = d->error_flag;
  a.data = (void*)pa.x; a.stride_b = pa.x_sb; a.stride_s = pa.x_ss;
  a.scale = (void*)pa.xs; a.sc_sb = pa.xs_sb; a.sc_ss = pa.xs_ss;
  a.zero = (void*)pa.xz;
  a.split = pa.split; a.a_int8 = pa.a_int8;
  a.data2 = (void*)pa.x2; a.stride2_b = pa.x2_sb; a.stride2_s = pa.x2_ss;
  a.scale2 = (void*)pa.xs2; a.sc2_sb = pa.xs2_sb; a.sc2_ss = pa.xs2_ss;
  return STARKV_OK;
}

int starkv_v_append(const starkv_v_append_desc* d, void* stream) {
  VAppendArgs a;
  const int st = build_v_append(d, a);
  return st ? st : launch_v_append(a, d->dtype, (hipStream_t)stream);
}

int starkv_decode_append(const starkv_k_append_desc* k, const starkv_v_append_desc* v,
                         const starkv_rope_apply_desc* q, void* stream) {
  StepAppendArgs a = {};
  int st;
  if ((st = build_k_append(k, a.k)) || (st = build_v_append(v, a.v))) return st;
  if (q && (st = build_rope_apply(q, a.r))) return st;
  if (v->dtype != k->dtype || (q && q->dtype != k->dtype)) return STARKV_ERR_DTYPE;
  a.has_rope = q != nullptr;
  const int64_t nb = ceil_div((int64_t)k->batch * k->k.n_kv_heads * k->n_tokens, 4) +
                     ceil_div((int64_t)v->batch * v->n_tokens * ceil_div(v->v.rank, 64), 4) +
                     (q ? ceil_div((int64_t)q->batch * q->n_heads * q->n_tokens * 64, 256) : 0);
  if (nb > INT32_MAX) return STARKV_ERR_LIMIT;
  return launch_step_append(a, k->dtype, (hipStream_t)stream);
}

// rows of act-dtype values: data 16-byte aligned, strides multiples of 8 elements
static bool rows16(const void* p, int64_t stride) { return al(p, 16) && stride >= 0 && stride % 8 == 0; }

int starkv_rms_norm(const starkv_rms_norm_desc* d, void* stream) {
  if (!d) return STARKV_ERR_NULL;
  if (d->rows < 0 || d->hidden < 8 || d->hidden % 8) return STARKV_ERR_SHAPE;
  if (d->hidden > NORM_MAX_HIDDEN) return STARKV_ERR_LIMIT;
  if (d->dtype != STARKV_F16 && d->dtype != STARKV_BF16) return STARKV_ERR_DTYPE;
  if (!d->x || !d->weight || !d->out || (d->residual_out && !d->residual)) return STARKV_ERR_NULL;
  if (!(d->eps >= 0.f)) return STARKV_ERR_SHAPE;
  if (!rows16(d->x, d->x_stride) || !rows16(d->out, d->out_stride) || !al(d->weight, 16) ||
      (d->residual && !rows16(d->residual, d->residual_stride)) ||
      (d->residual_out && !rows16(d->residual_out, d->residual_out_stride)))
    return STARKV_ERR_ALIGN;
  NormArgs a = {};
  a.x = d->x; a.xs = d->x_stride;
  a.res = d->residual; a.rs = d->residual_stride;
  a.res_out = d->residual_out; a.ros = d->residual_out_stride;
  a.w = d->weight; a.out = d->out; a.os = d->out_stride;
  a.rows = d->rows; a.H = d->hidden; a.eps = d->eps;
  return launch_rms_norm(a, d->dtype, (hipStream_t)stream);
}

int starkv_silu_mul(const starkv_silu_mul_desc* d, void* stream) {
  if (!d) return STARKV_ERR_NULL;
  if (d->rows < 0 || d->width < 8 || d->width % 8) return STARKV_ERR_SHAPE;
  if (d->dtype != STARKV_F16 && d->dtype != STARKV_BF16) return STARKV_ERR_DTYPE;
  if (!d->gate || !d->up || !d->out) return STARKV_ERR_NULL;
  if (!rows16(d->gate, d->gate_stride) || !rows16(d->up, d->up_stride) || !rows16(d->out, d->out_stride))
    return STARKV_ERR_ALIGN;
  if ((int64_t)d->rows * (d->width / 8) > MAX_THREADS_1D) return STARKV_ERR_LIMIT;
  SiluMulArgs a = {};
  a.g = d->gate; a.gs = d->gate_stride; a.u = d->up; a.us = d->up_stride;
  a.out = d->out; a.os = d->out_stride; a.rows = d->rows; a.W = d->width;
  return launch_silu_mul(a, d->dtype, (hipStream_t)stream);
}

int starkv_skinny_gemm(const starkv_skinny_gemm_desc* d, void* stream) {
  if (!d) return STARKV_ERR_NULL;
  if (d->m < 1 || d->k < 64 || d->k % 64 || d->n < 16 || d->n % 16) return STARKV_ERR_SHAPE;
  if (d->m > GEMM_MAX_M) return STARKV_ERR_LIMIT;
  if (d->epilogue < GEMM_STORE || d->epilogue > GEMM_SILU_MUL) return STARKV_ERR_SHAPE;
  if (d->epilogue == GEMM_SILU_MUL && d->n % 32) return STARKV_ERR_SHAPE;
  if (d->dtype != STARKV_F16 && d->dtype != STARKV_BF16) return STARKV_ERR_DTYPE;
  if (!d->x || !d->w || !d->out) return STARKV_ERR_NULL;
  if (d->x_stride < d->k || (!d->w_packed && d->w_stride < d->k)) return STARKV_ERR_SHAPE;
  const int n_out = d->epilogue == GEMM_SILU_MUL ? d->n / 2 : d->n;
  if (d->out_stride < n_out) return STARKV_ERR_SHAPE;
  if (!rows16(d->x, d->x_stride) || !al(d->w, 16) || (!d->w_packed && !rows16(d->w, d->w_stride)) || !al(d->out, 2))
    return STARKV_ERR_ALIGN;
  GemmArgs a = {};
  a.x = d->x; a.xs = d->x_stride; a.w = d->w; a.ws = d->w_stride; a.out = d->out; a.os = d->out_stride;
  a.wpk = d->w_packed != 0;
  if (d->rms && !(d->rms_eps >= 0.f)) return STARKV_ERR_SHAPE;
  a.rms = d->rms != 0; a.rms_eps = d->rms_eps;
  a.M = d->m; a.N = d->n; a.K = d->k; a.half_rows = d->n / 2;
  return launch_skinny_gemm(a, d->dtype, d->epilogue, (hipStream_t)stream);
}

}  // extern "C"

extern "C" {

size_t starkv_prefill_workspace_bytes(const starkv_prefill_desc* d) {
  int gs = 0;
  PrefillPlan P;
  if (validate_prefill(d, &gs, &P)) return 0;
  return P.total;
}

// Launch the repacks the plan asks for and point the kernel arguments at the
// aligned copies (latent offsets: elements for dense, bytes for quantised).
static int prefill_repack(const starkv_prefill_desc* d, const PrefillPlan& P, PFArgs& a, char* ws, hipStream_t s) {
  const starkv_klatent& k = d->k;
  const int Hkv = k.n_kv_heads, B = d->batch, S = (int)P.S;
  int st;
  auto set = [&](RepackArgs& r, int kind, const void* src, int64_t src_sb, int H, int S_, char* dst, int pitch) {
    r = RepackArgs{};
    r.kind = kind; r.src = (const uint8_t*)src; r.src_sb = src_sb; r.H = H; r.S = S_;
    r.dst = (uint8_t*)dst; r.pitch = pitch; r.dst_sb = (int64_t)H * S_ * pitch;
  };
  if (P.rk) {
    const bool dense = k.format == STARKV_FMT_DENSE;
    const int es = dense ? 2 : 1;
    const bool two = k.format == STARKV_FMT_INT4_REF && k.split > 0;
    const int split = dense ? 128 : (two ? k.split : 128);
    RepackArgs r;
    set(r, P.k_kind1, k.data, k.stride_b * es, Hkv, S, ws + P.off_k1, P.k_p1);
    for (int h = 0; h < Hkv; ++h) {
      r.src_off[h] = k.head_offset[h] * es; r.src_pitch[h] = k.pos_stride[h] * es;
      r.nel[h] = std::min(k.rank[h], split);
    }
    if ((st = launch_repack(r, B, s))) return st;
    a.kx = r.dst; a.kx_sb = r.dst_sb / es;
    for (int h = 0; h < Hkv; ++h) { a.kxoff[h] = (int64_t)h * S * P.k_p1 / es; a.kxpitch[h] = P.k_p1 / es; }
    if (P.k_p2) {
      set(r, RP_NIB, k.data2, k.stride2_b, Hkv, S, ws + P.off_k2, P.k_p2);
      for (int h = 0; h < Hkv; ++h) {
        const bool lo = k.rank[h] > split;
        r.src_off[h] = lo ? k.head_offset2[h] : 0; r.src_pitch[h] = lo ? k.pos_stride2[h] : 0;
        r.nel[h] = lo ? k.rank[h] - split : 0;
      }
      if ((st = launch_repack(r, B, s))) return st;
      a.kx2 = r.dst; a.kx2_sb = r.dst_sb;
      for (int h = 0; h < Hkv; ++h) { a.kxoff2[h] = (int64_t)h * S * P.k_p2; a.kxpitch2[h] = P.k_p2; }
    }
  }
  if (P.rv) {
    const starkv_vlatent& v = d->v;
    const bool dense = v.format == STARKV_FMT_DENSE;
    const int es = dense ? 2 : 1;
    PVArgs vb = {};
    int vq = 0;
    if ((st = validate_v(v, vb, &vq))) return st;
    RepackArgs r;
    set(r, P.v_kind1, v.data, v.stride_b * es, 1, S, ws + P.off_v1, P.v_p1);
    r.src_off[0] = 0; r.src_pitch[0] = v.stride_s * es;
    r.nel[0] = vq == VQ_BLOCK ? vb.split : v.rank;
    if ((st = launch_repack(r, B, s))) return st;
    a.vx = r.dst; a.vx_sb = r.dst_sb / es; a.vx_ss = P.v_p1 / es;
    if (P.v_p2) {
      set(r, RP_NIB, v.data2, v.stride2_b, 1, S, ws + P.off_v2, P.v_p2);
      r.src_off[0] = 0; r.src_pitch[0] = v.stride2_s;
      r.nel[0] = v.rank - vb.split;
      if ((st = launch_repack(r, B, s))) return st;
      a.vx2 = r.dst; a.vx2_sb = r.dst_sb; a.vx2_ss = P.v_p2;
    }
  }
  if (P.ru) {
    RepackArgs r;
    set(r, RP_HALF, d->uv, 0, 1, Hkv * HEAD_DIM, ws + P.off_u, P.u_p);
    r.src_off[0] = 0; r.src_pitch[0] = d->uv_row_stride * 2;
    r.nel[0] = d->v.rank;
    if ((st = launch_repack(r, 1, s))) return st;
    a.uv = r.dst; a.uv_rs = P.u_p / 2;
  }
  return STARKV_OK;
}

static int prefill_impl(const starkv_prefill_desc* d, void* workspace, size_t workspace_bytes, void* stream,
                        void* const* events) {
  int gs = 0, st;
  PrefillPlan P;
  if ((st = validate_prefill(d, &gs, &P))) return st;
  const size_t kvb = P.kvb;
  if (!workspace || workspace_bytes < P.total) return STARKV_ERR_WORKSPACE;
  if (!al(workspace, 256)) return STARKV_ERR_ALIGN;
  const starkv_klatent& k = d->k;
  PFArgs a = {};
  a.S = d->pos0 + d->n_tokens; a.S_pad = (int)P.S_pad;
  a.Hkv = k.n_kv_heads; a.Hq = d->n_q_heads; a.gs = gs; a.T = d->n_tokens; a.pos0 = d->pos0;
  a.kx = k.data; a.kx_sb = k.stride_b; a.k_i8 = k.format == STARKV_FMT_INT8_SYM;
  a.kscale = k.scale; a.ks_sb = k.scale_stride_b; a.ks_sh = k.scale_stride_h;
  // reference split format: ranks [0, ksplit) int8 or int4 in data, the rest int4 in data2
  const bool ktwo = k.format == STARKV_FMT_INT4_REF && k.split > 0;
  a.k_ref = k.format == STARKV_FMT_INT4_REF;
  a.ksplit = ktwo ? k.split : 128;
  a.k_a8 = ktwo && k.split_format == STARKV_FMT_INT8_SYM;
  a.kx2 = k.data2; a.kx2_sb = k.stride2_b;
  a.kscale2 = k.scale2; a.ks2_sb = k.scale2_stride_b; a.ks2_sh = k.scale2_stride_h;
  for (int h = 0; h < k.n_kv_heads; ++h) {
    a.krank[h] = k.rank[h];
    a.kxoff[h] = k.head_offset[h]; a.kxpitch[h] = k.pos_stride[h];
    const bool lo = ktwo && k.rank[h] > k.split;
    a.kxoff2[h] = lo ? k.head_offset2[h] : 0; a.kxpitch2[h] = lo ? k.pos_stride2[h] : 0;
    a.bkoff[h] = k.bk_head_offset[h];
  }
  a.bk = k.bk; a.bk_rs = k.bk_row_stride;
  const starkv_vlatent& v = d->v;
  a.vx = v.data; a.vx_sb = v.stride_b; a.vx_ss = v.stride_s;
  a.v_g64 = v.format == STARKV_FMT_INT4_G64; a.Rv = v.rank;
  a.vscale = v.scale; a.vzero = v.zero; a.vs_sb = v.scale_stride_b; a.vs_ss = v.scale_stride_s;
  {
    // per-token blocks: the split and block formats as validate_v reads them
    PVArgs vb = {};
    int vq = 0;
    if ((st = validate_v(v, vb, &vq))) return st;
    a.v_blk = vq == VQ_BLOCK;
    a.vsplit = vb.split; a.v_a8 = vb.a_int8;
    a.vx2 = vb.x2; a.vx2_sb = vb.x2_sb; a.vx2_ss = vb.x2_ss;
    a.vscale2 = vb.xs2; a.vs2_sb = vb.xs2_sb; a.vs2_ss = vb.xs2_ss;
  }
  a.uv = d->uv; a.uv_rs = d->uv_row_stride;
  a.rope = d->rope_table;
  a.kbuf = workspace; a.vbuf = (char*)workspace + kvb;
  a.q = d->q; a.q_sb = d->q_stride_b; a.q_sh = d->q_stride_h; a.q_st = d->q_stride_t;
  a.scale_log2 = d->scale * 1.4426950408889634f;
  a.out = d->out; a.o_sb = d->out_stride_b; a.o_sh = d->out_stride_h; a.o_st = d->out_stride_t;
  hipStream_t s = (hipStream_t)stream;
  if (events && (st = (int)hipEventRecord((hipEvent_t)events[0], s))) return st;
  if ((st = prefill_repack(d, P, a, (char*)workspace, s))) return st;
  if ((st = launch_prefill(a, d->dtype, d->batch, s, events ? (hipEvent_t)events[1] : nullptr))) return st;
  if (events && (st = (int)hipEventRecord((hipEvent_t)events[2], s))) return st;
  return STARKV_OK;
}

int starkv_prefill_attention(const starkv_prefill_desc* d, void* workspace, size_t workspace_bytes, void* stream) {
  return prefill_impl(d, workspace, workspace_bytes, stream, nullptr);
}

int starkv_prefill_attention_timed(const starkv_prefill_desc* d, void* workspace, size_t workspace_bytes,
                                   void* stream, void* const* events) {
  if (!events || !events[0] || !events[1] || !events[2]) return STARKV_ERR_NULL;
  return prefill_impl(d, workspace, workspace_bytes, stream, events);
}

}  // extern "C"
