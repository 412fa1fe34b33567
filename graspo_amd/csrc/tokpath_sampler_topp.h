// tokpath_sampler_topp.h -- the top-p sampler for bf16 rows (gfx950).
//
// Serves sampling rows with top-p active (0 < P < 1) and no top-k, on
// 16-byte aligned bf16 rows of 65536 <= V <= 2^18 with 0 < T <= 1024: every
// decode step of the reference's _next_token_from_logits(logits,
// temperature, top_p) (src/graspo/backends/graspoflow/tensor_utils.py:649-683)
// and the structured-output rows with an allow mask.  One workgroup of 1024
// threads per row reads the row once; the answer follows the contract of
// include/graspo_tokpath.h bit for bit.
//
// 1. Pilot.  Stream chunks are handed out in an order that starts the 16
//    waves at 16 evenly spaced places of the row.  Their first chunks (16384
//    tokens) are a sample: a two-pass radix select over the allowed tokens'
//    16-bit order keys picks theta, a value with about 4096 allowed tokens of
//    the row at or above it.
// 2. Stream.  Per allowed token one LDS add into a 16-bit count per bf16
//    value: unpenalised and penalised tokens (history ids, an LDS bitmap) in
//    two histograms of 16384 values (exponents [87, 151) of both signs),
//    zeros in two counters.  Allowed tokens whose processed value before
//    temperature (x, or pen(x) for a history id) reaches theta go with their
//    id into an LDS pool.  The raw log-sum-exp is folded for the logprob.
// 3. Totals.  m = the largest processed logit y.  Thread t owns 16 value
//    bins (thread 0 the largest values) and the penalised values whose y
//    lies between its bins; its weight total (DETEXP_FIX(y - m) per distinct
//    value times the count) and count total go through one block scan in
//    descending order.
// 4. Cut and draw.  The thread whose range holds floor(P W) (then
//    floor(u W')) is resolved by one wave: its at most 64 distinct values
//    sorted by y, a wave scan, and an integer quotient inside the tied
//    values (all tokens of one value share one weight).
// 5. Ids.  The k-th token of the cut value and the j-th of the drawn value,
//    in id order: from the pool (the matching entries set bits of an id
//    bitmap; a scan of popcounts finds the k-th), or, for a value below
//    theta, from a rescan of the row.
// Outside these bounds -- a value outside the bins, a count that overflows
// 16 bits, more than 46 penalised values in one resolved range, a processed
// logit outside the bins' range -- the row is handed over to the row-wise
// path, which runs in a second launch (a block-uniform decision, taken
// before any output of the row is written).
#pragma once

namespace gtp {
namespace topp {

constexpr int kB = 1024;             // threads per row
constexpr int kW = kB / kWave;       // waves per row
constexpr int kG = 2;                // vectors per lane per chunk
constexpr int kChunk = kWave * kG;   // vectors per chunk
constexpr int kBins = 16384;         // bf16 values with biased exponent in [87, 151), both signs
constexpr uint32_t kELo = 87;
constexpr int kPer = kBins / kB;     // bins per thread
constexpr int kPool = 8192;          // captured tokens
constexpr uint32_t kTarget = 4096;   // tokens the pilot aims to capture
constexpr int kPenLanes = 46;        // penalised values one resolved range may hold
constexpr int64_t kMinV = 65536;

struct Level {
  float y;              // processed logit of the value
  int32_t ubin;         // unpenalised bin of the value, or -1
  int32_t pbin;         // penalised raw bin whose y ties, or -1
  int32_t zero_u;       // 1: the unpenalised zeros belong to the level
  int32_t zero_p;       // 1: the penalised zeros belong to the level
  uint32_t n;           // tokens of the level
  uint32_t k;           // position of the wanted token in id order
  uint32_t n_before;    // tokens before the level
  unsigned long long s_before;  // weight before the level
  unsigned long long w;         // weight of one token of the level
};

struct alignas(16) Smem {
  uint32_t cnt[kBins / 2];                // allowed unpenalised tokens per value (16-bit halves)
  uint32_t pcnt[kBins / 2];               // allowed penalised tokens per raw value
  uint32_t pen[GTP_SAMPLER_MAX_V / 32];   // penalised ids
  uint32_t qid[kPool];                    // pool: id, bit 31 set for a penalised token
  uint16_t qh[kPool];                     // pool: bf16 pattern
  uint32_t sel[2][256];                   // pilot radix histograms
  float red_f[kW][3];
  uint32_t red_u[kW][2];
  unsigned long long red_w[kW];
  Level lv[2];                            // the cut (0) and the drawn (1) value
  int32_t id_out[2];
  uint32_t scan_n[kW][2];                 // rescan: matches per wave
  uint32_t chunk_ctr;
  uint32_t pool_n;
  uint32_t drop_key;     // largest ord32 key of a capture that found the pool full, 0: none
  uint32_t theta_sel[2];
  uint32_t n_counted;    // allowed tokens added to the two histograms
  uint32_t zc, pz;       // allowed unpenalised / penalised zeros
  unsigned long long o_ew[2];  // the resolved ranges: weight and count before them,
  uint32_t o_ec[2];            // their penalised raw bins [o_pl, o_ph]
  int32_t o_pl[2], o_ph[2];
  uint32_t flags;        // bit 0: allowed value outside the bins; bit 1: bad history id
  int32_t owner[2];
  int32_t bad;           // fallback decided by a single wave
};

__device__ __forceinline__ int bin_of(uint32_t h) {  // -1 outside the bins
  const uint32_t idx = (h & 0x7FFFu) - (kELo << 7);
  if (idx >= 64u * 128u) return -1;
  return (h & 0x8000u) ? (int)(kBins / 2 - 1 - idx) : (int)(kBins / 2 + idx);
}
__device__ __forceinline__ uint32_t bin_bits(int b) {
  return b >= kBins / 2 ? (uint32_t)(b - kBins / 2) + (kELo << 7)
                        : 0x8000u | ((uint32_t)(kBins / 2 - 1 - b) + (kELo << 7));
}
__device__ __forceinline__ float bin_x(int b) { return u2f(bin_bits(b) << 16); }
__device__ __forceinline__ uint32_t count16(const uint32_t* c, int b) {
  return (c[b >> 1] >> ((b & 1) * 16)) & 0xFFFFu;
}

// Block-wide exclusive scan in thread order of (u64, u32); every thread gets
// its exclusive prefix and the totals.
__device__ __forceinline__ void block_scan2(Smem& sm, unsigned long long w, uint32_t c,
                                            unsigned long long& ew, uint32_t& ec,
                                            unsigned long long& tw, uint32_t& tc) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const unsigned long long iw = wave_scan_u64(w);
  const uint32_t ic = wave_scan_u32(c);
  __syncthreads();
  if (lane == kWave - 1) {
    sm.red_w[wid] = iw;
    sm.red_u[wid][0] = ic;
  }
  __syncthreads();
  unsigned long long bw = 0ull, allw = 0ull;
  uint32_t bc = 0u, allc = 0u;
#pragma unroll
  for (int i = 0; i < kW; ++i) {
    const unsigned long long vw = sm.red_w[i];
    const uint32_t vc = sm.red_u[i][0];
    if (i < wid) {
      bw += vw;
      bc += vc;
    }
    allw += vw;
    allc += vc;
  }
  ew = bw + iw - w;
  ec = bc + ic - c;
  tw = allw;
  tc = allc;
}

// Block maximum of a u32 (every thread gets it).
__device__ __forceinline__ uint32_t block_max_u32(Smem& sm, uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t w = __shfl_xor(v, o, kWave);
    v = w > v ? w : v;
  }
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) sm.red_u[wid][1] = v;
  __syncthreads();
  uint32_t r = sm.red_u[0][1];
#pragma unroll
  for (int i = 1; i < kW; ++i) r = sm.red_u[i][1] > r ? sm.red_u[i][1] : r;
  return r;
}

template <bool kMask>
struct Row {
  const uint16_t* __restrict__ x;
  const uint32_t* __restrict__ mask;
  int64_t V, nvec;
  bool use_pen;
  float rho, Tc;
  // processed logits (contract steps: penalty, then temperature), zeros canonical
  __device__ __forceinline__ float pen_v(float x) const { return x < 0.0f ? x * rho : x / rho; }
  __device__ __forceinline__ float y_of(float v) const { return v / Tc + 0.0f; }
  __device__ __forceinline__ float ybin(int b) const { return y_of(bin_x(b)); }
  __device__ __forceinline__ float ypen(int p) const { return y_of(pen_v(bin_x(p))); }
  __device__ __forceinline__ bool allowed(int64_t id) const {
    return !kMask || ((mask[id >> 5] >> (id & 31)) & 1u);
  }
};

// smallest bin b with ybin(b) >= y (kBins when y is above every bin)
template <bool kMask>
__device__ __forceinline__ int ceil_bin(const Row<kMask>& r, float y) {
  int g = bin_of(bf16_round_up(y * r.Tc));
  if (g < 0) {
    int lo = 0, hi = kBins;  // first bin with ybin >= y in [lo, hi]
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (r.ybin(mid) >= y) hi = mid;
      else lo = mid + 1;
    }
    return lo;
  }
  while (g > 0 && r.ybin(g - 1) >= y) --g;
  while (g < kBins && r.ybin(g) < y) ++g;
  return g;
}

// Resolve the crossing of `X` (a weight position) inside thread `t`'s range:
// one wave sorts the range's distinct values by y, scans their weights and
// finds the value and the position inside it.  `ex_w` / `ex_c` are the
// weight and count before the range.  Returns false when the range holds too
// many penalised values (the caller falls back).
template <bool kMask>
__device__ __forceinline__ bool resolve_range(const Smem& sm, const Row<kMask>& r, int t, float m,
                              unsigned long long X, unsigned long long ex_w, uint32_t ex_c,
                              int pl, int ph, Level& out) {
  const int lane = threadIdx.x & (kWave - 1);
  const int hi = kBins - 1 - kPer * t;
  // entries: lanes 0..15 the unpenalised bins hi - lane, lanes 16..61 the
  // penalised raw bins pl.., lanes 62 / 63 the unpenalised / penalised zeros
  const int np = ph >= pl ? ph - pl + 1 : 0;
  if (np > kPenLanes) return false;
  const int zero_owner = (kBins - 1 - kBins / 2) / kPer;
  float y = kNegInf;
  uint32_t c = 0u;
  int kind = -1, ref = -1;
  if (lane < kPer) {
    kind = 0;
    ref = hi - lane;
    c = count16(sm.cnt, ref);
    y = r.ybin(ref);
  } else if (lane < kPer + np) {
    kind = 1;
    ref = pl + (lane - kPer);
    c = count16(sm.pcnt, ref);
    y = r.ypen(ref);
  } else if (t == zero_owner && lane >= kWave - 2) {
    kind = lane == kWave - 2 ? 2 : 3;
    c = lane == kWave - 2 ? sm.zc : sm.pz;
    y = 0.0f;
  }
  if (c == 0u) {
    y = kNegInf;
    kind = -1;
  }
  const unsigned long long w1 = c ? detexp_fix(y - m) : 0ull;
  // sort by (y desc, lane asc): rank by counting, then a permute
  const unsigned long long key = ((unsigned long long)ord32(y) << 32) | (uint32_t)(kWave - 1 - lane);
  uint32_t rank = 0;
  for (int j = 0; j < kWave; ++j) {
    const uint32_t khi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(key >> 32), j);
    const uint32_t klo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, j);
    const unsigned long long kk = ((unsigned long long)khi << 32) | klo;
    rank += kk > key ? 1u : 0u;
  }
  // lane `rank` receives this lane's entry (ds_permute scatters by address)
  auto scatter_u32 = [&](uint32_t v) -> uint32_t {
    return (uint32_t)__builtin_amdgcn_ds_permute((int)(rank * 4u), (int)v);
  };
  const float ys = u2f(scatter_u32(f2u(y)));
  const uint32_t cs = scatter_u32(c);
  const int kinds = (int)scatter_u32((uint32_t)kind);
  const int refs = (int)scatter_u32((uint32_t)ref);
  const unsigned long long ws = ((unsigned long long)scatter_u32((uint32_t)(w1 >> 32)) << 32) |
                                scatter_u32((uint32_t)w1);
  const unsigned long long iw = wave_scan_u64((unsigned long long)cs * ws);
  const uint32_t ic = wave_scan_u32(cs);
  const unsigned long long rel = X - ex_w;
  const unsigned long long past = __ballot(iw > rel);
  if (!past) return false;  // cannot happen: X lies inside the range
  const int e = __builtin_ctzll(past);
  const float ye = u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(ys), e));
  const unsigned long long grp = __ballot(ys == ye && cs != 0u);
  const int gs = __builtin_ctzll(grp);
  const unsigned long long iw_b =
      gs ? (((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(iw >> 32), gs - 1)
             << 32) |
            (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)iw, gs - 1))
         : 0ull;
  const uint32_t ic_b = gs ? (uint32_t)__builtin_amdgcn_readlane((int)ic, gs - 1) : 0u;
  const bool in_grp = (grp >> lane) & 1ull;
  // the group's members (at most one unpenalised bin, one penalised bin and
  // the two zero counts) and its size
  uint32_t gn = in_grp ? cs : 0u;
  gn = wave_sum_u32(gn);
  int ub = -1, pb = -1, zu = 0, zp = 0;
  const unsigned long long b0 = __ballot(in_grp && kinds == 0);
  const unsigned long long b1 = __ballot(in_grp && kinds == 1);
  if (b0) ub = __builtin_amdgcn_readlane(refs, __builtin_ctzll(b0));
  if (b1) pb = __builtin_amdgcn_readlane(refs, __builtin_ctzll(b1));
  zu = __ballot(in_grp && kinds == 2) ? 1 : 0;
  zp = __ballot(in_grp && kinds == 3) ? 1 : 0;
  const unsigned long long wt = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(ws >> 32), e) << 32) |
                                (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)ws, e);
  out.y = ye;
  out.ubin = ub;
  out.pbin = pb;
  out.zero_u = zu;
  out.zero_p = zp;
  out.n = gn;
  out.s_before = ex_w + iw_b;
  out.n_before = ex_c + ic_b;
  out.w = wt;
  const unsigned long long q = (X - out.s_before) / wt;
  out.k = (uint32_t)q;
  return q < gn;
}

// Level membership of an allowed token with bf16 pattern h.
__device__ __forceinline__ bool level_has(const Level& L, bool pen, uint32_t h) {
  if ((h & 0x7FFFu) == 0u) return pen ? L.zero_p != 0 : L.zero_u != 0;
  return pen ? (L.pbin >= 0 && h == bin_bits(L.pbin)) : (L.ubin >= 0 && h == bin_bits(L.ubin));
}

// Every token of the level is in the pool: each of its values before
// temperature is at or above theta and above every capture the full pool
// dropped.
template <bool kMask>
__device__ __forceinline__ bool level_in_pool(const Smem& sm, const Row<kMask>& r, const Level& L,
                                              float theta) {
  bool ok = true;
  auto check = [&](float v) {
    v = v + 0.0f;
    ok = ok && v >= theta && (sm.drop_key == 0u || ord32(v) > sm.drop_key);
  };
  if (L.ubin >= 0) check(bin_x(L.ubin));
  if (L.pbin >= 0) check(r.pen_v(bin_x(L.pbin)));
  if (L.zero_u || L.zero_p) check(0.0f);
  return ok;
}

// Ids of the two levels' wanted tokens by a rescan of the row (block-wide):
// pass 1 counts each level's tokens in 16 equal ranges, one per wave; pass 2
// walks the range that holds the wanted token.  Writes sm.id_out[0..1].
template <bool kMask>
__device__ __forceinline__ void rescan_ids(Smem& sm, const Row<kMask>& r) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const int64_t nvec = r.nvec, V = r.V;
  const int64_t span = (nvec + kW - 1) / kW;
  const int64_t v0 = wid * span, v1 = v0 + span < nvec ? v0 + span : nvec;
  const Level L0 = sm.lv[0], L1 = sm.lv[1];
  // matches of one vector (or, for v == nvec, of the tail tokens), as two 8-bit masks
  auto vec_matches = [&](int64_t v, uint32_t& m0, uint32_t& m1) __attribute__((always_inline)) {
    m0 = m1 = 0u;
    if (v < nvec) {
      const u32x4 q = *reinterpret_cast<const u32x4*>(r.x + v * 8);
      const uint32_t wds[4] = {q.x, q.y, q.z, q.w};
      const uint32_t ab = kMask ? (r.mask[v >> 2] >> ((v & 3) * 8)) & 0xFFu : 0xFFu;
      const uint32_t pb = r.use_pen ? (sm.pen[v >> 2] >> ((v & 3) * 8)) & 0xFFu : 0u;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t h = (j & 1) ? wds[j >> 1] >> 16 : wds[j >> 1] & 0xFFFFu;
        const bool on = (ab >> j) & 1u, pn = (pb >> j) & 1u;
        m0 |= (on && level_has(L0, pn, h)) ? 1u << j : 0u;
        m1 |= (on && level_has(L1, pn, h)) ? 1u << j : 0u;
      }
    } else {
      for (int64_t id = nvec * 8; id < V; ++id) {
        const int j = (int)(id - nvec * 8);
        const uint32_t h = r.x[id];
        const bool on = r.allowed(id);
        const bool pn = r.use_pen && ((sm.pen[id >> 5] >> (id & 31)) & 1u);
        m0 |= (on && level_has(L0, pn, h)) ? 1u << j : 0u;
        m1 |= (on && level_has(L1, pn, h)) ? 1u << j : 0u;
      }
    }
  };
  const bool has_tail = wid == kW - 1 && nvec * 8 < V;
  // pass 1
  uint32_t c0 = 0u, c1 = 0u;
  for (int64_t v = v0 + lane; v < v1; v += kWave) {
    uint32_t m0, m1;
    vec_matches(v, m0, m1);
    c0 += __builtin_popcount(m0);
    c1 += __builtin_popcount(m1);
  }
  if (has_tail && lane == 0) {
    uint32_t m0, m1;
    vec_matches(nvec, m0, m1);
    c0 += __builtin_popcount(m0);
    c1 += __builtin_popcount(m1);
  }
  c0 = wave_sum_u32(c0);
  c1 = wave_sum_u32(c1);
  if (lane == 0) {
    sm.scan_n[wid][0] = c0;
    sm.scan_n[wid][1] = c1;
  }
  __syncthreads();
  // pass 2: the wave whose range holds the wanted token of a level finds it
  for (int l = 0; l < 2; ++l) {
    const uint32_t k = l ? L1.k : L0.k;
    uint32_t before = 0u;
    for (int w = 0; w < wid; ++w) before += sm.scan_n[w][l];
    if (!(before <= k && k < before + sm.scan_n[wid][l])) continue;
    uint32_t run = before;
    for (int64_t vb = v0; vb < v1 + (has_tail ? 1 : 0); vb += kWave) {
      const int64_t v = vb + lane;
      uint32_t m0 = 0u, m1 = 0u;
      if (v < v1 || (has_tail && v == nvec)) vec_matches(v, m0, m1);
      const uint32_t mm = l ? m1 : m0;
      const uint32_t n = __builtin_popcount(mm);
      const uint32_t incl = wave_scan_u32(n);
      const uint32_t tot = lane63_u32(incl);
      if (run + tot > k) {
        const uint32_t ex = run + incl - n;
        if (n && ex <= k && k < ex + n) {
          uint32_t mk = mm;
          for (uint32_t i = 0; i < k - ex; ++i) mk &= mk - 1u;
          sm.id_out[l] = (int32_t)(v * 8 + __builtin_ctz(mk));
        }
        break;
      }
      run += tot;
    }
  }
  __syncthreads();
}

// One row; false when the row needs the row-wise path (a block-uniform
// decision, taken before any output is written).
template <bool kMask>
__device__ __forceinline__ bool topp_row(const SamplerArgs& a, int64_t b, Smem& sm) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  Row<kMask> r;
  r.x = reinterpret_cast<const uint16_t*>(a.logits) + b * a.row_stride;
  r.mask = kMask ? a.mask + b * a.mask_stride : nullptr;
  r.V = a.V;
  r.nvec = a.V / 8;
  r.use_pen = a.hist && a.hist_len > 0 && a.rho != 1.0f;
  r.rho = a.rho;
  r.Tc = a.T > 1e-6f ? a.T : 1e-6f;
  const float u = a.uniforms[b];
  const int64_t V = a.V, nvec = r.nvec;
  const uint32_t nchunks = (uint32_t)((nvec + kChunk - 1) / kChunk);
  const uint32_t per = nchunks / kW;
  // chunk c of the dynamic schedule -> chunk of the row: the first kW chunks
  // handed out start kW evenly spaced regions (the pilot sample)
  auto perm = [&](uint32_t c) -> uint32_t { return c < per * kW ? (c % kW) * per + c / kW : c; };

  // ---- 0. clear
  for (int i = tid; i < kBins / 2; i += kB) {
    sm.cnt[i] = 0u;
    sm.pcnt[i] = 0u;
  }
  if (r.use_pen)
    for (int64_t i = tid; i < (V + 31) / 32; i += kB) sm.pen[i] = 0u;
  if (tid < 512) sm.sel[tid >> 8][tid & 255] = 0u;
  if (tid == 0) {
    sm.owner[0] = -1;
    sm.owner[1] = -1;
    sm.chunk_ctr = 0u;
    sm.pool_n = 0u;
    sm.drop_key = 0u;
    sm.n_counted = 0u;
    sm.zc = 0u;
    sm.pz = 0u;
    sm.flags = 0u;
    sm.bad = 0;
  }
  __syncthreads();

  // ---- 1. the first two chunks in flight, then the history bitmap
  const uint32_t last = (uint32_t)(nvec - 1);
  const uint32_t last_word = (uint32_t)((V - 1) >> 5);
  auto grab = [&]() -> uint32_t {
    uint32_t c = 0;
    if (lane == 0) c = atomicAdd(&sm.chunk_ctr, 1u);
    return __builtin_amdgcn_readfirstlane(c);
  };
  auto issue = [&](u32x4(&buf)[kG], uint32_t& sw, uint32_t chunk) {
    const uint32_t pc = chunk < nchunks ? perm(chunk) : 0u;
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      uint32_t vi = pc * kChunk + (uint32_t)(k * kWave + lane);
      vi = vi < last ? vi : last;
      buf[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(r.x) + vi);
    }
    if (kMask) {  // the chunk's 32 mask words, one per lane (lanes 32..63 repeat them)
      uint32_t w = pc * (kChunk * 8 / 32) + (uint32_t)(lane & 31);
      sw = r.mask[w < last_word ? w : last_word];
    }
  };
  u32x4 qa[kG], qb[kG];
  uint32_t swa = 0xFFFFFFFFu, swb = 0xFFFFFFFFu;
  uint32_t ca = grab();
  issue(qa, swa, ca);
  uint32_t cb = grab();
  issue(qb, swb, cb);
  bool bad_hist = false;
  if (a.hist && a.hist_len > 0) {
    const int32_t* h = a.hist + b * a.hist_stride;
    for (int64_t j = tid; j < a.hist_len; j += kB) {
      const int32_t id = h[j];
      if (id >= V) bad_hist = true;
      else if (id >= 0 && r.use_pen) atomicOr(&sm.pen[id >> 5], 1u << (id & 31));
    }
  }
  if (bad_hist) atomicOr(&sm.flags, 2u);

  // allow bits of vector k of a chunk for this lane (vector k*64 + lane); a
  // cross-lane read, so every lane of the wave calls it (a lane past the
  // row's end would otherwise hand its neighbours a zero byte)
  auto allow_byte = [&](uint32_t sw, int k) -> uint32_t {
    if (!kMask) return 0xFFu;
    const uint32_t w = (uint32_t)__shfl((int)sw, k * (kWave / 4) + lane / 4, kWave);
    return (w >> ((lane & 3) * 8)) & 0xFFu;
  };

  // ---- 2. pilot: theta from the first chunk of every wave
  {
    uint32_t keys[kG][8];
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      const uint32_t pc = perm(ca);
      const uint32_t vi = pc * kChunk + (uint32_t)(k * kWave + lane);
      const uint32_t ab_all = allow_byte(swa, k);
      const uint32_t ab = vi < (uint32_t)nvec ? ab_all : 0u;
      const uint32_t wds[4] = {qa[k].x, qa[k].y, qa[k].z, qa[k].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t h = (j & 1) ? wds[j >> 1] >> 16 : wds[j >> 1] & 0xFFFFu;
        keys[k][j] = ((ab >> j) & 1u) ? ord16(h) : 0u;
        if (keys[k][j]) atomicAdd(&sm.sel[0][keys[k][j] >> 8], 1u);
      }
    }
    const uint32_t ks = (uint32_t)(((uint64_t)kTarget * (uint64_t)(kW * kChunk * 8) + (uint64_t)V - 1) /
                                   (uint64_t)V);
    __syncthreads();  // also completes the history bitmap
    auto pick = [&](const uint32_t* hist, uint32_t want, uint32_t& bin, uint32_t& rem) {
      // descending over 256 bins, 4 per lane: the bin holding the want-th key
      uint32_t c[4], s4 = 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c[i] = hist[255 - 4 * lane - i];
        s4 += c[i];
      }
      const uint32_t incl = wave_scan_u32(s4);
      const unsigned long long hit = __ballot(incl >= want);
      bin = 0xFFFFFFFFu;
      rem = 0u;
      if (!hit) return;
      const int l = __builtin_ctzll(hit);
      if (lane == l) {
        uint32_t run = incl - s4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (bin == 0xFFFFFFFFu && run + c[i] >= want) {
            bin = (uint32_t)(255 - 4 * lane - i);
            rem = want - run;
          }
          run += c[i];
        }
      }
      bin = (uint32_t)__builtin_amdgcn_readlane((int)bin, l);
      rem = (uint32_t)__builtin_amdgcn_readlane((int)rem, l);
    };
    if (wid == 0) {
      uint32_t hb, rem;
      pick(sm.sel[0], ks, hb, rem);
      if (lane == 0) {
        sm.theta_sel[0] = hb;
        sm.theta_sel[1] = rem;
      }
    }
    __syncthreads();
    const uint32_t hb = sm.theta_sel[0];
    if (hb != 0xFFFFFFFFu) {
#pragma unroll
      for (int k = 0; k < kG; ++k)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (keys[k][j] && (keys[k][j] >> 8) == hb) atomicAdd(&sm.sel[1][keys[k][j] & 0xFFu], 1u);
    }
    __syncthreads();
    if (wid == 0 && hb != 0xFFFFFFFFu) {
      uint32_t lb, rem2;
      pick(sm.sel[1], sm.theta_sel[1], lb, rem2);
      if (lane == 0) sm.theta_sel[0] = (hb << 8) | lb;
    } else if (wid == 0 && lane == 0) {
      sm.theta_sel[0] = 0xFFFFFFFFu;  // fewer allowed sample tokens than wanted: capture all
    }
    __syncthreads();
  }
  const uint32_t tkey = sm.theta_sel[0];
  const float theta = tkey == 0xFFFFFFFFu ? kNegInf : u2f(unord16(tkey) << 16);
  // vectors whose maximum is below th_lo hold no capture (rho < 1 lifts
  // penalised values, so there every vector is tested)
  const float th_lo = (r.use_pen && r.rho < 1.0f) ? kNegInf : theta;

  // ---- 3. stream
  Lse3 st{kNegInf, 0.0f, 0.0f};
  uint32_t counted = 0u;
  bool spill = false;
  auto count_token = [&](uint32_t h, bool pn) __attribute__((always_inline)) {
    const int bn = bin_of(h);
    if (bn >= 0) {
      atomicAdd((pn ? sm.pcnt : sm.cnt) + (bn >> 1), 1u << ((bn & 1) * 16));
      ++counted;
    } else if ((h & 0x7FFFu) == 0u) {
      atomicAdd(pn ? &sm.pz : &sm.zc, 1u);
    } else if (h != 0xFF80u) {
      spill = true;  // NaN, +inf, or a value outside the bins
    }
  };
  auto capture = [&](uint32_t id, uint32_t h, bool pn, uint32_t slot, float v) __attribute__((always_inline)) {
    if (slot < (uint32_t)kPool) {
      sm.qid[slot] = id | (pn ? 0x80000000u : 0u);
      sm.qh[slot] = (uint16_t)h;
    } else {
      atomicMax(&sm.drop_key, ord32(v + 0.0f));
    }
  };
  auto consume = [&](const u32x4(&buf)[kG], uint32_t sw, uint32_t chunk) __attribute__((always_inline)) {
    const uint32_t pc = perm(chunk);
    float x[kG][8], vm[kG];
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      Vec<uint16_t>::cvt(buf[k], x[k]);
      const uint32_t vi = pc * kChunk + (uint32_t)(k * kWave + lane);
      if (vi >= (uint32_t)nvec) {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[k][j] = kNegInf;
      }
      vm[k] = vec_max<8>(x[k]);
    }
    float cm = vm[0];
#pragma unroll
    for (int k = 1; k < kG; ++k) cm = max3raw(cm, vm[k], vm[k]);
    lse_fold_block_max<false, kG, 8>(st, x, cm);
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      const uint32_t vi = pc * kChunk + (uint32_t)(k * kWave + lane);
      const uint32_t ab_all = allow_byte(sw, k);
      const uint32_t ab = vi < (uint32_t)nvec ? ab_all : 0u;
      const uint32_t pb = r.use_pen ? (sm.pen[(vi < last ? vi : last) >> 2] >> ((vi & 3) * 8)) & 0xFFu : 0u;
      const uint32_t wds[4] = {buf[k].x, buf[k].y, buf[k].z, buf[k].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t h = (j & 1) ? wds[j >> 1] >> 16 : wds[j >> 1] & 0xFFFFu;
        if ((ab >> j) & 1u) count_token(h, (pb >> j) & 1u);
      }
      uint32_t cap = 0u;
      if (ab && vm[k] >= th_lo) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float v = ((pb >> j) & 1u) ? r.pen_v(x[k][j]) : x[k][j];
          cap |= (((ab >> j) & 1u) && v >= theta) ? 1u << j : 0u;
        }
      }
      if (__ballot(cap != 0u)) {
        const uint32_t n = __builtin_popcount(cap);
        const uint32_t incl = wave_scan_u32(n);
        uint32_t base = 0u;
        if (lane == 0) base = atomicAdd(&sm.pool_n, lane63_u32(incl));
        else (void)lane63_u32(incl);
        base = __builtin_amdgcn_readfirstlane(base);
        uint32_t slot = base + incl - n;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if ((cap >> j) & 1u) {
            const uint32_t h = (j & 1) ? wds[j >> 1] >> 16 : wds[j >> 1] & 0xFFFFu;
            const bool pn = (pb >> j) & 1u;
            capture(vi * 8u + (uint32_t)j, h, pn, slot, pn ? r.pen_v(x[k][j]) : x[k][j]);
            ++slot;
          }
        }
      }
    }
  };
  while (ca < nchunks) {
    consume(qa, swa, ca);
    if (cb >= nchunks) break;
    ca = grab();
    issue(qa, swa, ca);
    consume(qb, swb, cb);
    cb = grab();
    if (ca >= nchunks) break;
    issue(qb, swb, cb);
  }
  if (cb < nchunks && ca >= nchunks) consume(qb, swb, cb);
  // tail tokens (V not a multiple of 8)
  for (int64_t id = nvec * 8 + tid; id < V; id += kB) {
    const uint32_t h = r.x[id];
    const float xv = u2f(h << 16);
    float x1[1][4] = {{xv, kNegInf, kNegInf, kNegInf}};
    lse_fold_block_max<false, 1, 4>(st, x1, xv);
    if (r.allowed(id)) {
      const bool pn = r.use_pen && ((sm.pen[id >> 5] >> (id & 31)) & 1u);
      count_token(h, pn);
      const float v = pn ? r.pen_v(xv) : xv;
      if (v >= theta) capture((uint32_t)id, h, pn, atomicAdd(&sm.pool_n, 1u), v);
    }
  }
  if (spill) atomicOr(&sm.flags, 1u);
  {
    const uint32_t cs = wave_sum_u32(counted);
    if (lane == 0) atomicAdd(&sm.n_counted, cs);
  }
  const Lse3 rl = block_lse3<kB>(st, sm.red_f);  // (its barrier publishes the stream's LDS writes)

  // ---- 4. row status
  const float lse_m = rl.m, lse_ln = __builtin_amdgcn_logf(rl.s) * kLn2;
  int32_t status = GTP_ROW_OK;
  if (rl.s != rl.s || rl.m == kPosInf) status = GTP_ROW_NONFINITE;
  else if (sm.flags & 2u) status = GTP_ROW_BAD_HISTORY;
  else if (!(u >= 0.0f && u < 1.0f)) status = GTP_ROW_BAD_UNIFORM;
  if (status != GTP_ROW_OK) {
    if (tid == 0) write_row(a, b, status, -1, 0.f, 0.f, 0, 0.f, -1);
    return true;
  }
  if (sm.flags & 1u) return false;

  // ---- 5. m, weights and the block scan
  const int hi = kBins - 1 - kPer * tid, lo = hi - (kPer - 1);
  uint32_t cu[kPer / 2], cp[kPer / 2];
#pragma unroll
  for (int i = 0; i < kPer / 2; ++i) {
    cu[i] = sm.cnt[(lo >> 1) + i];
    cp[i] = sm.pcnt[(lo >> 1) + i];
  }
  // count of bin hi - i
  auto cnt_u = [&](int i) -> uint32_t { return (cu[kPer / 2 - 1 - (i >> 1)] >> ((i & 1) ? 0 : 16)) & 0xFFFFu; };
  auto cnt_p = [&](int i) -> uint32_t { return (cp[kPer / 2 - 1 - (i >> 1)] >> ((i & 1) ? 0 : 16)) & 0xFFFFu; };
  uint32_t mk = 0u;  // ord32 key of the largest processed logit (0: none)
  bool bad_y = false;
#pragma unroll
  for (int i = kPer - 1; i >= 0; --i) {
    if (cnt_u(i)) mk = ord32(r.ybin(hi - i));
  }
  {
    float yp = kNegInf;
    bool any = false;
#pragma unroll
    for (int i = kPer - 1; i >= 0; --i) {
      if (cnt_p(i)) {
        yp = r.ypen(hi - i);
        any = true;
      }
    }
    if (any) {
      if (!(yp > kNegInf && yp < kPosInf)) bad_y = true;
      else mk = ord32(yp) > mk ? ord32(yp) : mk;
    }
  }
  const int zero_owner = (kBins - 1 - kBins / 2) / kPer;
  const uint32_t zt = sm.zc + sm.pz;
  if (tid == zero_owner && zt) mk = ord32(0.0f) > mk ? ord32(0.0f) : mk;
  if (bad_y) atomicOr(&sm.flags, 1u);
  mk = block_max_u32(sm, mk);
  if (sm.flags & 1u) return false;
  if (mk == 0u) {
    if (tid == 0) write_row(a, b, GTP_ROW_EMPTY, -1, 0.f, 0.f, 0, 0.f, -1);
    return true;
  }
  const float m = unord32(mk);
  unsigned long long Wt = 0ull;
  uint32_t Nt = 0u;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const uint32_t c = cnt_u(i);
    if (c) {
      Wt += (unsigned long long)c * detexp_fix(r.ybin(hi - i) - m);
      Nt += c;
    }
  }
  // penalised raw bins whose y lies in this thread's range: ceil_bin(ypen(p))
  // in [lo, hi], i.e. ybin(lo - 1) < ypen(p) <= ybin(hi); ypen grows with p
  int pl = 0, ph = -1;
  if (r.use_pen) {
    const float ylo = lo > 0 ? r.ybin(lo - 1) : kNegInf, yhi = r.ybin(hi);
    int a0 = 0, a1 = kBins;  // first p with ypen(p) > ylo
    while (a0 < a1) {
      const int mid = (a0 + a1) >> 1;
      if (r.ypen(mid) > ylo) a1 = mid;
      else a0 = mid + 1;
    }
    int b0 = 0, b1 = kBins;  // first p with ypen(p) > yhi
    while (b0 < b1) {
      const int mid = (b0 + b1) >> 1;
      if (r.ypen(mid) > yhi) b1 = mid;
      else b0 = mid + 1;
    }
    pl = a0;
    ph = b0 - 1;
    for (int p = pl; p <= ph; ++p) {
      const uint32_t c = count16(sm.pcnt, p);
      if (c) {
        Wt += (unsigned long long)c * detexp_fix(r.ypen(p) - m);
        Nt += c;
      }
    }
  }
  if (tid == zero_owner && zt) {
    Wt += (unsigned long long)zt * detexp_fix(0.0f - m);
    Nt += zt;
  }
  unsigned long long ew, W;
  uint32_t ec, N;
  block_scan2(sm, Wt, Nt, ew, ec, W, N);
  // every counted token has an owner (no count overflowed 16 bits, no
  // penalised value above the bins)
  if (N != sm.n_counted + zt) return false;

  // ---- 6. the cut: the thread whose range holds floor(P W)
  const unsigned long long F = floor_mul(a.P, W);
  if (ew <= F && F < ew + Wt) {
    sm.owner[0] = tid;
    sm.o_ew[0] = ew;
    sm.o_ec[0] = ec;
    sm.o_pl[0] = pl;
    sm.o_ph[0] = ph;
  }
  __syncthreads();
  if (wid == 0) {
    Level L;
    const bool ok = sm.owner[0] >= 0 &&
                    resolve_range<kMask>(sm, r, sm.owner[0], m, F, sm.o_ew[0], sm.o_ec[0],
                                         sm.o_pl[0], sm.o_ph[0], L);
    if (lane == 0) {
      sm.lv[0] = L;
      sm.bad = ok && !(L.pbin >= 0 && L.zero_p) ? 0 : 1;
    }
  }
  __syncthreads();
  if (sm.bad) return false;
  const Level L0 = sm.lv[0];
  const uint32_t R = L0.n_before + L0.k + 1u;
  const unsigned long long Wp = L0.s_before + (unsigned long long)(L0.k + 1u) * L0.w;

  // ---- 7. the draw: floor(u W') among the kept tokens
  const unsigned long long U = floor_mul(u, Wp);
  if (ew <= U && U < ew + Wt) {
    sm.owner[1] = tid;
    sm.o_ew[1] = ew;
    sm.o_ec[1] = ec;
    sm.o_pl[1] = pl;
    sm.o_ph[1] = ph;
  }
  __syncthreads();
  if (wid == 0) {
    Level L;
    const bool ok = sm.owner[1] >= 0 &&
                    resolve_range<kMask>(sm, r, sm.owner[1], m, U, sm.o_ew[1], sm.o_ec[1],
                                         sm.o_pl[1], sm.o_ph[1], L);
    if (lane == 0) {
      sm.lv[1] = L;
      sm.bad = ok && !(L.pbin >= 0 && L.zero_p) ? 0 : 1;
    }
  }
  __syncthreads();
  if (sm.bad) return false;
  const Level L1 = sm.lv[1];

  // ---- 8. ids: from the pool when it holds both values, else a rescan
  if (level_in_pool<kMask>(sm, r, L0, theta) && level_in_pool<kMask>(sm, r, L1, theta)) {
    uint32_t* bm0 = sm.cnt;   // id bitmaps of the two levels (the counts are no longer needed)
    uint32_t* bm1 = sm.pcnt;
    for (int i = tid; i < kBins / 2; i += kB) {
      bm0[i] = 0u;
      bm1[i] = 0u;
    }
    __syncthreads();
    const uint32_t np = sm.pool_n < (uint32_t)kPool ? sm.pool_n : (uint32_t)kPool;
    for (uint32_t s2 = tid; s2 < np; s2 += kB) {
      const uint32_t q = sm.qid[s2], h = sm.qh[s2];
      const uint32_t id = q & 0x7FFFFFFFu;
      const bool pn = q >> 31;
      if (level_has(L0, pn, h)) atomicOr(&bm0[id >> 5], 1u << (id & 31));
      if (level_has(L1, pn, h)) atomicOr(&bm1[id >> 5], 1u << (id & 31));
    }
    __syncthreads();
    // thread t: words 8t .. 8t + 7 of each bitmap
    uint32_t w0[8], w1[8], p0 = 0u, p1 = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      w0[i] = bm0[8 * tid + i];
      w1[i] = bm1[8 * tid + i];
      p0 += __builtin_popcount(w0[i]);
      p1 += __builtin_popcount(w1[i]);
    }
    unsigned long long e0, t0;
    uint32_t e1, t1;
    block_scan2(sm, p0, p1, e0, e1, t0, t1);
    if (t0 != L0.n || t1 != L1.n) return false;
    // the k-th set bit of this thread's 8 words (unrolled: no indexed registers)
    auto find = [&](const uint32_t(&wv)[8], uint32_t k) -> int32_t {
      int32_t id = -1;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t pc = __builtin_popcount(wv[i]);
        if (id < 0 && k < pc) {
          uint32_t x = wv[i];
          for (uint32_t j = 0; j < k; ++j) x &= x - 1u;
          id = (int32_t)((8 * tid + i) * 32 + __builtin_ctz(x));
        }
        k = id < 0 ? k - pc : k;
      }
      return id;
    };
    if (e0 <= L0.k && L0.k < e0 + p0) sm.id_out[0] = find(w0, (uint32_t)(L0.k - e0));
    if (e1 <= L1.k && L1.k < e1 + p1) sm.id_out[1] = find(w1, L1.k - e1);
    __syncthreads();
  } else {
    rescan_ids<kMask>(sm, r);
  }

  // ---- 9. outputs
  if (tid == 0) {
    const int32_t id_thr = sm.id_out[0], id_draw = sm.id_out[1];
    const bool dp = r.use_pen && ((sm.pen[id_draw >> 5] >> (id_draw & 31)) & 1u);
    const int32_t bn = dp ? L1.pbin : L1.ubin;
    const float x_draw = bn >= 0 ? bin_x(bn) : 0.0f;
    const float slp = __builtin_amdgcn_logf((float)((double)L1.w / (double)Wp)) * kLn2;
    write_row(a, b, GTP_ROW_OK, id_draw, raw_logprob(x_draw, lse_m, lse_ln), slp, (int32_t)R,
              L0.y, id_thr);
  }
  return true;
}

}  // namespace topp

// One row per workgroup.  A row outside the top-p path's bounds is handed
// over: its index goes to handover[1 + n] with n = handover[0]++, and
// sampler_handover_kernel, launched right after on the same stream, runs the
// row-wise path for the listed rows and returns handover[0] to zero.  The
// row-wise path's registers thus never weigh on this kernel.
template <bool kMask>
__global__ __launch_bounds__(topp::kB) void sampler_topp_kernel(SamplerArgs a,
                                                                uint32_t* __restrict__ handover) {
  __shared__ topp::Smem sm;
  const int64_t b = blockIdx.x;
  if (!topp::topp_row<kMask>(a, b, sm) && threadIdx.x == 0)
    handover[1 + atomicAdd(handover, 1u)] = (uint32_t)b;
}

}  // namespace gtp
