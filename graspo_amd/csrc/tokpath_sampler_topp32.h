// tokpath_sampler_topp32.h -- the top-p sampler for fp32 rows (gfx950).
//
// Serves sampling rows with top-p active (0 < P < 1) and no top-k on
// 16-byte aligned fp32 rows of 65536 <= V <= 2^18: the reference's decode
// step _next_token_from_logits(logits.float(), temperature, top_p)
// (src/graspo/backends/graspoflow/tensor_utils.py:649-683) whether or not
// the values are bf16 values, with the repetition penalty and the allow mask
// of the contract in include/graspo_tokpath.h, bit for bit.  One workgroup of
// 1024 threads per row reads the row twice.
//
// The fixed-point weights DETEXP_FIX(y - m) of distinct fp32 values differ,
// so the total W needs every token's weight, and m (the largest y) is known
// only after a full read: two reads are the least an exact fp32 top-p needs.
//
// 0. Pilot.  The largest allowed x' of each wave's first chunk (16 evenly
//    spaced places of the row) gives r0 = that / T + 1/2.
// 1. Read 1.  Per token: the largest allowed x' (m = that / T exactly:
//    division by T is monotone), the raw maximum, the non-finite flag and the
//    raw sum of exponentials for the log-softmax; allowed tokens with
//    ya = x' * (1/T) >= r0 go to a top list (x', id) -- a few tokens for most
//    rows -- the others are counted in 2048 bins of width 1/64 in ya below
//    r0, the last bin open below (its weights are zero).  ya is within
//    3 * 2^-24 |y| of y and monotone in x', so a bin is an interval of x'.
// 2. Candidate bins.  With m known, each bin's weight lies within
//    count * e^(edges - m); the top list's weights are exact.  The smallest
//    prefix of bins whose lower bound exceeds P times the upper bound of W
//    holds the top-p cut (and so the draw) for certain; one more bin is
//    taken so that the group at the cut always has its lower neighbour.
//    The candidate bins get slot ranges in an LDS array (a counting sort).
// 3. Read 2 (chunks in reverse order, the most recently read first): W as
//    the sum of every allowed token's weight (DETEXP_FIX in fp64: exact, and
//    exact sums below 2^53 per thread), and each candidate (y, id) into its
//    bin's slot range with the bin's exact weight.
// 4. Cut and draw.  The group (top list or bin) whose weight interval holds
//    floor(P W) is ranked exactly by (y desc, id asc), then floor(u W') the
//    same.  Equal y of different x' can straddle a bin edge: the group's y
//    range must lie strictly between its neighbours' (|y| < 2^15 keeps one
//    fp32 step of y below half a bin, so a tie can only meet a neighbour).
// Outside these bounds (a NaN or +inf in the row, y = +inf, |y| >= 2^15, a
// top list or candidate set beyond its capacity, a tie across a group edge,
// a group of more than 1024 tokens at the cut) the row is handed over to the
// row-wise path, a block-uniform decision taken before any output of the row
// is written.
#pragma once

namespace gtp {
namespace tp32 {

constexpr int kB = 1024;              // threads per row
constexpr int kW = kB / kWave;        // waves per row
constexpr int kG = 4;                 // 16-byte vectors (4 tokens) per lane per chunk
constexpr int kChunk = kWave * kG;    // vectors per chunk (1024 tokens, 32 mask words)
constexpr int kNB = 2048;             // bins below r0
constexpr float kS = 64.0f;           // bins per unit of y
constexpr int kCap = 8192;            // candidate slots (the top list first)
constexpr int kTopCap = 512;          // top list
constexpr float kDelta = 0.5f;        // r0 above the sample's largest y
constexpr int kRankMax = 1024;        // largest group ranked at the cut or the draw
constexpr float kYMax = 32768.0f;     // |m|, |r0| below this
constexpr int64_t kMinV = 65536;
constexpr int kPenWords = GTP_SAMPLER_MAX_V / 32;

struct alignas(16) Smem {
  uint32_t cnt[kNB + kWave];      // read 1: tokens per bin (then a spare word per lane); then slot ends
  union {
    double wsum[kNB];                // read 2: candidate bins' weights (exact integers below 2^53)
    unsigned long long wpre[kNB];    // then the weight before each bin
  };
  float cy[kCap];                 // candidates: y (the top list: x' until converted)
  uint32_t cid[kCap];             // ... and id
  unsigned long long rw[kRankMax];  // weights of a ranked group
  uint32_t pen[kPenWords];        // penalised ids
  unsigned long long red_w[kW];
  double red_d[kW][2];
  float red_f[kW][4];
  uint32_t red_u[kW][2];
  unsigned long long w_top;       // exact weight of the top list
  unsigned long long total;       // ... plus the candidate bins'
  // the group at a weight position (search), then the token found in it
  int32_t g_v, g_s0, g_n;
  uint32_t g_nbefore;
  unsigned long long g_base;
  uint32_t t_min, t_max, t_prev, t_next;  // tie check (ord32 keys)
  int32_t res_id[2];
  float res_y[2];
  uint32_t res_r[2];              // tokens before the found one
  unsigned long long res_s[2];    // weight before it
  unsigned long long res_w[2];    // its weight
  uint32_t top_n, ctr, flags, fin;
  uint32_t nc;                    // candidates
  int32_t vth;                    // last candidate bin
  float u;
};

// 4 allow (or penalty) bits of vector k of a chunk for this lane, from the
// chunk's 32 words held one per lane (lanes 32..63 repeat them)
__device__ __forceinline__ uint32_t nibble(uint32_t sw, int k, int lane) {
  const uint32_t w = (uint32_t)__shfl((int)sw, k * (kWave / 8) + (lane >> 3), kWave);
  return (w >> ((lane & 7) * 4)) & 0xFu;
}

// DETEXP_FIX(d) for d in [-30.5, 0] as the fp64 value of the integer: the
// contract's fp32 steps to p and n, then p * 2^(n + 40) (exact in fp64)
// rounded to an integer, ties to even.  Equal to detexp_fix for every fp32 d
// in [-30, 0] and zero below (checked over all of them); callers clamp d at
// -30.5 (every weight below -30 is zero).
__device__ __forceinline__ double detexp_fix_f64(float d) {
  const float n = __builtin_rintf(d * 0x1.715476p+0f);
  float r = __builtin_fmaf(-n, 0x1.62e4p-1f, d);
  r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0x1p-1f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_rint(__builtin_ldexp((double)p, (int)n + 40));
}

__device__ __forceinline__ double shfl_up_f64(double v, int o) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const uint32_t lo = __shfl_up((uint32_t)u, o, kWave), hi = __shfl_up((uint32_t)(u >> 32), o, kWave);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double wave_scan_f64(double x) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const double v = shfl_up_f64(x, o);
    if (lane >= o) x += v;
  }
  return x;
}
__device__ __forceinline__ double lane63_f64(double v) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  return __builtin_bit_cast(double, lane63_u64(u));
}

// Block sum of a u64 (every thread gets it).
__device__ __forceinline__ unsigned long long block_sum_u64(Smem& sm, unsigned long long w) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const unsigned long long iw = wave_scan_u64(w);
  __syncthreads();
  if (lane == kWave - 1) sm.red_w[wid] = iw;
  __syncthreads();
  w = 0ull;
#pragma unroll
  for (int i = 0; i < kW; ++i) w += sm.red_w[i];
  return w;
}

// Rank the group of n tokens at candidate slots [s0, s0 + n) by (y desc,
// id asc) and find the one whose weight interval holds X - base (base: the
// weight before the group; X - base below the group's weight).  n <= 64:
// wave 0 alone; n <= kRankMax: the whole block.  The result goes to slot l
// of the res_* fields.
__device__ __forceinline__ void rank_group(Smem& sm, float m, int s0, int n, unsigned long long base,
                                           uint32_t nbefore, unsigned long long X, int l) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  if (n <= kWave) {
    if (tid < kWave) {
      const bool in = lane < n;
      const float y = in ? sm.cy[s0 + lane] : kNegInf;
      const uint32_t id = in ? sm.cid[s0 + lane] : 0u;
      const unsigned long long k = in ? rank_key(y, (int32_t)id) : 0ull;
      const unsigned long long w = in ? detexp_fix(y - m) : 0ull;
      unsigned long long s = 0ull;
      uint32_t r = 0u;
      for (int j = 0; j < n; ++j) {
        const unsigned long long kj =
            ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), j) << 32) |
            (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, j);
        const unsigned long long wj =
            ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(w >> 32), j) << 32) |
            (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)w, j);
        const bool before = kj > k;
        s += before ? wj : 0ull;
        r += before ? 1u : 0u;
      }
      if (in && base + s <= X && X < base + s + w) {
        sm.res_id[l] = (int32_t)id;
        sm.res_y[l] = y;
        sm.res_r[l] = nbefore + r;
        sm.res_s[l] = base + s;
        sm.res_w[l] = w;
      }
    }
    __syncthreads();
    return;
  }
  const bool in = tid < n;
  float y = kNegInf;
  uint32_t id = 0u;
  unsigned long long k = 0ull, w = 0ull;
  if (in) {
    y = sm.cy[s0 + tid];
    id = sm.cid[s0 + tid];
    k = rank_key(y, (int32_t)id);
    w = detexp_fix(y - m);
    sm.rw[tid] = w;
  }
  __syncthreads();
  unsigned long long s = 0ull;
  uint32_t r = 0u;
  if (in) {
    for (int j = 0; j < n; ++j) {
      const unsigned long long kj = rank_key(sm.cy[s0 + j], (int32_t)sm.cid[s0 + j]);
      const bool before = kj > k;
      s += before ? sm.rw[j] : 0ull;
      r += before ? 1u : 0u;
    }
    if (base + s <= X && X < base + s + w) {
      sm.res_id[l] = (int32_t)id;
      sm.res_y[l] = y;
      sm.res_r[l] = nbefore + r;
      sm.res_s[l] = base + s;
      sm.res_w[l] = w;
    }
  }
  __syncthreads();
}

// Slot range [s0, s0 + n) of group g: -1 the top list, v >= 0 candidate bin
// v (cnt[v] holds the end of bin v's slots after read 2).
__device__ __forceinline__ void group_range(const Smem& sm, int g, int& s0, int& n) {
  if (g < 0) {
    s0 = 0;
    n = (int)sm.top_n;
  } else {
    s0 = g ? (int)sm.cnt[g - 1] : (int)sm.top_n;
    n = (int)sm.cnt[g] - s0;
  }
}

// True when group g's y values lie strictly between those of its neighbours
// (g - 1 above, g + 1 below; the top list has no group above): then no tie
// in y crosses its edges and ranking it alone is exact.
__device__ __forceinline__ bool tie_free(Smem& sm, int g) {
  const int tid = threadIdx.x;
  if (tid == 0) {
    sm.t_min = 0xFFFFFFFFu;
    sm.t_max = 0u;
    sm.t_prev = 0xFFFFFFFFu;
    sm.t_next = 0u;
  }
  __syncthreads();
  int s0, n;
  group_range(sm, g, s0, n);
  uint32_t mn = 0xFFFFFFFFu, mx = 0u;
  for (int i = tid; i < n; i += kB) {
    const uint32_t k = ord32(sm.cy[s0 + i]);
    mn = k < mn ? k : mn;
    mx = k > mx ? k : mx;
  }
  if (tid < n) {  // (only threads that saw a token: no 1024-way atomic on one word)
    atomicMin(&sm.t_min, mn);
    atomicMax(&sm.t_max, mx);
  }
  if (g >= 0) {  // the group above: its smallest y
    int p0, pn;
    group_range(sm, g - 1, p0, pn);
    uint32_t pm = 0xFFFFFFFFu;
    for (int i = tid; i < pn; i += kB) {
      const uint32_t k = ord32(sm.cy[p0 + i]);
      pm = k < pm ? k : pm;
    }
    if (tid < pn) atomicMin(&sm.t_prev, pm);
  }
  {  // the group below: its largest y
    int q0, qn;
    group_range(sm, g + 1, q0, qn);
    uint32_t qm = 0u;
    for (int i = tid; i < qn; i += kB) {
      const uint32_t k = ord32(sm.cy[q0 + i]);
      qm = k > qm ? k : qm;
    }
    if (tid < qn) atomicMax(&sm.t_next, qm);
  }
  __syncthreads();
  const bool ok = sm.t_max < sm.t_prev && sm.t_min > sm.t_next;
  __syncthreads();
  return ok;
}

// The group whose weight interval holds X (wave 0; X below sm.total): the
// top list when X < w_top, else the last candidate bin v <= vth with
// prefix(v) <= X.  Writes g_* .
__device__ __forceinline__ void find_group(Smem& sm, unsigned long long X, int vth) {
  const int lane = threadIdx.x & (kWave - 1);
  int v = -1;
  if (X >= sm.w_top) {
    // wpre[v]: the weight before bin v (non-decreasing in v)
    const int p1 = lane * 32;
    const unsigned long long b1 = __ballot(p1 <= vth && sm.wpre[p1] <= X);
    const int base = (63 - __builtin_clzll(b1)) * 32;  // (bit 0 is set: wpre[0] = w_top <= X)
    const int p2 = base + (lane & 31);
    const unsigned long long b2 = __ballot(lane < 32 && p2 <= vth && sm.wpre[p2] <= X);
    v = base + (63 - __builtin_clzll(b2));
  }
  if (lane == 0) {
    int s0, n;
    group_range(sm, v, s0, n);
    sm.g_v = v;
    sm.g_s0 = s0;
    sm.g_n = n;
    sm.g_nbefore = (uint32_t)s0;
    sm.g_base = v < 0 ? 0ull : sm.wpre[v];
  }
}

// One row; false when the row must be handed over to the row-wise path (a
// block-uniform decision, taken before any output is written).
// kMode bit 0: repetition penalty; bit 1: allow mask.
template <int kMode>
__device__ __forceinline__ bool topp32_row(const SamplerArgs& a, int64_t b, Smem& sm) {
  constexpr bool kPen = (kMode & 1) != 0, kMask = (kMode & 2) != 0;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  const float* xr = reinterpret_cast<const float*>(a.logits) + b * a.row_stride;
  const u32x4* xv = reinterpret_cast<const u32x4*>(xr);
  const uint32_t* mrow = kMask ? a.mask + b * a.mask_stride : nullptr;
  const int64_t V = a.V;
  const uint32_t nvec = (uint32_t)(V / 4);  // whole vectors (the rest: the tail)
  const uint32_t nchunks = (nvec + kChunk - 1) / kChunk;
  const uint32_t per = nchunks / kW;
  const uint32_t last = nvec - 1u;
  const uint32_t last_word = (uint32_t)((V - 1) >> 5);
  const float Tc = a.T > 1e-6f ? a.T : 1e-6f;
  const float rT = 1.0f / Tc;
  const float bh = div_by_t_bound(Tc);
  const float rho = a.rho;
  // schedule index -> chunk: the first kW start kW evenly spaced regions
  auto perm = [&](uint32_t c) -> uint32_t { return c < per * kW ? (c % kW) * per + c / kW : c; };
  auto issue = [&](u32x4(&buf)[kG], uint32_t& sw, uint32_t pc, auto nt_c) {
    constexpr bool nt = decltype(nt_c)::value;
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      uint32_t vi = pc * kChunk + (uint32_t)(k * kWave + lane);
      vi = vi < last ? vi : last;
      buf[k] = nt ? __builtin_nontemporal_load(xv + vi) : xv[vi];
    }
    if (kMask) {
      const uint32_t w = pc * (kChunk * 4 / 32) + (uint32_t)(lane & 31);
      sw = mrow[w < last_word ? w : last_word];
    }
  };
  auto xpen = [&](float x, bool pn) -> float {
    float xp = x;
    if (kPen && pn) xp = x < 0.0f ? x * rho : x / rho;
    return xp;
  };

  // ---- first chunks in flight (read 1 keeps four per wave in flight: its
  // work per chunk is shorter than the memory latency), then the clear and
  // the history bitmap
  u32x4 qa[kG], qb[kG], qc[kG], qd[kG];
  uint32_t swa = 0xFFFFFFFFu, swb = 0xFFFFFFFFu, swc = 0xFFFFFFFFu, swd = 0xFFFFFFFFu;
  uint32_t ca = (uint32_t)wid, cb = (uint32_t)(kW + wid);
  // (with an allow mask, three: the mask words take the registers of a fourth)
  constexpr bool kFour = !kMask;
  uint32_t cc = (uint32_t)(2 * kW + wid), cd = kFour ? (uint32_t)(3 * kW + wid) : nchunks;
  using T_ = std::true_type;
  using F_ = std::false_type;
  if (ca < nchunks) issue(qa, swa, perm(ca), T_{});
  if (cb < nchunks) issue(qb, swb, perm(cb), T_{});
  if (cc < nchunks) issue(qc, swc, perm(cc), T_{});
  if (kFour && cd < nchunks) issue(qd, swd, perm(cd), T_{});
  for (int i = tid; i < kNB + kWave; i += kB) sm.cnt[i] = 0u;
  if (kPen)
    for (int64_t i = tid; i < (V + 31) / 32; i += kB) sm.pen[i] = 0u;
  if (tid == 0) {
    sm.u = a.uniforms[b];
    sm.fin = a.finished && a.finished[b];
    sm.top_n = 0u;
    sm.ctr = (kFour ? 4u : 3u) * kW;
    sm.flags = 0u;
    sm.vth = -2;
    sm.res_id[0] = sm.res_id[1] = -1;
  }
  __syncthreads();
  if (a.hist && a.hist_len > 0) {
    const int32_t* h = a.hist + b * a.hist_stride;
    bool bad_hist = false;
    for (int64_t j = tid; j < a.hist_len; j += kB) {
      const int32_t id = h[j];
      if (id >= V) bad_hist = true;
      else if (kPen && id >= 0) atomicOr(&sm.pen[id >> 5], 1u << (id & 31));
    }
    if (bad_hist) atomicOr(&sm.flags, 2u);
  }
  __syncthreads();

  // per vector k of a chunk: valid (a whole vector of the row), allow and
  // penalty bits
  auto bits = [&](uint32_t sw, uint32_t pc, int k, bool& valid, uint32_t& ab, uint32_t& pb,
                  bool partial = true) {
    const uint32_t vi = pc * kChunk + (uint32_t)(k * kWave + lane);
    valid = !partial || vi < nvec;
    ab = kMask ? nibble(sw, k, lane) : 0xFu;
    if (!valid) ab = 0u;
    pb = kPen ? (sm.pen[(vi < last ? vi : last) >> 3] >> ((vi & 7u) * 4u)) & 0xFu : 0u;
  };

  // ---- 0. pilot: the largest allowed x' and raw value of the first chunk
  float r0, nref;
  {
    float mx = kNegInf, mr = kNegInf;
    if (ca < nchunks) {
      const uint32_t pc = perm(ca);
#pragma unroll
      for (int k = 0; k < kG; ++k) {
        bool valid;
        uint32_t ab, pb;
        bits(swa, pc, k, valid, ab, pb);
        const uint32_t wd[4] = {qa[k].x, qa[k].y, qa[k].z, qa[k].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x = u2f(wd[j]);
          const float xp = xpen(x, (pb >> j) & 1u);
          if ((ab >> j) & 1u) mx = fmaxf(mx, xp);
          if (valid) mr = fmaxf(mr, x);
        }
      }
    }
    mx = wave_max_f(mx);
    mr = wave_max_f(mr);
    if (lane == 0) {
      sm.red_f[wid][0] = mx;
      sm.red_f[wid][1] = mr;
    }
    __syncthreads();
    mx = mr = kNegInf;
#pragma unroll
    for (int i = 0; i < kW; ++i) {
      mx = fmaxf(mx, sm.red_f[i][0]);
      mr = fmaxf(mr, sm.red_f[i][1]);
    }
    // (no allowed token in the sample: every token is binned at the bottom,
    // and the row is handed over after the read)
    r0 = mx == kNegInf ? kPosInf : mx / Tc + kDelta;
    nref = -(mr * kLog2e);  // the raw sum is taken relative to mr
  }
  // row constants in scalar registers
  auto sgpr = [](float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
  };
  r0 = sgpr(r0);
  nref = sgpr(nref);
  auto bin_of = [&](float ya) -> int {
    return (int)fminf(fmaxf((r0 - ya) * kS, 0.0f), (float)(kNB - 1));
  };
  // a chunk's kind: `partial` when it holds vectors past the row's end
  // (the last chunk of a row whose vectors do not fill it)
  const bool ragged = (nvec % kChunk) != 0;
  auto is_partial = [&](uint32_t pc) { return ragged && pc == nchunks - 1u; };

  // ---- 1. read 1: maxima, the flag, the raw sum, the top list, bin counts
  float mxp = kNegInf, rx = kNegInf, ls = 0.0f;
  bool nf = false;
  auto top_add = [&](bool c, float xp, uint32_t id) __attribute__((always_inline)) {
    const unsigned long long bal = __ballot(c);
    if (!bal) return;
    uint32_t base = 0u;
    if (lane == 0) base = atomicAdd(&sm.top_n, (uint32_t)__builtin_popcountll(bal));
    base = (uint32_t)__builtin_amdgcn_readlane((int)base, 0);
    if (c) {
      const uint32_t slot =
          base + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
      if (slot < (uint32_t)kTopCap) {
        sm.cy[slot] = xp;
        sm.cid[slot] = id;
      }
    }
  };
  // one token: the maxima, the flag and the raw sum; its bin count (tokens
  // that are not counted go to the lane's own spare word, so masked tokens
  // meet no bank conflict); `anyt`: an allowed token at or above r0
  auto tok1 = [&](float x, bool valid, bool al, bool pn, bool& anyt) __attribute__((always_inline)) {
    nf = nf || (valid && !(x < kPosInf));
    rx = valid ? fmaxf(rx, x) : rx;
    ls += valid ? __builtin_amdgcn_exp2f(__builtin_fmaf(x, kLog2e, nref)) : 0.0f;
    const float xp = xpen(x, pn);
    mxp = al ? fmaxf(mxp, xp) : mxp;
    const float ya = xp * rT;
    const bool top = ya >= r0;
    anyt = anyt || (al && top);
    atomicAdd(&sm.cnt[al && !top ? bin_of(ya) : kNB + lane], 1u);
  };
  auto work1 = [&](const u32x4(&buf)[kG], uint32_t sw, uint32_t pc, auto partial_c)
                   __attribute__((always_inline)) {
    constexpr bool partial = decltype(partial_c)::value;
    bool anyt = false;
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      bool valid;
      uint32_t ab, pb;
      bits(sw, pc, k, valid, ab, pb, partial);
      const uint32_t wd[4] = {buf[k].x, buf[k].y, buf[k].z, buf[k].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) tok1(u2f(wd[j]), valid, (ab >> j) & 1u, (pb >> j) & 1u, anyt);
    }
    if (__ballot(anyt)) {  // (rare) the chunk's top tokens to the top list
#pragma unroll 1
      for (int k = 0; k < kG; ++k) {
        bool valid;
        uint32_t ab, pb;
        bits(sw, pc, k, valid, ab, pb);
        const uint32_t vi = pc * kChunk + (uint32_t)(k * kWave + lane);
        const uint32_t wd[4] = {buf[k].x, buf[k].y, buf[k].z, buf[k].w};
        for (int j = 0; j < 4; ++j) {
          const float xp = xpen(u2f(wd[j]), (pb >> j) & 1u);
          top_add(((ab >> j) & 1u) && xp * rT >= r0, xp, vi * 4u + (uint32_t)j);
        }
      }
    }
  };
  auto run1 = [&](const u32x4(&buf)[kG], uint32_t sw, uint32_t pc) __attribute__((always_inline)) {
    if (is_partial(pc)) work1(buf, sw, pc, T_{});
    else work1(buf, sw, pc, F_{});
  };
  auto grab = [&]() -> uint32_t {
    uint32_t c = 0;
    if (lane == 0) c = atomicAdd(&sm.ctr, 1u);
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)c);
  };
  // a ring of four buffers: each is refilled right after its chunk is done
  // (the schedule hands out increasing indices, so a buffer past the row's
  // end can precede others that still hold chunks)
  while (ca < nchunks || cb < nchunks || cc < nchunks || cd < nchunks) {
    if (ca < nchunks) {
      run1(qa, swa, perm(ca));
      ca = grab();
      if (ca < nchunks) issue(qa, swa, perm(ca), T_{});
    }
    if (cb < nchunks) {
      run1(qb, swb, perm(cb));
      cb = grab();
      if (cb < nchunks) issue(qb, swb, perm(cb), T_{});
    }
    if (cc < nchunks) {
      run1(qc, swc, perm(cc));
      cc = grab();
      if (cc < nchunks) issue(qc, swc, perm(cc), T_{});
    }
    if (kFour && cd < nchunks) {
      run1(qd, swd, perm(cd));
      cd = grab();
      if (cd < nchunks) issue(qd, swd, perm(cd), T_{});
    }
  }
  // tail tokens (V not a multiple of 4): lane 0 of wave 0
  const int ntail = (int)(V - (int64_t)nvec * 4);
  auto tail_token = [&](int j, float& x, bool& in, bool& al, bool& pn) {
    const uint32_t id = nvec * 4u + (uint32_t)j;
    in = lane == 0 && j < ntail;
    x = in ? xr[id] : kNegInf;
    al = in && (!kMask || ((mrow[id >> 5] >> (id & 31u)) & 1u));
    pn = kPen && in && ((sm.pen[id >> 5] >> (id & 31u)) & 1u);
  };
  if (ntail > 0 && wid == 0) {
    bool anyt = false;
    for (int j = 0; j < ntail; ++j) {
      float x;
      bool in, al, pn;
      tail_token(j, x, in, al, pn);
      tok1(x, in, al, pn, anyt);
    }
    for (int j = 0; j < ntail; ++j) {
      float x;
      bool in, al, pn;
      tail_token(j, x, in, al, pn);
      const float xp = xpen(x, pn);
      top_add(al && xp * rT >= r0, xp, nvec * 4u + (uint32_t)j);
    }
  }
  // the reductions
  {
    const float a1 = wave_max_f(mxp), a2 = wave_max_f(rx), a3 = wave_sum_f(ls);
    const bool f = __ballot(nf) != 0ull;
    if (lane == 0) {
      sm.red_f[wid][0] = a1;
      sm.red_f[wid][1] = a2;
      sm.red_f[wid][2] = a3;
      sm.red_u[wid][0] = f ? 1u : 0u;
    }
    __syncthreads();
    if (tid == 0) sm.ctr = 2u * kW;  // (read 2's chunk counter: every wave has left read 1)
    mxp = rx = kNegInf;
    ls = 0.0f;
    nf = false;
#pragma unroll
    for (int i = 0; i < kW; ++i) {
      mxp = fmaxf(mxp, sm.red_f[i][0]);
      rx = fmaxf(rx, sm.red_f[i][1]);
      ls += sm.red_f[i][2];
      nf = nf || sm.red_u[i][0] != 0u;
    }
  }
  if (nf) return false;  // NaN or +inf: the row-wise path writes the status
  const float u = sm.u;
  int32_t status = GTP_ROW_OK;
  if (sm.flags & 2u) status = GTP_ROW_BAD_HISTORY;
  else if (!(u >= 0.0f && u < 1.0f)) status = GTP_ROW_BAD_UNIFORM;
  else if (mxp == kNegInf) status = GTP_ROW_EMPTY;
  if (status != GTP_ROW_OK) {
    if (tid == 0) write_row_f(a, b, sm.fin != 0u, status, -1, 0.f, 0.f, 0, 0.f, -1);
    return true;
  }
  const float m = sgpr(mxp / Tc + 0.0f);  // the largest y: division by T is monotone
  if (!(fabsf(m) < kYMax && fabsf(r0) < kYMax)) return false;
  const uint32_t n_top = sm.top_n;
  if (n_top > (uint32_t)kTopCap) return false;
  // the raw log-sum-exp relative to the pilot's raw maximum; taken again in
  // read 2 (relative to the row's) if that overflowed
  const bool raw_again = __builtin_amdgcn_readfirstlane(!(ls < kPosInf && ls > 0.0f) ? 1 : 0) != 0;
  rx = sgpr(rx);
  const float raw_m = raw_again ? rx : -nref * kLn2;

  // ---- 2. candidate bins
  {
    unsigned long long wt = 0ull;
    for (uint32_t i = tid; i < n_top; i += kB) {
      const float y = sm.cy[i] / Tc + 0.0f;  // (x' -> y in place)
      sm.cy[i] = y;
      wt += detexp_fix(y - m);
    }
    wt = block_sum_u64(sm, wt);
    // bin v holds r0 - ya in [v / 64 - e, (v + 1) / 64 + e] (e bounds the
    // rounding of r0 - ya and |y - ya| <= 3 * 2^-24 |y|); its tokens weigh
    // c e^(y - m) within 1e-5 plus 2^-41 each (DETEXP_FIX's polynomial and
    // rounding; fp32 exponentials); zero below m - 30
    const float e = 4e-6f + 2e-7f * (fabsf(r0) + 33.0f);
    const float rm = r0 - m;  // (exact enough: both below 2^15, e covers it)
    float lo2 = 0.0f, hi2 = 0.0f;
    uint32_t c2 = 0u;
    float lo_own[2];
    uint32_t c_own[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int v = 2 * tid + q;
      const uint32_t c = sm.cnt[v];
      float lo = 0.0f, hi = 0.0f;
      if (c) {
        const float t = 0x1p-40f;
        const float dhi = rm - (float)v / kS + e;
        const float dlo = v == kNB - 1 ? -1e30f : rm - (float)(v + 1) / kS - e - 1e-6f;
        hi = dhi < -30.0f ? 0.0f
                          : (float)c * (__expf(fminf(dhi + 1e-6f, 0.0f)) * (1.0f + 1e-5f) + t);
        lo = dlo < -30.0f ? 0.0f : (float)c * (__expf(dlo) * (1.0f - 1e-5f) - t);
        lo = lo > 0.0f ? lo : 0.0f;
      }
      lo_own[q] = lo;
      c_own[q] = c;
      lo2 += lo;
      hi2 += hi;
      c2 += c;
    }
    // block scans of (count, lower bound) in bin order and the sum of the
    // upper bounds (fp64 sums)
    const double ilo = wave_scan_f64((double)lo2);
    const uint32_t ic = wave_scan_u32(c2);
    const double shi = lane63_f64(wave_scan_f64((double)hi2));
    __syncthreads();
    if (lane == kWave - 1) {
      sm.red_d[wid][0] = ilo;
      sm.red_d[wid][1] = shi;
      sm.red_u[wid][0] = ic;
    }
    if (tid == 0) sm.w_top = wt;
    __syncthreads();
    double blo = 0.0, hi_all = 0.0;
    uint32_t bc = 0u;
#pragma unroll
    for (int i = 0; i < kW; ++i) {
      if (i < wid) {
        blo += sm.red_d[i][0];
        bc += sm.red_u[i][0];
      }
      hi_all += sm.red_d[i][1];
    }
    const double wtop = (double)wt * 0x1p-40;
    // (fp32 terms summed in fp64: 1e-5 of margin covers their rounding)
    const double target = (double)a.P * (wtop + hi_all * (1.0 + 1e-5)) * (1.0 + 1e-9);
    double acc = wtop + (blo + ilo - (double)lo2) * (1.0 - 1e-5);  // lower bound before my bins
    uint32_t cbefore = bc + ic - c2;  // tokens in the bins before mine
    // the crossing bin, plus one (the cut's group has its lower neighbour)
    if (tid == 0 && wtop > target) {
      sm.vth = 0;
      sm.nc = n_top + sm.cnt[0];
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const double prev = acc;
      acc += (double)lo_own[q] * (1.0 - 1e-5);
      const int v = 2 * tid + q;
      if (!(wtop > target) && prev <= target && acc > target) {
        sm.vth = v + 1;
        sm.nc = n_top + cbefore + c_own[q] + (v + 1 < kNB ? sm.cnt[v + 1] : 0u);
      }
      cbefore += c_own[q];
    }
    __syncthreads();
    const int vth = sm.vth;
    if (vth < 0 || vth >= kNB - 1 || sm.nc > (uint32_t)kCap) return false;
    // slot offsets of the candidate bins, their weights zeroed
    uint32_t s = n_top + bc + ic - c2;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int v = 2 * tid + q;
      if (v <= vth) {
        sm.cnt[v] = s;
        sm.wsum[v] = 0.0;
      }
      s += c_own[q];
    }
    __syncthreads();
  }
  const int vth = __builtin_amdgcn_readfirstlane(sm.vth);
  // read 2's candidate pre-test: ya at or above t_lo holds every candidate
  // bin (bin_of(ya) <= vth needs r0 - ya < (vth + 1) / 64 within rounding)
  const float t_lo = r0 - (float)(vth + 1) / kS - 1e-3f;
  const float t_lo_y = sgpr(t_lo - 1e-3f - 2e-7f * (fabsf(r0) + 33.0f));

  // ---- 3. read 2: W, the candidates (and the raw sum if read 1's overflowed)
  double wacc = 0.0;
  float ls2 = 0.0f;
  auto tok2 = [&](float x, uint32_t id, bool valid, bool al, bool pn) __attribute__((always_inline)) {
    if (raw_again) ls2 += valid ? __builtin_amdgcn_exp2f((x - rx) * kLog2e) : 0.0f;
    const float xp = xpen(x, pn);
    const float y = div_by_t(xp, Tc, rT, bh);  // xp / Tc (-0 is canonicalised where it is stored)
    const float d = fmaxf(al ? y - m : -100.0f, -30.5f);
    const double w = detexp_fix_f64(d);
    wacc += w;
    // candidates have ya >= t_lo, so y >= t_lo_y (|y - ya| <= 3 * 2^-24 |y|)
    if (al && y >= t_lo_y) {  // (few tokens: the candidate bins)
      const float ya = xp * rT;
      const int v = bin_of(ya);
      if (ya < r0 && v <= vth) {
        const uint32_t slot = atomicAdd(&sm.cnt[v], 1u);
        sm.cy[slot] = y + 0.0f;
        sm.cid[slot] = id;
        atomicAdd(&sm.wsum[v], w);
      }
    }
  };
  auto work2 = [&](const u32x4(&buf)[kG], uint32_t sw, uint32_t pc, auto partial_c)
                   __attribute__((always_inline)) {
    constexpr bool partial = decltype(partial_c)::value;
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      bool valid;
      uint32_t ab, pb;
      bits(sw, pc, k, valid, ab, pb, partial);
      const uint32_t vi = pc * kChunk + (uint32_t)(k * kWave + lane);
      const uint32_t wd[4] = {buf[k].x, buf[k].y, buf[k].z, buf[k].w};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        tok2(u2f(wd[j]), vi * 4u + (uint32_t)j, valid, (ab >> j) & 1u, (pb >> j) & 1u);
    }
  };
  auto run2 = [&](const u32x4(&buf)[kG], uint32_t sw, uint32_t pc) __attribute__((always_inline)) {
    if (is_partial(pc)) work2(buf, sw, pc, T_{});
    else work2(buf, sw, pc, F_{});
  };
  {
    // chunks in reverse order: the last ones read come first
    auto rev = [&](uint32_t c) { return nchunks - 1u - c; };
    ca = (uint32_t)wid;
    cb = (uint32_t)(kW + wid);
    if (ca < nchunks) issue(qa, swa, rev(ca), T_{});
    if (cb < nchunks) issue(qb, swb, rev(cb), T_{});
    if (ca < nchunks) run2(qa, swa, rev(ca));
    while (true) {
      if (cb >= nchunks) break;
      ca = grab();
      if (ca < nchunks) issue(qa, swa, rev(ca), T_{});
      run2(qb, swb, rev(cb));
      if (ca >= nchunks) break;
      cb = grab();
      if (cb < nchunks) issue(qb, swb, rev(cb), T_{});
      run2(qa, swa, rev(ca));
    }
    if (ntail > 0 && wid == 0) {
      for (int j = 0; j < ntail; ++j) {
        float x;
        bool in, al, pn;
        tail_token(j, x, in, al, pn);
        tok2(x, nvec * 4u + (uint32_t)j, in, al, pn);
      }
    }
  }
  // (a thread's sum of at most 256 weights below 2^41 is an exact fp64 integer)
  const unsigned long long W = block_sum_u64(sm, (unsigned long long)wacc);
  float lse_m = raw_m, lse_s = ls;
  if (raw_again) {
    const float s2 = wave_sum_f(ls2);
    if (lane == 0) sm.red_f[wid][3] = s2;
    __syncthreads();
    lse_s = 0.0f;
#pragma unroll
    for (int i = 0; i < kW; ++i) lse_s += sm.red_f[i][3];
  }
  const float lse_ln = __builtin_amdgcn_logf(lse_s) * kLn2;

  // ---- 4. prefixes of the candidate bins, then the cut and the draw
  {
    unsigned long long w0 = 0ull, w1 = 0ull;
    if (2 * tid <= vth) w0 = (unsigned long long)sm.wsum[2 * tid];
    if (2 * tid + 1 <= vth) w1 = (unsigned long long)sm.wsum[2 * tid + 1];
    const unsigned long long own = w0 + w1;
    const unsigned long long iw = wave_scan_u64(own);
    __syncthreads();
    if (lane == kWave - 1) sm.red_w[wid] = iw;
    __syncthreads();
    unsigned long long bw = 0ull, all = 0ull;
#pragma unroll
    for (int i = 0; i < kW; ++i) {
      if (i < wid) bw += sm.red_w[i];
      all += sm.red_w[i];
    }
    const unsigned long long ex = sm.w_top + bw + iw - own;
    if (2 * tid <= vth) sm.wpre[2 * tid] = ex;
    if (2 * tid + 1 <= vth) sm.wpre[2 * tid + 1] = ex + w0;
    if (tid == 0) sm.total = sm.w_top + all;
    __syncthreads();
  }
  for (int l = 0; l < 2; ++l) {
    // the cut at floor(P W), then the draw at floor(u W')
    const unsigned long long X =
        l == 0 ? floor_mul(a.P, W) : floor_mul(u, sm.res_s[0] + sm.res_w[0]);
    if (X >= sm.total) return false;  // (the bounds make this impossible)
    if (wid == 0) find_group(sm, X, vth);
    __syncthreads();
    const int g = sm.g_v, n = sm.g_n;
    if (g >= vth || n > kRankMax || !tie_free(sm, g)) return false;
    rank_group(sm, m, sm.g_s0, n, sm.g_base, sm.g_nbefore, X, l);
    if (sm.res_id[l] < 0) return false;
  }
  if (tid == 0) {
    const unsigned long long Wp = sm.res_s[0] + sm.res_w[0];
    const int32_t id_draw = sm.res_id[1];
    const float slp = __builtin_amdgcn_logf((float)((double)sm.res_w[1] / (double)Wp)) * kLn2;
    write_row_f(a, b, sm.fin != 0u, GTP_ROW_OK, id_draw, raw_logprob(xr[id_draw], lse_m, lse_ln), slp,
                (int32_t)(sm.res_r[0] + 1u), sm.res_y[0], sm.res_id[0]);
  }
  return true;
}

}  // namespace tp32

// One row per workgroup; a row outside the fp32 top-p path's bounds
// (topp32_row returns false, the same in every thread, before any output is
// written) runs the row-wise path in the same workgroup and LDS, so the call
// is one launch.
// kMode bit 0: repetition penalty active; bit 1: allow mask.
template <int kMode>
__global__ __launch_bounds__(tp32::kB) void sampler_topp32_kernel(SamplerArgs a) {
  __shared__ union {
    tp32::Smem t;
    SamplerSmem g;
  } smu;
  const int64_t b = blockIdx.x;
  if (!tp32::topp32_row<kMode>(a, b, smu.t)) {
    __syncthreads();  // every thread is done with the top-p state
    rowwise_row<float>(a, b, smu.g);
  }
}

}  // namespace gtp
