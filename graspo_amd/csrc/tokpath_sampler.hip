// tokpath_sampler.hip -- the rollout sampler (gfx950).
//
// One workgroup of 1024 threads per row; the whole row state lives in LDS.
//
// Stream pass (the only HBM read of the row).  Each thread loads 8 groups of
// 8 logits per iteration (16-byte vectors) and, fused into the read:
//   * folds the raw row into an online log-sum-exp (for the logprob output;
//     a NaN or +inf anywhere poisons the sum and marks the row non-finite);
//   * stores for every group the bf16-rounded-up maximum of its allowed
//     logits as a 16-bit order key in LDS (an upper bound of every processed
//     logit of the group, since the repetition penalty only lowers values
//     when rho >= 1);
//   * keeps a per-thread lower bound: the max over its groups that hold no
//     penalised allowed token (there the processed logit equals the raw one).
//
// Candidate path (1 <= top_k <= 256, or greedy).  The K-th largest of the
// 1024 thread lower bounds (LDS radix select over 16-bit keys) is a value tau
// that at least K distinct tokens reach, so every token of the top-K has
// y >= y(tau).  Only groups whose upper-bound key passes are re-read (a few
// hundred bytes from L2/MALL); their tokens get the exact penalty and the
// exact IEEE division by the temperature and are ranked exactly by
// (y desc, id asc).  Fixed-point weights, top-p cut and the draw are then
// integer prefix sums over at most K entries.
//
// General path (top-p only, top_k > 256, rho < 1, or candidate overflow).
// Re-reads the row from L2/MALL: (A) exact max, (B) count and fixed-point
// weight histograms over 2048 bins of (m - y) * 64, (C) collect only the
// bins that can hold the top-k cut, the top-p cut and the draw, rank them
// exactly.  If those bins hold more than 2048 tokens (heavy exact ties) a
// weighted radix descent over the 64-bit (y, id) key resolves each cut with
// one re-read per 8-bit digit.
//
// Every path evaluates the same contract as include/graspo_tokpath.h; the
// selection strategy only decides which tokens are looked at exactly.
//
// Replaces _next_token_from_logits / _sample_next_token
// (src/graspo/backends/graspoflow/tensor_utils.py:649-683).
#include "tokpath_sampler_internal.h"

namespace gtp {

constexpr int kSB = 1024;           // threads per row
constexpr int kSW = kSB / kWave;    // waves per row
constexpr int kSG = 8;              // groups per thread per stream iteration
constexpr int kKFast = 256;         // largest top-k of the candidate path
constexpr int kCandCap = 1024;      // candidate slots (<= kSB: one per thread when ranking)
constexpr int kMaxGroups = GTP_SAMPLER_MAX_V / 8;
constexpr int kPenWords = GTP_SAMPLER_MAX_V / 32;
constexpr int kNB = 2048;           // general-path bins
constexpr float kBinScale = 64.0f;  // bins per nat
constexpr int kCollectCap = 2048;


struct GeneralSmem {
  uint32_t ccum[kNB];            // bin counts, then inclusive prefix
  unsigned long long wcum[kNB];  // bin weights, then inclusive prefix
  unsigned long long ckey[kCollectCap];
  unsigned long long cw[kCollectCap];  // weight, then in-bin inclusive cumulative
  uint32_t crank[kCollectCap];
  uint16_t cbin[kCollectCap];
};
struct RadixSmem {
  unsigned long long hw[256];
  uint32_t hc[256];
};

struct SamplerSmem {
  uint32_t pen[kPenWords];
  union {
    uint16_t gkey[kMaxGroups];
    GeneralSmem gen;
    RadixSmem rad;
  } u;
  unsigned long long cand_key[kCandCap];
  float cand_x[kCandCap];
  int32_t order[kKFast];
  unsigned long long incl[kKFast];
  uint32_t hist16[256];
  float red_f[kSW];
  float red_g[kSW];
  unsigned long long red_u[kSW];
  int32_t ncand;
  int32_t sel_bucket;
  int32_t sel_above;
  int32_t imin;
  unsigned long long sel_w_above;
  unsigned long long sel_total_w;
  uint32_t sel_total_c;
};

// --------------------------------------------------------- block helpers

__device__ __forceinline__ float block_max(SamplerSmem& sm, float v) {
  v = wave_max(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) sm.red_f[wid] = v;
  __syncthreads();
  float r = sm.red_f[0];
#pragma unroll
  for (int w = 1; w < kSW; ++w) r = fmaxf(r, sm.red_f[w]);
  return r;
}

__device__ __forceinline__ uint32_t block_sum_u32(SamplerSmem& sm, uint32_t v) {
  v = wave_sum_u32(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) sm.red_u[wid] = v;
  __syncthreads();
  uint32_t r = 0;
#pragma unroll
  for (int w = 0; w < kSW; ++w) r += (uint32_t)sm.red_u[w];
  return r;
}

__device__ __forceinline__ LseState block_lse(SamplerSmem& sm, LseState v) {
  v = wave_lse(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) {
    sm.red_f[wid] = v.m;
    sm.red_g[wid] = v.s;
  }
  __syncthreads();
  LseState r{sm.red_f[0], sm.red_g[0]};
#pragma unroll
  for (int w = 1; w < kSW; ++w) r = lse_merge(r, LseState{sm.red_f[w], sm.red_g[w]});
  return r;
}

// Fold 8*NG raw logits into a per-thread log-sum-exp (base-2 sums).
template <int NG>
__device__ __forceinline__ void lse_fold(LseState& st, const float (&x)[NG][8], float cm) {
  if (st.m == kNegInf) {
    bool nan = false;
#pragma unroll
    for (int k = 0; k < NG; ++k)
#pragma unroll
      for (int j = 0; j < 8; ++j) nan |= (x[k][j] != x[k][j]);
    if (nan) st.s = __builtin_nanf("");
  }
  const float mn = fmaxf(st.m, cm);
  if (mn == kNegInf) return;
  if (mn != st.m && st.s > 0.0f) st.s *= __builtin_amdgcn_exp2f((st.m - mn) * kLog2e);
  st.m = mn;
  const float mL = mn * kLog2e;
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < NG; ++k)
#pragma unroll
    for (int j = 0; j < 8; ++j) s += __builtin_amdgcn_exp2f(__builtin_fmaf(x[k][j], kLog2e, -mL));
  st.s += s;
}

// Wave 0 finds, in a 256-bucket histogram walked from the top bucket down,
// the bucket holding the element at 0-based position `target`; writes the
// bucket and the count above it.  Caller syncs before and after.
__device__ __forceinline__ void select_bucket_u32(SamplerSmem& sm, const uint32_t* hist,
                                                  uint32_t target) {
  if (threadIdx.x >= kWave) return;
  const int lane = threadIdx.x;
  uint32_t c[4];
  uint32_t tot = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    c[q] = hist[255 - 4 * lane - q];
    tot += c[q];
  }
  uint32_t incl = tot;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    uint32_t w = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += w;
  }
  uint32_t above = incl - tot;
  if (above <= target && target < incl) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (target < above + c[q]) {
        sm.sel_bucket = 255 - 4 * lane - q;
        sm.sel_above = (int32_t)above;
        break;
      }
      above += c[q];
    }
  }
}

// Same for 64-bit weights: the bucket where the inclusive cumulative weight
// first exceeds `target`.  Also returns the counts above (hc).
__device__ __forceinline__ void select_bucket_w(SamplerSmem& sm, const unsigned long long* hw,
                                                const uint32_t* hc, unsigned long long target) {
  if (threadIdx.x >= kWave) return;
  const int lane = threadIdx.x;
  unsigned long long w[4];
  uint32_t c[4];
  unsigned long long tot = 0;
  uint32_t ctot = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    w[q] = hw[255 - 4 * lane - q];
    c[q] = hc[255 - 4 * lane - q];
    tot += w[q];
    ctot += c[q];
  }
  unsigned long long incl = wave_incl_scan_u64(tot);
  uint32_t cincl = ctot;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    uint32_t v = __shfl_up(cincl, o, kWave);
    if (lane >= o) cincl += v;
  }
  unsigned long long above = incl - tot;
  uint32_t cabove = cincl - ctot;
  if (above <= target && target < incl) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (target < above + w[q]) {
        sm.sel_bucket = 255 - 4 * lane - q;
        sm.sel_above = (int32_t)cabove;
        sm.sel_w_above = above;
        break;
      }
      above += w[q];
      cabove += c[q];
    }
  }
}

// ------------------------------------------------------------ row context

template <typename T>
struct Row {
  const T* x;
  const uint32_t* mask;  // row of the allow mask or nullptr
  int64_t V;
  int64_t ngroups;
  bool vec_ok;
  bool greedy;
  bool use_pen;
  float Tc;
  float rho;

  __device__ __forceinline__ uint32_t mask_byte(int64_t G) const {
    return mask ? (mask[G >> 2] >> ((G & 3) * 8)) & 0xFFu : 0xFFu;
  }
  __device__ __forceinline__ uint32_t pen_byte(const SamplerSmem& sm, int64_t G) const {
    return use_pen ? (sm.pen[G >> 2] >> ((G & 3) * 8)) & 0xFFu : 0u;
  }
  // exact processed logit y of one element (contract steps S1, S4)
  __device__ __forceinline__ float process(float x, bool pen) const {
    float xp = x;
    if (pen) xp = (x < 0.0f) ? x * rho : x / rho;
    float y = greedy ? xp : xp / Tc;
    return y + 0.0f;
  }
};

// Visit every allowed token with a finite processed logit:
// f(id, y, x_raw).  Row re-read (L2/MALL resident after the stream pass).
template <typename T, typename F>
__device__ __forceinline__ void for_each_valid(const Row<T>& r, const SamplerSmem& sm, F&& f) {
  for (int64_t G = threadIdx.x; G < r.ngroups; G += kSB) {
    const uint32_t mb = r.mask_byte(G);
    if (mb == 0u) continue;
    float x[8];
    load_group<T>(r.x, G, r.V, r.vec_ok, x);
    const uint32_t pb = r.pen_byte(sm, G);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t e = G * 8 + j;
      if (e < r.V && ((mb >> j) & 1u)) {
        const float y = r.process(x[j], (pb >> j) & 1u);
        if (y > kNegInf) f((int32_t)e, y, x[j]);
      }
    }
  }
}

// Write the outputs of a row.
__device__ __forceinline__ void write_row(const SamplerArgs& a, int64_t b, int32_t status, int64_t id,
                                          float lp, float slp, int32_t kept, float tv, int32_t tid) {
  const bool fin = a.finished && a.finished[b];
  if (status != GTP_ROW_OK) {
    a.out_ids[b] = fin ? a.pad_id : -1;
    if (a.out_lp) a.out_lp[b] = __builtin_nanf("");
    if (a.out_slp) a.out_slp[b] = __builtin_nanf("");
    if (a.out_kept) a.out_kept[b] = 0;
    if (a.out_tv) a.out_tv[b] = 0.0f;
    if (a.out_tid) a.out_tid[b] = -1;
  } else {
    a.out_ids[b] = fin ? a.pad_id : id;
    if (a.out_lp) a.out_lp[b] = lp;
    if (a.out_slp) a.out_slp[b] = slp;
    if (a.out_kept) a.out_kept[b] = kept;
    if (a.out_tv) a.out_tv[b] = tv;
    if (a.out_tid) a.out_tid[b] = tid;
  }
  if (a.out_status) a.out_status[b] = status;
}

// ------------------------------------------------------ radix descent path
// Weighted search over the 64-bit rank key of valid tokens with
// key >= kmin: the token at which the inclusive cumulative (count or
// fixed-point weight, in order) first exceeds the target.  When
// `target_from_total` is set the target is floor(frac * total) with the
// total taken from the first digit's histogram.  Returns the key; fills the
// count before it (rank), the weight before it and the set's totals.
struct RadixResult {
  unsigned long long key;
  uint32_t rank;
  unsigned long long w_before;
  unsigned long long w_self;
  unsigned long long total_w;
  uint32_t total_c;
};

template <typename T>
__device__ RadixResult radix_search(SamplerSmem& sm, const Row<T>& r, float m, bool weighted,
                                    unsigned long long kmin, bool target_from_total, float frac,
                                    unsigned long long target) {
  unsigned long long prefix = 0, pmask = 0, w_before = 0;
  uint32_t rank = 0;
  RadixResult res{};
  for (int shift = 56; shift >= 0; shift -= 8) {
    __syncthreads();
    for (int i = threadIdx.x; i < 256; i += kSB) {
      sm.u.rad.hw[i] = 0;
      sm.u.rad.hc[i] = 0;
    }
    if (threadIdx.x == 0) {
      sm.sel_bucket = 0;
      sm.sel_above = 0;
      sm.sel_w_above = 0;
    }
    __syncthreads();
    for_each_valid<T>(r, sm, [&](int32_t id, float y, float) {
      const unsigned long long k = rank_key(y, id);
      if (k < kmin || (k & pmask) != prefix) return;
      const uint32_t dg = (uint32_t)(k >> shift) & 0xFFu;
      const unsigned long long w = weighted ? detexp_fix(y - m) : 1ull;
      atomicAdd(&sm.u.rad.hw[dg], w);
      atomicAdd(&sm.u.rad.hc[dg], 1u);
    });
    __syncthreads();
    if (shift == 56) {
      if (threadIdx.x < kWave) {
        unsigned long long tw = 0;
        uint32_t tc = 0;
        for (int q = 0; q < 4; ++q) {
          tw += sm.u.rad.hw[threadIdx.x * 4 + q];
          tc += sm.u.rad.hc[threadIdx.x * 4 + q];
        }
        for (int o = 32; o > 0; o >>= 1) {
          tw += shfl_xor_u64(tw, o);
          tc += __shfl_xor(tc, o, kWave);
        }
        if (threadIdx.x == 0) {
          sm.sel_total_w = tw;
          sm.sel_total_c = tc;
        }
      }
      __syncthreads();
      res.total_w = sm.sel_total_w;
      res.total_c = sm.sel_total_c;
      if (target_from_total) target = floor_mul(frac, res.total_w);
    }
    select_bucket_w(sm, sm.u.rad.hw, sm.u.rad.hc, target);
    __syncthreads();
    const uint32_t dg = (uint32_t)sm.sel_bucket & 0xFFu;
    target -= sm.sel_w_above;
    w_before += sm.sel_w_above;
    rank += (uint32_t)sm.sel_above;
    prefix |= (unsigned long long)dg << shift;
    pmask |= 0xFFull << shift;
    if (shift == 0) res.w_self = sm.u.rad.hw[dg];
  }
  __syncthreads();
  res.key = prefix;
  res.rank = rank;
  res.w_before = w_before;
  return res;
}

// ---------------------------------------------------------------- kernel

template <typename T>
__global__ __launch_bounds__(kSB) void sampler_rowwise_kernel(SamplerArgs a) {
  __shared__ SamplerSmem sm;
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;

  Row<T> r;
  r.x = reinterpret_cast<const T*>(a.logits) + b * a.row_stride;
  r.mask = a.mask ? a.mask + b * a.mask_stride : nullptr;
  r.V = a.V;
  r.ngroups = (a.V + 7) / 8;
  r.vec_ok = (reinterpret_cast<uintptr_t>(r.x) & 15u) == 0;
  r.greedy = !(a.T > 0.0f);
  r.Tc = a.T > 1e-6f ? a.T : 1e-6f;
  r.rho = a.rho;
  r.use_pen = a.hist && a.hist_len > 0 && a.rho != 1.0f;
  const float u = r.greedy ? 0.0f : a.uniforms[b];

  // ---- 0. penalty bitmap and history check
  const int64_t nwords = (a.V + 31) / 32;
  if (r.use_pen)
    for (int64_t w = tid; w < nwords; w += kSB) sm.pen[w] = 0u;
  if (tid == 0) sm.ncand = 0;
  __syncthreads();
  bool bad_hist = false;
  if (a.hist && a.hist_len > 0) {
    const int32_t* h = a.hist + b * a.hist_stride;
    for (int64_t j = tid; j < a.hist_len; j += kSB) {
      const int32_t id = h[j];
      if (id >= a.V) bad_hist = true;
      else if (id >= 0 && r.use_pen) atomicOr(&sm.pen[id >> 5], 1u << (id & 31));
    }
  }
  bad_hist = __syncthreads_or(bad_hist);

  // ---- 1. stream pass
  LseState ls{kNegInf, 0.0f};
  float tl = kNegInf;
  constexpr int64_t kStep = (int64_t)kSB * kSG;
  for (int64_t base = 0; base < r.ngroups; base += kStep) {
    float x[kSG][8];
    uint32_t mb[kSG], pb[kSG];
#pragma unroll
    for (int k = 0; k < kSG; ++k) {
      const int64_t G = base + k * kSB + tid;
      if (G < r.ngroups) {
        load_group<T>(r.x, G, r.V, r.vec_ok, x[k]);
        mb[k] = r.mask_byte(G);
        pb[k] = r.pen_byte(sm, G);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[k][j] = kNegInf;
        mb[k] = 0u;
        pb[k] = 0u;
      }
    }
    float cm = kNegInf;
#pragma unroll
    for (int k = 0; k < kSG; ++k) {
      const int64_t G = base + k * kSB + tid;
      float ghi;
      if (a.mask) {
        ghi = kNegInf;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t keep = (uint32_t)(((int32_t)(mb[k] << (31 - j))) >> 31);
          ghi = fmaxf(ghi, u2f((f2u(x[k][j]) & keep) | (0xFF800000u & ~keep)));
        }
        cm = fmaxf(cm, max8(x[k]));
      } else {
        ghi = max8(x[k]);
        cm = fmaxf(cm, ghi);
      }
      if (G < r.ngroups) sm.u.gkey[G] = (uint16_t)ord16(bf16_round_up(ghi));
      if ((mb[k] & pb[k]) == 0u) tl = fmaxf(tl, ghi);
    }
    lse_fold<kSG>(ls, x, cm);
  }
  const LseState row_lse = block_lse(sm, ls);
  const float lse_raw = row_lse.m + __builtin_amdgcn_logf(row_lse.s) * kLn2;
  const bool nonfinite = (row_lse.s != row_lse.s) || row_lse.m == kPosInf;

  int32_t status = GTP_ROW_OK;
  if (nonfinite) status = GTP_ROW_NONFINITE;
  else if (bad_hist) status = GTP_ROW_BAD_HISTORY;
  else if (!r.greedy && !(u >= 0.0f && u < 1.0f)) status = GTP_ROW_BAD_UNIFORM;
  if (status != GTP_ROW_OK) {
    if (tid == 0) write_row(a, b, status, -1, 0.f, 0.f, 0, 0.f, -1);
    return;
  }

  const int32_t Keff = r.greedy ? 1 : a.K;
  const bool p_active = !r.greedy && a.P > 0.0f && a.P < 1.0f;
  bool general = !(Keff >= 1 && Keff <= kKFast) || (r.use_pen && a.rho < 1.0f);

  if (!general) {
    // ---- 2. tau = Keff-th largest thread lower bound (16-bit keys)
    const uint32_t mykey = ord16(bf16_round_down(tl));
    if (tid < 256) sm.hist16[tid] = 0u;
    if (tid == 0) {
      sm.sel_bucket = 0;
      sm.sel_above = 0;
    }
    __syncthreads();
    atomicAdd(&sm.hist16[mykey >> 8], 1u);
    __syncthreads();
    select_bucket_u32(sm, sm.hist16, (uint32_t)(Keff - 1));
    __syncthreads();
    const uint32_t b1 = (uint32_t)sm.sel_bucket & 0xFFu;
    const uint32_t t1 = (uint32_t)(Keff - 1) - (uint32_t)sm.sel_above;
    __syncthreads();
    if (tid < 256) sm.hist16[tid] = 0u;
    if (tid == 0) {
      sm.sel_bucket = 0;
      sm.sel_above = 0;
    }
    __syncthreads();
    if ((mykey >> 8) == b1) atomicAdd(&sm.hist16[mykey & 0xFFu], 1u);
    __syncthreads();
    select_bucket_u32(sm, sm.hist16, t1);
    __syncthreads();
    const uint32_t tau_key = (b1 << 8) | ((uint32_t)sm.sel_bucket & 0xFFu);
    const float tau = u2f(unord16(tau_key) << 16);
    const float y_tau = r.greedy ? tau : (tau / r.Tc) + 0.0f;
    // smallest group key whose upper bound can reach y_tau (monotone search;
    // keys at or below -inf's key never pass)
    uint32_t lo = 0x0080u, hi = 0xFF81u;
    while (lo < hi) {
      const uint32_t mid = (lo + hi) >> 1;
      const float gv = u2f(unord16(mid) << 16);
      const float gy = r.greedy ? gv : (gv / r.Tc) + 0.0f;
      if (gy >= y_tau) hi = mid;
      else lo = mid + 1;
    }
    const uint32_t gk_thr = lo;

    // ---- 3. re-read passing groups, exact candidates
    for (int64_t base = 0; base < r.ngroups; base += kStep) {
#pragma unroll
      for (int k = 0; k < kSG; ++k) {
        const int64_t G = base + k * kSB + tid;
        if (G < r.ngroups && (uint32_t)sm.u.gkey[G] >= gk_thr) {
          float x[8];
          load_group<T>(r.x, G, r.V, r.vec_ok, x);
          const uint32_t mbits = r.mask_byte(G), pbits = r.pen_byte(sm, G);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int64_t e = G * 8 + j;
            if (e < r.V && ((mbits >> j) & 1u)) {
              const float y = r.process(x[j], (pbits >> j) & 1u);
              if (y > kNegInf && y >= y_tau) {
                const int slot = atomicAdd(&sm.ncand, 1);
                if (slot < kCandCap) {
                  sm.cand_key[slot] = rank_key(y, (int32_t)e);
                  sm.cand_x[slot] = x[j];
                }
              }
            }
          }
        }
      }
    }
    __syncthreads();
    const int nc = sm.ncand;
    if (nc > kCandCap) {
      general = true;
    } else if (nc == 0) {
      if (tid == 0) write_row(a, b, GTP_ROW_EMPTY, -1, 0.f, 0.f, 0, 0.f, -1);
      return;
    } else {
      const int nk = Keff < nc ? Keff : nc;
      // ---- 4. exact rank among candidates (one candidate per thread)
      if (tid < nc) {
        const unsigned long long ki = sm.cand_key[tid];
        int rk = 0;
        for (int j = 0; j < nc; ++j) rk += (sm.cand_key[j] > ki) ? 1 : 0;
        if (rk < nk) sm.order[rk] = tid;
      }
      __syncthreads();
      const unsigned long long k0 = sm.cand_key[sm.order[0]];
      const float m = rank_key_y(k0);
      if (m == kPosInf) {
        if (tid == 0) write_row(a, b, GTP_ROW_NONFINITE, -1, 0.f, 0.f, 0, 0.f, -1);
        return;
      }
      if (r.greedy) {
        if (tid == 0) {
          const int32_t id = rank_key_id(k0);
          write_row(a, b, GTP_ROW_OK, id, sm.cand_x[sm.order[0]] - lse_raw, 0.0f, 1, m, id);
        }
        return;
      }
      // ---- 5. fixed-point weights, inclusive prefix (wave 0, 4 per lane)
      if (tid < nk) sm.incl[tid] = detexp_fix(rank_key_y(sm.cand_key[sm.order[tid]]) - m);
      __syncthreads();
      if (tid < kWave) {
        unsigned long long v[4], tot = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int rr = tid * 4 + q;
          v[q] = rr < nk ? sm.incl[rr] : 0ull;
          tot += v[q];
        }
        unsigned long long run = wave_incl_scan_u64(tot) - tot;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int rr = tid * 4 + q;
          run += v[q];
          if (rr < nk) sm.incl[rr] = run;
        }
      }
      __syncthreads();
      if (tid == 0) {
        const unsigned long long Wk = sm.incl[nk - 1];
        int R = nk;
        if (p_active) {
          const unsigned long long F = floor_mul(a.P, Wk);
          // R = 1 + #{r < nk-1 : incl[r] <= F}
          int lo2 = 0, hi2 = nk - 1;
          while (lo2 < hi2) {
            const int mid = (lo2 + hi2) >> 1;
            if (sm.incl[mid] <= F) lo2 = mid + 1;
            else hi2 = mid;
          }
          R = lo2 + 1;
        }
        const unsigned long long Wp = sm.incl[R - 1];
        const unsigned long long U = floor_mul(u, Wp);
        int lo3 = 0, hi3 = R - 1;
        while (lo3 < hi3) {
          const int mid = (lo3 + hi3) >> 1;
          if (sm.incl[mid] <= U) lo3 = mid + 1;
          else hi3 = mid;
        }
        const int rs = lo3;
        const unsigned long long ws = sm.incl[rs] - (rs ? sm.incl[rs - 1] : 0ull);
        const int ci = sm.order[rs];
        const int32_t id = rank_key_id(sm.cand_key[ci]);
        const unsigned long long kt = sm.cand_key[sm.order[R - 1]];
        const float slp = (float)::log((double)ws / (double)Wp);
        write_row(a, b, GTP_ROW_OK, id, sm.cand_x[ci] - lse_raw, slp, R, rank_key_y(kt),
                  rank_key_id(kt));
      }
      return;
    }
  }

  // ================================================================ general
  __syncthreads();
  // (A) exact max of the processed logits of valid tokens
  float ymax = kNegInf;
  for_each_valid<T>(r, sm, [&](int32_t, float y, float) { ymax = fmaxf(ymax, y); });
  const float m = block_max(sm, ymax);
  if (m == kNegInf) {
    if (tid == 0) write_row(a, b, GTP_ROW_EMPTY, -1, 0.f, 0.f, 0, 0.f, -1);
    return;
  }
  if (m == kPosInf) {
    if (tid == 0) write_row(a, b, GTP_ROW_NONFINITE, -1, 0.f, 0.f, 0, 0.f, -1);
    return;
  }
  GeneralSmem& g = sm.u.gen;
  // (B) bin histograms
  __syncthreads();
  for (int i = tid; i < kNB; i += kSB) {
    g.ccum[i] = 0u;
    g.wcum[i] = 0ull;
  }
  __syncthreads();
  auto bin_of = [&](float y) -> int {
    const float d = (m - y) * kBinScale;
    return d < (float)(kNB - 1) ? (int)d : kNB - 1;
  };
  for_each_valid<T>(r, sm, [&](int32_t, float y, float) {
    const int bn = bin_of(y);
    atomicAdd(&g.ccum[bn], 1u);
    if (!r.greedy) atomicAdd(&g.wcum[bn], detexp_fix(y - m));
  });
  __syncthreads();
  // inclusive prefix over bins: wave 0, 32 bins per lane
  if (tid < kWave) {
    constexpr int per = kNB / kWave;
    uint32_t ct = 0;
    unsigned long long wt = 0;
    for (int q = 0; q < per; ++q) {
      ct += g.ccum[tid * per + q];
      wt += g.wcum[tid * per + q];
    }
    uint32_t cex = ct;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      uint32_t v = __shfl_up(cex, o, kWave);
      if (tid >= o) cex += v;
    }
    cex -= ct;
    unsigned long long wex = wave_incl_scan_u64(wt) - wt;
    for (int q = 0; q < per; ++q) {
      cex += g.ccum[tid * per + q];
      wex += g.wcum[tid * per + q];
      g.ccum[tid * per + q] = cex;
      g.wcum[tid * per + q] = wex;
    }
  }
  __syncthreads();
  const uint32_t n_valid = g.ccum[kNB - 1];
  const unsigned long long W_all = g.wcum[kNB - 1];
  const bool k_active = Keff > 0 && (uint32_t)Keff < n_valid;
  const uint32_t nk = k_active ? (uint32_t)Keff : n_valid;
  // bin search helpers (first bin with cumulative > v)
  auto first_bin_c = [&](uint32_t v) -> int {
    int lo = 0, hi = kNB - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (g.ccum[mid] > v) hi = mid;
      else lo = mid + 1;
    }
    return lo;
  };
  auto first_bin_w = [&](unsigned long long v) -> int {
    int lo = 0, hi = kNB - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (g.wcum[mid] > v) hi = mid;
      else lo = mid + 1;
    }
    return lo;
  };
  auto wex_bin = [&](int bn) -> unsigned long long { return bn ? g.wcum[bn - 1] : 0ull; };
  auto cex_bin = [&](int bn) -> uint32_t { return bn ? g.ccum[bn - 1] : 0u; };
  // bins that can hold the k cut, the p cut, the draw and the last kept rank
  const int b_k = first_bin_c(nk - 1);
  unsigned long long Wk_lo = W_all, Wk_hi = W_all;
  if (k_active) {
    Wk_lo = wex_bin(b_k);
    Wk_hi = g.wcum[b_k];
  }
  int bp_lo = b_k, bp_hi = b_k;
  if (p_active) {
    const int x1 = first_bin_w(floor_mul(a.P, Wk_lo));
    const int x2 = first_bin_w(floor_mul(a.P, Wk_hi));
    bp_lo = x1 < b_k ? x1 : b_k;
    bp_hi = x2 < b_k ? x2 : b_k;
  }
  int bu_lo = 0, bu_hi = bp_hi;
  if (!r.greedy) {
    const unsigned long long Wp_lo = wex_bin(bp_lo);
    unsigned long long Wp_hi = g.wcum[bp_hi];
    if (Wp_hi > Wk_hi) Wp_hi = Wk_hi;
    const int y1 = first_bin_w(floor_mul(u, Wp_lo));
    const int y2 = first_bin_w(floor_mul(u, Wp_hi));
    bu_lo = y1 < bp_hi ? y1 : bp_hi;
    bu_hi = y2 < bp_hi ? y2 : bp_hi;
  } else {
    bu_lo = 0;
    bu_hi = 0;
  }
  auto in_need = [&](int bn) -> bool {
    return bn == b_k || (bn >= bp_lo && bn <= bp_hi) || (bn >= bu_lo && bn <= bu_hi);
  };
  uint32_t need_local = 0;
  for (int bn = tid; bn < kNB; bn += kSB)
    if (in_need(bn)) need_local += g.ccum[bn] - cex_bin(bn);
  const uint32_t need_count = block_sum_u32(sm, need_local);
  int64_t id_draw = -1, id_thr = -1;
  float y_thr = 0.0f;
  int32_t kept = 0;
  double slp = 0.0;
  if (need_count <= (uint32_t)kCollectCap) {
    // (C) collect the needed bins and rank them exactly
    if (tid == 0) sm.ncand = 0;
    __syncthreads();
    for_each_valid<T>(r, sm, [&](int32_t id, float y, float) {
      const int bn = bin_of(y);
      if (!in_need(bn)) return;
      const int slot = atomicAdd(&sm.ncand, 1);
      if (slot < kCollectCap) {
        g.ckey[slot] = rank_key(y, id);
        g.cw[slot] = r.greedy ? 0ull : detexp_fix(y - m);
        g.cbin[slot] = (uint16_t)bn;
      }
    });
    __syncthreads();
    const int nc = sm.ncand < kCollectCap ? sm.ncand : kCollectCap;
    // in-bin rank and in-bin inclusive weight (O(n^2) over collected tokens)
    unsigned long long my_cum[2] = {0, 0};
    uint32_t my_rank[2] = {0, 0};
    for (int s2 = 0; s2 < 2; ++s2) {
      const int i = tid + s2 * kSB;
      if (i < nc) {
        const unsigned long long ki = g.ckey[i];
        const uint16_t bi = g.cbin[i];
        uint32_t rk = 0;
        unsigned long long wc = g.cw[i];
        for (int j = 0; j < nc; ++j) {
          if (g.cbin[j] == bi && g.ckey[j] > ki) {
            rk++;
            wc += g.cw[j];
          }
        }
        my_rank[s2] = cex_bin(bi) + rk;
        my_cum[s2] = wex_bin(bi) + wc;
      }
    }
    __syncthreads();
    for (int s2 = 0; s2 < 2; ++s2) {
      const int i = tid + s2 * kSB;
      if (i < nc) {
        g.crank[i] = my_rank[s2];
        g.cw[i] = my_cum[s2];  // now: inclusive cumulative weight at this token
      }
    }
    __syncthreads();
    // resolution: every lookup is "the collected token with rank == R" or
    // "the lowest-ranked collected token with cumulative > F among rank < N"
    auto rank_lookup = [&](uint32_t want) -> int {  // index of token with crank == want
      if (tid == 0) sm.imin = -1;
      __syncthreads();
      for (int i = tid; i < nc; i += kSB)
        if (g.crank[i] == want) sm.imin = i;
      __syncthreads();
      const int found = sm.imin;
      __syncthreads();
      return found < 0 ? 0 : found;  // a miss would be a logic error: stay in bounds
    };
    auto first_above = [&](unsigned long long F, uint32_t limit) -> int {  // returns index
      if (tid == 0) sm.imin = 0x7FFFFFFF;
      __syncthreads();
      for (int i = tid; i < nc; i += kSB)
        if (g.crank[i] < limit && g.cw[i] > F) atomicMin(&sm.imin, (int32_t)g.crank[i]);
      __syncthreads();
      const int want = sm.imin;
      __syncthreads();
      return rank_lookup(want == 0x7FFFFFFF ? 0u : (uint32_t)want);
    };
    if (r.greedy) {
      const int i0 = rank_lookup(0);
      id_draw = rank_key_id(g.ckey[i0]);
      id_thr = id_draw;
      y_thr = rank_key_y(g.ckey[i0]);
      kept = 1;
      slp = 0.0;
    } else {
      unsigned long long Wk = W_all;
      if (k_active) Wk = g.cw[rank_lookup(nk - 1)];
      int i_cut;
      if (p_active) i_cut = first_above(floor_mul(a.P, Wk), nk);
      else i_cut = rank_lookup(nk - 1);
      const unsigned long long Wp = g.cw[i_cut];
      kept = (int32_t)(g.crank[i_cut] + 1u);
      id_thr = rank_key_id(g.ckey[i_cut]);
      y_thr = rank_key_y(g.ckey[i_cut]);
      const int i_u = first_above(floor_mul(u, Wp), (uint32_t)kept);
      id_draw = rank_key_id(g.ckey[i_u]);
      const unsigned long long w_u = detexp_fix(rank_key_y(g.ckey[i_u]) - m);
      slp = ::log((double)w_u / (double)Wp);
    }
  } else {
    // radix descent fallback (heavy exact ties): one re-read per digit
    const unsigned long long kNone = 0ull;
    if (r.greedy) {
      RadixResult t0 = radix_search<T>(sm, r, m, false, kNone, false, 0.f, 0ull);
      id_draw = rank_key_id(t0.key);
      id_thr = id_draw;
      y_thr = rank_key_y(t0.key);
      kept = 1;
      slp = 0.0;
    } else {
      unsigned long long kmin = kNone;
      if (k_active) kmin = radix_search<T>(sm, r, m, false, kNone, false, 0.f, nk - 1).key;
      RadixResult cut;
      if (p_active) {
        cut = radix_search<T>(sm, r, m, true, kmin, true, a.P, 0ull);
      } else {
        // last kept = the lowest key of the kept set: rank nk-1 by count
        RadixResult c = radix_search<T>(sm, r, m, false, kmin, false, 0.f, nk - 1);
        cut = c;
        cut.w_before = 0;  // recomputed below from the weighted totals
      }
      kept = (int32_t)(cut.rank + 1u);
      id_thr = rank_key_id(cut.key);
      y_thr = rank_key_y(cut.key);
      RadixResult drw = radix_search<T>(sm, r, m, true, cut.key, true, u, 0ull);
      // drw.total_w = weight of the kept set = W'
      id_draw = rank_key_id(drw.key);
      slp = ::log((double)drw.w_self / (double)drw.total_w);
    }
  }
  if (tid == 0) {
    const bool in_row = id_draw >= 0 && id_draw < r.V;
    const float xd = in_row ? Elem<T>::get(r.x, id_draw) : __builtin_nanf("");
    write_row(a, b, GTP_ROW_OK, id_draw, xd - lse_raw, (float)slp, kept, y_thr, (int32_t)id_thr);
  }
}

}  // namespace gtp

using namespace gtp;

namespace gtp {

// One workgroup of 1024 threads per row; handles every row layout, vocabulary
// and parameter combination the contract allows.
int launch_sampler_general(const SamplerArgs& a, int dtype, int64_t B, hipStream_t s) {
  const dim3 grid((unsigned)B), block(kSB);
  switch (dtype) {
    case GTP_DTYPE_BF16:
      hipLaunchKernelGGL(sampler_rowwise_kernel<uint16_t>, grid, block, 0, s, a);
      break;
    case GTP_DTYPE_F16:
      hipLaunchKernelGGL(sampler_rowwise_kernel<_Float16>, grid, block, 0, s, a);
      break;
    case GTP_DTYPE_F32:
      hipLaunchKernelGGL(sampler_rowwise_kernel<float>, grid, block, 0, s, a);
      break;
    default:
      return GTP_ERR_INVALID_ARGUMENT;
  }
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}

}  // namespace gtp
