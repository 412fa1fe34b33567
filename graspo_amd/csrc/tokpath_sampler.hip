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
#include "tokpath_stream.h"

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

__device__ __forceinline__ unsigned long long block_max_u64(SamplerSmem& sm, unsigned long long v) {
  v = wave_max_u64(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) sm.red_u[wid] = v;
  __syncthreads();
  unsigned long long r = sm.red_u[0];
#pragma unroll
  for (int w = 1; w < kSW; ++w) r = sm.red_u[w] > r ? sm.red_u[w] : r;
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
  const float mb = mn;
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < NG; ++k)
#pragma unroll
    for (int j = 0; j < 8; ++j) s += __builtin_amdgcn_exp2f((x[k][j] - mb) * kLog2e);
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

// Visit every group of 8 tokens that holds an allowed one: f(G, v[8], valid)
// with, for kY, the processed logits y of all 8 (computed without a
// per-element branch: a penalised and an unpenalised element differ in a
// select) and `valid` the mask of the allowed tokens with y > -inf; without
// kY, v holds the penalised logits x' before the temperature (no division)
// and `valid` the allowed tokens with x' > -inf.  The loads run kAhead
// groups ahead of their use (a pass over an fp32 batch re-reads it from
// HBM: [256, 248320] fp32 outgrows the last-level cache).
template <typename T, bool kY, typename F>
__device__ __forceinline__ void for_each_group8(const Row<T>& r, const SamplerSmem& sm, F&& f) {
  constexpr int kAhead = 3;
  float xb[kAhead][8];
  uint32_t mbb[kAhead];
  auto fetch = [&](int64_t G, float (&x)[8], uint32_t& mb) {
    mb = G < r.ngroups ? r.mask_byte(G) : 0u;
    if (mb != 0u) load_group<T>(r.x, G, r.V, r.vec_ok, x);
  };
#pragma unroll
  for (int q = 0; q < kAhead; ++q) fetch((int64_t)threadIdx.x + (int64_t)q * kSB, xb[q], mbb[q]);
  for (int64_t G0 = threadIdx.x; G0 < r.ngroups; G0 += (int64_t)kAhead * kSB) {
#pragma unroll
    for (int q = 0; q < kAhead; ++q) {
      const int64_t G = G0 + (int64_t)q * kSB;
      const uint32_t mb = mbb[q];
      float x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = xb[q][j];
      fetch(G + (int64_t)kAhead * kSB, xb[q], mbb[q]);
      if (mb == 0u) continue;
      const uint32_t pb = r.pen_byte(sm, G);
      if (pb != 0u) {  // (penalised tokens are rare: only their groups divide by rho)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float q2 = (x[j] < 0.0f) ? x[j] * r.rho : x[j] / r.rho;
          x[j] = ((pb >> j) & 1u) ? q2 : x[j];
        }
      }
      float v[8];
      uint32_t valid = 0u;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float yy = kY ? (r.greedy ? x[j] : x[j] / r.Tc) + 0.0f : x[j];
        v[j] = yy;
        const bool ok = G * 8 + j < r.V && ((mb >> j) & 1u) && yy > kNegInf;
        valid |= (ok ? 1u : 0u) << j;
      }
      f(G, v, valid);
    }
  }
}

// Write the outputs of a row.
// (`fin`: the row's finished flag, read by the caller)
__device__ __forceinline__ void write_row_f(const SamplerArgs& a, int64_t b, bool fin, int32_t status,
                                            int64_t id, float lp, float slp, int32_t kept, float tv,
                                            int32_t tid) {
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
__device__ __forceinline__ void write_row(const SamplerArgs& a, int64_t b, int32_t status, int64_t id,
                                          float lp, float slp, int32_t kept, float tv, int32_t tid) {
  write_row_f(a, b, a.finished && a.finished[b], status, id, lp, slp, kept, tv, tid);
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

// One row (block-uniform; every thread of the 1024-thread workgroup calls it).
// NG: groups per thread per stream step (fewer registers for a smaller NG)
template <typename T, int NG = kSG>
__device__ __forceinline__ void rowwise_row(const SamplerArgs& a, int64_t b, SamplerSmem& sm) {
  const int tid = threadIdx.x;

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
  float xpmax = kNegInf;  // max of the allowed penalised logits x' (the general path's m)
  constexpr int64_t kStep = (int64_t)kSB * NG;
  for (int64_t base = 0; base < r.ngroups; base += kStep) {
    float x[NG][8];
    uint32_t mb[NG], pb[NG];
#pragma unroll
    for (int k = 0; k < NG; ++k) {
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
    for (int k = 0; k < NG; ++k) {
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
      if ((mb[k] & pb[k]) == 0u) {
        tl = fmaxf(tl, ghi);
        xpmax = fmaxf(xpmax, ghi);
      } else {  // (rare: a group with an allowed penalised token)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float xj = x[k][j];
          const float xp = ((pb[k] >> j) & 1u) ? ((xj < 0.0f) ? xj * r.rho : xj / r.rho) : xj;
          if ((mb[k] >> j) & 1u) xpmax = fmaxf(xpmax, xp);
        }
      }
    }
    lse_fold<NG>(ls, x, cm);
  }
  const LseState row_lse = block_lse(sm, ls);
  // logprob = x - m - ln s, rounded once (raw_logprob)
  const float lse_m = row_lse.m, lse_ln = __builtin_amdgcn_logf(row_lse.s) * kLn2;
  const bool nonfinite = (row_lse.s != row_lse.s) || row_lse.m == kPosInf;

  // A row without an answer on the ordered paths (block-uniform call):
  // greedy rows take the argmax semantics of greedy_argmax_rescan (wave 0
  // scans the row; sm.pen already holds the penalised ids), other rows
  // report `st`.
  auto fail = [&](int32_t st) __attribute__((always_inline)) {
    if (r.greedy && !bad_hist) {
      if (tid < kWave) greedy_argmax_rescan<T>(a, b, sm.pen, false, nonfinite, lse_m, lse_ln);
      return;
    }
    if (tid == 0) write_row(a, b, r.greedy ? GTP_ROW_BAD_HISTORY : st, -1, 0.f, 0.f, 0, 0.f, -1);
  };
  int32_t status = GTP_ROW_OK;
  if (nonfinite) status = GTP_ROW_NONFINITE;
  else if (bad_hist) status = GTP_ROW_BAD_HISTORY;
  else if (!r.greedy && !(u >= 0.0f && u < 1.0f)) status = GTP_ROW_BAD_UNIFORM;
  if (status != GTP_ROW_OK) {
    fail(status);
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
      for (int k = 0; k < NG; ++k) {
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
      fail(GTP_ROW_EMPTY);
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
        fail(GTP_ROW_NONFINITE);
        return;
      }
      if (r.greedy) {
        if (tid == 0) {
          const int32_t id = rank_key_id(k0);
          write_row(a, b, GTP_ROW_OK, id, raw_logprob(sm.cand_x[sm.order[0]], lse_m, lse_ln), 0.0f, 1, m, id);
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
        write_row(a, b, GTP_ROW_OK, id, raw_logprob(sm.cand_x[ci], lse_m, lse_ln), slp, R, rank_key_y(kt),
                  rank_key_id(kt));
      }
      return;
    }
  }

  // ================================================================ general
  __syncthreads();
  // (A) exact max of the processed logits of valid tokens.  Dividing by
  // T > 0 with rounding to nearest is monotone, so the max of y = x' / T is
  // the quotient of the max of x', taken in the stream pass: one division
  // per row, no re-read.  (A token whose y alone overflows to -inf cannot
  // hold the max unless every token does, and then the row is empty either
  // way.)
  const float xm = block_max(sm, xpmax);
  const float m = (xm == kNegInf || r.greedy) ? xm : xm / r.Tc + 0.0f;
  if (m == kNegInf) {
    fail(GTP_ROW_EMPTY);
    return;
  }
  if (m == kPosInf) {
    fail(GTP_ROW_NONFINITE);
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
  // (B), with the row's last valid token in order (the lowest rank key):
  // the last kept rank of a row with neither top-k nor top-p (only looked
  // for without top-p)
  const bool want_last = !r.greedy && !p_active;
  unsigned long long nkey_last = 0ull;  // ~(lowest rank key)
  for_each_group8<T, true>(r, sm, [&](int64_t G, const float (&y)[8], uint32_t valid) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int bn = bin_of(y[j]);
      // (a masked element's y may exceed m: its unused weight is taken at d <= 0)
      const unsigned long long w = r.greedy ? 0ull : detexp_fix(fminf(y[j] - m, 0.0f));
      const bool ok = (valid >> j) & 1u;
      if (ok) {
        atomicAdd(&g.ccum[bn], 1u);
        if (!r.greedy) atomicAdd(&g.wcum[bn], w);
      }
      if (want_last) {
        const unsigned long long nk = ok ? ~rank_key(y[j], (int32_t)(G * 8 + j)) : 0ull;
        nkey_last = nk > nkey_last ? nk : nkey_last;
      }
    }
  });
  const unsigned long long key_last = ~block_max_u64(sm, nkey_last);
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
  // without top-k and top-p every valid token is kept: the last kept rank is
  // key_last and the kept weight is W_all, so no bin needs collecting for
  // the cut (the bottom bin can hold most of the row)
  const bool keep_all = !r.greedy && !k_active && !p_active;
  if (p_active) {
    const int x1 = first_bin_w(floor_mul(a.P, Wk_lo));
    const int x2 = first_bin_w(floor_mul(a.P, Wk_hi));
    bp_lo = x1 < b_k ? x1 : b_k;
    bp_hi = x2 < b_k ? x2 : b_k;
  }
  int bu_lo = 0, bu_hi = bp_hi;
  if (!r.greedy) {
    unsigned long long Wp_lo = wex_bin(bp_lo);
    unsigned long long Wp_hi = g.wcum[bp_hi];
    if (Wp_hi > Wk_hi) Wp_hi = Wk_hi;
    if (keep_all) Wp_lo = Wp_hi = W_all;
    const int y1 = first_bin_w(floor_mul(u, Wp_lo));
    const int y2 = first_bin_w(floor_mul(u, Wp_hi));
    bu_lo = y1 < bp_hi ? y1 : bp_hi;
    bu_hi = y2 < bp_hi ? y2 : bp_hi;
  } else {
    bu_lo = 0;
    bu_hi = 0;
  }
  // the k cut's bin only matters with top-k (greedy: Keff = 1), the p cut's
  // only when some rank can be cut
  auto in_need = [&](int bn) -> bool {
    return (k_active && bn == b_k) || (!keep_all && bn >= bp_lo && bn <= bp_hi) ||
           (bn >= bu_lo && bn <= bu_hi);
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
    // the needed bins lie in [nb_lo, nb_hi]: y in (m - (nb_hi + 1) / 64,
    // m - nb_lo / 64], widened by a bin and 2^-20 relative and mapped to x'
    // (x' = y T up to rounding), so only tokens near those bins divide
    int nb_lo = kNB, nb_hi = -1;
    auto widen = [&](int lo, int hi) {
      nb_lo = lo < nb_lo ? lo : nb_lo;
      nb_hi = hi > nb_hi ? hi : nb_hi;
    };
    if (k_active) widen(b_k, b_k);
    if (!keep_all) widen(bp_lo, bp_hi);
    widen(bu_lo, bu_hi);
    const float y_hi = m - (float)nb_lo / kBinScale + 1.0f / kBinScale;
    const float y_lo = nb_hi >= kNB - 1 ? kNegInf : m - (float)(nb_hi + 2) / kBinScale;
    auto pad = [](float v, float dir) { return v + dir * (fabsf(v) * 0x1p-20f + 0x1p-100f); };
    const float sc = r.greedy ? 1.0f : r.Tc;
    const float x_hi = pad(pad(y_hi, 1.0f) * sc, 1.0f);
    const float x_lo = y_lo == kNegInf ? kNegInf : pad(pad(y_lo, -1.0f) * sc, -1.0f);
    for_each_group8<T, false>(r, sm, [&](int64_t G, const float (&xp)[8], uint32_t valid) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (!((valid >> j) & 1u) || xp[j] < x_lo || xp[j] > x_hi) continue;
        const float y = (r.greedy ? xp[j] : xp[j] / r.Tc) + 0.0f;
        if (!(y > kNegInf)) continue;
        const int bn = bin_of(y);
        if (in_need(bn)) {
          const int slot = atomicAdd(&sm.ncand, 1);
          if (slot < kCollectCap) {
            g.ckey[slot] = rank_key(y, (int32_t)(G * 8 + j));
            g.cw[slot] = r.greedy ? 0ull : detexp_fix(y - m);
            g.cbin[slot] = (uint16_t)bn;
          }
        }
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
      unsigned long long Wk = W_all, Wp = W_all;
      if (k_active) Wk = g.cw[rank_lookup(nk - 1)];
      if (keep_all) {
        kept = (int32_t)n_valid;
        id_thr = rank_key_id(key_last);
        y_thr = rank_key_y(key_last);
      } else {
        const int i_cut = p_active ? first_above(floor_mul(a.P, Wk), nk) : rank_lookup(nk - 1);
        Wp = g.cw[i_cut];
        kept = (int32_t)(g.crank[i_cut] + 1u);
        id_thr = rank_key_id(g.ckey[i_cut]);
        y_thr = rank_key_y(g.ckey[i_cut]);
      }
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
    write_row(a, b, GTP_ROW_OK, id_draw, raw_logprob(xd, lse_m, lse_ln), (float)slp, kept, y_thr, (int32_t)id_thr);
  }
}

template <typename T>
__global__ __launch_bounds__(kSB) void sampler_rowwise_kernel(SamplerArgs a) {
  __shared__ SamplerSmem sm;
  rowwise_row<T>(a, (int64_t)blockIdx.x, sm);
}

// ============================================================ value histogram
//
// Rows of bf16 logits with T > 0 on 16-byte aligned rows (top-p with or
// without top-k, any top-k): all allowed tokens with the same bf16 bit
// pattern and the same penalty state have the same processed logit and the
// same fixed-point weight, so the exact totals and prefix sums of the
// contract are sums over the row's distinct values, not over its tokens.
//
// 1. One streaming pass (the only full HBM read): the raw log-sum-exp, and
//    a count per bf16 value (16384 bins: both signs, biased exponents
//    [87, 151), i.e. 2^-40 <= |x| < 2^24).  Values outside the bins are
//    "singletons" kept with their raw value and id.  Afterwards each
//    distinct penalised history id moves from its value's count to a second
//    count per value (penalised values: y = pen(x) / T).
// 2. m = the largest processed logit.  A segment is 16 value bins (one per
//    thread); each penalised value and each singleton joins the segment
//    whose value range holds its y.  A block scan in descending order gives
//    each segment the count and weight above it.
// 3. The top-k rank, the top-p cut, the last kept rank and the draw each
//    pick a segment from those totals; one wave resolves the order inside
//    it: its bins in value order, its extra items (penalised values and
//    singletons, sorted in registers) merged by position, and a penalised
//    value equal to a bin's y merged into that bin.  A run of tokens with
//    one value has one weight, so positions inside it are integer quotients.
// 4. A token of a bin is found by id: one coalesced rescan of the row lists
//    each wave's members of the two items in id order (a packed 16-bit
//    compare of 8 tokens against a pattern costs 13 instructions).
// Anything outside these bounds -- more singletons than the list holds, a
// singleton or penalised value exactly tied with another item at a cut,
// more than 64 extra items in one resolved segment, a non-finite processed
// logit -- runs the row-wise path for the row instead, in the same
// workgroup.
//
// Replaces _sample_next_token (src/graspo/backends/graspoflow/tensor_utils.py:671-683)
// for these rows.

constexpr int kHBins = 16384;
constexpr uint32_t kHELo = 87;
constexpr int kHSegBins = kHBins / kSB;  // 16 bins per thread and per segment
constexpr int kHSCap = 512;              // singletons of a row
constexpr int kHXCap = 64;               // extra items of one resolved segment
constexpr int kHItems = kHSegBins + kHXCap;
constexpr int kHPenSpan = 2048;          // penalised-value bins one segment may span
constexpr int kHG = 2;                   // vectors per thread per stream step
constexpr uint32_t kNoPattern = 0x10000u;  // matches no 16-bit pattern
constexpr int kHListCap = 512;

// Set lanes of a wave mask below this lane.
__device__ __forceinline__ uint32_t lanes_below(unsigned long long m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Lane-wise minimum of the two unsigned 16-bit halves (v_pk_min_u16; the
// compiler turns the generic form into compares and selects).
__device__ __forceinline__ uint32_t pk_min_u16(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_pk_min_u16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}           // ids of one item one wave lists in the rescan

struct alignas(16) HistSmem {
  uint32_t cnt[kHBins + kWave];          // allowed unpenalised tokens per value (+ a spill word per lane)
  uint32_t pcnt2[kHBins / 2];            // allowed penalised tokens per value, 16 bits each
  uint32_t pen[GTP_SAMPLER_MAX_V / 32];  // penalised ids
  uint32_t sid[kHSCap];                  // singleton id
  float sx[kHSCap];                      // singleton raw logit
  uint16_t sbin[kHSCap];                 // largest bin whose y <= the singleton's y (0xFFFF: none)
  unsigned long long segw[kSB];          // weight of the extra items of each segment
  uint32_t segc[kSB];
  uint32_t seg_plo[kSB];                 // penalised bins placed in each segment: [plo, phi)
  uint32_t seg_phi[kSB];
  // the resolved segment (wave 0)
  unsigned long long it_w[kHItems];      // per-token weight of each item, in rank order
  uint32_t it_c[kHItems];                // tokens in the item
  int32_t it_ref[kHItems];               // bin b, kHBins + penalised bin p, or -1 - singleton slot
  int32_t it_aux[kHItems];               // penalised bin merged into bin b, or -1
  uint32_t xcode[kHXCap];                // extra items: kHBins + p, or singleton slot
  int32_t aux_q[kHSegBins];
  float rys[kHSegBins];                  // y and unpenalised count of its bins
  uint32_t rcs[kHSegBins];
  float red3[kSW][3];
  uint32_t red_u[kSW];
  uint32_t red_v[kSW];
  unsigned long long red_w[kSW];
  float red_m[kSW];
  uint32_t ns;
  uint32_t chunk_ctr;
  int32_t seg_pick;
  int32_t fallback;
  uint32_t pick_c;
  unsigned long long pick_w;
  int32_t res_ref, res_aux, res_j;
  uint32_t res_c, res_cb;
  unsigned long long res_wb, res_w;
  int32_t id_out[2];
  int32_t walk_w[2];
  uint32_t walk_lo[2];
};
static_assert(sizeof(HistSmem) <= 160 * 1024, "one workgroup per CU");
static_assert(2 * kSW * kHListCap <= kHBins + kWave, "the id lists fit in the bin counts");

// Block maximum of a float (every thread gets it).
__device__ __forceinline__ float block_max_hist(HistSmem& sm, float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) sm.red_m[threadIdx.x / kWave] = v;
  __syncthreads();
  float r = sm.red_m[0];
#pragma unroll
  for (int w = 1; w < kSW; ++w) r = fmaxf(r, sm.red_m[w]);
  return r;
}

__device__ __forceinline__ int hbin_of(uint32_t h) {
  const uint32_t mag = h & 0x7FFFu, e = mag >> 7;
  if (e < kHELo || e >= kHELo + 64u) return -1;
  const int idx = (int)(mag - (kHELo << 7));
  return (h & 0x8000u) ? (kHBins / 2 - 1 - idx) : (kHBins / 2 + idx);
}
__device__ __forceinline__ uint32_t hbin_bits(int b) {
  return b >= kHBins / 2 ? (uint32_t)(b - kHBins / 2) + (kHELo << 7)
                         : 0x8000u | ((uint32_t)(kHBins / 2 - 1 - b) + (kHELo << 7));
}
__device__ __forceinline__ uint32_t pcnt_of(const HistSmem& sm, int p) {
  return (sm.pcnt2[p >> 1] >> ((p & 1) * 16)) & 0xFFFFu;
}

// Position of the n-th (from 0) set bit of an 8-bit mask.
__device__ __forceinline__ uint32_t nth_bit(uint32_t m, uint32_t n) {
#pragma unroll
  for (uint32_t i = 0; i < 8; ++i)
    if (i < n) m &= m - 1u;
  return (uint32_t)__builtin_ctz(m);
}

// wave sort of 64-bit keys, descending (one per lane)
__device__ __forceinline__ unsigned long long wave_sort_desc_u64(unsigned long long v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int k = 2; k <= kWave; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j >= 1; j >>= 1) {
      const unsigned long long w = __shfl_xor(v, j, kWave);
      const bool desc = (lane & k) == 0;
      const bool lower = (lane & j) == 0;
      v = desc == lower ? (v > w ? v : w) : (v < w ? v : w);
    }
  }
  return v;
}

// One row; false when the row needs the row-wise path instead.  Without a
// mask every token is counted in the bins or kept as a singleton, so the
// raw log-sum-exp comes from the counts (one exp per distinct value) and
// the stream does no floating-point work; with a mask the stream folds it
// token by token.
template <typename T, bool kMask>
__device__ __forceinline__ bool hist_row(const SamplerArgs& a, int64_t b, HistSmem& sm) {
  static_assert(sizeof(T) == 2, "bf16 rows only");
  constexpr bool kLseStream = kMask;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  const T* __restrict__ row = reinterpret_cast<const T*>(a.logits) + b * a.row_stride;
  const uint32_t* __restrict__ mrow = kMask ? a.mask + b * a.mask_stride : nullptr;
  const int64_t V = a.V, nvec = V / 8;
  const bool use_pen = a.hist && a.hist_len > 0 && a.rho != 1.0f;
  const float Tc = a.T > 1e-6f ? a.T : 1e-6f;
  const float rho = a.rho;
  const float u = a.uniforms[b];
  auto xbin = [&](int bn) __attribute__((always_inline)) -> float {
    return u2f(hbin_bits(bn) << 16);
  };
  auto ybin = [&](int bn) __attribute__((always_inline)) -> float { return xbin(bn) / Tc + 0.0f; };
  auto ypen = [&](float x) __attribute__((always_inline)) -> float {
    const float xp = x < 0.0f ? x * rho : x / rho;
    return xp / Tc + 0.0f;
  };
  auto ypbin = [&](int p) __attribute__((always_inline)) -> float { return ypen(xbin(p)); };
  auto is_pen = [&](int64_t id) __attribute__((always_inline)) -> bool {
    return use_pen && ((sm.pen[id >> 5] >> (id & 31)) & 1u);
  };
  auto allowed = [&](int64_t id) __attribute__((always_inline)) -> bool {
    return !kMask || ((mrow[id >> 5] >> (id & 31)) & 1u);
  };
  // largest bin whose y <= y (-1: none): from the bin of y * T (within a
  // bin or two of the answer), else by bisection
  auto place = [&](float y) __attribute__((always_inline)) -> int {
    int g = hbin_of(f2u(y * Tc) >> 16);
    if (g >= 0) {
      while (g + 1 < kHBins && ybin(g + 1) <= y) ++g;
      while (g >= 0 && ybin(g) > y) --g;
      return g;
    }
    int lo = 0, hi = kHBins - 1, bf = -1;
    while (lo <= hi) {
      const int mid = (lo + hi) >> 1;
      if (ybin(mid) <= y) {
        bf = mid;
        lo = mid + 1;
      } else {
        hi = mid - 1;
      }
    }
    return bf;
  };

  // ---- 0. clear
  for (int i = tid; i < kHBins + kWave; i += kSB) sm.cnt[i] = 0u;
  for (int i = tid; i < kHBins / 2; i += kSB) sm.pcnt2[i] = 0u;
  if (use_pen)
    for (int i = tid; i < (int)((V + 31) / 32); i += kSB) sm.pen[i] = 0u;
  sm.segw[tid] = 0ull;
  sm.segc[tid] = 0u;
  sm.seg_plo[tid] = 0xFFFFu;
  sm.seg_phi[tid] = 0u;
  if (tid < kHSegBins) sm.aux_q[tid] = -1;
  if (tid == 0) {
    sm.ns = 0u;
    sm.chunk_ctr = 0u;
    sm.fallback = 0;
  }
  __syncthreads();

  // ---- 1. stream: value counts, singletons (and with a mask the raw
  // log-sum-exp)
  Lse3 st{kNegInf, 0.0f, 0.0f};
  auto single = [&](int64_t id, float x) __attribute__((always_inline)) {
    const uint32_t slot = atomicAdd(&sm.ns, 1u);
    if (slot < (uint32_t)kHSCap) {
      sm.sid[slot] = (uint32_t)id;
      sm.sx[slot] = x;
    }
  };
  auto fold = [&](float(&x)[kHG][8], const u32x4(&raw)[kHG], uint32_t sw, int64_t vbase,
                  bool last) __attribute__((always_inline)) {
    if (kLseStream) {
      float gm[kHG];
#pragma unroll
      for (int k = 0; k < kHG; ++k) gm[k] = vec_max<8>(x[k]);
      if (last) {
#pragma unroll
        for (int k = 0; k < kHG; ++k)
          if (vbase + (int64_t)k * kWave >= nvec) {
            gm[k] = kNegInf;
#pragma unroll
            for (int j = 0; j < 8; ++j) x[k][j] = kNegInf;
          }
      }
      float cm = gm[0];
#pragma unroll
      for (int k = 1; k + 1 < kHG; k += 2) cm = max3raw(cm, gm[k], gm[k + 1]);
      if (!(kHG & 1)) cm = max3raw(cm, gm[kHG - 1], gm[kHG - 1]);
      lse_fold_block_max<false, kHG, 8>(st, x, cm);
    }
#pragma unroll
    for (int k = 0; k < kHG; ++k) {
      const int64_t vi = vbase + (int64_t)k * kWave;
      uint32_t ab = 0xFFu;
      if (kMask) {
        const uint32_t o = (uint32_t)(k * kWave + lane) * 8u;
        ab = ((uint32_t)__shfl((int)sw, (int)(o >> 5), kWave) >> (o & 31u)) & 0xFFu;
      }
      if (last && vi >= nvec) ab = 0u;
      const uint32_t wds[4] = {raw[k].x, raw[k].y, raw[k].z, raw[k].w};
      uint32_t sg = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        // bin = 2^13 + (idx ^ sign): 2^13 + idx for x > 0, 2^13 - 1 - idx for x < 0
        const uint32_t w = wds[j >> 1];
        const uint32_t h = (j & 1) ? w >> 16 : w & 0xFFFFu;
        const uint32_t mag = h & 0x7FFFu;
        const uint32_t sgn = (j & 1) ? (uint32_t)((int32_t)w >> 31)
                                     : (uint32_t)((int32_t)(w << 16) >> 31);
        const uint32_t idx = mag - (kHELo << 7);
        const bool in = idx < 64u * 128u;
        const bool ok = (ab >> j) & 1u;
        // tokens outside the bins and masked tokens count in the lane's spill word
        atomicAdd(&sm.cnt[in && ok ? (idx ^ sgn) + kHBins / 2 : kHBins + lane], 1u);
        // kept one by one: allowed tokens outside the bins except -inf
        // (NaN and +inf among them make the row non-finite)
        sg |= (ok && !in && h != 0xFF80u) ? (1u << j) : 0u;
      }
      if (sg) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if ((sg >> j) & 1u) single(vi * 8 + j, x[k][j]);
      }
    }
  };
  stream_chunks<T, kHG, false, kMask>(row, 0, nvec, mrow, &sm.chunk_ctr, fold);
  for (int64_t id = nvec * 8 + tid; id < V; id += kSB) {
    const float xv = Elem<T>::get(row, id);
    if (kLseStream) {
      float x1[1][4] = {{xv, kNegInf, kNegInf, kNegInf}};
      lse_fold_block_max<false, 1, 4>(st, x1, xv);
    }
    if (allowed(id)) {
      const uint32_t h = f2u(xv) >> 16;
      const int bn = hbin_of(h);
      if (bn >= 0)
        atomicAdd(&sm.cnt[bn], 1u);
      else if (h != 0xFF80u)
        single(id, xv);
    }
  }
  float lm = st.m, ls = st.s;
  if (kLseStream)
    block_lse2<kSB>(lm, ls, sm.red3);  // its barrier completes the counts and singletons
  else
    __syncthreads();

  // ---- history: each distinct, allowed penalised id moves to the
  // penalised count of its value (singletons read the bitmap later)
  bool bad_hist = false;
  if (a.hist && a.hist_len > 0) {
    const int32_t* hr = a.hist + b * a.hist_stride;
    for (int64_t j = tid; j < a.hist_len; j += kSB) {
      const int32_t id = hr[j];
      if (id >= V) {
        bad_hist = true;
      } else if (id >= 0 && use_pen) {
        const uint32_t bit = 1u << (id & 31);
        const uint32_t old = atomicOr(&sm.pen[id >> 5], bit);
        if (!(old & bit) && allowed(id)) {
          const int bn = hbin_of((uint32_t)row[id]);
          if (bn >= 0) {
            atomicSub(&sm.cnt[bn], 1u);
            atomicAdd(&sm.pcnt2[bn >> 1], 1u << ((bn & 1) * 16));
          }
        }
      }
    }
  }
  bad_hist = __syncthreads_or(bad_hist);
  const uint32_t ns = sm.ns;
  if (!kLseStream && ns > (uint32_t)kHSCap) return false;  // the count-based sum needs them all

  // ---- 2. the bins, in blocks of 64 values: wave w takes blocks w, w + 16,
  // ... (so dense value ranges spread over all waves) and skips empty
  // blocks; a row of 16 lanes covers one segment.
  // Pass A: raw log-sum-exp terms from the counts (without a mask), each
  // segment's unpenalised count, the lane's highest bins with tokens.
  float lm_l = kNegInf, ls_l = 0.0f;
  int top_u = -1, lo_p = -1, hi_p = -1;
#pragma unroll 1
  for (int kb = 0; kb < kHBins / kSB; ++kb) {
    const int bb = kb * kSB + wid * kWave + lane;
    const uint32_t c = sm.cnt[bb], pc = pcnt_of(sm, bb);
    if (__ballot((c | pc) != 0u) == 0ull) continue;
    if (c) top_u = bb;
    if (pc) {
      hi_p = bb;
      if (lo_p < 0) lo_p = bb;
    }
    if (!kLseStream && (c | pc)) {  // values rise with kb: each is the lane's new maximum
      const float x = xbin(bb);
      ls_l = ls_l * __builtin_amdgcn_exp2f((lm_l - x) * kLog2e) + (float)(c + pc);
      lm_l = x;
    }
    const uint32_t rs = row_scan_u32(c);
    if ((lane & 15) == 15) sm.segc[bb >> 4] = rs;
  }
  if (!kLseStream) {
    // singletons (a NaN one makes the sum NaN, an infinite one the maximum)
    for (uint32_t s = tid; s < ns; s += kSB) {
      const float x = sm.sx[s];
      if (x > lm_l) {
        ls_l = ls_l * __builtin_amdgcn_exp2f((lm_l - x) * kLog2e) + 1.0f;
        lm_l = x;
      } else {
        ls_l += __builtin_amdgcn_exp2f((x - lm_l) * kLog2e);
      }
    }
    const float mw = wave_max_f(lm_l);
    float sw = ls_l * __builtin_amdgcn_exp2f((lm_l - mw) * kLog2e);
    if (!(lm_l > kNegInf)) sw = ls_l;  // no terms (0), or a NaN sum
    sw = wave_sum_f(sw);
    if (lane == 0) {
      sm.red3[wid][0] = mw;
      sm.red3[wid][1] = sw;
    }
    __syncthreads();
    float mb = kNegInf;
#pragma unroll
    for (int w = 0; w < kSW; ++w) mb = fmaxf(mb, sm.red3[w][0]);
    float sb = 0.0f;
#pragma unroll
    for (int w = 0; w < kSW; ++w) {
      const float mwv = sm.red3[w][0], swv = sm.red3[w][1];
      sb += mwv > kNegInf ? swv * __builtin_amdgcn_exp2f((mwv - mb) * kLog2e) : swv;
    }
    lm = mb;
    ls = sb;
  }
  // logprob = x - m - ln s, rounded once (raw_logprob)
  const float lse_m = lm, lse_ln = __builtin_amdgcn_logf(ls) * kLn2;
  int32_t status = GTP_ROW_OK;
  if (ls != ls || lm == kPosInf)
    status = GTP_ROW_NONFINITE;
  else if (bad_hist)
    status = GTP_ROW_BAD_HISTORY;
  else if (!(u >= 0.0f && u < 1.0f))
    status = GTP_ROW_BAD_UNIFORM;
  if (status != GTP_ROW_OK) {
    if (tid == 0) write_row(a, b, status, -1, 0.f, 0.f, 0, 0.f, -1);
    return true;
  }
  if (ns > (uint32_t)kHSCap) return false;

  // m = the largest processed logit (y of penalised values is monotone in
  // the value: a lane's extremes bound it, and show an overflow to +-inf)
  float ymax = top_u >= 0 ? ybin(top_u) : kNegInf;
  bool odd = false;
  if (hi_p >= 0) {
    const float yh = ypbin(hi_p), yl = ypbin(lo_p);
    odd = !(yh < kPosInf && yl > kNegInf);
    ymax = fmaxf(ymax, yh);
  }
  for (uint32_t s = tid; s < ns; s += kSB) {
    const float x = sm.sx[s];
    const float y = is_pen(sm.sid[s]) ? ypen(x) : x / Tc + 0.0f;
    odd |= !(y > kNegInf && y < kPosInf);
    ymax = fmaxf(ymax, y);
  }
  ymax = wave_max_f(ymax);
  odd = __ballot(odd) != 0ull;
  __syncthreads();
  if (lane == 0) {
    sm.red_m[wid] = ymax;
    sm.red_u[wid] = odd ? 1u : 0u;
  }
  __syncthreads();
  float m = kNegInf;
  uint32_t any_odd = 0;
#pragma unroll
  for (int w = 0; w < kSW; ++w) {
    m = fmaxf(m, sm.red_m[w]);
    any_odd |= sm.red_u[w];
  }
  if (any_odd) return false;
  // Pass B: weights.  Bins sum per segment (row of 16 lanes); penalised
  // values and singletons join the segment of the largest bin at or below
  // their y, and a segment records the range of penalised values it got.
#pragma unroll 1
  for (int kb = 0; kb < kHBins / kSB; ++kb) {
    const int bb = kb * kSB + wid * kWave + lane;
    const uint32_t c = sm.cnt[bb], pc = pcnt_of(sm, bb);
    if (__ballot((c | pc) != 0u) == 0ull) continue;
    const unsigned long long w = c ? (unsigned long long)c * detexp_fix(ybin(bb) - m) : 0ull;
    const unsigned long long rw = row_scan_u64(w);
    if ((lane & 15) == 15 && rw) atomicAdd(&sm.segw[bb >> 4], rw);
    if (pc) {
      const float y = ypbin(bb);
      const int bf = place(y);
      const int sg = bf < 0 ? 0 : bf / kHSegBins;
      atomicMin(&sm.seg_plo[sg], (uint32_t)bb);
      atomicMax(&sm.seg_phi[sg], (uint32_t)bb + 1u);
      atomicAdd(&sm.segw[sg], (unsigned long long)pc * detexp_fix(y - m));
      atomicAdd(&sm.segc[sg], pc);
    }
  }
  for (uint32_t s = tid; s < ns; s += kSB) {
    const float x = sm.sx[s];
    const float y = is_pen(sm.sid[s]) ? ypen(x) : x / Tc + 0.0f;
    const int bf = place(y);
    sm.sbin[s] = bf < 0 ? (uint16_t)0xFFFFu : (uint16_t)bf;
    const int sg = bf < 0 ? 0 : bf / kHSegBins;
    atomicAdd(&sm.segw[sg], detexp_fix(y - m));
    atomicAdd(&sm.segc[sg], 1u);
  }
  __syncthreads();
  const unsigned long long W_t = sm.segw[tid];
  const uint32_t C_t = sm.segc[tid];
  // count / weight of all segments above this one (descending order)
  unsigned long long aW, W_all;
  uint32_t aC, n_valid;
  {
    const unsigned long long iw = wave_scan_u64(W_t);
    const uint32_t ic = wave_scan_u32(C_t);
    const unsigned long long tw = lane63_u64(iw);
    const uint32_t tc = lane63_u32(ic);
    if (lane == 0) {
      sm.red_w[wid] = tw;
      sm.red_u[wid] = tc;
    }
    __syncthreads();
    unsigned long long hw = 0;
    uint32_t hc = 0;
    W_all = 0;
    n_valid = 0;
#pragma unroll
    for (int w = 0; w < kSW; ++w) {
      if (w > wid) {
        hw += sm.red_w[w];
        hc += sm.red_u[w];
      }
      W_all += sm.red_w[w];
      n_valid += sm.red_u[w];
    }
    aW = hw + (tw - iw);
    aC = hc + (tc - ic);
  }
  if (n_valid == 0u) {
    if (tid == 0) write_row(a, b, GTP_ROW_EMPTY, -1, 0.f, 0.f, 0, 0.f, -1);
    return true;
  }

  // ---- 3. searches.  pick(): the segment whose interval holds the target
  // (its count and weight above broadcast with it).
  auto pick = [&](bool mine) __attribute__((always_inline)) {
    __syncthreads();
    if (tid == 0) sm.seg_pick = -1;
    __syncthreads();
    if (mine) {
      sm.seg_pick = tid;
      sm.pick_c = aC;
      sm.pick_w = aW;
    }
    __syncthreads();
  };
  // Resolve segment t (wave 0): its items in rank order.  mode 0: the item
  // holding in-segment rank v; mode 1: the item holding in-segment weight
  // offset v (the rank inside it is an integer quotient).  Returns false
  // (block-uniform) when the segment is outside the bounds of this path.
  auto resolve = [&](int t, int mode, unsigned long long v)
                     __attribute__((always_inline)) -> bool {
    __syncthreads();
    if (wid == 0) {
      const int b0 = t * kHSegBins;
      const int plo = (int)sm.seg_plo[t], phi = (int)sm.seg_phi[t];
      bool bad = phi - plo > kHPenSpan;
      // extra items: the penalised values placed here, and the segment's
      // singletons
      uint32_t k = 0, k_pen = 0;
      if (!bad) {
        for (int base = plo; base < phi; base += kWave) {
          const int p = base + lane;
          const bool ext = p < phi && pcnt_of(sm, p) != 0u;
          const unsigned long long mk = __ballot(ext);
          const uint32_t pos = k + (uint32_t)__builtin_popcountll(mk & ((1ull << lane) - 1ull));
          if (ext && pos < (uint32_t)kHXCap) sm.xcode[pos] = (uint32_t)(kHBins + p);
          k += (uint32_t)__builtin_popcountll(mk);
        }
        k_pen = k;
        for (uint32_t base = 0; base < ns; base += kWave) {
          const uint32_t s = base + (uint32_t)lane;
          bool in = false;
          if (s < ns) {
            const uint32_t sb = sm.sbin[s];
            in = (sb == 0xFFFFu ? 0 : (int)sb / kHSegBins) == t;
          }
          const unsigned long long mk = __ballot(in);
          const uint32_t pos = k + (uint32_t)__builtin_popcountll(mk & ((1ull << lane) - 1ull));
          if (in && pos < (uint32_t)kHXCap) sm.xcode[pos] = s;
          k += (uint32_t)__builtin_popcountll(mk);
        }
        bad = k > (uint32_t)kHXCap;
      }
      wave_lds_sync();
      if (!bad && k == 0) {
        // no extra items: the segment's bins in descending order (lane l
        // holds bin 15 - l), counted and weighed by scans in registers
        const int q = kHSegBins - 1 - lane;
        const uint32_t c = lane < kHSegBins ? sm.cnt[b0 + q] : 0u;
        const unsigned long long w = c ? detexp_fix(ybin(b0 + q) - m) : 0ull;
        const unsigned long long wt = (unsigned long long)c * w;
        const uint32_t cb = wave_scan_u32(c) - c;
        const unsigned long long wb = wave_scan_u64(wt) - wt;
        const bool hit = mode == 0 ? (v >= cb && v < (unsigned long long)cb + c)
                                   : (v >= wb && v < wb + wt);
        if (hit) {
          sm.res_ref = b0 + q;
          sm.res_aux = -1;
          sm.res_j = (int32_t)(mode == 0 ? v - cb : (v - wb) / w);  // w > 0 on a weight hit
          sm.res_c = c;
          sm.res_cb = cb;
          sm.res_wb = wb;
          sm.res_w = w;
        }
        if (lane == 0) sm.fallback = 0;
      } else {
      // the segment's bins, in scalar registers
      float ys[kHSegBins];
      uint32_t cs[kHSegBins];
      unsigned long long wq[kHSegBins];
      {
        const float yl = lane < kHSegBins ? ybin(b0 + lane) : 0.0f;
        const uint32_t cl = lane < kHSegBins ? sm.cnt[b0 + lane] : 0u;
        const unsigned long long wl = cl ? detexp_fix(yl - m) : 0ull;
#pragma unroll
        for (int q = 0; q < kHSegBins; ++q) {
          ys[q] = u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(yl), q));
          cs[q] = (uint32_t)__builtin_amdgcn_readlane((int)cl, q);
          wq[q] = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(wl >> 32), q)
                   << 32) |
                  (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)wl, q);
        }
      }
      // extras sorted by rank: key = (ord y, ~tag), tag = id << 12 | slot for
      // a singleton, 2^30 | p for a penalised value.  Penalised values come
      // in rising order, so without singletons reading them backwards sorts
      // them.
      const bool have = !bad && (uint32_t)lane < k;
      const bool presorted = k_pen == k;
      unsigned long long key = 0;
      if (have) {
        const uint32_t code = sm.xcode[presorted ? k - 1u - (uint32_t)lane : (uint32_t)lane];
        float y;
        uint32_t tag;
        if (code >= (uint32_t)kHBins) {
          const int p = (int)code - kHBins;
          y = ypbin(p);
          tag = 0x40000000u | (uint32_t)p;
        } else {
          const uint32_t id = sm.sid[code];
          const float x = sm.sx[code];
          y = is_pen(id) ? ypen(x) : x / Tc + 0.0f;
          tag = (id << 12) | code;
        }
        key = ((unsigned long long)ord32(y) << 32) | (unsigned long long)(0xFFFFFFFFu - tag);
      }
      if (k > 1u && !bad && !presorted) key = wave_sort_desc_u64(key);
      const uint32_t tag_me = 0xFFFFFFFFu - (uint32_t)key;
      const uint32_t oy_me = (uint32_t)(key >> 32);
      const float y_me = have ? unord32(oy_me) : kNegInf;
      const bool pen_item = have && (tag_me & 0x40000000u);
      // a penalised value equal to a bin with tokens merges into it; other
      // equalities the item order cannot express leave this path
      int merge_q = -1;
      uint32_t nb_above = 0;
      bool tie = false;
#pragma unroll
      for (int q = 0; q < kHSegBins; ++q) {
        if (cs[q]) {
          nb_above += ys[q] > y_me ? 1u : 0u;
          if (have && ys[q] == y_me) {
            if (pen_item)
              merge_q = q;
            else
              tie = true;
          }
        }
      }
      {
        const uint32_t oy_next = (uint32_t)__shfl_down((int)oy_me, 1, kWave);
        const bool pen_next = __shfl_down((int)pen_item, 1, kWave) != 0;
        tie |= have && (uint32_t)lane + 1u < k && oy_next == oy_me && (pen_item || pen_next);
      }
      bad |= __ballot(tie) != 0ull;
      const unsigned long long merged = __ballot(merge_q >= 0);
      const bool own = have && merge_q < 0;  // an item of its own
      const uint32_t rank_me =
          (uint32_t)__builtin_popcountll(__ballot(own) & ((1ull << lane) - 1ull));
      const uint32_t n_own_x = (uint32_t)__builtin_popcountll(__ballot(own));
      if (!bad) {
        if (merge_q >= 0) sm.aux_q[merge_q] = (int32_t)(tag_me & 0x3FFFFu);
        if (own) {
          const uint32_t pos = rank_me + nb_above;
          sm.it_w[pos] = detexp_fix(y_me - m);
          if (pen_item) {
            const int p = (int)(tag_me & 0x3FFFFu);
            sm.it_c[pos] = pcnt_of(sm, p);
            sm.it_ref[pos] = kHBins + p;
          } else {
            sm.it_c[pos] = 1u;
            sm.it_ref[pos] = -1 - (int32_t)(tag_me & 0xFFFu);
          }
          sm.it_aux[pos] = -1;
        }
        wave_lds_sync();
        uint32_t nzb = 0;
#pragma unroll
        for (int q = kHSegBins - 1; q >= 0; --q) {
          if (cs[q]) {
            const unsigned long long above_x = __ballot(own && y_me > ys[q]);
            if (lane == 0) {
              const uint32_t pos = nzb + (uint32_t)__builtin_popcountll(above_x);
              const int32_t ax = merged ? sm.aux_q[q] : -1;
              sm.it_w[pos] = wq[q];
              sm.it_c[pos] = cs[q] + (ax >= 0 ? pcnt_of(sm, ax) : 0u);
              sm.it_ref[pos] = b0 + q;
              sm.it_aux[pos] = ax;
            }
            ++nzb;
          }
        }
        wave_lds_sync();
        const uint32_t n_it = nzb + n_own_x;
        uint32_t c2[2] = {0u, 0u};
        unsigned long long w2[2] = {0ull, 0ull}, wt2[2] = {0ull, 0ull};
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const uint32_t i = 2u * (uint32_t)lane + (uint32_t)q;
          if (i < n_it) {
            c2[q] = sm.it_c[i];
            w2[q] = sm.it_w[i];
            wt2[q] = (unsigned long long)c2[q] * w2[q];
          }
        }
        const uint32_t lc = c2[0] + c2[1];
        const unsigned long long lw = wt2[0] + wt2[1];
        uint32_t cb = wave_scan_u32(lc) - lc;
        unsigned long long wb = wave_scan_u64(lw) - lw;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const uint32_t i = 2u * (uint32_t)lane + (uint32_t)q;
          if (i < n_it) {
            bool hit = false;
            uint32_t jj = 0;
            if (mode == 0) {
              hit = v >= cb && v < (unsigned long long)cb + c2[q];
              jj = (uint32_t)(v - cb);
            } else {
              hit = v >= wb && v < wb + wt2[q];
              if (hit) jj = (uint32_t)((v - wb) / w2[q]);  // w2 > 0 on a hit
            }
            if (hit) {
              sm.res_ref = sm.it_ref[i];
              sm.res_aux = sm.it_aux[i];
              sm.res_j = (int32_t)jj;
              sm.res_c = c2[q];
              sm.res_cb = cb;
              sm.res_wb = wb;
              sm.res_w = w2[q];
            }
            cb += c2[q];
            wb += wt2[q];
          }
        }
      }
      if (lane < kHSegBins) sm.aux_q[lane] = -1;
      if (lane == 0) sm.fallback = bad ? 1 : 0;
      }
    }
    __syncthreads();
    return sm.fallback == 0;
  };
  const bool p_active = a.P > 0.0f && a.P < 1.0f;
  const bool k_active = a.K >= 1 && (uint32_t)a.K < n_valid;
  const uint32_t nk = k_active ? (uint32_t)a.K : n_valid;
  // Three searches over the rank order, one resolved segment each
  // (S_r: the weight of the ranks before r):
  // (0) top-k: the rank nk - 1, W_K = S_nk;
  // (1) top-p: the rank r* whose weight interval holds F = floor(P W_K).
  //     #{r : S_r <= F} = r* + 1, so R = min(nk, r* + 1), and when r* + 1
  //     <= nk, r* is the last kept rank with W' = S_{r*+1}; otherwise the
  //     last kept rank is (0)'s with W' = W_K.  Without top-p, R = nk and
  //     the last kept rank is (0)'s or, without top-k, the last valid rank.
  // (2) the draw: the rank whose weight interval holds U = floor(u W').
  unsigned long long W_K = W_all, Wp = 0, w_draw = 0;
  uint32_t R = nk;
  int32_t thr_ref = 0, thr_aux = -1, thr_j = 0, drw_ref = 0, drw_aux = -1, drw_j = 0;
  bool have_thr = false;
  for (int step = 0; step < 4; ++step) {
    if ((step == 0 && !k_active) || (step == 1 && !p_active) || (step == 2 && have_thr)) continue;
    // step 2: the last valid rank (neither top-k nor top-p active)
    const int mode = step == 0 || step == 2 ? 0 : 1;
    const unsigned long long target = step == 0   ? (unsigned long long)(nk - 1u)
                                      : step == 1 ? floor_mul(a.P, W_K)
                                      : step == 2 ? (unsigned long long)(nk - 1u)
                                                  : floor_mul(u, Wp);
    pick(mode == 0 ? (C_t && aC <= target && target < (unsigned long long)aC + C_t)
                   : (W_t && aW <= target && target < aW + W_t));
    if (sm.seg_pick < 0) return false;
    if (!resolve(sm.seg_pick, mode, target - (mode == 0 ? sm.pick_c : sm.pick_w))) return false;
    const unsigned long long S_after =
        sm.pick_w + sm.res_wb + (unsigned long long)(sm.res_j + 1) * sm.res_w;
    if (step == 0 || step == 2 ||
        (step == 1 && sm.pick_c + sm.res_cb + (uint32_t)sm.res_j + 1u <= nk)) {
      if (step == 0) W_K = S_after;
      if (step == 1) R = sm.pick_c + sm.res_cb + (uint32_t)sm.res_j + 1u;
      thr_ref = sm.res_ref;
      thr_aux = sm.res_aux;
      thr_j = sm.res_j;
      Wp = S_after;
      have_thr = step != 0 || !p_active;
    } else if (step == 1) {
      have_thr = true;  // the top-k cut binds: (0)'s rank and W' = W_K stay
    } else {
      drw_ref = sm.res_ref;
      drw_aux = sm.res_aux;
      drw_j = sm.res_j;
      w_draw = sm.res_w;
    }
  }

  // ---- 4. ids: a singleton's is known; otherwise the j-th token, in id
  // order, among the allowed tokens with the item's bit pattern (unpenalised
  // for a bin, penalised for a penalised value; both for a merged bin).
  // Wave w rescans the w-th sixteenth of the row, 64 consecutive vectors a
  // step, one a lane; a step with no token equal to a pattern costs only the
  // compares.  The members found in a step are appended to the wave's list
  // of each item in id order (a prefix over the lanes), so the j-th member
  // is read from the list of the wave whose count covers j.  A list holds
  // kHListCap ids (in the bin counts' storage, read no more); a member past
  // that is found by scanning the wave's range again for that position only.
  uint32_t hu1 = kNoPattern, hp1 = kNoPattern, hu2 = kNoPattern, hp2 = kNoPattern;
  if (thr_ref >= kHBins) {
    hp1 = hbin_bits(thr_ref - kHBins);
  } else if (thr_ref >= 0) {
    hu1 = hbin_bits(thr_ref);
    if (thr_aux >= 0) hp1 = hbin_bits(thr_aux);
  }
  if (drw_ref >= kHBins) {
    hp2 = hbin_bits(drw_ref - kHBins);
  } else if (drw_ref >= 0) {
    hu2 = hbin_bits(drw_ref);
    if (drw_aux >= 0) hp2 = hbin_bits(drw_aux);
  }
  const bool need1 = thr_ref >= 0, need2 = drw_ref >= 0;
  __syncthreads();
  if (tid == 0) {
    sm.id_out[0] = need1 ? -1 : (int32_t)sm.sid[-1 - thr_ref];
    sm.id_out[1] = need2 ? -1 : (int32_t)sm.sid[-1 - drw_ref];
    sm.walk_w[0] = sm.walk_w[1] = -1;
  }
  if (need1 || need2) {
    const int64_t nv8 = (V + 7) / 8;
    const int64_t wspan = ((nv8 + kSW - 1) / kSW + 7) & ~(int64_t)7;  // whole 128-byte lines
    // Bit j set: token j of the vector w (tokens 2k and 2k+1 in the low and
    // high half of word k) differs from the pattern pp (the 16-bit pattern in
    // both halves).  Per word a packed 16-bit min(w ^ pp, 1) is 0 in a
    // matching half and 1 otherwise; the halves' bits are then interleaved.
    auto nomatch = [](const u32x4& w, uint32_t pp) __attribute__((always_inline)) -> uint32_t {
      const uint32_t z0 = pk_min_u16(w.x ^ pp, 0x00010001u), z1 = pk_min_u16(w.y ^ pp, 0x00010001u);
      const uint32_t z2 = pk_min_u16(w.z ^ pp, 0x00010001u), z3 = pk_min_u16(w.w ^ pp, 0x00010001u);
      const uint32_t q = z0 | (z1 << 2) | (z2 << 4) | (z3 << 6);  // even tokens at 0-6, odd at 16-22
      return (q & 0xFFFFu) | (q >> 15);
    };
    // the patterns are the same in every lane: keep them in scalar registers
    const uint32_t pu1 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(hu1 * 0x10001u));
    const uint32_t pp1 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(hp1 * 0x10001u));
    const uint32_t pu2 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(hu2 * 0x10001u));
    const uint32_t pp2 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(hp2 * 0x10001u));
    const uint32_t hp1s = (uint32_t)__builtin_amdgcn_readfirstlane((int)hp1);
    const uint32_t hp2s = (uint32_t)__builtin_amdgcn_readfirstlane((int)hp2);
    // kNoPattern * 0x10001 = 0x10000 (no 16-bit pattern): the item has no such tokens
    const int en_u1 = __builtin_amdgcn_readfirstlane((int)(pu1 != 0x10000u));
    const int en_u2 = __builtin_amdgcn_readfirstlane((int)(pu2 != 0x10000u));
    const int en_p = __builtin_amdgcn_readfirstlane((int)(pp1 != 0x10000u || pp2 != 0x10000u));
    // Members of the two items among the 8 tokens of vector vi (w; valid:
    // the tokens inside the row): low byte item 1, high byte item 2.  A
    // penalised token is a member when it has the item's penalised pattern
    // (few tokens are penalised: each is compared by itself), any other when
    // it has the unpenalised one; kNoPattern matches nothing.
    auto members = [&](const u32x4& w, int64_t vi, uint32_t valid, uint32_t okw, uint32_t pnw)
        __attribute__((always_inline)) -> uint32_t {
      const int64_t e0 = vi * 8;
      uint32_t ok = valid;
      if (kMask) ok &= okw >> (e0 & 31);
      const uint32_t pn = use_pen ? (pnw >> (e0 & 31)) & 0xFFu : 0u;
      const uint32_t nu1 = en_u1 ? nomatch(w, pu1) : 0xFFu;
      const uint32_t nu2 = en_u2 ? nomatch(w, pu2) : 0xFFu;
      uint32_t mp = 0;  // penalised members: item 1 in the low byte, item 2 in the high byte
      if (en_p) {
        for (uint32_t m = pn & ok; m; m &= m - 1u) {
          const uint32_t j = (uint32_t)__builtin_ctz(m);
          const uint32_t wk = j < 4u ? (j < 2u ? w.x : w.y) : (j < 6u ? w.z : w.w);
          const uint32_t h = (wk >> ((j & 1u) * 16u)) & 0xFFFFu;
          mp |= ((h == hp1s ? 1u : 0u) | (h == hp2s ? 0x100u : 0u)) << j;
        }
      }
      const uint32_t keep = ~pn & ok;
      return ((~nu1 & keep) | ((~nu2 & keep) << 8) | mp) & 0xFFFFu;
    };
    // This wave's pass over the vectors [r0, r1): member p (from 0, in id
    // order) of item k goes to dst_k[p - lo_k] when p - lo_k < cap_k; n_k
    // returns the item's members in the range.
    auto collect = [&](int64_t r0, int64_t r1, int32_t* dst1, uint32_t lo1, uint32_t cap1,
                       int32_t* dst2, uint32_t lo2, uint32_t cap2, uint32_t& n1, uint32_t& n2)
        __attribute__((always_inline)) {
      constexpr int kU = 8;
      const int64_t vend = r1 < nvec ? r1 : nvec;  // full vectors of the range end here
      n1 = 0;
      n2 = 0;
#pragma unroll 1
      for (int64_t s = r0; s < r1; s += (int64_t)kWave * kU) {
        u32x4 buf[kU];
        uint32_t okw[kU] = {}, pnw[kU] = {};
        if (vend > r0) {
#pragma unroll
          for (int i = 0; i < kU; ++i) {
            const int64_t vi = s + i * kWave + lane, vc = vi < vend ? vi : vend - 1;
            buf[i] = *reinterpret_cast<const u32x4*>(row + vc * 8);
            if (kMask) okw[i] = mrow[vc >> 2];
          }
          if (use_pen) {
#pragma unroll
            for (int i = 0; i < kU; ++i) {
              const int64_t vi = s + i * kWave + lane;
              pnw[i] = sm.pen[(vi < vend ? vi : vend - 1) >> 2];
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < kU; ++i) buf[i] = u32x4{0u, 0u, 0u, 0u};  // no full vector in the range
        }
#pragma unroll
        for (int i = 0; i < kU; ++i) {
          const int64_t vi = s + i * kWave + lane;
          u32x4 w = buf[i];
          uint32_t valid = 0xFFu, okv = kMask ? okw[i] : 0u, pnv = use_pen ? pnw[i] : 0u;
          if (vi >= vend) {
            // the partial last vector, or past the range
            valid = 0u;
            w = u32x4{0u, 0u, 0u, 0u};
            if (vi < r1) {
              const int64_t e0 = vi * 8;
              uint32_t hv[8];
#pragma unroll
              for (int j = 0; j < 8; ++j) hv[j] = e0 + j < V ? (uint32_t)row[e0 + j] : 0u;
              w = u32x4{hv[0] | hv[1] << 16, hv[2] | hv[3] << 16, hv[4] | hv[5] << 16, hv[6] | hv[7] << 16};
              valid = (1u << (uint32_t)(V - e0)) - 1u;
              if (kMask) okv = mrow[e0 >> 5];
              if (use_pen) pnv = sm.pen[e0 >> 5];
            }
          }
          const uint32_t mm = members(w, vi < r1 ? vi : r1 - 1, valid, okv, pnv);  // past the range: none
          if (__ballot(mm != 0u)) {
            const uint32_t m1 = mm & 0xFFu, m2 = mm >> 8;
            const uint32_t c = (uint32_t)__builtin_popcount(m1) | ((uint32_t)__builtin_popcount(m2) << 16);
            uint32_t ex, tot;
            if (__ballot((c & 0xFFFEFFFEu) != 0u)) {
              // a lane with two members of an item: both counts in one scan (a
              // step holds at most 512 members of an item)
              const uint32_t inc = wave_scan_u32(c);
              tot = lane63_u32(inc);
              ex = inc - c;
            } else {
              // at most one member of each item a lane: the lanes below with one
              const unsigned long long b1 = __ballot(m1 != 0u), b2 = __ballot(m2 != 0u);
              ex = lanes_below(b1) | (lanes_below(b2) << 16);
              tot = (uint32_t)__builtin_popcountll(b1) | ((uint32_t)__builtin_popcountll(b2) << 16);
            }
            // p - lo in unsigned arithmetic: positions before lo wrap past cap
            uint32_t q1 = n1 + (ex & 0xFFFFu) - lo1, q2 = n2 + (ex >> 16) - lo2;
            for (uint32_t m = m1; m; m &= m - 1u, ++q1)
              if (q1 < cap1) dst1[q1] = (int32_t)(vi * 8 + __builtin_ctz(m));
            for (uint32_t m = m2; m; m &= m - 1u, ++q2)
              if (q2 < cap2) dst2[q2] = (int32_t)(vi * 8 + __builtin_ctz(m));
            n1 += tot & 0xFFFFu;
            n2 += tot >> 16;
          }
        }
      }
    };
    int32_t* const lists = reinterpret_cast<int32_t*>(sm.cnt);
    auto wave_range = [&](int w, int64_t& r0, int64_t& r1) __attribute__((always_inline)) {
      r0 = (int64_t)w * wspan < nv8 ? (int64_t)w * wspan : nv8;
      r1 = r0 + wspan < nv8 ? r0 + wspan : nv8;
    };
    {
      int64_t r0, r1;
      wave_range(wid, r0, r1);
      int32_t* const l1 = lists + (size_t)wid * 2 * kHListCap;
      uint32_t n1, n2;
      collect(r0, r1, l1, 0u, need1 ? (uint32_t)kHListCap : 0u, l1 + kHListCap, 0u,
              need2 ? (uint32_t)kHListCap : 0u, n1, n2);
      if (lane == 0) {
        sm.red_u[wid] = n1;
        sm.red_v[wid] = n2;
      }
    }
    __syncthreads();
    if (wid == 0) {
#pragma unroll
      for (int which = 0; which < 2; ++which) {
        if (which == 0 ? need1 : need2) {
          const uint32_t jt = (uint32_t)(which == 0 ? thr_j : drw_j);
          const uint32_t n = lane < kSW ? (which == 0 ? sm.red_u[lane] : sm.red_v[lane]) : 0u;
          const uint32_t inc = wave_scan_u32(n), ex = inc - n;
          if (jt >= ex && jt < inc) {
            if (jt - ex < (uint32_t)kHListCap) {
              sm.id_out[which] = lists[(size_t)lane * 2 * kHListCap + which * kHListCap + (jt - ex)];
            } else {
              sm.walk_w[which] = lane;
              sm.walk_lo[which] = jt - ex;
            }
          }
        }
      }
    }
    __syncthreads();
    if (wid < 2 && sm.walk_w[wid] >= 0) {  // a list too short: wave k finds item k's member
      int64_t r0, r1;
      wave_range(sm.walk_w[wid], r0, r1);
      const uint32_t lo = sm.walk_lo[wid];
      uint32_t n1, n2;
      collect(r0, r1, &sm.id_out[0], lo, wid == 0 ? 1u : 0u, &sm.id_out[1], lo, wid == 1 ? 1u : 0u,
              n1, n2);
    }
  }
  __syncthreads();
  const int32_t id_thr = sm.id_out[0], id_draw = sm.id_out[1];
  if (id_thr < 0 || id_draw < 0) return false;  // not reached: every item has its tokens
  if (tid == 0) {
    float y_thr;
    if (thr_ref >= kHBins) {
      y_thr = ypbin(thr_ref - kHBins);
    } else if (thr_ref >= 0) {
      y_thr = ybin(thr_ref);
    } else {
      const uint32_t s = (uint32_t)(-1 - thr_ref);
      y_thr = is_pen(sm.sid[s]) ? ypen(sm.sx[s]) : sm.sx[s] / Tc + 0.0f;
    }
    const float x_draw = u2f((uint32_t)row[id_draw] << 16);
    const float slp = (float)::log((double)w_draw / (double)Wp);
    write_row(a, b, GTP_ROW_OK, id_draw, raw_logprob(x_draw, lse_m, lse_ln), slp, (int32_t)R, y_thr, id_thr);
  }
  return true;
}

template <typename T, bool kMask>
__global__ __launch_bounds__(kSB) void sampler_hist_kernel(SamplerArgs a) {
  __shared__ union {
    HistSmem h;
    SamplerSmem g;
  } smu;
  const int64_t b = blockIdx.x;
  if (!hist_row<T, kMask>(a, b, smu.h)) {
    __syncthreads();
    rowwise_row<T>(a, b, smu.g);
  }
}

}  // namespace gtp

#include "tokpath_sampler_topp.h"
#include "tokpath_sampler_topp32.h"
#include "tokpath_sampler_topps.h"

using namespace gtp;

namespace gtp {

// Top-p rows without top-k that the top-p kernels take (bf16 or fp32).
bool topp_takes(int dtype, int64_t B, int64_t V, const gtp_sampler_params* p) {
  const bool top_p = p->top_p > 0.0f && p->top_p < 1.0f && (p->top_k <= 0 || (int64_t)p->top_k >= V);
  return (dtype == GTP_DTYPE_BF16 || dtype == GTP_DTYPE_F32) && p->temperature > 0.0f &&
         p->temperature <= 1024.0f && top_p && V >= topp::kMinV && V <= GTP_SAMPLER_MAX_V && B > 0;
}

ToppSplit plan_topp_split(int dtype, int64_t B, int64_t V, const gtp_sampler_params* p, size_t cap) {
  ToppSplit pl{0, 0, 0};
  if (dtype != GTP_DTYPE_BF16 || !topp_takes(dtype, B, V, p) || B > kToppSplitMaxB) return pl;
  const int64_t nvec = V / 8;
  int64_t S = (device_cus() + B - 1) / B;
  if (S > topps::kMaxS) S = topps::kMaxS;
  for (; S >= 2; --S) {
    // slices start on allow-mask word boundaries: vps a multiple of 8 vectors
    const int64_t vps = ((nvec + S - 1) / S + 7) / 8 * 8;
    const int64_t se = (nvec + vps - 1) / vps;
    const size_t hb = ((size_t)B * se * topps::kHdrWords * 4 + 255) / 256 * 256;
    const size_t bytes = kWsZeroBytes + hb + (size_t)B * se * topps::kSlotWords * 4;
    if (se >= 2 && bytes <= cap) {
      pl.S = (int)se;
      pl.vps = vps;
      pl.bytes = bytes;
      break;
    }
  }
  return pl;
}

size_t topp_workspace_bytes(int dtype, int64_t B, int64_t V, const gtp_sampler_params* p, size_t cap) {
  if (!topp_takes(dtype, B, V, p)) return 0;
  const ToppSplit sp = plan_topp_split(dtype, B, V, p, cap);
  return sp.S ? sp.bytes : 0;
}

GeneralRoute route_general(int dtype, int64_t B, int64_t V, bool aligned, int64_t hist_len,
                           bool has_mask, const gtp_sampler_params* p, bool has_ws,
                           size_t workspace_bytes) {
  GeneralRoute r{GTP_ROUTE_ROWWISE, ToppSplit{0, 0, 0}};
  // top-p rows without top-k: the top-p kernels (each runs the row-wise path
  // itself for a row outside its bounds)
  const bool tp = topp_takes(dtype, B, V, p);
  const bool pen = hist_len > 0 && p->repetition_penalty != 1.0f;
  // (penalised counts are 16-bit: at most 65535 history entries)
  // (rows with a mask and no penalty: the split kernel gains nothing from
  // 32 rows on, [64, 151936] 43.4 against 42.1 us)
  if (tp && aligned && dtype == GTP_DTYPE_BF16 && hist_len <= 65535 && has_ws &&
      (pen || !has_mask || B <= 32)) {
    // few bf16 rows: each row split over S workgroups (the workspace holds
    // their counters, headers and slots)
    const ToppSplit sp = plan_topp_split(dtype, B, V, p, workspace_bytes);
    if (sp.S >= 2) {
      r.route = GTP_ROUTE_TOPP_SPLIT;
      r.split = sp;
      return r;
    }
  }
  if (tp && aligned && dtype == GTP_DTYPE_F32) {
    r.route = GTP_ROUTE_TOPP32;  // two reads, the candidates of the cut in LDS
    return r;
  }
  if (tp && aligned && dtype == GTP_DTYPE_BF16 && hist_len <= 65535) {
    r.route = GTP_ROUTE_TOPP;
    return r;
  }
  // bf16 sampling rows on 16-byte aligned rows: the value-histogram kernel
  // (temperature bounded so that distinct bf16 values keep distinct, normal
  // y = x / T)
  if (dtype == GTP_DTYPE_BF16 && aligned && p->temperature > 0.0f && p->temperature <= 1024.0f &&
      hist_len <= 65535)
    r.route = GTP_ROUTE_HIST;
  return r;
}

// One workgroup of 1024 threads per row; handles every row layout, vocabulary
// and parameter combination the contract allows.
int launch_sampler_general(const SamplerArgs& a, int dtype, int64_t B, hipStream_t s,
                           void* workspace, size_t workspace_bytes) {
  const dim3 grid((unsigned)B), block(kSB);
  const int64_t es = dtype == GTP_DTYPE_F32 ? 4 : 2;
  const bool aligned = (reinterpret_cast<uintptr_t>(a.logits) & 15u) == 0 &&
                       ((a.row_stride * es) & 15) == 0;
  gtp_sampler_params p{a.T, a.K, a.P, a.rho};
  const bool pen = a.hist && a.hist_len > 0 && a.rho != 1.0f;
  const int mode = (a.mask ? 2 : 0) | (pen ? 1 : 0);
  const GeneralRoute r = route_general(dtype, B, a.V, aligned, a.hist ? a.hist_len : 0,
                                       a.mask != nullptr, &p, workspace != nullptr,
                                       workspace_bytes);
  switch (r.route) {
    case GTP_ROUTE_TOPP_SPLIT: {
      unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
      const dim3 sgrid((unsigned)r.split.S, (unsigned)B);
      switch (mode) {
        case 0: launch_timed(sampler_topps_kernel<0>, sgrid, block, s, a, ws, r.split.vps); break;
        case 1: launch_timed(sampler_topps_kernel<1>, sgrid, block, s, a, ws, r.split.vps); break;
        case 2: launch_timed(sampler_topps_kernel<2>, sgrid, block, s, a, ws, r.split.vps); break;
        default: launch_timed(sampler_topps_kernel<3>, sgrid, block, s, a, ws, r.split.vps); break;
      }
      break;
    }
    case GTP_ROUTE_TOPP32:
      switch (mode) {
        case 0: launch_timed(sampler_topp32_kernel<0>, grid, block, s, a); break;
        case 1: launch_timed(sampler_topp32_kernel<1>, grid, block, s, a); break;
        case 2: launch_timed(sampler_topp32_kernel<2>, grid, block, s, a); break;
        default: launch_timed(sampler_topp32_kernel<3>, grid, block, s, a); break;
      }
      break;
    case GTP_ROUTE_TOPP:
      switch (mode) {
        case 0: launch_timed(sampler_topp_kernel<0>, grid, block, s, a); break;
        case 1: launch_timed(sampler_topp_kernel<1>, grid, block, s, a); break;
        case 2: launch_timed(sampler_topp_kernel<2>, grid, block, s, a); break;
        default: launch_timed(sampler_topp_kernel<3>, grid, block, s, a); break;
      }
      break;
    case GTP_ROUTE_HIST:
      if (a.mask)
        launch_timed(sampler_hist_kernel<uint16_t, true>, grid, block, s, a);
      else
        launch_timed(sampler_hist_kernel<uint16_t, false>, grid, block, s, a);
      break;
    default:
      switch (dtype) {
        case GTP_DTYPE_BF16:
          launch_timed(sampler_rowwise_kernel<uint16_t>, grid, block, s, a);
          break;
        case GTP_DTYPE_F16:
          launch_timed(sampler_rowwise_kernel<_Float16>, grid, block, s, a);
          break;
        case GTP_DTYPE_F32:
          launch_timed(sampler_rowwise_kernel<float>, grid, block, s, a);
          break;
        default:
          return GTP_ERR_INVALID_ARGUMENT;
      }
  }
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}

}  // namespace gtp
