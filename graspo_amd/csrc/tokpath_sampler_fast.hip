// tokpath_sampler_fast.hip -- the rollout sampler for greedy and top-k rows
// (1 <= k <= 128) on 16-byte aligned rows (gfx950).
//
// One workgroup of 1024 threads per CU.  A row is split into S slices
// (S = ceil(CUs / B), so a B >= 256 batch is one row per workgroup and every
// workgroup of the launch is resident at once): all slices stream together,
// and the selection tails run after the memory system has drained.
//
// 1. Stream (the only HBM read of the slice; tokpath_stream.h).  Per step a
//    wave takes the next chunk of 64 x 5 vectors (8 bf16/fp16 or 4 fp32
//    logits each) from an LDS counter, so all waves finish together, and
//    folds it into an online log-sum-exp of the raw logits (the logprob output) and writes,
//    per vector, a 16-bit order key of its raw maximum rounded up to bf16
//    into LDS.  The slice's allow-mask words are staged in LDS by the stream
//    prologue; a vector with no allowed token gets key 0 and is never looked
//    at again.  History ids are loaded in the prologue and set the slice's
//    penalty bitmap (LDS) after the stream.
// 2. Select.  A processed logit is never above the processed value of its
//    vector's key: the penalty lowers logits when rho >= 1 (for rho < 1 the
//    bound is raised to match), and division by the temperature is monotone.
//    So for a key threshold tau, every token of a vector with key < tau has
//    y <= Y_out = bound(key tau-1).  tau comes from a 256-bin LDS histogram
//    of the keys, sized so that about k / (allowed density) vectors pass; only
//    those vectors are re-read (L2), their tokens get the exact penalty, mask
//    and IEEE division by the temperature, and those with y > Y_out are kept.
//    Once at least k such tokens exist, the slice's top-k (by y desc, id asc)
//    is among them; otherwise tau is moved using the measured hit rate, and
//    finally every vector is taken.  The top k of the kept tokens are ranked
//    by counting (<= 256 tokens) or an 8-bit radix select on the 64-bit
//    (y, id) key (re-reading the passing vectors per digit if more than 1024
//    tokens pass, e.g. under massive exact ties).
// 3. With S == 1 the workgroup finishes the row from LDS.  Otherwise it
//    publishes its sorted top-k and (m, s) to the workspace and the last
//    workgroup of the row to arrive (an epoch-tagged counter advanced with
//    compare-and-swap, so no workgroup ever waits on another) merges the S
//    lists by binary-search ranks.
// 4. Finish: fixed-point weights (DETEXP_FIX), exact top-p cut and
//    inverse-CDF draw over the sorted top-k, outputs.
//
// Every output follows the contract of include/graspo_tokpath.h bit for bit;
// the threshold logic only decides which tokens are evaluated exactly.
//
// Replaces _next_token_from_logits / _sample_next_token
// (src/graspo/backends/graspoflow/tensor_utils.py:649-683).
#include <atomic>

#include "tokpath_sampler_internal.h"
#include "tokpath_stream.h"

namespace gtp {

constexpr int kFT = 1024;                   // threads per workgroup (one per CU)
constexpr int kFWaves = kFT / kWave;
constexpr int kFG = 5;                      // vectors per thread per stream step
constexpr int kSliceVecs = 32768;           // most vectors in one slice (2^18 bf16 tokens)
constexpr int kFastK = 128;                 // largest kept set of this path
constexpr int kCand = 1024;                 // candidate slots (slice and merge)
constexpr int kSel = 2048;                  // re-read list entries per round
constexpr int kPenWords = kSliceVecs * 8 / 32 + 2;
constexpr int kMaxSlices = 64;
constexpr size_t kSlotBytes = 16 + (size_t)kFastK * 16;

struct SliceHead {
  float m;
  float s;
  uint32_t n;
  uint32_t flags;  // bit 0: a history id >= V (reported by slice 0)
};
struct SliceEnt {
  unsigned long long key;
  float x;
  uint32_t pad;
};

struct FastArgs {
  SamplerArgs a;
  int64_t vps;            // vectors per slice
  unsigned char* ws;      // [B] counters (256-byte padded), then B * S slots
  size_t cnt_bytes;
  uint32_t epoch;         // 1..65535, different for consecutive calls
  int32_t Kc;             // entries per slice list (1 when greedy)
  int32_t greedy;
  int32_t use_pen;
  int32_t p_active;
  float Tc;
};

struct FastSmem {
  union {
    uint16_t gkey[kSliceVecs];       // per-vector order keys of the slice
    uint32_t soff[kMaxSlices + 1];   // merge: start of each slice's list in ckey / cx
  } u;
  uint32_t pen[kPenWords];           // penalty bitmap of the slice's tokens
  uint32_t maskw[kPenWords];         // allow-mask words of the slice's tokens
  unsigned long long ckey[kCand];    // candidates (slice), lists (merge)
  float cx[kCand];
  uint16_t sel[kSel];
  unsigned long long skey[kFastK];   // the slice's survivors before sorting
  float sx[kFastK];
  unsigned long long fkey[kFastK];   // the row's top-k, sorted
  float fx[kFastK];
  unsigned long long incl[kFastK];   // inclusive prefix of the fixed-point weights
  uint32_t hist[256];
  float red[kFWaves][3];
  uint32_t redu[kFWaves];
  uint32_t redx[kFWaves][5];
  uint32_t ngt;
  uint32_t chunk_ctr;  // next stream chunk (per-wave dynamic schedule)
  int32_t bucket;
  uint32_t above;
  int32_t flag;
  unsigned long long found;
};
static_assert(sizeof(FastSmem) <= 160 * 1024, "one workgroup per CU");

// ------------------------------------------------------------------ helpers

template <int E>
__device__ __forceinline__ float vec_max(const float (&x)[E]) {
  if constexpr (E == 8) {
    float m = max3raw(x[0], x[1], x[2]);
    m = max3raw(m, x[3], x[4]);
    m = max3raw(m, x[5], x[6]);
    return max3raw(m, x[7], x[7]);
  } else {
    const float m = max3raw(x[0], x[1], x[2]);
    return max3raw(m, x[3], x[3]);
  }
}

// Order key of a vector maximum: its bf16 rounding toward +inf.
template <typename T>
__device__ __forceinline__ uint32_t vec_key(float gm) {
  if constexpr (Elem<T>::kDtype == GTP_DTYPE_BF16)
    return ord16(f2u(gm) >> 16);  // a bf16 maximum is already a bf16 value
  else
    return ord16(bf16_round_up(gm));
}

__device__ __forceinline__ float key_value(uint32_t k) { return u2f(unord16(k) << 16); }

struct Proc {
  int greedy;
  int use_pen;
  float rho;
  float Tc;
  // processed logit (contract steps: penalty, then temperature), zeros canonical
  __device__ __forceinline__ float y(float x, bool pen) const {
    float xp = x;
    if (pen) xp = (x < 0.0f) ? x * rho : x / rho;
    const float v = greedy ? xp : xp / Tc;
    return v + 0.0f;
  }
  // largest processed logit any raw x <= v can reach
  __device__ __forceinline__ float ub(float v) const {
    float vp = v;
    if (use_pen && rho < 1.0f) vp = (v > 0.0f) ? v / rho : v * rho;
    const float r = greedy ? vp : vp / Tc;
    return r + 0.0f;
  }
};

// Exclusive prefix sum over the threads of the block (in thread order).
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* red, uint32_t* total) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  uint32_t incl = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t w = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += w;
  }
  __syncthreads();
  if (lane == kWave - 1) red[wid] = incl;
  __syncthreads();
  uint32_t before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kFWaves; ++w) {
    if (w < wid) before += red[w];
    tot += red[w];
  }
  *total = tot;
  return before + incl - v;
}

// Wave 0: the bucket (walking 255 -> 0) that holds 0-based position `target`
// of a 256-bucket count histogram, and the count above it; nothing is written
// when the histogram holds no more than `target` entries.  Callers sync
// before and after.
__device__ __forceinline__ void find_bucket(FastSmem& sm, uint32_t target) {
  if (threadIdx.x >= kWave) return;
  const int lane = threadIdx.x;
  uint32_t c[4], tot = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    c[q] = sm.hist[255 - 4 * lane - q];
    tot += c[q];
  }
  uint32_t incl = tot;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t w = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += w;
  }
  uint32_t above = incl - tot;
  if (above <= target && target < incl) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (target < above + c[q]) {
        sm.bucket = 255 - 4 * lane - q;
        sm.above = above;
        break;
      }
      above += c[q];
    }
  }
}

// Write one row's outputs (status != OK: id -1, or the pad id when finished).
__device__ __forceinline__ void write_out(const SamplerArgs& a, int64_t b, int32_t status,
                                          int64_t id, float lp, float slp, int32_t kept, float tv,
                                          int32_t tid) {
  const bool fin = a.finished && a.finished[b];
  const bool ok = status == GTP_ROW_OK;
  a.out_ids[b] = fin ? a.pad_id : (ok ? id : -1);
  if (a.out_lp) a.out_lp[b] = ok ? lp : __builtin_nanf("");
  if (a.out_slp) a.out_slp[b] = ok ? slp : __builtin_nanf("");
  if (a.out_kept) a.out_kept[b] = ok ? kept : 0;
  if (a.out_tv) a.out_tv[b] = ok ? tv : 0.0f;
  if (a.out_tid) a.out_tid[b] = ok ? tid : -1;
  if (a.out_status) a.out_status[b] = status;
}

// ------------------------------------------------------------ slice context
//
// The selection tail runs once per workgroup, straight from a cold
// instruction cache, so its code is kept short: rolled loops, one exact
// evaluation site, and the rare paths (heavy ties, long candidate lists, the
// multi-slice merge) out of line.

template <typename T>
struct Slice {
  static constexpr int E = Vec<T>::kE;
  const T* row;
  const uint32_t* mrow;  // allow-mask row or nullptr
  Proc proc;
  int64_t v0, v1;        // vectors [v0, v1)
  int nv;
  int64_t tail0;         // first tail token (last slice only; == V otherwise)
  int64_t V;
  uint32_t w0;           // first penalty word of the slice

  __device__ __forceinline__ uint32_t mask_bits(const FastSmem& sm, int64_t e0, int n) const {
    return mrow ? (sm.maskw[(uint32_t)(e0 >> 5) - w0] >> (e0 & 31)) & ((1u << n) - 1u)
                : (1u << n) - 1u;
  }
  __device__ __forceinline__ uint32_t pen_bits(const FastSmem& sm, int64_t e0, int n) const {
    return (sm.pen[(uint32_t)(e0 >> 5) - w0] >> (e0 & 31)) & ((1u << n) - 1u);
  }
};

// Element j of a loaded 16-byte vector.
template <typename T>
__device__ __forceinline__ float vec_elem(const u32x4& v, int j) {
  if constexpr (Vec<T>::kE == 4) {
    const uint32_t w = j < 2 ? (j == 0 ? v.x : v.y) : (j == 2 ? v.z : v.w);
    return u2f(w);
  } else {
    const int q = j >> 1;
    const uint32_t w = q < 2 ? (q == 0 ? v.x : v.y) : (q == 2 ? v.z : v.w);
    const uint32_t h = (j & 1) ? (w >> 16) : (w & 0xFFFFu);
    if constexpr (Elem<T>::kDtype == GTP_DTYPE_BF16)
      return u2f(h << 16);
    else
      return f16_to_f32((uint16_t)h);
  }
}

// Slice offsets of the vectors whose key is >= tau, in key order of the
// slice, positions [base, base + kSel) of that list written to sm.sel.
// Returns the length of the whole list.  Block-uniform.
__device__ __forceinline__ uint32_t select_vectors(FastSmem& sm, int nv, uint32_t tau,
                                                   uint32_t base) {
  const u32x4* keys = reinterpret_cast<const u32x4*>(sm.u.gkey);
  const int nchunk = (nv + 7) >> 3;
  uint32_t mine = 0;
  for (int j = threadIdx.x; j < nchunk; j += kFT) {
    const u32x4 w = keys[j];
    const uint32_t k[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int q = 0; q < 4; ++q)
      mine += ((k[q] & 0xFFFFu) >= tau ? 1u : 0u) + ((k[q] >> 16) >= tau ? 1u : 0u);
  }
  uint32_t total;
  uint32_t pos = block_excl_scan(mine, sm.redu, &total);
  for (int j = threadIdx.x; j < nchunk && pos < base + kSel; j += kFT) {
    const u32x4 w = keys[j];
    const uint32_t k[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t key = (e & 1) ? (k[e >> 1] >> 16) : (k[e >> 1] & 0xFFFFu);
      if (key >= tau) {
        if (pos >= base && pos < base + kSel) sm.sel[pos - base] = (uint16_t)(j * 8 + e);
        ++pos;
      }
    }
  }
  __syncthreads();
  return total;
}

// f(id, y, x) for every valid token with y > yout of the listed vectors
// sm.sel[0, n).  yout = ub(xout), so a raw x <= xout never passes: only the
// few tokens above xout pay for the exact penalty and IEEE division.
template <typename T, typename F>
__device__ __forceinline__ void emit_listed(const FastSmem& sm, const Slice<T>& c, uint32_t n,
                                            float xout, float yout, F& f) {
  constexpr int E = Vec<T>::kE;
  const u32x4* rv = reinterpret_cast<const u32x4*>(c.row);
  for (uint32_t p = threadIdx.x; p < n; p += kFT) {
    const int64_t vi = c.v0 + sm.sel[p];
    const u32x4 v = rv[vi];
    const int64_t e0 = vi * E;
    const uint32_t mb = c.mask_bits(sm, e0, E);
    const uint32_t pb = c.proc.use_pen ? c.pen_bits(sm, e0, E) : 0u;
    uint32_t cand = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) cand |= (vec_elem<T>(v, j) > xout ? 1u : 0u) << j;
    cand &= mb;
    while (cand) {
      const int j = __builtin_ctz(cand);
      cand &= cand - 1u;
      const float x = vec_elem<T>(v, j);
      const float y = c.proc.y(x, (pb >> j) & 1u);
      if (y > yout) f((int32_t)(e0 + j), y, x);
    }
  }
}

template <typename T, typename F>
__device__ __forceinline__ void emit_tail(const FastSmem& sm, const Slice<T>& c, float xout,
                                          float yout, F& f) {
  for (int64_t id = c.tail0 + threadIdx.x; id < c.V; id += kFT) {
    if (!c.mask_bits(sm, id, 1)) continue;
    const float x = Elem<T>::get(c.row, id);
    if (!(x > xout)) continue;
    const bool pen = c.proc.use_pen && c.pen_bits(sm, id, 1);
    const float y = c.proc.y(x, pen);
    if (y > yout) f((int32_t)id, y, x);
  }
}

// f for every valid token with y > yout in the vectors whose key is >= tau
// and in the tail (any list length).  Block-uniform.
template <typename T, typename F>
__device__ __forceinline__ void for_each_candidate(FastSmem& sm, const Slice<T>& c, uint32_t tau,
                                                   float xout, float yout, F f) {
  uint32_t total = select_vectors(sm, c.nv, tau, 0);
  for (uint32_t base = 0; base < total; base += kSel) {
    if (base > 0) select_vectors(sm, c.nv, tau, base);
    const uint32_t n = total - base < (uint32_t)kSel ? total - base : (uint32_t)kSel;
    emit_listed<T>(sm, c, n, xout, yout, f);
    __syncthreads();
  }
  emit_tail<T>(sm, c, xout, yout, f);
  __syncthreads();
}

// k-th largest (1-based) of n >= k distinct 64-bit keys.  `hist_pass(prefix,
// pmask, shift)` adds, for every key with (key & pmask) == prefix, one count
// to sm.hist[(key >> shift) & 255]; `find_one(prefix, pmask)` stores the
// unique key with that prefix in sm.found.  Block-uniform.
template <typename HistPass, typename FindOne>
__device__ __forceinline__ unsigned long long radix_kth(FastSmem& sm, uint32_t k,
                                                        HistPass hist_pass, FindOne find_one) {
  unsigned long long prefix = 0, pmask = 0;
  uint32_t target = k - 1;
  for (int shift = 56; shift >= 0; shift -= 8) {
    __syncthreads();
    if (threadIdx.x < 256) sm.hist[threadIdx.x] = 0u;
    __syncthreads();
    hist_pass(prefix, pmask, shift);
    __syncthreads();
    find_bucket(sm, target);
    __syncthreads();
    const uint32_t d = (uint32_t)sm.bucket & 0xFFu;
    const uint32_t in_bucket = sm.hist[d];
    target -= sm.above;
    prefix |= (unsigned long long)d << shift;
    pmask |= 0xFFull << shift;
    if (in_bucket == 1u && shift > 0) {
      __syncthreads();
      find_one(prefix, pmask);
      __syncthreads();
      return sm.found;
    }
  }
  return prefix;
}

// Rank of each of n <= kFT distinct keys by counting (one broadcast LDS read
// per wave per key); entries of rank < k go to out(rank, key, x).
// Block-uniform; callers sync before (keys complete).
template <typename Out>
__device__ __forceinline__ void rank_sort_small(const unsigned long long* keys, const float* xs,
                                                uint32_t n, uint32_t k, Out out) {
  if (threadIdx.x < n) {
    const unsigned long long ki = keys[threadIdx.x];
    uint32_t rk = 0;
#pragma unroll 8
    for (uint32_t j = 0; j < n; ++j) rk += keys[j] > ki ? 1u : 0u;
    if (rk < k) out(rk, ki, xs[threadIdx.x]);
  }
}

// The slice's top Kc into sm.skey / sm.sx (unsorted) when more than 256
// tokens beat Y_out: radix select in LDS (<= kCand of them), or, past that
// (massive exact ties), the same select re-reading the passing vectors once
// per digit.  Rare: not executed on the common path.
template <typename T>
__device__ __forceinline__ void select_top_slow(FastSmem& sm, const Slice<T>& c, uint32_t ngt,
                                             uint32_t Kc, uint32_t tau, float xout, float yout) {
  const int tid = threadIdx.x;
  if (ngt <= (uint32_t)kCand) {
    const unsigned long long kth = radix_kth(
        sm, Kc,
        [&](unsigned long long prefix, unsigned long long pmask, int shift) {
          for (uint32_t i = tid; i < ngt; i += kFT) {
            const unsigned long long k = sm.ckey[i];
            if ((k & pmask) == prefix) atomicAdd(&sm.hist[(k >> shift) & 0xFFu], 1u);
          }
        },
        [&](unsigned long long prefix, unsigned long long pmask) {
          for (uint32_t i = tid; i < ngt; i += kFT)
            if ((sm.ckey[i] & pmask) == prefix) sm.found = sm.ckey[i];
        });
    if (tid == 0) sm.ngt = 0u;
    __syncthreads();
    for (uint32_t i = tid; i < ngt; i += kFT) {
      if (sm.ckey[i] >= kth) {
        const uint32_t slot = atomicAdd(&sm.ngt, 1u);
        sm.skey[slot] = sm.ckey[i];
        sm.sx[slot] = sm.cx[i];
      }
    }
  } else {
    const unsigned long long kth = radix_kth(
        sm, Kc,
        [&](unsigned long long prefix, unsigned long long pmask, int shift) {
          for_each_candidate<T>(sm, c, tau, xout, yout, [&](int32_t id, float y, float) {
            const unsigned long long k = rank_key(y, id);
            if ((k & pmask) == prefix) atomicAdd(&sm.hist[(k >> shift) & 0xFFu], 1u);
          });
        },
        [&](unsigned long long prefix, unsigned long long pmask) {
          for_each_candidate<T>(sm, c, tau, xout, yout, [&](int32_t id, float y, float) {
            const unsigned long long k = rank_key(y, id);
            if ((k & pmask) == prefix) sm.found = k;
          });
        });
    if (tid == 0) sm.ngt = 0u;
    __syncthreads();
    for_each_candidate<T>(sm, c, tau, xout, yout, [&](int32_t id, float y, float x) {
      const unsigned long long k = rank_key(y, id);
      if (k >= kth) {
        const uint32_t slot = atomicAdd(&sm.ngt, 1u);
        sm.skey[slot] = k;
        sm.sx[slot] = x;
      }
    });
  }
  __syncthreads();
}

// Finish a row from its sorted top nk (sm.fkey / sm.fx): status, greedy pick
// or fixed-point top-p cut and draw, outputs.  Block-uniform.
__device__ __forceinline__ void finish_row(FastSmem& sm, const FastArgs& fa, int64_t b,
                                        const Lse3& row_lse, bool bad_hist, uint32_t nk) {
  const SamplerArgs& a = fa.a;
  const int tid = threadIdx.x;
  const float u = fa.greedy ? 0.0f : a.uniforms[b];
  const float lse_raw = row_lse.m + __builtin_amdgcn_logf(row_lse.s) * kLn2;
  int32_t status = GTP_ROW_OK;
  if (row_lse.s != row_lse.s || row_lse.m == kPosInf)
    status = GTP_ROW_NONFINITE;
  else if (bad_hist)
    status = GTP_ROW_BAD_HISTORY;
  else if (!fa.greedy && !(u >= 0.0f && u < 1.0f))
    status = GTP_ROW_BAD_UNIFORM;
  else if (nk == 0u)
    status = GTP_ROW_EMPTY;
  else if (rank_key_y(sm.fkey[0]) == kPosInf)
    status = GTP_ROW_NONFINITE;
  if (status != GTP_ROW_OK) {
    if (tid == 0) write_out(a, b, status, -1, 0.f, 0.f, 0, 0.f, -1);
    return;
  }
  const unsigned long long k0 = sm.fkey[0];
  const float m = rank_key_y(k0);
  if (fa.greedy) {
    if (tid == 0) {
      const int32_t id = rank_key_id(k0);
      write_out(a, b, GTP_ROW_OK, id, sm.fx[0] - lse_raw, 0.0f, 1, m, id);
    }
    return;
  }
  // fixed-point weights and their inclusive prefix (wave 0, 2 ranks per lane)
  if (tid < kWave) {
    unsigned long long v[2], tot = 0;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t r = (uint32_t)tid * 2u + q;
      v[q] = r < nk ? detexp_fix(rank_key_y(sm.fkey[r]) - m) : 0ull;
      tot += v[q];
    }
    unsigned long long run = wave_incl_scan_u64(tot) - tot;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t r = (uint32_t)tid * 2u + q;
      run += v[q];
      if (r < nk) sm.incl[r] = run;
    }
  }
  __syncthreads();
  if (tid == 0) {
    const unsigned long long Wk = sm.incl[nk - 1];
    int R = (int)nk;
    if (fa.p_active) {
      const unsigned long long F = floor_mul(a.P, Wk);
      int lo = 0, hi = (int)nk - 1;  // R = 1 + #{r < nk-1 : incl[r] <= F}
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sm.incl[mid] <= F) lo = mid + 1;
        else hi = mid;
      }
      R = lo + 1;
    }
    const unsigned long long Wp = sm.incl[R - 1];
    const unsigned long long U = floor_mul(u, Wp);
    int lo = 0, hi = R - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (sm.incl[mid] <= U) lo = mid + 1;
      else hi = mid;
    }
    const int rs = lo;
    const unsigned long long ws = sm.incl[rs] - (rs ? sm.incl[rs - 1] : 0ull);
    const unsigned long long kt = sm.fkey[R - 1];
    const float slp = __builtin_amdgcn_logf((float)((double)ws / (double)Wp)) * kLn2;
    write_out(a, b, GTP_ROW_OK, rank_key_id(sm.fkey[rs]), sm.fx[rs] - lse_raw, slp, R,
              rank_key_y(kt), rank_key_id(kt));
  }
}

// The last workgroup of a split row: gather the S sorted lists, rank the
// union by binary search, finish.  Block-uniform.
__device__ __forceinline__ void merge_row(FastSmem& sm, const FastArgs& fa, int64_t b, int S) {
  const int tid = threadIdx.x;
  const uint32_t Kc = (uint32_t)fa.Kc;
  const unsigned char* slots = fa.ws + fa.cnt_bytes + (size_t)b * S * kSlotBytes;
  Lse3 part{kNegInf, 0.0f, 0.0f};
  uint32_t my_n = 0, my_flags = 0;
  if (tid < S) {
    const SliceHead* hj = reinterpret_cast<const SliceHead*>(slots + (size_t)tid * kSlotBytes);
    part = Lse3{hj->m, hj->s, 0.0f};
    my_n = hj->n;
    my_flags = hj->flags;
  }
  const Lse3 row_lse = block_lse3<kFT>(part, sm.red);
  const bool any_bad_hist = __syncthreads_or(my_flags & 1u);
  uint32_t total;
  const uint32_t my_off = block_excl_scan(my_n, sm.redu, &total);
  if (tid < S) sm.u.soff[tid] = my_off;
  if (tid == 0) sm.u.soff[S] = total;
  __syncthreads();
  for (uint32_t t = tid; t < total; t += kFT) {
    int lo = 0, hi = S - 1;  // slice j with soff[j] <= t < soff[j+1]
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (sm.u.soff[mid] <= t) lo = mid;
      else hi = mid - 1;
    }
    const SliceEnt* ej =
        reinterpret_cast<const SliceEnt*>(slots + (size_t)lo * kSlotBytes + sizeof(SliceHead));
    const SliceEnt e = ej[t - sm.u.soff[lo]];
    sm.ckey[t] = e.key;
    sm.cx[t] = e.x;
  }
  __syncthreads();
  // rank in the union = index in its own list + entries of the other
  // (descending, distinct) lists above it
  const uint32_t nk = total < Kc ? total : Kc;
  for (uint32_t t = tid; t < total; t += kFT) {
    int lo = 0, hi = S - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (sm.u.soff[mid] <= t) lo = mid;
      else hi = mid - 1;
    }
    const int j = lo;
    const unsigned long long kt = sm.ckey[t];
    uint32_t rk = t - sm.u.soff[j];
    for (int j2 = 0; j2 < S && rk < Kc; ++j2) {
      if (j2 == j) continue;
      uint32_t l2 = sm.u.soff[j2], h2 = sm.u.soff[j2 + 1];  // first entry below kt
      while (l2 < h2) {
        const uint32_t mid = (l2 + h2) >> 1;
        if (sm.ckey[mid] > kt) l2 = mid + 1;
        else h2 = mid;
      }
      rk += l2 - sm.u.soff[j2];
    }
    if (rk < Kc) {
      sm.fkey[rk] = kt;
      sm.fx[rk] = sm.cx[t];
    }
  }
  __syncthreads();
  finish_row(sm, fa, b, row_lse, any_bad_hist, nk);
}

// --------------------------------------------------------------- the kernel

template <typename T>
__global__ __launch_bounds__(kFT) void sampler_split_kernel(FastArgs fa) {
  constexpr int E = Vec<T>::kE;
  constexpr int kHistPer = 4;  // history ids per thread per batch
  __shared__ FastSmem sm;
  const SamplerArgs& a = fa.a;
  const int tid = threadIdx.x;
  const int s = blockIdx.x, S = gridDim.x;
  const int64_t b = blockIdx.y;

  Slice<T> c;
  c.row = reinterpret_cast<const T*>(a.logits) + b * a.row_stride;
  c.mrow = a.mask ? a.mask + b * a.mask_stride : nullptr;
  c.proc = Proc{fa.greedy, fa.use_pen, a.rho, fa.Tc};
  c.V = a.V;
  const int64_t nvec = a.V / E;
  c.v0 = (int64_t)s * fa.vps;
  c.v1 = c.v0 + fa.vps < nvec ? c.v0 + fa.vps : nvec;
  c.nv = (int)(c.v1 - c.v0);
  c.tail0 = s == S - 1 ? nvec * E : a.V;
  const int64_t e0 = c.v0 * E;
  const int64_t e1 = s == S - 1 ? a.V : c.v1 * E;
  c.w0 = (uint32_t)(e0 >> 5);
  const int nw = (int)(((e1 - 1) >> 5) - (e0 >> 5) + 1);
  const bool read_hist = a.hist && a.hist_len > 0 && (fa.use_pen || s == 0);
  const int32_t* hrow = a.hist + b * a.hist_stride;
  if (tid == 0) sm.chunk_ctr = 0u;
  __syncthreads();

  // ---- 0. (stream prologue) history ids into registers, penalty bitmap
  // cleared; the bitmap is filled after the stream, so nothing here waits
  // The allow-mask words of the slice are staged in LDS: one batched load
  // overlapping the first stream round trip, then a barrier before any fold.
  constexpr int kMaskPer = (kPenWords + kFT - 1) / kFT;
  int32_t hv[kHistPer];
  auto setup = [&]() {
    uint32_t mw[kMaskPer];
    if (c.mrow) {
#pragma unroll
      for (int q = 0; q < kMaskPer; ++q) {
        const int i = tid + q * kFT;
        mw[q] = i < nw ? c.mrow[c.w0 + i] : 0u;
      }
    }
    if (read_hist) {
#pragma unroll
      for (int q = 0; q < kHistPer; ++q) {
        const int64_t j = tid + (int64_t)q * kFT;
        hv[q] = j < a.hist_len ? hrow[j] : -1;
      }
    }
    if (fa.use_pen)
      for (int i = tid; i < nw; i += kFT) sm.pen[i] = 0u;
    if (c.mrow) {
#pragma unroll
      for (int q = 0; q < kMaskPer; ++q) {
        const int i = tid + q * kFT;
        if (i < nw) sm.maskw[i] = mw[q];
      }
      __syncthreads();
    }
  };

  // ---- 1. stream: raw log-sum-exp and per-vector keys
  Lse3 st{kNegInf, 0.0f, 0.0f};
  uint32_t nz = 0, allowed = 0;
  float rmax = kNegInf;  // largest vector maximum (its key is the slice's largest)
  auto fold = [&](float(&x)[kFG][E], const uint32_t(&)[kFG], int64_t vbase, bool last) {
    float gm[kFG];
#pragma unroll
    for (int k = 0; k < kFG; ++k) gm[k] = vec_max<E>(x[k]);
    if (last) {
#pragma unroll
      for (int k = 0; k < kFG; ++k)
        if (vbase + (int64_t)k * kWave >= c.v1) {
          gm[k] = kNegInf;
#pragma unroll
          for (int j = 0; j < E; ++j) x[k][j] = kNegInf;
        }
    }
    float cm = gm[0];
#pragma unroll
    for (int k = 1; k + 1 < kFG; k += 2) cm = max3raw(cm, gm[k], gm[k + 1]);
    if (!(kFG & 1)) cm = max3raw(cm, gm[kFG - 1], gm[kFG - 1]);
    lse_fold_block_max<false, kFG, E>(st, x, cm);
#pragma unroll
    for (int k = 0; k < kFG; ++k) {
      const int64_t vi = vbase + (int64_t)k * kWave;
      if (!last || vi < c.v1) {
        uint32_t key = vec_key<T>(gm[k]);
        if (c.mrow) {
          const uint32_t mb = c.mask_bits(sm, vi * E, E);
          if (mb == 0u) {
            key = 0u;
            gm[k] = kNegInf;
          } else {
            ++nz;
            allowed += __builtin_popcount(mb);
          }
        }
        sm.u.gkey[vi - c.v0] = (uint16_t)key;
        rmax = max3raw(rmax, gm[k], gm[k]);
      }
    }
  };
  // non-temporal: the row is read once; the few vectors re-read during
  // selection come back from the MALL
  stream_vectors_dyn<T, kFG, true, false>(c.row, c.v0, c.v1, nullptr, 0, &sm.chunk_ctr, fold,
                                         setup);
  for (int64_t id = c.tail0 + tid; id < a.V; id += kFT) {
    float x[1][4] = {{Elem<T>::get(c.row, id), kNegInf, kNegInf, kNegInf}};
    lse_fold_block_max<false, 1, 4>(st, x, x[0][0]);
  }
  // keys past the slice inside its last 16-byte chunk read as 0
  if (tid < 8 && c.nv + tid < ((c.nv + 7) & ~7)) sm.u.gkey[c.nv + tid] = 0;

  // one combined block reduction: (m, s), the largest vector maximum, nz,
  // allowed.  Its barrier also orders the bitmap clearing before the history
  // atomics below.
  Lse3 lse;
  uint32_t kmax;
  {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const Lse3 w{__shfl_xor(st.m, o, kWave), __shfl_xor(st.s, o, kWave), 0.0f};
      st = lse3_merge(st, w);
      rmax = fmaxf(rmax, __shfl_xor(rmax, o, kWave));
      nz += __shfl_xor(nz, o, kWave);
      allowed += __shfl_xor(allowed, o, kWave);
    }
    const int lane = tid & (kWave - 1), wid = tid / kWave;
    if (lane == 0) {
      sm.redx[wid][0] = f2u(st.m);
      sm.redx[wid][1] = f2u(st.s);
      sm.redx[wid][2] = f2u(rmax);
      sm.redx[wid][3] = nz;
      sm.redx[wid][4] = allowed;
    }
    __syncthreads();
    lse = Lse3{kNegInf, 0.0f, 0.0f};
    rmax = kNegInf;
    nz = 0;
    allowed = 0;
    for (int w = 0; w < kFWaves; ++w) {
      lse = lse3_merge(lse, Lse3{u2f(sm.redx[w][0]), u2f(sm.redx[w][1]), 0.0f});
      rmax = fmaxf(rmax, u2f(sm.redx[w][2]));
      nz += sm.redx[w][3];
      allowed += sm.redx[w][4];
    }
    kmax = rmax > kNegInf ? vec_key<T>(rmax) : 0u;
    if (!c.mrow) {
      nz = (uint32_t)c.nv;
      allowed = (uint32_t)c.nv * E;
    }
  }
  // penalty bitmap of the slice from the history ids
  bool bad_hist = false;
  if (read_hist) {
    for (int64_t j0 = 0; j0 < a.hist_len; j0 += (int64_t)kHistPer * kFT) {
      if (j0 > 0) {
        for (int q = 0; q < kHistPer; ++q) {
          const int64_t j = j0 + tid + (int64_t)q * kFT;
          hv[q] = j < a.hist_len ? hrow[j] : -1;
        }
      }
      for (int q = 0; q < kHistPer; ++q) {
        const int32_t id = hv[q];
        if (id >= a.V) {
          bad_hist = true;
        } else if (fa.use_pen && id >= e0 && id < e1) {
          atomicOr(&sm.pen[(uint32_t)(id >> 5) - c.w0], 1u << (id & 31));
        }
      }
    }
  }
  bad_hist = __syncthreads_or(bad_hist);

  // ---- 2. select the slice's top Kc
  const uint32_t Kc = (uint32_t)fa.Kc;
  uint32_t tau = 1u;
  float xout = kNegInf, yout = kNegInf;
  uint32_t ngt = 0;
  const bool has_tail = c.tail0 < a.V;
  if (kmax > 0u || has_tail) {
    // allowed tokens per vector among vectors with one: roughly the chance
    // that a re-read vector contributes a token above the threshold
    const float dens = nz ? (float)allowed / (float)(nz * E) : 1.0f;
    uint32_t need = (uint32_t)__builtin_ceilf(2.0f * (float)Kc / dens) + 32u;
    // large slices histogram a 1-in-8 sample of the keys (the threshold only
    // steers how many vectors are re-read; exactness is checked below)
    const bool sampled = c.nv > 8192;
    const u32x4* keys = reinterpret_cast<const u32x4*>(sm.u.gkey);
    const int nchunk = (c.nv + 7) >> 3;
    int shift = 0;
    for (int attempt = 0; attempt < 4; ++attempt) {
      if (attempt < 3 && kmax > 1u) {
        __syncthreads();
        if (tid < 256) sm.hist[tid] = 0u;
        if (tid == 0) {
          sm.bucket = 0;  // fewer than `need` keys in range: take the whole range
          sm.above = 0;
        }
        __syncthreads();
        for (int j = tid; j < nchunk; j += kFT) {
          const u32x4 w = keys[j];
          const uint32_t kk[4] = {w.x, w.y, w.z, w.w};
          for (int e = 0; e < (sampled ? 1 : 8); ++e) {
            const uint32_t k = (e & 1) ? (kk[e >> 1] >> 16) : (kk[e >> 1] & 0xFFFFu);
            if (k >= 1u) {
              const uint32_t d = (kmax - k) >> shift;
              if (d < 256u) atomicAdd(&sm.hist[255 - d], 1u);
            }
          }
        }
        __syncthreads();
        // bucket (from the top) where the count of passing vectors reaches need
        const uint32_t need_h = sampled ? (need + 7u) / 8u : need;
        find_bucket(sm, need_h - 1u);
        __syncthreads();
        const uint32_t bt = 255u - (uint32_t)sm.bucket;  // distance bin from kmax
        const int64_t lo = (int64_t)kmax - (int64_t)((bt + 1u) << shift) + 1;
        tau = lo > 1 ? (uint32_t)lo : 1u;
      } else {
        tau = 1u;
      }
      xout = tau > 1u ? key_value(tau - 1u) : kNegInf;
      yout = tau > 1u ? c.proc.ub(xout) : kNegInf;
      if (tid == 0) sm.ngt = 0u;
      __syncthreads();
      uint32_t nsel = 0;
      auto collect = [&](int32_t id, float y, float x) {
        const uint32_t slot = atomicAdd(&sm.ngt, 1u);
        if (slot < (uint32_t)kCand) {
          sm.ckey[slot] = rank_key(y, id);
          sm.cx[slot] = x;
        }
      };
      {
        const uint32_t total = select_vectors(sm, c.nv, tau, 0);
        nsel = total;
        for (uint32_t base = 0; base < total; base += kSel) {
          if (base > 0) select_vectors(sm, c.nv, tau, base);
          const uint32_t n = total - base < (uint32_t)kSel ? total - base : (uint32_t)kSel;
          emit_listed<T>(sm, c, n, xout, yout, collect);
          __syncthreads();
        }
        emit_tail<T>(sm, c, xout, yout, collect);
        __syncthreads();
      }
      ngt = sm.ngt;
      if (tau <= 1u || (ngt >= Kc && ngt <= (uint32_t)kCand)) break;
      // move the threshold by the measured rate of kept tokens per vector
      if (ngt > (uint32_t)kCand) {
        const uint64_t t = (uint64_t)nsel * (uint64_t)(kCand / 2) / ngt;
        need = t > Kc ? (uint32_t)t : Kc;
      } else if (ngt > 0u) {
        const uint64_t t = (uint64_t)nsel * 2u * Kc / ngt + 32u;
        need = t < 0x7FFFFFFFull ? (uint32_t)t : 0x7FFFFFFFu;
      } else {
        need = need < 0x0FFFFFFFu ? need * 8u + 64u : 0x7FFFFFFFu;
      }
      shift = need > 4096u ? 3 : (need > 1024u ? 1 : 0);
    }
  }

  // ---- 3. the slice's top min(ngt, Kc), sorted by rank
  const uint32_t nout = ngt < Kc ? ngt : Kc;
  // this slice's workspace slot (only rows split over several slices have one)
  SliceHead* head = S > 1 ? reinterpret_cast<SliceHead*>(fa.ws + fa.cnt_bytes +
                                                         ((size_t)b * S + s) * kSlotBytes)
                          : nullptr;
  SliceEnt* ent = S > 1 ? reinterpret_cast<SliceEnt*>(head + 1) : nullptr;
  auto put = [&](uint32_t r, unsigned long long k, float x) {
    if (S == 1) {
      sm.fkey[r] = k;
      sm.fx[r] = x;
    } else {
      ent[r].key = k;
      ent[r].x = x;
    }
  };
  if (ngt <= 256u) {
    rank_sort_small(sm.ckey, sm.cx, ngt, Kc, put);
  } else {
    select_top_slow<T>(sm, c, ngt, Kc, tau, xout, yout);
    rank_sort_small(sm.skey, sm.sx, Kc, Kc, put);
  }
  __syncthreads();
  if (S == 1) {
    finish_row(sm, fa, b, lse, bad_hist, nout);
    return;
  }
  if (tid == 0) {
    head->m = lse.m;
    head->s = lse.s;
    head->n = nout;
    head->flags = (s == 0 && bad_hist) ? 1u : 0u;
  }

  // ---- 4. the last workgroup of the row to arrive merges.  The barrier
  // completes every wave's stores to L2; one release fence (an L2 write-back)
  // by the thread that bumps the counter publishes them device-wide, and the
  // merging workgroup's acquire fence (L2 invalidate) makes the other
  // workgroups' slots visible before any of its waves reads them.
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    uint32_t* cnt = reinterpret_cast<uint32_t*>(fa.ws) + b;
    uint32_t old = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t arrived;
    while (true) {
      const uint32_t nw2 = (old >> 16) == fa.epoch ? old + 1u : (fa.epoch << 16) | 1u;
      const uint32_t prev = atomicCAS(cnt, old, nw2);
      if (prev == old) {
        arrived = nw2 & 0xFFFFu;
        break;
      }
      old = prev;
    }
    const bool last = arrived == (uint32_t)S;
    if (last) __threadfence();
    sm.flag = last ? 1 : 0;
  }
  __syncthreads();
  if (!sm.flag) return;
  merge_row(sm, fa, b, S);
}

// ------------------------------------------------------------------ planning

struct FastPlan {
  bool fast;
  int S;
  int64_t vps;
  size_t cnt_bytes;
  size_t ws_bytes;
};

int elem_size(int dtype) { return dtype == GTP_DTYPE_F32 ? 4 : 2; }

// Compute units of the current device (cached per device): the launch aims
// at one resident workgroup per CU so that every slice streams at once and
// the selection tails run after the memory system has drained.
int64_t device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

FastPlan plan_fast(int dtype, int64_t B, int64_t V, const gtp_sampler_params* p, bool aligned) {
  FastPlan pl{false, 0, 0, 0, 0};
  const bool greedy = !(p->temperature > 0.0f);
  const int64_t Kc = greedy ? 1 : p->top_k;
  const int E = 16 / elem_size(dtype);
  const int64_t nvec = V / E;
  if (!aligned || Kc < 1 || Kc > kFastK || nvec < 64 || B < 1 || B > 0xFFFF) return pl;
  const int64_t s_min = (nvec + kSliceVecs - 1) / kSliceVecs;
  const int64_t s_cap = kCand / Kc < kMaxSlices ? kCand / Kc : kMaxSlices;
  if (s_min > s_cap) return pl;
  const int64_t cus = device_cus();
  int64_t S = (cus + B - 1) / B;
  const int64_t s_small = nvec / 1024 > 1 ? nvec / 1024 : 1;  // slices of >= 1024 vectors
  if (S > s_small) S = s_small;
  if (S > s_cap) S = s_cap;
  if (S < s_min) S = s_min;
  if (S < 1) S = 1;
  const int64_t vps = (nvec + S - 1) / S;
  S = (nvec + vps - 1) / vps;
  pl.fast = true;
  pl.S = (int)S;
  pl.vps = vps;
  if (S > 1) {
    pl.cnt_bytes = (((size_t)B * 4 + 255) / 256) * 256;
    pl.ws_bytes = pl.cnt_bytes + (size_t)B * S * kSlotBytes;
  }
  return pl;
}

std::atomic<uint32_t> g_epoch{0};

}  // namespace gtp

using namespace gtp;

extern "C" size_t gtp_sample_workspace_bytes(int dtype, int64_t B, int64_t V,
                                             const gtp_sampler_params* params) {
  if (!params || B <= 0 || V <= 0) return 0;
  const FastPlan pl = plan_fast(dtype, B, V, params, true);
  return pl.fast ? pl.ws_bytes : 0;
}

extern "C" int gtp_sample_rows(const void* logits, int dtype, int64_t B, int64_t V,
                               int64_t row_stride, const int32_t* history, int64_t hist_len,
                               int64_t hist_stride, const uint32_t* allow_mask, int64_t mask_stride,
                               const float* uniforms, const gtp_sampler_params* params,
                               const uint8_t* finished, int64_t pad_token_id, int64_t* out_ids,
                               float* out_logprob, float* out_sampled_logprob, int32_t* out_kept,
                               float* out_thresh_value, int32_t* out_thresh_id, int32_t* out_status,
                               void* workspace, size_t workspace_bytes, void* stream) {
  if (!params || B < 0 || V <= 0 || row_stride < V) return GTP_ERR_INVALID_ARGUMENT;
  if (dtype != GTP_DTYPE_F32 && dtype != GTP_DTYPE_BF16 && dtype != GTP_DTYPE_F16)
    return GTP_ERR_INVALID_ARGUMENT;
  if (B > 0 && (!logits || !out_ids)) return GTP_ERR_INVALID_ARGUMENT;
  if (!(params->repetition_penalty > 0.0f)) return GTP_ERR_INVALID_ARGUMENT;
  if (allow_mask && mask_stride < (V + 31) / 32) return GTP_ERR_INVALID_ARGUMENT;
  if (hist_len < 0) return GTP_ERR_INVALID_ARGUMENT;
  if (history && hist_len > 0 && hist_stride < hist_len) return GTP_ERR_INVALID_ARGUMENT;
  const bool greedy = !(params->temperature > 0.0f);
  if (!greedy && !uniforms) return GTP_ERR_INVALID_ARGUMENT;
  if (V > GTP_SAMPLER_MAX_V || B > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  if (B == 0) return GTP_OK;
  SamplerArgs a;
  a.logits = logits;
  a.V = V;
  a.row_stride = row_stride;
  a.hist = history;
  a.hist_len = history ? hist_len : 0;
  a.hist_stride = hist_stride;
  a.mask = allow_mask;
  a.mask_stride = mask_stride;
  a.uniforms = uniforms;
  a.T = params->temperature;
  a.K = params->top_k;
  a.P = params->top_p;
  a.rho = params->repetition_penalty;
  a.finished = finished;
  a.pad_id = pad_token_id;
  a.out_ids = out_ids;
  a.out_lp = out_logprob;
  a.out_slp = out_sampled_logprob;
  a.out_kept = out_kept;
  a.out_tv = out_thresh_value;
  a.out_tid = out_thresh_id;
  a.out_status = out_status;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);

  const int es = elem_size(dtype);
  const bool aligned = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0 &&
                       ((row_stride * es) & 15) == 0;
  const FastPlan pl = plan_fast(dtype, B, V, params, aligned);
  if (!pl.fast) return launch_sampler_general(a, dtype, B, st);
  if (pl.ws_bytes > 0 && (!workspace || workspace_bytes < pl.ws_bytes))
    return GTP_ERR_INVALID_ARGUMENT;

  FastArgs fa;
  fa.a = a;
  fa.vps = pl.vps;
  fa.ws = reinterpret_cast<unsigned char*>(workspace);
  fa.cnt_bytes = pl.cnt_bytes;
  fa.epoch = (g_epoch.fetch_add(1u, std::memory_order_relaxed) % 0xFFFFu) + 1u;
  fa.greedy = greedy ? 1 : 0;
  fa.Kc = greedy ? 1 : params->top_k;
  fa.use_pen = (history && hist_len > 0 && params->repetition_penalty != 1.0f) ? 1 : 0;
  fa.p_active = (!greedy && params->top_p > 0.0f && params->top_p < 1.0f) ? 1 : 0;
  fa.Tc = params->temperature > 1e-6f ? params->temperature : 1e-6f;
  const dim3 grid((unsigned)pl.S, (unsigned)B), block(kFT);
  switch (dtype) {
    case GTP_DTYPE_BF16:
      hipLaunchKernelGGL(sampler_split_kernel<uint16_t>, grid, block, 0, st, fa);
      break;
    case GTP_DTYPE_F16:
      hipLaunchKernelGGL(sampler_split_kernel<_Float16>, grid, block, 0, st, fa);
      break;
    default:
      hipLaunchKernelGGL(sampler_split_kernel<float>, grid, block, 0, st, fa);
      break;
  }
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}
