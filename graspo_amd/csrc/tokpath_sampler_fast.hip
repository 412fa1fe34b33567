// tokpath_sampler_fast.hip -- the rollout sampler for greedy and top-k rows
// (1 <= k <= 128) on 16-byte aligned rows (gfx950).
//
// One workgroup of 1024 threads per CU.  A row is split into S slices
// (S = ceil(CUs / B), so a B >= 256 batch is one row per workgroup and every
// workgroup of the launch is resident at once).
//
// 1. Pilot.  Each thread first loads 4 vectors (8 bf16/fp16 or 4 fp32 logits
//    each) from the start of the slice -- before any other load, so they
//    come back first -- and takes the largest allowed one, lowered by the
//    largest possible penalty.  Each wave sorts its 64 values in registers
//    and posts its top 16; the last wave to post picks the Kc-th largest,
//    theta1.  Those values belong to distinct tokens, so at least Kc allowed
//    tokens have a penalised logit >= theta1.  No block barrier is involved:
//    a wave issues its first stream chunks as soon as it has posted, and
//    only waits for theta with those loads in flight.
// 2. Stream (the only HBM read of the slice; tokpath_stream.h).  Waves take
//    chunks of 64 x 4 vectors from an LDS counter (each lane also brings one
//    allow-mask word of the chunk; slices start on word boundaries) and fold
//    them into an online log-sum-exp of the raw logits (the logprob output).
//    A vector whose maximum reaches theta (theta1 mapped back through the
//    penalty's largest increase and lowered by 2^-12) is queued -- raw, with
//    its slice index and allow bits -- in its wave's LDS queue, which is
//    drained 64 vectors at a time, one per lane: the allowed tokens with
//    x >= theta enter an LDS pool of (id, x).  A vector below theta costs one
//    compare.  History ids set a penalty bitmap in LDS while the first
//    chunks are in flight.
// 3. Resolve.  The pooled tokens get the exact penalty, mask and IEEE
//    division by the temperature.  A token left out has x < theta, so its
//    processed logit is <= ub(theta); when at least Kc pooled tokens beat
//    that bound, the slice's top Kc (by y desc, id asc) is among them.  A
//    1024-bin histogram of 16-bit keys (wave 0 finds the Kc-th) trims the
//    pool before ranking by counting (<= 256 tokens) or an 8-bit radix select
//    on the 64-bit (y, id) key.  When the pool overflowed or does not
//    separate (e.g. massive exact ties), the slice falls back to per-vector
//    keys re-read from HBM and a threshold search over them.
// 4. With S == 1 the workgroup finishes the row from LDS.  Otherwise it
//    publishes its sorted top-k and (m, s) to the workspace and the last
//    workgroup of the row to arrive (a per-row counter in the workspace,
//    which that workgroup returns to zero, so no workgroup ever waits on
//    another and the workspace is ready for the next call) merges the S
//    lists by binary-search ranks.
// 5. Finish (one wave): fixed-point weights (DETEXP_FIX), exact top-p cut
//    and inverse-CDF draw over the sorted top-k, counted with ballots.
//
// Every output follows the contract of include/graspo_tokpath.h bit for bit;
// the threshold logic only decides which tokens are evaluated exactly.
//
// Replaces _next_token_from_logits / _sample_next_token
// (src/graspo/backends/graspoflow/tensor_utils.py:649-683).
#include <atomic>
#include <mutex>

#include "tokpath_sampler_internal.h"
#include "tokpath_stream.h"

namespace gtp {

constexpr int kFT = 1024;                   // threads per workgroup (one per CU)
constexpr int kFWaves = kFT / kWave;
constexpr int kTT = 256;                    // threads of the ranking tail (one wave per SIMD)
constexpr int kFG = 4;                      // vectors per thread per stream step
constexpr int kSliceVecs = 32768;           // most vectors in one slice (2^18 bf16 tokens)
constexpr int kFastK = 128;                 // largest kept set of this path
constexpr int kCand = 2048;                 // candidate slots of a slice (the capture pool)
constexpr int kMergeCand = 1024;            // entries of all slice lists of a row
constexpr int kPHist = 1024;                // bins of the final 16-bit key filter
constexpr int kWTop = 16;                   // pilot keys each wave posts (its largest)
constexpr int kQCap = 128;                  // queued vectors per wave (drained at 64)
// pilot vectors per thread (fp16 converts in more registers)
template <typename T>
constexpr int kNPof = Elem<T>::kDtype == GTP_DTYPE_F16 ? 3 : 4;
constexpr int kSel = 2048;                  // re-read list entries per round
constexpr int kPenWords = kSliceVecs * 8 / 32 + 2;
// at most 8 slices per row: with few rows (B <= 16) one slice of a row
// streams fast enough on its own and merging more lists costs more than the
// slices save (fp32 [8, 151936], top-k 50: 25-27 us for 1 to 8 slices, 34 us
// for 20)
constexpr int kMaxSlices = 8;
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
  int32_t Kc;             // entries per slice list (1 when greedy)
  int32_t greedy;
  int32_t use_pen;
  int32_t p_active;
  float Tc;
};

struct FastSmem {
  union {
    struct {                          // during the stream
      u32x4 qv[kFWaves][kQCap];       // each wave's queue of vectors whose maximum reached theta
      uint32_t qi[kFWaves][kQCap];    // ... and their indices in the slice
    } st;
    struct {                          // fallback after the stream
      uint16_t gkey[kSliceVecs];      // per-vector order keys of the slice
      uint16_t sel[kSel];
    } fb;
    uint32_t soff[kMaxSlices + 1];    // merge: start of each slice's list in ckey / cx
  } u;
  uint32_t pen[kPenWords];           // penalty bitmap of the slice's tokens
  unsigned long long ckey[kCand];    // capture pool / candidates (slice), lists (merge)
  float cx[kCand];
  unsigned long long skey[kFastK];   // the slice's survivors before sorting
  float sx[kFastK];
  unsigned long long fkey[kFastK];   // the row's top-k, sorted
  float fx[kFastK];
  unsigned long long incl[kFastK];   // inclusive prefix of the fixed-point weights
  uint32_t hist[256];
  uint32_t phist[kPHist];            // final filter histogram
  uint32_t wtop[kFWaves * kWTop];    // each wave's largest pilot keys, descending
  float red[kFWaves][3];
  uint32_t redu[kFWaves];
  uint32_t redx[kFWaves][5];
  uint32_t ngt;
  uint32_t pool_n;     // tokens captured during the stream
  uint32_t kmax16;     // block maximum of 16-bit order keys (pilot, final filter)
  uint32_t parrive;    // waves that have posted their pilot keys
  uint32_t theta_ready;
  uint32_t theta_ord;  // ord32 of the capture threshold, once theta_ready
  uint32_t chunk_ctr;  // next stream chunk (per-wave dynamic schedule)
  int32_t bucket;
  uint32_t above;
  int32_t flag;
  unsigned long long found;
};
static_assert(sizeof(FastSmem) <= 160 * 1024, "one workgroup per CU");

// ------------------------------------------------------------------ helpers

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
  const uint32_t incl = wave_scan_u32(v);  // DPP, no LDS round trip
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
  const uint32_t incl = wave_scan_u32(tot);
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

// The calling wave (all 64 lanes): the bucket of an NB-bin histogram h (bin
// NB-1 on top) that holds 0-based position `target`, or -1 when h holds no
// more than `target` entries.  Returned to every lane.
template <int NB>
__device__ __forceinline__ int32_t wave_find_bucket(const uint32_t* h, uint32_t target,
                                                   uint32_t* above_out = nullptr) {
  constexpr int PL = NB / kWave;  // bins per lane, lane 0 holding the top ones
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t* hl = h + NB - PL * (lane + 1);  // this lane's bins, ascending
  uint32_t tot = 0;
#pragma unroll 8
  for (int q = 0; q < PL; ++q) tot += hl[q];
  const uint32_t incl = wave_scan_u32(tot);
  const bool here = incl - tot <= target && target < incl;
  const unsigned long long who = __ballot(here);
  if (!who) return -1;
  const int src = (int)__builtin_ctzll(who);
  // the holding lane walks its bins from the top
  int32_t bin = 0;
  uint32_t ab = 0;
  if (lane == src) {
    uint32_t above = incl - tot;
    for (int q = PL - 1; q >= 0; --q) {
      const uint32_t cq = hl[q];
      if (target < above + cq) {
        bin = NB - PL * (lane + 1) + q;
        ab = above;
        break;
      }
      above += cq;
    }
  }
  if (above_out) *above_out = (uint32_t)__builtin_amdgcn_readlane((int)ab, src);
  return __builtin_amdgcn_readlane(bin, src);
}

// Sort the 64 R values of a wave in descending order in registers (bitonic
// network; element r*64 + lane lives in v[r] of that lane).
template <int R>
__device__ __forceinline__ void wave_sort_desc(uint32_t (&v)[R]) {
  const int lane = threadIdx.x & (kWave - 1);
  constexpr int N = kWave * R;
  auto xch = [](uint32_t x, int j) __attribute__((always_inline)) -> uint32_t {
    switch (j) {
      case 1: return lane_xor<1>(x);
      case 2: return lane_xor<2>(x);
      case 4: return lane_xor<4>(x);
      case 8: return lane_xor<8>(x);
      case 16: return lane_xor<16>(x);
      default: return lane_xor<32>(x);
    }
  };
#pragma unroll
  for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j >= 1; j >>= 1) {
      if (j >= kWave) {
        const int jr = j / kWave;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if ((r & jr) == 0) {
            const bool desc = ((r * kWave + lane) & k) == 0;
            const uint32_t hi = max(v[r], v[r | jr]), lo = min(v[r], v[r | jr]);
            v[r] = desc ? hi : lo;
            v[r | jr] = desc ? lo : hi;
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint32_t w = xch(v[r], j);
          const bool desc = ((r * kWave + lane) & k) == 0;
          const bool lower = (lane & j) == 0;
          v[r] = desc == lower ? max(v[r], w) : min(v[r], w);
        }
      }
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

  // allow bits of tokens [e0, e0 + n), n <= 8, inside one mask word (global
  // read: only the rare paths look tokens up one by one)
  __device__ __forceinline__ uint32_t mask_bits(int64_t e0, int n) const {
    return mrow ? (mrow[e0 >> 5] >> (e0 & 31)) & ((1u << n) - 1u) : (1u << n) - 1u;
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
  const u32x4* keys = reinterpret_cast<const u32x4*>(sm.u.fb.gkey);
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
        if (pos >= base && pos < base + kSel) sm.u.fb.sel[pos - base] = (uint16_t)(j * 8 + e);
        ++pos;
      }
    }
  }
  __syncthreads();
  return total;
}

// f(id, y, x) for every valid token with y > yout of the listed vectors
// sm.u.fb.sel[0, n).  yout = ub(xout), so a raw x <= xout never passes: only the
// few tokens above xout pay for the exact penalty and IEEE division.
template <typename T, typename F>
__device__ __forceinline__ void emit_listed(const FastSmem& sm, const Slice<T>& c, uint32_t n,
                                            float xout, float yout, F& f) {
  constexpr int E = Vec<T>::kE;
  const u32x4* rv = reinterpret_cast<const u32x4*>(c.row);
  for (uint32_t p = threadIdx.x; p < n; p += kFT) {
    const int64_t vi = c.v0 + sm.u.fb.sel[p];
    const u32x4 v = rv[vi];
    const int64_t e0 = vi * E;
    const uint32_t mb = c.mask_bits(e0, E);
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
    if (!c.mask_bits(id, 1)) continue;
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

// Rank of each of n <= kFT / 4 distinct keys by counting: the four threads
// of a quad share a key and each counts the larger keys in a quarter of the
// list, summed within the quad (DPP); entries of rank < k go to
// out(rank, key, x).  Block-uniform; callers sync before (keys complete).
template <typename Out>
__device__ __forceinline__ void rank_sort_small(const unsigned long long* keys, const float* xs,
                                                uint32_t n, uint32_t k, Out out) {
  const uint32_t i = threadIdx.x >> 2, part = threadIdx.x & 3u;
  unsigned long long ki = 0;
  uint32_t rk = 0;
  if (i < n) {
    ki = keys[i];
#pragma unroll 4
    for (uint32_t j = part; j < n; j += 4u) rk += keys[j] > ki ? 1u : 0u;
  }
  rk += lane_xor<1>(rk);  // every lane takes part in the quad sums
  rk += lane_xor<2>(rk);
  if (i < n && part == 0u && rk < k) out(rk, ki, xs[i]);
}

// The slice's top Kc into sm.skey / sm.sx (unsorted) when more than 256
// tokens beat Y_out: radix select in LDS (<= kCand of them), or, past that
// (massive exact ties), the same select re-reading the passing vectors once
// per digit.  Rare: not executed on the common path.
template <typename T>
__device__ __forceinline__ void select_top_slow(FastSmem& sm, const Slice<T>& c, uint32_t ngt,
                                             uint32_t Kc, uint32_t tau, float xout, float yout,
                                             int nthr) {
  const int tid = threadIdx.x;
  if (ngt <= (uint32_t)kCand) {
    const unsigned long long kth = radix_kth(
        sm, Kc,
        [&](unsigned long long prefix, unsigned long long pmask, int shift) {
          for (uint32_t i = tid; tid < nthr && i < ngt; i += nthr) {
            const unsigned long long k = sm.ckey[i];
            if ((k & pmask) == prefix) atomicAdd(&sm.hist[(k >> shift) & 0xFFu], 1u);
          }
        },
        [&](unsigned long long prefix, unsigned long long pmask) {
          for (uint32_t i = tid; tid < nthr && i < ngt; i += nthr)
            if ((sm.ckey[i] & pmask) == prefix) sm.found = sm.ckey[i];
        });
    if (tid == 0) sm.ngt = 0u;
    __syncthreads();
    for (uint32_t i = tid; tid < nthr && i < ngt; i += nthr) {
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
// or fixed-point top-p cut and draw, outputs.  Wave 0 only (lane r/2 holds
// the weights of ranks r); the cut and the draw are counts of prefix sums
// below a bound, taken with ballots.  Callers sync before (lists complete).
template <typename T>
__device__ __forceinline__ void finish_row(FastSmem& sm, const FastArgs& fa, int64_t b,
                                           float u, float lm, float ls, bool bad_hist,
                                           uint32_t nk) {
  const SamplerArgs& a = fa.a;
  const int lane = threadIdx.x;
  if (lane >= kWave) return;
  // logprob = x - m - ln s, rounded once (raw_logprob)
  const float lse_m = lm, lse_ln = __builtin_amdgcn_logf(ls) * kLn2;
  const bool raw_nonfinite = ls != ls || lm == kPosInf;
  int32_t status = GTP_ROW_OK;
  if (raw_nonfinite)
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
    if (fa.greedy && !bad_hist) {  // argmax semantics for NaN, +inf and all -inf rows
      greedy_argmax_rescan<T>(a, b, sm.pen, true, raw_nonfinite, lse_m, lse_ln);
      return;
    }
    if (fa.greedy) status = GTP_ROW_BAD_HISTORY;
    if (lane == 0) write_out(a, b, status, -1, 0.f, 0.f, 0, 0.f, -1);
    return;
  }
  const unsigned long long k0 = sm.fkey[0];
  const float m = rank_key_y(k0);
  if (fa.greedy) {
    if (lane == 0) {
      const int32_t id = rank_key_id(k0);
      write_out(a, b, GTP_ROW_OK, id, raw_logprob(sm.fx[0], lse_m, lse_ln), 0.0f, 1, m, id);
    }
    return;
  }
  // fixed-point weights of ranks r0 = 2 lane, r1 = r0 + 1 and their
  // inclusive prefix sums i0, i1
  const uint32_t r0 = 2u * (uint32_t)lane, r1 = r0 + 1u;
  const unsigned long long w0 = r0 < nk ? detexp_fix(rank_key_y(sm.fkey[r0]) - m) : 0ull;
  const unsigned long long w1 = r1 < nk ? detexp_fix(rank_key_y(sm.fkey[r1]) - m) : 0ull;
  const unsigned long long i1 = wave_scan_u64(w0 + w1);
  const unsigned long long i0 = i1 - w1;
  auto incl_at = [&](uint32_t r) -> unsigned long long {  // r wave-uniform
    const unsigned long long v = (r & 1u) ? i1 : i0;
    const int l = (int)(r >> 1);
    return ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l)
            << 32) |
           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  };
  auto count_le = [&](uint32_t lim, unsigned long long bound) -> uint32_t {  // #{r < lim : incl[r] <= bound}
    const unsigned long long c0 = __ballot(r0 < lim && i0 <= bound);
    const unsigned long long c1 = __ballot(r1 < lim && i1 <= bound);
    return (uint32_t)(__builtin_popcountll(c0) + __builtin_popcountll(c1));
  };
  const unsigned long long Wk = incl_at(nk - 1u);
  const uint32_t R = fa.p_active ? 1u + count_le(nk - 1u, floor_mul(a.P, Wk)) : nk;
  const unsigned long long Wp = incl_at(R - 1u);
  const uint32_t rs = count_le(R - 1u, floor_mul(u, Wp));
  const unsigned long long hi = incl_at(rs);
  const unsigned long long lo = rs ? incl_at(rs - 1u) : 0ull;
  if (lane == 0) {
    const unsigned long long kt = sm.fkey[R - 1u];
    const float slp = __builtin_amdgcn_logf((float)((double)(hi - lo) / (double)Wp)) * kLn2;
    write_out(a, b, GTP_ROW_OK, rank_key_id(sm.fkey[rs]), raw_logprob(sm.fx[rs], lse_m, lse_ln), slp, (int32_t)R,
              rank_key_y(kt), rank_key_id(kt));
  }
}

// The last workgroup of a split row: gather the S sorted lists, rank the
// union by binary search, finish.  Block-uniform.
template <typename T>
__device__ __forceinline__ void merge_row(FastSmem& sm, const FastArgs& fa, int64_t b, float u,
                                          int S) {
  const int tid = threadIdx.x;
  const uint32_t Kc = (uint32_t)fa.Kc;
  const unsigned char* slots = fa.ws + fa.cnt_bytes + (size_t)b * S * kSlotBytes;
  float lm = kNegInf, ls = 0.0f;
  uint32_t my_n = 0, my_flags = 0;
  if (tid < S) {
    const SliceHead* hj = reinterpret_cast<const SliceHead*>(slots + (size_t)tid * kSlotBytes);
    lm = hj->m;
    ls = hj->s;
    my_n = hj->n;
    my_flags = hj->flags;
  }
  block_lse2<kFT>(lm, ls, sm.red);
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
  finish_row<T>(sm, fa, b, u, lm, ls, any_bad_hist, nk);
}

// --------------------------------------------------------------- the kernel

template <typename T, bool kMask>
__global__ __launch_bounds__(kFT) void sampler_split_kernel(FastArgs fa) {
  constexpr int E = Vec<T>::kE;
  constexpr int kHistPer = 4;  // history ids per thread per batch
  constexpr int kNP = kNPof<T>;
  __shared__ FastSmem sm;
  const SamplerArgs& a = fa.a;
  const int tid = threadIdx.x;
  const int s = blockIdx.x, S = gridDim.x;
  const int64_t b = blockIdx.y;
  const uint32_t Kc = (uint32_t)fa.Kc;

  Slice<T> c;
  c.row = reinterpret_cast<const T*>(a.logits) + b * a.row_stride;
  c.mrow = kMask ? a.mask + b * a.mask_stride : nullptr;
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

  // ---- 0. the first global requests go out before anything else: the first
  // batch of history ids here, the pilot vectors in the stream; then (the
  // stream's prologue) counters, histograms and penalty bitmap are cleared
  const int lane = tid & (kWave - 1);
  // the row's uniform, needed only by the finish: requested first, so that no
  // global load sits on the path after the stream
  const float u_row = fa.greedy ? 0.0f : a.uniforms[b];
  int32_t hv[kHistPer];
#pragma unroll
  for (int q = 0; q < kHistPer; ++q) {
    const int64_t j = tid + (int64_t)q * kFT;
    hv[q] = read_hist && j < a.hist_len ? hrow[j] : -1;
  }
  bool bad_hist = false;
  auto hist_bits = [&](int32_t id) {
    if (id >= a.V)
      bad_hist = true;
    else if (fa.use_pen && id >= e0 && id < e1)
      atomicOr(&sm.pen[(uint32_t)(id >> 5) - c.w0], 1u << (id & 31));
  };
  auto prologue = [&]() {
    if (tid == 0) {
      sm.chunk_ctr = 0u;
      sm.pool_n = 0u;
      sm.kmax16 = 0u;
      sm.bucket = -1;
      sm.parrive = 0u;
      sm.theta_ready = 0u;
    }
    for (int i = tid; i < kPHist; i += kFT) sm.phist[i] = 0u;
    if (fa.use_pen)
      for (int i = tid; i < nw; i += kFT) sm.pen[i] = 0u;
    __syncthreads();
    // history ids past the first kHistPer x 1024 (long histories only)
    if (read_hist)
      for (int64_t j = (int64_t)kHistPer * kFT + tid; j < a.hist_len; j += kFT) hist_bits(hrow[j]);
  };

  // ---- 1. stream with a prefix pilot.
  // Every token of the slice is folded into the raw log-sum-exp (the logprob
  // output).  The pilot -- the slice's first kNP x 1024 vectors, requested
  // before the rest -- sets the capture threshold: theta1 is the Kc-th
  // largest, over the 1024 threads, of the thread's largest allowed
  // penalised pilot logit (rounded down to bf16).  Threads hold disjoint
  // tokens, so at least Kc allowed tokens have a penalised logit >= theta1,
  // and a token can only outrank them if its raw value reaches theta
  // (theta1 mapped back through the penalty's largest increase and lowered
  // by 2^-12).  Every allowed token with x >= theta is captured into the LDS
  // pool (ckey holds the id, cx the raw logit); a lane whose block maximum
  // is below theta only pays one compare.  Exactness is checked after the
  // stream.
  Lse3 st{kNegInf, 0.0f, 0.0f};
  float theta = kNegInf;
  auto allow_bits = [&](uint32_t sw, int64_t vi) -> uint32_t {
    if constexpr (kMask)
      return (sw >> ((uint32_t)(vi * E) & 31u)) & ((1u << E) - 1u);
    else
      return (1u << E) - 1u;
  };
  auto capture = [&](const float(&xv)[E], uint32_t sw, int64_t vi) __attribute__((always_inline)) {
    uint32_t cand = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) cand |= (xv[j] >= theta && xv[j] > kNegInf ? 1u : 0u) << j;
    cand &= allow_bits(sw, vi);
    while (cand) {
      const int j = __builtin_ctz(cand);
      cand &= cand - 1u;
      float xj = xv[0];  // xv[j] without a dynamic register index
#pragma unroll
      for (int q = 1; q < E; ++q) xj = q == j ? xv[q] : xj;
      const uint32_t slot = atomicAdd(&sm.pool_n, 1u);
      if (slot < (uint32_t)kCand) {
        sm.ckey[slot] = (unsigned long long)(uint32_t)(vi * E + j);
        sm.cx[slot] = xj;
      }
    }
  };
  // lower bound of the penalised value of raw x (the history is not consulted)
  auto lb_pen = [&](float x) __attribute__((always_inline)) -> float {
    return (fa.use_pen && a.rho >= 1.0f) ? (x < 0.0f ? x * a.rho : x / a.rho) : x;
  };
  // raw capture threshold for a 16-bit key t16 that at least Kc allowed
  // penalised logits reach: the smallest raw x whose penalised value can reach
  // it, lowered by 2^-12 (so that after the division by T every left-out token
  // stays strictly below those Kc)
  auto raw_of = [&](uint32_t t16) __attribute__((always_inline)) -> float {
    if (!t16) return kNegInf;
    float t1 = unord32(t16 << 16);
    if (fa.use_pen && a.rho < 1.0f) t1 = t1 > 0.0f ? t1 * a.rho : t1 / a.rho;
    return t1 - __builtin_fabsf(t1) * 0x1p-12f - 0x1p-100f;
  };
  // the Kc-th largest of 64 * R keys held by the wave (v: R per lane)
  auto kth_key = [&](auto& v) __attribute__((always_inline)) -> uint32_t {
    wave_sort_desc(v);
    const uint32_t r = (Kc - 1u) / kWave, l = (Kc - 1u) % kWave;
    const uint32_t vr = r == 0 ? v[0] : v[1];  // Kc <= 128 <= 64 R
    return (uint32_t)__builtin_amdgcn_readlane((int)vr, (int)l);
  };
  // the thread's pilot key and the wave's arrival; the last wave to arrive
  // turns the 1024 keys into the threshold (no block barrier: waves that
  // arrive first go on issuing their own loads)
  auto pre = [&](const u32x4(&pv)[kNP], const uint32_t(&psw)[kNP], int64_t np) {
    float mx = kNegInf;  // the thread's largest allowed raw pilot logit
#pragma unroll
    for (int q = 0; q < kNP; ++q) {
      const int64_t rel = (int64_t)q * kFT + tid;
      if (rel < np) {
        float x[1][E];
        Vec<T>::cvt(pv[q], x[0]);
        lse_fold_block_max<false, 1, E>(st, x, vec_max<E>(x[0]));
        const uint32_t mb = allow_bits(psw[q], c.v0 + rel);
#pragma unroll
        for (int j = 0; j < E; ++j) mx = ((mb >> j) & 1u) ? max3raw(mx, x[0][j], x[0][j]) : mx;
      }
    }
    // lower bound of its penalised value (the history bitmap is not needed)
    const float lv = mx > kNegInf ? lb_pen(mx) : kNegInf;
    // the wave's 16 largest keys (0: no allowed token) to LDS
    uint32_t k16[1] = {lv > kNegInf ? ord32(lv) >> 16 : 0u};
    wave_sort_desc<1>(k16);
    if (lane < kWTop) sm.wtop[(tid / kWave) * kWTop + lane] = k16[0];
    uint32_t arrived = 0;
    if (lane == 0)
      arrived = __hip_atomic_fetch_add(&sm.parrive, 1u, __ATOMIC_ACQ_REL,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane(arrived) != (uint32_t)kFWaves - 1u) return;
    // last wave: theta1 = the Kc-th largest of the posted keys.  They are
    // keys of distinct threads, so at least Kc threads reach it (exact
    // unless one wave held more than 16 of the Kc largest).  (Taking theta
    // from the first waves to post instead makes it ready ~2 us earlier but
    // doubles the pool, and with a penalty and no mask overflows it.)
    uint32_t t16;
    if (Kc <= (uint32_t)kWave) {
      uint32_t v[2];  // the 8 largest keys of each wave suffice
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int e = q * kWave + lane;
        v[q] = sm.wtop[(e / 8) * kWTop + (e % 8)];
      }
      t16 = kth_key(v);
    } else {
      uint32_t v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = sm.wtop[q * kWave + lane];
      t16 = kth_key(v);
    }
    if (lane == 0) {
      sm.theta_ord = ord32(raw_of(t16));
      __hip_atomic_store(&sm.theta_ready, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  // with the first chunks in flight: the first history batch into the
  // penalty bitmap, then the threshold, then the pilot's own tokens
  auto post = [&](const u32x4(&pv)[kNP], const uint32_t(&psw)[kNP], int64_t np) {
#pragma unroll
    for (int q = 0; q < kHistPer; ++q)
      if (hv[q] >= 0) hist_bits(hv[q]);
    while (__hip_atomic_load(&sm.theta_ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0u)
      __builtin_amdgcn_s_sleep(1);
    theta = unord32(__hip_atomic_load(&sm.theta_ord, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
#pragma unroll
    for (int q = 0; q < kNP; ++q) {
      const int64_t rel = (int64_t)q * kFT + tid;
      if (rel < np) {
        float x[E];
        Vec<T>::cvt(pv[q], x);
        if (vec_max<E>(x) >= theta) capture(x, psw[q], c.v0 + rel);
      }
    }
  };
  // Vectors whose maximum reaches theta are queued (raw, with their slice
  // index) per wave and drained 64 at a time, one per lane, so the per-token
  // tests run at full width however sparse the hits are.
  const int wid = tid / kWave;
  uint32_t qn = 0;  // wave-uniform queue length
  auto drain = [&](uint32_t n) __attribute__((always_inline)) {
    if ((uint32_t)lane < n) {
      const u32x4 rv = sm.u.st.qv[wid][lane];
      const uint32_t qi = sm.u.st.qi[wid][lane];
      const int64_t vi = c.v0 + (qi >> 8);
      const uint32_t ab = qi & 0xFFu;
      float xv[E];
      Vec<T>::cvt(rv, xv);
      uint32_t cand = 0;
#pragma unroll
      for (int j = 0; j < E; ++j) cand |= (xv[j] >= theta && xv[j] > kNegInf ? 1u : 0u) << j;
      cand &= ab;
      while (cand) {
        const int j = __builtin_ctz(cand);
        cand &= cand - 1u;
        float xj = xv[0];
#pragma unroll
        for (int q = 1; q < E; ++q) xj = q == j ? xv[q] : xj;
        const uint32_t slot = atomicAdd(&sm.pool_n, 1u);
        if (slot < (uint32_t)kCand) {
          sm.ckey[slot] = (unsigned long long)(uint32_t)(vi * E + j);
          sm.cx[slot] = xj;
        }
      }
    }
    // the rest (< 64 entries) moves to the front
    const uint32_t rest = qn - n;
    if ((uint32_t)lane < rest) {
      const u32x4 t = sm.u.st.qv[wid][n + lane];
      const uint32_t ti = sm.u.st.qi[wid][n + lane];
      sm.u.st.qv[wid][lane] = t;
      sm.u.st.qi[wid][lane] = ti;
    }
    qn = rest;
  };
  auto fold = [&](float(&x)[kFG][E], const u32x4(&raw)[kFG], const uint32_t(&sw)[kFG],
                  int64_t vbase,
                  bool last) {
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
      // this vector's allow bits (its word came with its data); with a mask
      // the hit test uses the largest allowed value (a test on the raw
      // maximum queues about ten times as many vectors, and their drains
      // cost more than this)
      uint32_t ab = (1u << E) - 1u;
      float gh = gm[k];
      if (kMask) {
        ab = allow_bits(sw[k], vbase + (int64_t)k * kWave);
        float xm[E];
#pragma unroll
        for (int j = 0; j < E; ++j) xm[j] = (ab >> j) & 1u ? x[k][j] : kNegInf;
        gh = vec_max<E>(xm);
      }
      const bool hit = gh >= theta && gh > kNegInf;
      const unsigned long long m = __ballot(hit);
      if (m) {
        if (hit) {
          const uint32_t pos = qn + (uint32_t)__builtin_popcountll(m & ((1ull << lane) - 1ull));
          sm.u.st.qv[wid][pos] = raw[k];
          sm.u.st.qi[wid][pos] = ((uint32_t)(vbase + (int64_t)k * kWave - c.v0) << 8) | ab;
        }
        qn += (uint32_t)__builtin_popcountll(m);
        if (qn >= (uint32_t)kWave) drain((uint32_t)kWave);
      }
    }
  };
  // non-temporal: the row is read once
  stream_vectors_prefix<T, kFT, kNP, kFG, true, kMask>(c.row, c.v0, c.v1, c.mrow, &sm.chunk_ctr,
                                                    prologue, pre, post, fold);
  if (qn) drain(qn);
  // tokens past the last whole vector (last slice only)
  for (int64_t id = c.tail0 + tid; id < a.V; id += kFT) {
    float x[1][4] = {{Elem<T>::get(c.row, id), kNegInf, kNegInf, kNegInf}};
    lse_fold_block_max<false, 1, 4>(st, x, x[0][0]);
    const float xv = x[0][0];
    if (xv >= theta && xv > kNegInf && c.mask_bits(id, 1)) {
      const uint32_t slot = atomicAdd(&sm.pool_n, 1u);
      if (slot < (uint32_t)kCand) {
        sm.ckey[slot] = (unsigned long long)(uint32_t)id;
        sm.cx[slot] = xv;
      }
    }
  }
  // each wave's raw (m, s) goes to LDS with the barrier below; only the
  // finish (or the slice's head) needs the merged value, so no barrier of its
  // own sits on the path
  {
    float wm = st.m, ws = st.s;
    wave_lse2(wm, ws);
    if (lane == 0) {
      sm.red[wid][0] = wm;
      sm.red[wid][1] = ws;
    }
  }
  bad_hist = __syncthreads_or(bad_hist);  // also completes the pool, the bitmap and the sums
  // the merged raw log-sum-exp, for the calling wave (wave 0 uses it)
  auto merged_lse = [&](float& lm, float& ls) __attribute__((always_inline)) {
    lm = lane < kFWaves ? sm.red[lane][0] : kNegInf;
    ls = lane < kFWaves ? sm.red[lane][1] : 0.0f;
    wave_lse2(lm, ls);
  };

  // ---- 2. resolve the pool: exact processed logits and order keys.  Every
  // token left out has x < theta, so its processed logit is <= yex; the pool
  // holds the slice's top Kc when at least Kc pooled tokens beat yex (or when
  // theta is -inf and every allowed token was pooled).  Of those, a 16-bit
  // key histogram keeps the ones at or above the Kc-th key for ranking.
  const uint32_t pool_n = sm.pool_n;
  const uint32_t npool = pool_n < (uint32_t)kCand ? pool_n : (uint32_t)kCand;
  const float yex = theta > kNegInf ? c.proc.ub(theta) : kNegInf;
  constexpr int kPer = kCand / kFT;
  unsigned long long pk[kPer];
  float px[kPer];
  uint32_t pk16[kPer];
  uint32_t nval = 0, mx16 = 0;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const uint32_t i = (uint32_t)tid + (uint32_t)q * kFT;
    pk[q] = 0ull;
    px[q] = 0.0f;
    pk16[q] = 0u;
    if (i < npool) {
      const int32_t id = (int32_t)(uint32_t)sm.ckey[i];
      const float x = sm.cx[i];
      const bool pen = fa.use_pen && ((sm.pen[(uint32_t)(id >> 5) - c.w0] >> (id & 31)) & 1u);
      const float y = c.proc.y(x, pen);
      if (y > yex) {
        pk[q] = rank_key(y, id);
        px[q] = x;
        pk16[q] = ord32(y) >> 16;
        ++nval;
        mx16 = max(mx16, pk16[q]);
      }
    }
  }
  nval = lane63_u32(wave_scan_u32(nval));
  mx16 = (uint32_t)wave_max_f((float)mx16);  // 16-bit keys are exact in fp32
  if (lane == 0) {
    sm.redu[tid / kWave] = nval;
    if (mx16) atomicMax(&sm.kmax16, mx16);
  }
  __syncthreads();
  uint32_t nbeat = 0;
#pragma unroll
  for (int w = 0; w < kFWaves; ++w) nbeat += sm.redu[w];
  const bool pool_exact = pool_n <= (uint32_t)kCand && (theta == kNegInf || nbeat >= Kc);
  uint32_t tau = 1u;
  float xout = kNegInf, yout = kNegInf;
  uint32_t ngt = 0;
  int nthr = kFT;  // threads that take part from here on
  if (pool_exact) {
    // keys at or above the Kc-th key (16-bit), found by wave 0
    uint32_t t16 = 0;
    if (nbeat > 256u) {
      const uint32_t km = sm.kmax16;
#pragma unroll
      for (int q = 0; q < kPer; ++q)
        if (pk[q] && km - pk16[q] < (uint32_t)kPHist) atomicAdd(&sm.phist[kPHist - 1 - (km - pk16[q])], 1u);
      __syncthreads();
      if (tid < kWave) {
        const int32_t bk = wave_find_bucket<kPHist>(sm.phist, Kc - 1u);
        if (tid == 0) sm.bucket = bk;
      }
      __syncthreads();
      if (sm.bucket >= 0) t16 = km - (uint32_t)(kPHist - 1 - sm.bucket);
    }
    // compaction into ckey / cx (every thread has read its pool entries
    // before the barrier above): one slot reservation per wave
    if (tid == 0) sm.ngt = 0u;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const bool keep = pk[q] && pk16[q] >= t16;
      const unsigned long long m = __ballot(keep);
      uint32_t base = 0;
      if (lane == 0 && m) base = atomicAdd(&sm.ngt, (uint32_t)__builtin_popcountll(m));
      base = __builtin_amdgcn_readfirstlane(base);
      if (keep) {
        const uint32_t slot = base + (uint32_t)__builtin_popcountll(m & ((1ull << lane) - 1ull));
        sm.ckey[slot] = pk[q];
        sm.cx[slot] = px[q];
      }
    }
    __syncthreads();
    ngt = sm.ngt;
    // a whole row in this workgroup: ranking and finish use one wave per
    // SIMD; the other waves only pass the barriers
    if (S == 1) nthr = kTT;
  } else {
    // ---- 2b. fallback (pool overflow or no separation, e.g. massive exact
    // ties): per-vector keys of the slice re-read from HBM, then the
    // threshold search below.
    uint32_t nz = 0, allowed = 0;
    float rmax = kNegInf;
    const u32x4* rv = reinterpret_cast<const u32x4*>(c.row);
    for (int64_t vi = c.v0 + tid; vi < c.v1; vi += kFT) {
      float xv[E];
      Vec<T>::cvt(rv[vi], xv);
      float g = vec_max<E>(xv);
      uint32_t key = vec_key<T>(g);
      if (kMask) {
        const uint32_t mb = c.mask_bits(vi * E, E);
        if (mb == 0u) {
          key = 0u;
          g = kNegInf;
        } else {
          ++nz;
          allowed += __builtin_popcount(mb);
        }
      }
      sm.u.fb.gkey[vi - c.v0] = (uint16_t)key;
      rmax = max3raw(rmax, g, g);
    }
    // keys past the slice inside its last 16-byte chunk read as 0
    if (tid < 8 && c.nv + tid < ((c.nv + 7) & ~7)) sm.u.fb.gkey[c.nv + tid] = 0;
    uint32_t kmax;
    {
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        rmax = fmaxf(rmax, __shfl_xor(rmax, o, kWave));
        nz += __shfl_xor(nz, o, kWave);
        allowed += __shfl_xor(allowed, o, kWave);
      }
      const int lane = tid & (kWave - 1), wid = tid / kWave;
      __syncthreads();
      if (lane == 0) {
        sm.redx[wid][2] = f2u(rmax);
        sm.redx[wid][3] = nz;
        sm.redx[wid][4] = allowed;
      }
      __syncthreads();
      rmax = kNegInf;
      nz = 0;
      allowed = 0;
      for (int w = 0; w < kFWaves; ++w) {
        rmax = fmaxf(rmax, u2f(sm.redx[w][2]));
        nz += sm.redx[w][3];
        allowed += sm.redx[w][4];
      }
      kmax = rmax > kNegInf ? vec_key<T>(rmax) : 0u;
      if (!kMask) {
        nz = (uint32_t)c.nv;
        allowed = (uint32_t)c.nv * E;
      }
    }
    const bool has_tail = c.tail0 < a.V;
    if (kmax > 0u || has_tail) {
      // allowed tokens per vector among vectors with one: roughly the chance
      // that a re-read vector contributes a token above the threshold
      const float dens = nz ? (float)allowed / (float)(nz * E) : 1.0f;
      uint32_t need = (uint32_t)__builtin_ceilf(2.0f * (float)Kc / dens) + 32u;
      // large slices histogram a 1-in-8 sample of the keys (the threshold only
      // steers how many vectors are re-read; exactness is checked below)
      const bool sampled = c.nv > 8192;
      const u32x4* keys = reinterpret_cast<const u32x4*>(sm.u.fb.gkey);
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
    select_top_slow<T>(sm, c, ngt, Kc, tau, xout, yout, nthr);
    rank_sort_small(sm.skey, sm.sx, Kc, Kc, put);
  }
  __syncthreads();
  if (S == 1) {
    if (tid >= kWave) return;
    float lm, ls;
    merged_lse(lm, ls);
    finish_row<T>(sm, fa, b, u_row, lm, ls, bad_hist, nout);
    return;
  }
  if (tid < kWave) {
    float lm, ls;
    merged_lse(lm, ls);
    if (tid == 0) {
      head->m = lm;
      head->s = ls;
      head->n = nout;
      head->flags = (s == 0 && bad_hist) ? 1u : 0u;
    }
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
    const uint32_t arrived = atomicAdd(cnt, 1u) + 1u;
    const bool last = arrived == (uint32_t)S;
    if (last) {
      // Every workgroup of the row has arrived, so nothing else touches the
      // counter in this launch: return it to zero for the next call.
      __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __threadfence();
    }
    sm.flag = last ? 1 : 0;
  }
  __syncthreads();
  if (!sm.flag) return;
  merge_row<T>(sm, fa, b, u_row, S);
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
// Threads that race on a device's first call both store the same value.
int64_t device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

FastPlan plan_fast(int dtype, int64_t B, int64_t V, const gtp_sampler_params* p, bool aligned) {
  FastPlan pl{false, 0, 0, 0, 0};
  const bool greedy = !(p->temperature > 0.0f);
  const int64_t Kc = greedy ? 1 : p->top_k;
  const int E = 16 / elem_size(dtype);
  const int64_t nvec = V / E;
  if (!aligned || Kc < 1 || Kc > kFastK || nvec < 64 || B < 1 || B > 0xFFFF) return pl;
  const int64_t s_min = (nvec + kSliceVecs - 1) / kSliceVecs;
  const int64_t s_cap = kMergeCand / Kc < kMaxSlices ? kMergeCand / Kc : kMaxSlices;
  if (s_min > s_cap) return pl;
  const int64_t cus = device_cus();
  int64_t S = (cus + B - 1) / B;
  const int64_t s_small = nvec / 1024 > 1 ? nvec / 1024 : 1;  // slices of >= 1024 vectors
  if (S > s_small) S = s_small;
  if (S > s_cap) S = s_cap;
  if (S < s_min) S = s_min;
  if (S < 1) S = 1;
  // slices start on allow-mask word boundaries: vps a multiple of 8 vectors
  const int64_t vps = ((nvec + S - 1) / S + 7) / 8 * 8;
  S = (nvec + vps - 1) / vps;
  pl.fast = true;
  pl.S = (int)S;
  pl.vps = vps;
  if (S > 1) {
    // the arrival counters of every split call on this device (S > 1 needs
    // B < CUs) lie in one fixed region before the slots: calls whose B
    // differs never find another call's slot data in their counters
    const int64_t nc = B > cus ? B : cus;
    pl.cnt_bytes = (((size_t)nc * 4 + 255) / 256) * 256;
    if (pl.cnt_bytes < kWsZeroBytes) pl.cnt_bytes = kWsZeroBytes;
    pl.ws_bytes = pl.cnt_bytes + (size_t)B * S * kSlotBytes;
  }
  return pl;
}

}  // namespace gtp

using namespace gtp;

extern "C" size_t gtp_sample_workspace_bytes(int dtype, int64_t B, int64_t V,
                                             const gtp_sampler_params* params) {
  if (!params || B <= 0 || V <= 0 || V > GTP_SAMPLER_MAX_V || B > 0x7FFFFFFFll) return 0;
  const FastPlan pl = plan_fast(dtype, B, V, params, true);
  return pl.fast ? pl.ws_bytes : topp_workspace_bytes(dtype, B, V, params, SIZE_MAX);
}

extern "C" int gtp_sample_route(int dtype, int64_t B, int64_t V, int aligned, int64_t hist_len,
                                int has_mask, const gtp_sampler_params* params,
                                size_t workspace_bytes, int32_t* out_route, int32_t* out_slices) {
  if (!params || !out_route || B <= 0 || V <= 0 || hist_len < 0) return GTP_ERR_INVALID_ARGUMENT;
  if (dtype != GTP_DTYPE_F32 && dtype != GTP_DTYPE_BF16 && dtype != GTP_DTYPE_F16)
    return GTP_ERR_INVALID_ARGUMENT;
  if (V > GTP_SAMPLER_MAX_V || B > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  const FastPlan pl = plan_fast(dtype, B, V, params, aligned != 0);
  if (pl.fast) {
    *out_route = GTP_ROUTE_SPLIT_TOPK;
    if (out_slices) *out_slices = pl.S;
    return GTP_OK;
  }
  const GeneralRoute r = route_general(dtype, B, V, aligned != 0, hist_len, has_mask != 0, params,
                                       workspace_bytes > 0, workspace_bytes);
  *out_route = r.route;
  if (out_slices) *out_slices = r.route == GTP_ROUTE_TOPP_SPLIT ? r.split.S : 1;
  return GTP_OK;
}

namespace gtp {

// gtp_sample_rows with its workspace; `clear_counters` zeroes the per-row
// arrival counters first (a fill kernel, so a captured graph holds no memset
// node), for a workspace whose previous contents the call cannot vouch for.
int sample_rows_impl(const void* logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
                     const int32_t* history, int64_t hist_len, int64_t hist_stride,
                     const uint32_t* allow_mask, int64_t mask_stride, const float* uniforms,
                     const gtp_sampler_params* params, const uint8_t* finished,
                     int64_t pad_token_id, int64_t* out_ids, float* out_logprob,
                     float* out_sampled_logprob, int32_t* out_kept, float* out_thresh_value,
                     int32_t* out_thresh_id, int32_t* out_status, void* workspace,
                     size_t workspace_bytes, bool clear_counters, void* stream);

}  // namespace gtp

extern "C" int gtp_sample_rows(const void* logits, int dtype, int64_t B, int64_t V,
                               int64_t row_stride, const int32_t* history, int64_t hist_len,
                               int64_t hist_stride, const uint32_t* allow_mask, int64_t mask_stride,
                               const float* uniforms, const gtp_sampler_params* params,
                               const uint8_t* finished, int64_t pad_token_id, int64_t* out_ids,
                               float* out_logprob, float* out_sampled_logprob, int32_t* out_kept,
                               float* out_thresh_value, int32_t* out_thresh_id, int32_t* out_status,
                               void* workspace, size_t workspace_bytes, void* stream) {
  return sample_rows_impl(logits, dtype, B, V, row_stride, history, hist_len, hist_stride,
                          allow_mask, mask_stride, uniforms, params, finished, pad_token_id,
                          out_ids, out_logprob, out_sampled_logprob, out_kept, out_thresh_value,
                          out_thresh_id, out_status, workspace, workspace_bytes, false, stream);
}

// ------------------------------------------------ the entry point without allocation
//
// gtp_sample_rows_noalloc runs gtp_sample_rows with the library's own
// workspace: a file-scope device array of GTP_NOALLOC_SCRATCH_BYTES, one copy
// per GPU for the life of the process.  Host code never passes the array's
// name to a kernel (on the host it is a stand-in, not a device address): the
// first call on each device, with that device current, looks up that
// device's copy with hipGetSymbolAddress and keeps the address in a
// per-device table, and every launch takes the address from the table.
static __device__ __align__(256) unsigned char scratch[GTP_NOALLOC_SCRATCH_BYTES];

namespace gtp {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// This device's copy of `scratch`, or nullptr when it cannot be found.
void* scratch_for_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace gtp

extern "C" int gtp_sample_rows_noalloc(const void* logits, int dtype, int64_t B, int64_t V,
                                       int64_t row_stride, const int32_t* history,
                                       int64_t hist_len, int64_t hist_stride,
                                       const uint32_t* allow_mask, int64_t mask_stride,
                                       const float* uniforms, const gtp_sampler_params* params,
                                       const uint8_t* finished, int64_t pad_token_id,
                                       int64_t* out_ids, float* out_logprob,
                                       float* out_sampled_logprob, int32_t* out_kept,
                                       float* out_thresh_value, int32_t* out_thresh_id,
                                       int32_t* out_status, void* stream) {
  if (!params || B < 0 || V <= 0) return GTP_ERR_INVALID_ARGUMENT;
  if (B == 0) return GTP_OK;
  size_t need = gtp_sample_workspace_bytes(dtype, B, V, params);
  if (need > GTP_NOALLOC_SCRATCH_BYTES && !plan_fast(dtype, B, V, params, true).fast)
    need = topp_workspace_bytes(dtype, B, V, params, GTP_NOALLOC_SCRATCH_BYTES);  // fewer slices
  if (need > GTP_NOALLOC_SCRATCH_BYTES) return GTP_ERR_UNSUPPORTED;
  void* ws = nullptr;
  if (need > 0) {
    ws = scratch_for_current_device();
    if (!ws) return GTP_ERR_LAUNCH;
  }
  return sample_rows_impl(logits, dtype, B, V, row_stride, history, hist_len, hist_stride,
                          allow_mask, mask_stride, uniforms, params, finished, pad_token_id,
                          out_ids, out_logprob, out_sampled_logprob, out_kept, out_thresh_value,
                          out_thresh_id, out_status, ws, GTP_NOALLOC_SCRATCH_BYTES, true, stream);
}

namespace gtp {

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

int sample_rows_impl(const void* logits, int dtype, int64_t B, int64_t V, int64_t row_stride,
                     const int32_t* history, int64_t hist_len, int64_t hist_stride,
                     const uint32_t* allow_mask, int64_t mask_stride, const float* uniforms,
                     const gtp_sampler_params* params, const uint8_t* finished,
                     int64_t pad_token_id, int64_t* out_ids, float* out_logprob,
                     float* out_sampled_logprob, int32_t* out_kept, float* out_thresh_value,
                     int32_t* out_thresh_id, int32_t* out_status, void* workspace,
                     size_t workspace_bytes, bool clear_counters, void* stream) {
  if (!params || B < 0 || V <= 0 || row_stride < V) return GTP_ERR_INVALID_ARGUMENT;
  if (dtype != GTP_DTYPE_F32 && dtype != GTP_DTYPE_BF16 && dtype != GTP_DTYPE_F16)
    return GTP_ERR_INVALID_ARGUMENT;
  if (B > 0 && (!logits || !out_ids)) return GTP_ERR_INVALID_ARGUMENT;
  if (!(params->repetition_penalty > 0.0f)) return GTP_ERR_INVALID_ARGUMENT;
  // bounded before any size arithmetic below
  if (V > GTP_SAMPLER_MAX_V || B > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  if (allow_mask && mask_stride < (V + 31) / 32) return GTP_ERR_INVALID_ARGUMENT;
  if (hist_len < 0) return GTP_ERR_INVALID_ARGUMENT;
  if (history && hist_len > 0 && hist_stride < hist_len) return GTP_ERR_INVALID_ARGUMENT;
  const bool greedy = !(params->temperature > 0.0f);
  if (!greedy && B > 0 && !uniforms) return GTP_ERR_INVALID_ARGUMENT;
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
  // the stride's byte count modulo 16, in unsigned arithmetic (any stride >= V is legal)
  const bool aligned = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0 &&
                       (((uint64_t)row_stride * (uint64_t)es) & 15u) == 0;
  const FastPlan pl = plan_fast(dtype, B, V, params, aligned);
  if (!pl.fast) {
    const size_t tw = topp_workspace_bytes(dtype, B, V, params, workspace_bytes);
    if (clear_counters && tw > 0 && workspace && workspace_bytes >= tw) {
      // the split top-p kernel's zero region (its per-row arrival counters)
      const int64_t nw = (int64_t)(kWsZeroBytes / 4);
      hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, st,
                         reinterpret_cast<uint32_t*>(workspace), nw);
    }
    return launch_sampler_general(a, dtype, B, st, workspace, workspace_bytes);
  }
  if (pl.ws_bytes > 0 && (!workspace || workspace_bytes < pl.ws_bytes))
    return GTP_ERR_INVALID_ARGUMENT;
  if (clear_counters && pl.ws_bytes > 0) {
    const int64_t nw = (int64_t)(pl.cnt_bytes / 4);
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<uint32_t*>(workspace), nw);
  }

  FastArgs fa;
  fa.a = a;
  fa.vps = pl.vps;
  fa.ws = reinterpret_cast<unsigned char*>(workspace);
  fa.cnt_bytes = pl.cnt_bytes;
  fa.greedy = greedy ? 1 : 0;
  fa.Kc = greedy ? 1 : params->top_k;
  fa.use_pen = (history && hist_len > 0 && params->repetition_penalty != 1.0f) ? 1 : 0;
  fa.p_active = (!greedy && params->top_p > 0.0f && params->top_p < 1.0f) ? 1 : 0;
  fa.Tc = params->temperature > 1e-6f ? params->temperature : 1e-6f;
  const dim3 grid((unsigned)pl.S, (unsigned)B), block(kFT);
  const bool m = allow_mask != nullptr;
  switch (dtype) {
    case GTP_DTYPE_BF16:
      if (m) launch_timed(sampler_split_kernel<uint16_t, true>, grid, block, st, fa);
      else launch_timed(sampler_split_kernel<uint16_t, false>, grid, block, st, fa);
      break;
    case GTP_DTYPE_F16:
      if (m) launch_timed(sampler_split_kernel<_Float16, true>, grid, block, st, fa);
      else launch_timed(sampler_split_kernel<_Float16, false>, grid, block, st, fa);
      break;
    default:
      if (m) launch_timed(sampler_split_kernel<float, true>, grid, block, st, fa);
      else launch_timed(sampler_split_kernel<float, false>, grid, block, st, fa);
      break;
  }
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}

}  // namespace gtp
