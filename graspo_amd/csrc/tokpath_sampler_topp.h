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
// Value bins.  A bf16 value with biased exponent in [87, 150) has a 13-bit
// magnitude index i; word i of a region holds two 16-bit counts, the
// positive value in the low half and the negative one in the high half.
// Per token the stream computes the byte offset of its word with packed
// 16-bit arithmetic on the token pair a 32-bit load returns (and, sub,
// min, shift: two tokens per instruction) and adds 1 or 0x10000 to it in
// LDS: about six instructions per token, no branch.  Zeros, values outside
// the exponent range, infinities and NaN fall into an escape word; a row
// with any escape is handed over.  Region A counts the allowed unpenalised
// tokens; region 2 counts the allowed penalised tokens (by raw value) or,
// with a mask and no penalty, the masked tokens (for the raw log-sum-exp).
// With both a mask and a penalty, masked tokens go to per-lane spill words
// and the raw log-sum-exp is folded per token.
//
// 1. Pilot.  The first chunk of each wave (16 evenly spaced places of the
//    row) is counted; one block scan over the counts picks theta, the value
//    with about 1200 sampled-to-scale allowed tokens at or above it.
// 2. Stream.  Counts per token; a vector (8 tokens) with an allowed token at
//    or above theta goes whole into an LDS pool (16 bytes and its index).
// 3. Totals.  Thread t owns the value bins 16t..16t+15 (descending values)
//    and the penalised values whose processed logit y lies between them;
//    its weight total (DETEXP_FIX(y - m) per value times the count) and
//    count go through one block scan in descending order.  The raw
//    log-sum-exp comes from the same counts.
// 4. Cut and draw.  One wave finds the thread whose range holds floor(P W)
//    (then floor(u W')) from the stored prefixes, ranks the range's values
//    by y and takes the position inside the tied value (all its tokens
//    share one weight) as an integer quotient.
// 5. Ids.  The k-th token (id order) of the cut value and the j-th of the
//    drawn value come from the pool when every token of both values is in
//    it; otherwise from one more read of the row.
// Outside these bounds (an escape, a 16-bit count overflow, a penalised
// value above every bin, more than 48 penalised values in one resolved
// range) the row is handed over to the row-wise path, which the same
// workgroup runs in the same launch; the decision is block-uniform and taken
// before any output of the row is written.
#pragma once

namespace gtp {
namespace topp {

typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef short ss2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ us2 as_us2(uint32_t w) { return __builtin_bit_cast(us2, w); }
__device__ __forceinline__ ss2 as_ss2(uint32_t w) { return __builtin_bit_cast(ss2, w); }
__device__ __forceinline__ uint32_t as_u32(us2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ uint32_t as_u32(ss2 v) { return __builtin_bit_cast(uint32_t, v); }

constexpr int kB = 1024;             // threads per row
constexpr int kW = kB / kWave;       // waves per row
constexpr int kG = 4;                // vectors per lane per chunk
constexpr int kChunk = kWave * kG;   // vectors per chunk (2048 tokens, 64 mask words)
constexpr uint32_t kELo = 87;        // smallest binned biased exponent
constexpr uint32_t kBase = kELo << 7;
constexpr uint32_t kNI = 63u * 128u;  // magnitude indices per sign (index 0: zero and tiny values)
constexpr int kNV = 2 * (int)kNI;     // value bins, index 0 = the largest value
constexpr int kPer = 16;              // value bins per owning thread
constexpr int kOwners = kNV / kPer;   // threads that own value bins
constexpr uint32_t kR2 = 8192;        // first word of region 2 (byte offset 32768)
constexpr uint32_t kJunk = 8160;      // word for vectors past the row's end
constexpr uint32_t kSpill = 16320;    // 64 per-lane spill words (mask and penalty)
constexpr int kHistWords = 16384;
constexpr int kPoolV = 3584;          // captured vectors (without a penalty)
constexpr int kPoolVPen = 1536;       // ... with one (the penalty bitmap takes the rest)
constexpr uint32_t kTarget = 2560;    // tokens the pilot aims to capture (without a penalty)
constexpr uint32_t kTargetPen = 1100;
constexpr int kPenLanes = 48;         // penalised values one resolved range may hold
constexpr int kSmall = 64;            // values with at most this many tokens rank from a list
constexpr int kRescanBuf = 512;       // ids one wave keeps per value in a rescan
constexpr int kRescanG = 4;           // vectors per lane per rescan step
constexpr int64_t kMinV = 65536;
constexpr uint32_t kNone = 0xFFFFFFFFu;

struct Level {
  float y;                      // processed logit of the value
  uint32_t hu;                  // bf16 bits of its unpenalised tokens, kNone: none
  uint32_t hp;                  // bf16 bits of its penalised tokens, kNone: none
  uint32_t n;                   // tokens of the value
  uint32_t k;                   // position of the wanted token in id order
  uint32_t n_before;            // tokens before the value
  unsigned long long s_before;  // weight before the value
  unsigned long long w;         // weight of one of its tokens
};

struct alignas(16) Smem {
  // counts (regions A and 2, junk and spill words); after the cut and the
  // draw: id lists, id bitmaps or rescan buffers
  uint32_t hist[kHistWords];
  // pool: captured vectors; with a penalty, entries [kPoolVPen, kPoolV)
  // hold the bitmap of penalised ids (GTP_SAMPLER_MAX_V bits)
  u32x4 qd[kPoolV];
  uint32_t qv[kPoolV];  // ... their vector index | allow byte << 16
  union {
    struct {
      unsigned long long w[kB];  // penalised values' weight per owning thread
      uint32_t c[kB];            // ... and count
    } own;
    struct {
      unsigned long long w[kB + 1];  // weight before each thread's range (then the total)
      uint32_t c[kB + 1];            // count before each thread's range
    } ex;
  } x;
  unsigned long long red_w[kW];
  uint32_t red_u[kW][4];
  float red_f[kW][3];
  Level lv[2];  // the cut (0) and the drawn (1) value
  int32_t id_out[2];
  uint32_t scan_n[kW][2];
  uint32_t seg_n[kW];  // pool entries of each wave's own segment
  uint32_t over_n;     // entries of the shared overflow area
  uint32_t list_n[2];
  uint32_t chunk_ctr;
  uint32_t drop_ord;  // largest ord16 key of a vector the full pool dropped, 0: none
  uint32_t theta;     // bf16 bits of theta, kNone: every allowed token is captured
  float u;            // the row's uniform and finished flag (read at the start)
  uint32_t fin;
  uint32_t flags;     // bit 0: hand over; bit 1: bad history id
  // the weight scan's totals (weight, count, region-2 count, raw (m, s))
  unsigned long long tot_w;
  uint32_t tot_n, tot_n2;
  float tot_m, tot_s;
  int32_t bad;
  __device__ __forceinline__ uint32_t* pen() { return reinterpret_cast<uint32_t*>(&qd[kPoolVPen]); }
  __device__ __forceinline__ const uint32_t* pen() const {
    return reinterpret_cast<const uint32_t*>(&qd[kPoolVPen]);
  }
};

// Magnitude index i of a bf16 value: 0 for zeros and values below 2^-40
// (the zero bin), mag - (kBase - 1) for the exponents [87, 150) (the last
// magnitude aside), kNI (the escape word) above.
// Value bin v (0 = the largest) <-> word, half and bf16 bits; the two zero
// bins (v = kNI - 1 and kNI) stand for the value 0.
constexpr int kZeroPos = (int)kNI - 1, kZeroNeg = (int)kNI;
__device__ __forceinline__ uint32_t vb_word(int v) {
  return v < (int)kNI ? kNI - 1u - (uint32_t)v : (uint32_t)v - kNI;
}
__device__ __forceinline__ uint32_t vb_shift(int v) { return v < (int)kNI ? 0u : 16u; }
__device__ __forceinline__ uint32_t vb_bits(int v) {  // (the zero bins: 0x0000 / 0x8000)
  const uint32_t i = vb_word(v);
  const uint32_t mag = i ? i + kBase - 1u : 0u;
  return v < (int)kNI ? mag : 0x8000u | mag;
}
__device__ __forceinline__ float vb_x(int v) { return vb_word(v) ? u2f(vb_bits(v) << 16) : 0.0f; }
__device__ __forceinline__ int vb_of(uint32_t h) {  // -1 outside the bins
  const uint32_t mag = h & 0x7FFFu;
  const uint32_t i = mag < kBase ? 0u : mag - (kBase - 1u);
  if (i >= kNI) return -1;
  return (h & 0x8000u) ? (int)(kNI + i) : (int)(kNI - 1u - i);
}
__device__ __forceinline__ uint32_t cnt(const Smem& sm, uint32_t region, int v) {
  return (sm.hist[region + vb_word(v)] >> vb_shift(v)) & 0xFFFFu;
}

// 0xFFFF in the low half when bit 2p of b is set, in the high half when bit
// 2p + 1 is
__device__ __forceinline__ uint32_t spread(uint32_t b, int p) {
  const uint32_t lo = (uint32_t)((int32_t)(b << (31 - 2 * p)) >> 31);
  const uint32_t hi = (uint32_t)((int32_t)(b << (30 - 2 * p)) >> 31);
  return (lo & 0xFFFFu) | (hi & 0xFFFF0000u);
}

// region-A word indices (two 16-bit halves) of a token pair: a saturating
// subtraction sends zeros and tiny values to index 0, a minimum sends the
// values above the range (and infinities, NaN) to the escape word
__device__ __forceinline__ uint32_t pair_words(uint32_t w) {
  const us2 i = __builtin_elementwise_sub_sat(as_us2(w & 0x7FFF7FFFu), (us2)(unsigned short)(kBase - 1u));
  return as_u32(__builtin_elementwise_min(i, (us2)(unsigned short)kNI));
}

__device__ __forceinline__ void lds_add(Smem& sm, uint32_t word, uint32_t v) {
  __hip_atomic_fetch_add(&sm.hist[word], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Block-wide exclusive scan in thread order of (u64, u32) plus a float sum;
// every thread gets its exclusive prefix and the totals.
__device__ __forceinline__ void block_scan2(Smem& sm, unsigned long long w, uint32_t c, float f,
                                            unsigned long long& ew, uint32_t& ec,
                                            unsigned long long& tw, uint32_t& tc, float& tf) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const unsigned long long iw = wave_scan_u64(w);
  const uint32_t ic = wave_scan_u32(c);
  const float sf = wave_sum_f(f);
  __syncthreads();
  if (lane == kWave - 1) {
    sm.red_w[wid] = iw;
    sm.red_u[wid][0] = ic;
    sm.red_f[wid][0] = sf;
  }
  __syncthreads();
  unsigned long long bw = 0ull, allw = 0ull;
  uint32_t bc = 0u, allc = 0u;
  float allf = 0.0f;
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
    allf += sm.red_f[i][0];
  }
  ew = bw + iw - w;
  ec = bc + ic - c;
  tw = allw;
  tc = allc;
  tf = allf;
}

// The weight step's block scan: exclusive prefix in thread order of the
// owners' (weight, count), the totals, the sum of n2 and the raw (m, s)
// merge (online with a mask and no penalty).  Wave 0 combines the 16 waves'
// partials in its lanes and hands the prefixes back through LDS, so no
// thread loops over all waves (the tail runs at one CU's issue rate).
template <int kMode>
__device__ __forceinline__ void weight_scan(Smem& sm, unsigned long long Wt, uint32_t Nt, uint32_t n2,
                                            float lm, float lsum, unsigned long long& ew, uint32_t& ec,
                                            unsigned long long& W, uint32_t& N, uint32_t& N2, float& lse_m,
                                            float& lse_s) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const unsigned long long iw = wave_scan_u64(Wt);
  const uint32_t ic = wave_scan_u32(Nt);
  const uint32_t s2 = wave_total_u32(n2);
  if (kMode == 2) wave_lse2(lm, lsum);
  else if (kMode != 3) lsum = wave_sum_f(lsum);
  __syncthreads();  // (own is read)
  if (lane == kWave - 1) {
    sm.red_w[wid] = iw;
    sm.red_u[wid][0] = ic;
    sm.red_u[wid][1] = s2;
    sm.red_f[wid][0] = lm;
    sm.red_f[wid][1] = lsum;
  }
  __syncthreads();
  if (wid == 0) {
    const bool in = lane < kW;
    const unsigned long long vw = in ? sm.red_w[lane] : 0ull;
    const uint32_t vc = in ? sm.red_u[lane][0] : 0u, v2 = in ? sm.red_u[lane][1] : 0u;
    const float fm = in ? sm.red_f[lane][0] : kNegInf, fs = in ? sm.red_f[lane][1] : 0.0f;
    const unsigned long long pw = wave_scan_u64(vw);
    const uint32_t pc = wave_scan_u32(vc);
    const uint32_t t2 = wave_total_u32(v2);
    const float mm = wave_max_f(fm);
    float ss = 0.0f;
    if (kMode == 2) ss = wave_sum_f(fs > 0.0f ? fs * __builtin_amdgcn_exp2f((fm - mm) * kLog2e) : 0.0f);
    else if (kMode != 3) ss = wave_sum_f(fs);
    if (in) {  // (this wave read its lanes' entries above)
      sm.red_w[lane] = pw - vw;
      sm.red_u[lane][2] = pc - vc;
    }
    if (lane == kWave - 1) {
      sm.tot_w = pw;
      sm.tot_n = pc;
      sm.tot_n2 = t2;
      sm.tot_m = mm;
      sm.tot_s = ss;
    }
  }
  __syncthreads();
  ew = sm.red_w[wid] + iw - Wt;
  ec = sm.red_u[wid][2] + ic - Nt;
  W = sm.tot_w;
  N = sm.tot_n;
  N2 = sm.tot_n2;
  lse_m = sm.tot_m;
  lse_s = sm.tot_s;
}

struct Row {
  const uint16_t* __restrict__ x;
  const uint32_t* __restrict__ mask;
  int64_t V, nvec;
  float rho, Tc;
  // processed logits (contract steps: penalty, then temperature), zeros canonical
  __device__ __forceinline__ float pen_v(float v) const { return v < 0.0f ? v * rho : v / rho; }
  __device__ __forceinline__ float y_of(float v) const { return v / Tc + 0.0f; }
  __device__ __forceinline__ float ybin(int v) const { return y_of(vb_x(v)); }
  __device__ __forceinline__ float ypen(int v) const { return y_of(pen_v(vb_x(v))); }
  __device__ __forceinline__ bool allowed(int64_t id) const {
    return !mask || ((mask[id >> 5] >> (id & 31)) & 1u);
  }
};

// Largest value bin v with ybin(v) >= y (the smallest binned value whose
// processed logit reaches y), or -1 when y lies above every bin.
__device__ __forceinline__ int ceil_v(const Row& r, float y) {
  int v = vb_of(bf16_round_up(y * r.Tc));
  if (v < 0) {
    if (!(r.ybin(0) >= y)) return -1;
    int lo = 0, hi = kNV - 1;  // ybin(lo) >= y; the answer lies in [lo, hi]
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (r.ybin(mid) >= y) lo = mid;
      else hi = mid - 1;
    }
    return lo;
  }
  while (v + 1 < kNV && r.ybin(v + 1) >= y) ++v;
  while (v >= 0 && r.ybin(v) < y) --v;
  return v;
}

// First value bin p in [0, kNV] with ypen(p) <= y (ypen falls as p grows),
// by the 64 lanes of a wave.  First one window of 64 bins around the raw
// value whose penalised, scaled logit is y (x = y T rho for y >= 0, y T / rho
// below): the predicate "p == kNV or ypen(p) <= y" is monotone, so when the
// window's first bin fails it (or is bin 0) and a later one passes, the
// first passing bin is the answer.  Otherwise rounds of 64 probes narrow
// 16128 candidates to one in three steps.  Wave-uniform result.
__device__ __forceinline__ int first_pen_le(const Row& r, float y) {
  const int lane = threadIdx.x & (kWave - 1);
  {
    const float xs = y * r.Tc;
    const int ve = vb_of(bf16_round_up(xs >= 0.0f ? xs * r.rho : xs / r.rho));
    if (ve >= 0) {
      int w0 = ve - kWave / 2;
      w0 = w0 < 0 ? 0 : (w0 > kNV - (kWave - 1) ? kNV - (kWave - 1) : w0);
      const int p = w0 + lane;  // <= kNV
      const unsigned long long pass = __ballot(p >= kNV || r.ypen(p) <= y);
      if (pass && (w0 == 0 || !(pass & 1ull))) return w0 + __builtin_ctzll(pass);
    }
  }
  int lo = 0, hi = kNV;  // the answer lies in [lo, hi]
  while (hi > lo) {
    const int span = hi - lo;
    // lane l probes lo + ceil((l + 1) span / 65) - 1: increasing, inside [lo, hi)
    const int probe = lo + (int)(((int64_t)(lane + 1) * span + 64) / 65) - 1;
    const bool le = r.ypen(probe) <= y;
    const unsigned long long hit = __ballot(le);
    const unsigned long long miss = __ballot(!le);
    const int nhi = hit ? __builtin_amdgcn_readlane(probe, __builtin_ctzll(hit)) : hi;
    const int nlo = miss ? __builtin_amdgcn_readlane(probe, 63 - __builtin_clzll(miss)) + 1 : lo;
    lo = nlo;
    hi = nhi;
  }
  return lo;
}

// Resolve the crossing of weight position X (one wave): the owning thread
// from the stored prefixes, then its range's values -- 16 bins and the
// penalised values whose y lies between them -- ranked by y, scanned, and
// the position inside the crossing value.  False: the row must be handed
// over.
template <int kMode>
__device__ __forceinline__ bool resolve(const Smem& sm, const Row& r, float m, unsigned long long X,
                                        Level& out) {
  const int lane = threadIdx.x & (kWave - 1);
  // owner: the last thread t with ex.w[t] <= X (ex.w[kOwners] is the total, > X)
  const unsigned long long b1 = __ballot(sm.x.ex.w[lane * kPer] <= X);
  const int base = (63 - __builtin_clzll(b1)) * kPer;
  const unsigned long long b2 = __ballot(lane < kPer && sm.x.ex.w[base + (lane & (kPer - 1))] <= X);
  const int t = base + (63 - __builtin_clzll(b2));
  if (t >= kOwners) return false;
  const unsigned long long ex_w = sm.x.ex.w[t];
  const uint32_t ex_c = sm.x.ex.c[t];
  const int v0 = t * kPer;
  int pa = 0, np = 0;
  if (kMode & 1) {
    const float hi_y = r.ybin(v0);
    pa = first_pen_le(r, hi_y);
    const int pe = v0 + kPer < kNV ? first_pen_le(r, r.ybin(v0 + kPer)) : kNV;
    np = pe - pa;
    if (np > kPenLanes) return false;
  }
  // entries: lanes 0..15 the bins v0 + lane (descending), lanes 16.. the
  // penalised raw bins pa, pa + 1, .. (descending y)
  float y = kNegInf;
  uint32_t c = 0u;
  int kind = -1, ref = -1;
  if (lane < kPer) {
    kind = 0;
    ref = v0 + lane;
    c = cnt(sm, 0u, ref);
    y = r.ybin(ref);
  } else if (lane < kPer + np) {
    kind = 1;
    ref = pa + (lane - kPer);
    c = cnt(sm, kR2, ref);
    y = r.ypen(ref);
  }
  if (c == 0u) {
    y = kNegInf;
    kind = -1;
  }
  const unsigned long long w1 = c ? detexp_fix(y - m) : 0ull;
  float ys;
  uint32_t cs;
  int kinds, refs;
  unsigned long long ws;
  if (kMode & 1) {
    // rank by (y desc, lane asc) and move every entry to its rank
    const uint32_t ky = ord32(y);
    uint32_t rank = 0;
#pragma unroll 8
    for (int j = 0; j < kWave; ++j) {
      const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)ky, j);
      rank += (kj > ky || (kj == ky && j < lane)) ? 1u : 0u;
    }
    auto scatter_u32 = [&](uint32_t v) -> uint32_t {
      return (uint32_t)__builtin_amdgcn_ds_permute((int)(rank * 4u), (int)v);
    };
    ys = u2f(scatter_u32(f2u(y)));
    cs = scatter_u32(c);
    kinds = (int)scatter_u32((uint32_t)kind);
    refs = (int)scatter_u32((uint32_t)ref);
    ws = ((unsigned long long)scatter_u32((uint32_t)(w1 >> 32)) << 32) | scatter_u32((uint32_t)w1);
  } else {
    // the 16 bins are in descending order already
    ys = y;
    cs = c;
    kinds = kind;
    refs = ref;
    ws = w1;
  }
  const unsigned long long iw = wave_scan_u64((unsigned long long)cs * ws);
  const uint32_t ic = wave_scan_u32(cs);
  const unsigned long long rel = X - ex_w;
  const unsigned long long past = __ballot(iw > rel);
  if (!past) return false;  // cannot happen: X lies inside the range
  const int e = __builtin_ctzll(past);
  const float ye = u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(ys), e));
  // the zero bins hold zeros and tiny values of one weight but distinct
  // order: a position inside them goes to the row-wise path
  if (ye == 0.0f) return false;
  const unsigned long long grp = __ballot(ys == ye && cs != 0u);
  const int gs = __builtin_ctzll(grp);
  const unsigned long long iw_b =
      gs ? (((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(iw >> 32), gs - 1)
             << 32) |
            (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)iw, gs - 1))
         : 0ull;
  const uint32_t ic_b = gs ? (uint32_t)__builtin_amdgcn_readlane((int)ic, gs - 1) : 0u;
  const bool in_grp = (grp >> lane) & 1ull;
  // the group's members (at most one unpenalised and one penalised value)
  const uint32_t gn = wave_total_u32(in_grp ? cs : 0u);
  const unsigned long long bu = __ballot(in_grp && kinds == 0);
  const unsigned long long bp = __ballot(in_grp && kinds == 1);
  const int ub = bu ? __builtin_amdgcn_readlane(refs, __builtin_ctzll(bu)) : -1;
  const int pb = bp ? __builtin_amdgcn_readlane(refs, __builtin_ctzll(bp)) : -1;
  const unsigned long long wt =
      ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(ws >> 32), e) << 32) |
      (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)ws, e);
  out.y = ye;
  out.hu = ub >= 0 ? vb_bits(ub) : kNone;
  out.hp = pb >= 0 ? vb_bits(pb) : kNone;
  out.n = gn;
  out.s_before = ex_w + iw_b;
  out.n_before = ex_c + ic_b;
  out.w = wt;
  // q = floor((X - s_before) / wt) < gn <= 2^18: a double estimate, then
  // exact integer corrections (every product stays below X < 2^63)
  const unsigned long long num = X - out.s_before;
  unsigned long long q = (unsigned long long)((double)num / (double)wt);
  while (q > 0 && q * wt > num) --q;
  while ((q + 1) * wt <= num) ++q;
  out.k = (uint32_t)q;
  return q < gn;
}

__device__ __forceinline__ bool in_level(const Level& L, bool pn, uint32_t h) {
  return h == (pn ? L.hp : L.hu);
}

// Ids of the two levels' wanted tokens (rank k0 of level 0, k1 of level 1,
// in id order) by one more read of the vectors [lo_a, hi_a) (and the
// vocabulary tail when `tail_a`) -- or, when `two`, of [lo_a, hi_a) for
// level 0 by waves 0-7 and [lo_b, hi_b) (tail_b) for level 1 by waves 8-15.
// Each wave walks a contiguous part of its range, counts its levels' tokens
// with packed 16-bit compares (bit 15 of a half is set where the half equals
// the level's pattern), keeps up to kRescanBuf matching ids per level in id
// order; the wave whose part holds a wanted token reads it from its buffer,
// or walks its part again when the buffer overflowed.  Writes
// sm.id_out[0..1].
template <int kMode>
__device__ __forceinline__ void rescan_ids(Smem& sm, const Row& r, int64_t lo_a, int64_t hi_a,
                                           bool tail_a, int64_t lo_b, int64_t hi_b, bool tail_b,
                                           uint32_t k0, uint32_t k1, bool two) {
  constexpr bool kPen = (kMode & 1) != 0, kMask = (kMode & 2) != 0;
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const int64_t nvec = r.nvec, V = r.V;
  const int grp = two && wid >= kW / 2 ? 1 : 0;  // (wave-uniform)
  const int ng = two ? kW / 2 : kW, wl = two ? wid % (kW / 2) : wid;
  const bool want0 = !two || grp == 0, want1 = !two || grp == 1;
  const int64_t lo = grp ? lo_b : lo_a, hi = grp ? hi_b : hi_a;
  const bool tail_here = grp ? tail_b : tail_a;
  const int64_t span = (hi - lo + ng - 1) / ng;
  const int64_t v0 = lo + wl * span < hi ? lo + wl * span : hi;
  const int64_t v1 = v0 + span < hi ? v0 + span : hi;
  Level L0 = sm.lv[0], L1 = sm.lv[1];
  if (!want0) L0.hu = L0.hp = kNone;
  if (!want1) L1.hu = L1.hp = kNone;
  uint32_t* buf0 = sm.hist + (0 * kW + wid) * kRescanBuf;
  uint32_t* buf1 = sm.hist + (1 * kW + wid) * kRescanBuf;
  // a level's value in both halves (0xFFFF, a NaN pattern, matches nothing
  // here: such rows never reach this point)
  auto pat = [](uint32_t h) { return h == kNone ? 0xFFFFFFFFu : h * 0x10001u; };
  const uint32_t u0 = pat(L0.hu), p0 = pat(L0.hp), u1 = pat(L1.hu), p1 = pat(L1.hp);
  auto zeq = [](uint32_t w, uint32_t pt) {
    const uint32_t x = w ^ pt;
    return as_u32(as_us2(x) - (us2)(unsigned short)1) & ~x & 0x80008000u;
  };
  // match bits (15 and 31 of each word) of vector v for both levels
  auto matches = [&](int64_t v, const u32x4& q, uint32_t(&m0)[4], uint32_t(&m1)[4])
                     __attribute__((always_inline)) {
    const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
    const uint32_t ab = kMask ? (r.mask[v >> 2] >> ((v & 3) * 8)) & 0xFFu : 0xFFu;
    const uint32_t pb = kPen ? (sm.pen()[v >> 2] >> ((v & 3) * 8)) & 0xFFu : 0u;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t a2 = kMask ? spread(ab, p) & 0x80008000u : 0x80008000u;
      if (kPen) {
        const uint32_t pn2 = spread(pb, p) & 0x80008000u;
        m0[p] = ((zeq(wd[p], u0) & ~pn2) | (zeq(wd[p], p0) & pn2)) & a2;
        m1[p] = ((zeq(wd[p], u1) & ~pn2) | (zeq(wd[p], p1) & pn2)) & a2;
      } else {
        m0[p] = zeq(wd[p], u0) & a2;
        m1[p] = zeq(wd[p], u1) & a2;
      }
    }
  };
  auto bits8 = [](const uint32_t(&m)[4]) {
    uint32_t b = 0u;
#pragma unroll
    for (int p = 0; p < 4; ++p) b |= (((m[p] >> 15) & 1u) << (2 * p)) | ((m[p] >> 31) << (2 * p + 1));
    return b;
  };
  auto count4 = [](const uint32_t(&m)[4]) {
    return (uint32_t)(__builtin_popcount(m[0]) + __builtin_popcount(m[1]) + __builtin_popcount(m[2]) +
                      __builtin_popcount(m[3]));
  };
  auto tail_matches = [&](uint32_t& t0, uint32_t& t1) {
    t0 = t1 = 0u;
    for (int64_t id = nvec * 8; id < V; ++id) {
      const int j = (int)(id - nvec * 8);
      const uint32_t h = r.x[id];
      const bool on = r.allowed(id);
      const bool pn = kPen && ((sm.pen()[id >> 5] >> (id & 31)) & 1u);
      t0 |= (on && in_level(L0, pn, h)) ? 1u << j : 0u;
      t1 |= (on && in_level(L1, pn, h)) ? 1u << j : 0u;
    }
  };
  const bool has_tail = tail_here && wl == ng - 1 && nvec * 8 < V;
  constexpr int64_t kStep = (int64_t)kWave * kRescanG;
  // append the set bits of mm (ids base + bit) at position ex onwards
  auto keep = [&](uint32_t* buf, uint32_t mm, uint32_t ex, int64_t base) {
    uint32_t i = ex;
    while (mm) {
      const int j = __builtin_ctz(mm);
      mm &= mm - 1u;
      if (i < (uint32_t)kRescanBuf) buf[i] = (uint32_t)(base + j);
      ++i;
    }
  };
  uint32_t run0 = 0u, run1 = 0u;
  for (int64_t vb = v0; vb < v1; vb += kStep) {
    u32x4 q[kRescanG];
#pragma unroll
    for (int g = 0; g < kRescanG; ++g) {
      const int64_t v = vb + g * kWave + lane;
      q[g] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(r.x) + (v < v1 ? v : v0));
    }
#pragma unroll
    for (int g = 0; g < kRescanG; ++g) {
      const int64_t v = vb + g * kWave + lane;
      uint32_t m0[4] = {0u, 0u, 0u, 0u}, m1[4] = {0u, 0u, 0u, 0u};
      if (v < v1) matches(v, q[g], m0, m1);
      const uint32_t n0 = count4(m0), n1 = count4(m1);
      if (!__ballot((n0 | n1) != 0u)) continue;
      const uint32_t i0 = wave_scan_u32(n0), i1 = wave_scan_u32(n1);
      if (n0) keep(buf0, bits8(m0), run0 + i0 - n0, v * 8);
      if (n1) keep(buf1, bits8(m1), run1 + i1 - n1, v * 8);
      run0 += lane63_u32(i0);
      run1 += lane63_u32(i1);
    }
  }
  if (has_tail) {
    uint32_t t0, t1;
    tail_matches(t0, t1);
    if (lane == 0) {
      keep(buf0, t0, run0, nvec * 8);
      keep(buf1, t1, run1, nvec * 8);
    }
    run0 += __builtin_popcount(t0);
    run1 += __builtin_popcount(t1);
  }
  if (lane == 0) {
    sm.scan_n[wid][0] = run0;
    sm.scan_n[wid][1] = run1;
  }
  __syncthreads();
  for (int l = 0; l < 2; ++l) {
    if (!(l ? want1 : want0)) continue;
    const uint32_t k = l ? k1 : k0;
    uint32_t before = 0u;
    for (int w = 0; w < wid; ++w) before += sm.scan_n[w][l];
    const uint32_t mine = sm.scan_n[wid][l];
    if (!(before <= k && k < before + mine)) continue;
    const uint32_t local = k - before;
    if (mine <= (uint32_t)kRescanBuf) {
      if (lane == 0) sm.id_out[l] = (int32_t)(l ? buf1 : buf0)[local];
      continue;
    }
    // the buffer overflowed: walk the range again up to the wanted match
    uint32_t run = 0u;
    bool done = false;
    for (int64_t vb = v0; vb < v1 && !done; vb += kWave) {
      const int64_t v = vb + lane;
      uint32_t m0[4] = {0u, 0u, 0u, 0u}, m1[4] = {0u, 0u, 0u, 0u};
      if (v < v1) matches(v, *reinterpret_cast<const u32x4*>(r.x + v * 8), m0, m1);
      const uint32_t mm = l ? bits8(m1) : bits8(m0);
      const uint32_t n = __builtin_popcount(mm);
      const uint32_t incl = wave_scan_u32(n);
      const uint32_t ex = run + incl - n;
      if (n && ex <= local && local < ex + n) {
        uint32_t mk = mm;
        for (uint32_t i = 0; i < local - ex; ++i) mk &= mk - 1u;
        sm.id_out[l] = (int32_t)(v * 8 + __builtin_ctz(mk));
      }
      run += lane63_u32(incl);
      done = run > local;
    }
    if (!done && has_tail && lane == 0) {  // the wanted token is in the tail
      uint32_t t0, t1;
      tail_matches(t0, t1);
      uint32_t mm = l ? t1 : t0;
      for (uint32_t i = 0; i < local - run; ++i) mm &= mm - 1u;
      sm.id_out[l] = (int32_t)(nvec * 8 + __builtin_ctz(mm));
    }
  }
  __syncthreads();
}

// One row; false when the row must be handed over to the row-wise path (a
// block-uniform decision, taken before any output is written).
// kMode bit 0: repetition penalty; bit 1: allow mask.
template <int kMode>
__device__ __forceinline__ bool topp_row(const SamplerArgs& a, int64_t b, Smem& sm) {
  constexpr bool kPen = (kMode & 1) != 0, kMask = (kMode & 2) != 0;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  Row r;
  r.x = reinterpret_cast<const uint16_t*>(a.logits) + b * a.row_stride;
  r.mask = kMask ? a.mask + b * a.mask_stride : nullptr;
  r.V = a.V;
  r.nvec = a.V / 8;
  r.rho = a.rho;
  r.Tc = a.T > 1e-6f ? a.T : 1e-6f;
  const int64_t V = a.V, nvec = r.nvec;
  const uint32_t nchunks = (uint32_t)((nvec + kChunk - 1) / kChunk);
  const uint32_t per = nchunks / kW;
  const bool ragged = (nvec % kChunk) != 0;  // the last chunk is partial
  // chunk c of the dynamic schedule -> chunk of the row: the first kW chunks
  // handed out start kW evenly spaced regions (the pilot sample)
  auto perm = [&](uint32_t c) -> uint32_t { return c < per * kW ? (c % kW) * per + c / kW : c; };
  // a thread's 16 bins are 16 consecutive words: visited in a per-thread
  // rotated order, the 64 lanes of a wave hit distinct LDS banks
  auto rot = [&](int j) -> int { return (j + (tid >> 2)) & (kPer - 1); };

  // ---- 0. the first two chunks of each wave in flight (chunks w and kW + w
  // of the schedule), then the clear
  const uint32_t last = (uint32_t)(nvec - 1);
  const uint32_t last_word = (uint32_t)((V - 1) >> 5);
  auto issue = [&](u32x4(&buf)[kG], uint32_t& sw, uint32_t chunk) {
    const uint32_t pc = perm(chunk);
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      uint32_t vi = pc * kChunk + (uint32_t)(k * kWave + lane);
      vi = vi < last ? vi : last;
      buf[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(r.x) + vi);
    }
    if (kMask) {  // the chunk's 64 mask words, one per lane
      const uint32_t w = pc * (kChunk * 8 / 32) + (uint32_t)lane;
      sw = r.mask[w < last_word ? w : last_word];
    }
  };
  u32x4 qa[kG], qb[kG];
  uint32_t swa = 0xFFFFFFFFu, swb = 0xFFFFFFFFu;
  uint32_t ca = (uint32_t)wid, cb = (uint32_t)(kW + wid);
  if (ca < nchunks) issue(qa, swa, ca);
  if (cb < nchunks) issue(qb, swb, cb);
  {
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int i = tid; i < kHistWords / 4; i += kB) reinterpret_cast<u32x4*>(sm.hist)[i] = z;
    if (kPen)
      for (int64_t i = tid; i < (V + 127) / 128; i += kB) reinterpret_cast<u32x4*>(sm.pen())[i] = z;
  }
  if (tid == 0) {
    // (read now: a global load after the stream waits behind the other
    // rows' traffic)
    sm.u = a.uniforms[b];
    sm.fin = a.finished && a.finished[b];
    sm.chunk_ctr = 2u * kW;
    sm.over_n = 0u;
    sm.drop_ord = 0u;
    sm.theta = kNone;
    sm.flags = 0u;
    sm.bad = 0;
    sm.list_n[0] = 0u;
    sm.list_n[1] = 0u;
    sm.id_out[0] = -1;
    sm.id_out[1] = -1;
  }
  __syncthreads();

  // ---- 1. the history bitmap
  auto grab = [&]() -> uint32_t {
    uint32_t c = 0;
    if (lane == 0) c = atomicAdd(&sm.chunk_ctr, 1u);
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)c);
  };
  if (a.hist && a.hist_len > 0) {
    const int32_t* h = a.hist + b * a.hist_stride;
    bool bad_hist = false;
    for (int64_t j = tid; j < a.hist_len; j += kB) {
      const int32_t id = h[j];
      if (id >= V) bad_hist = true;
      else if (kPen && id >= 0) atomicOr(&sm.pen()[id >> 5], 1u << (id & 31));
    }
    if (bad_hist) atomicOr(&sm.flags, 2u);
  }
  __syncthreads();  // the history bitmap is complete

  // allow bits of vector k of a chunk for this lane (vector k*64 + lane); a
  // cross-lane read, so every lane of the wave calls it
  auto allow_byte = [&](uint32_t sw, int k) -> uint32_t {
    const uint32_t w = (uint32_t)__shfl((int)sw, k * (kWave / 4) + lane / 4, kWave);
    return (w >> ((lane & 3) * 8)) & 0xFFu;
  };

  // ---- 2. stream state and a chunk's work
  Lse3 st{kNegInf, 0.0f, 0.0f};  // raw log-sum-exp per token (mask and penalty)
  const uint32_t junk2 = kJunk * 0x10001u;
  const uint32_t spill2 = (kSpill + (uint32_t)lane) * 0x10001u;
  // capture test: signed 16-bit compare of the raw bits against a theta >= 0,
  // order keys otherwise
  bool cap_signed = false;
  uint32_t cap_th2 = 0u;  // theta - 1 (signed) or ord16(theta) - 1, in both halves
  int th_s = 0;           // theta as a signed 16-bit pattern
  uint32_t th_o = 1u;     // ord16(theta) (1: every allowed token)
  uint32_t rmax = 0u;     // running maximum of the allowed tokens (packed, test's domain)
  // pool layout: 16 wave segments of kSegV entries, then a shared overflow
  // area of kOver entries
  constexpr uint32_t kCap = kPen ? kPoolVPen : kPoolV;
  constexpr uint32_t kSegV = kPen ? 64u : 160u;
  constexpr uint32_t kOver = kCap - kW * kSegV;
  uint32_t seg = 0u;  // this wave's pool entries so far (wave-uniform)
  // a vector whose test passed goes whole into this wave's pool segment (no
  // LDS round trip); past its end, into the overflow area (one LDS atomic
  // per wave and step); a full pool keeps the largest key it dropped
  auto append = [&](bool c, uint32_t vi, const u32x4& vec, uint32_t ab) __attribute__((always_inline)) {
    const unsigned long long bal = __ballot(c);
    if (!bal) return;
    const uint32_t base = seg, n = (uint32_t)__builtin_popcountll(bal);
    seg += n;
    const uint32_t first_over = base > kSegV ? base : kSegV;  // segment slot of the first overflow
    uint32_t obase = 0u;
    if (base + n > kSegV) {
      if (lane == 0) obase = atomicAdd(&sm.over_n, base + n - first_over);
      obase = (uint32_t)__builtin_amdgcn_readlane((int)obase, 0);
    }
    if (c) {
      const uint32_t slot = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                             __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
      const uint32_t o = obase + (slot - first_over);  // (used when slot >= kSegV)
      if (slot < kSegV || o < kOver) {
        const uint32_t e = slot < kSegV ? wid * kSegV + slot : kW * kSegV + o;
        sm.qd[e] = vec;
        sm.qv[e] = vi | (ab << 16);
      } else {
        const uint32_t wd[4] = {vec.x, vec.y, vec.z, vec.w};
        uint32_t mo = 0u;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t h = (j & 1) ? wd[j >> 1] >> 16 : wd[j >> 1] & 0xFFFFu;
          const uint32_t k = ((ab >> j) & 1u) ? ord16(h) : 0u;
          mo = k > mo ? k : mo;
        }
        atomicMax(&sm.drop_ord, mo);
      }
    }
  };
  // (partial, count, capture arrive as integral constants: each combination
  // compiles to its own branch-free body)
  auto work = [&](const u32x4(&buf)[kG], uint32_t sw, uint32_t chunk, auto partial_c, auto count_c,
                  auto capture_c) __attribute__((always_inline)) {
    constexpr bool partial = decltype(partial_c)::value;
    constexpr bool count = decltype(count_c)::value;
    constexpr bool capture = decltype(capture_c)::value;
    const uint32_t pc = perm(chunk);
    float xf[kG][8];
    float cm = kNegInf;
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      const uint32_t vi = pc * kChunk + (uint32_t)(k * kWave + lane);
      const bool valid = !partial || vi < (uint32_t)nvec;  // (always true for full chunks)
      uint32_t ab = kMask ? allow_byte(sw, k) : 0xFFu;
      if (partial && !valid) ab = 0u;
      const uint32_t pb =
          kPen ? (sm.pen()[(vi < last ? vi : last) >> 2] >> ((vi & 3) * 8)) & 0xFFu : 0u;
      const uint32_t wd[4] = {buf[k].x, buf[k].y, buf[k].z, buf[k].w};
      uint32_t mk[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) mk[p] = (kMask || partial) ? spread(ab, p) : 0xFFFFFFFFu;
      if constexpr (count) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t w = wd[p];
          uint32_t a2 = pair_words(w);  // region 2: + kR2 (bit 13 of each half)
          if (kMode == 1) a2 |= spread(pb, p) & 0x20002000u;
          if (kMode == 2) a2 |= ~mk[p] & 0x20002000u;
          if (kMode == 3) {
            a2 |= spread(pb, p) & 0x20002000u;
            a2 = (a2 & mk[p]) | (spill2 & ~mk[p]);
          }
          if (partial && !valid) a2 = junk2;
          // a negative value counts in the high half: 1 + 0xFFFF per negative token
          const uint32_t neg = as_u32(as_ss2(w) >> (ss2)(short)15);
          lds_add(sm, a2 & 0xFFFFu, (neg & 0xFFFFu) + 1u);
          lds_add(sm, a2 >> 16, (neg >> 16) + 1u);
        }
        if constexpr (kMode == 3) {
          Vec<uint16_t>::cvt(buf[k], xf[k]);
          if (partial && !valid) {
#pragma unroll
            for (int j = 0; j < 8; ++j) xf[k][j] = kNegInf;
          }
          cm = max3raw(cm, vec_max<8>(xf[k]), kNegInf);
        }
      }
      if constexpr (capture) {
        bool c;
        if (cap_signed) {
          ss2 mx;
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const uint32_t q = (kMask || partial) ? ((wd[p] & mk[p]) | (0x80008000u & ~mk[p])) : wd[p];
            mx = p ? __builtin_elementwise_max(mx, as_ss2(q)) : as_ss2(q);
          }
          rmax = as_u32(__builtin_elementwise_max(as_ss2(rmax), mx));
          mx = __builtin_elementwise_max(mx, as_ss2(cap_th2));
          c = as_u32(mx) != cap_th2;
        } else {
          us2 mx;
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const uint32_t neg = as_u32(as_ss2(wd[p]) >> (ss2)(short)15);
            uint32_t q = wd[p] ^ (neg | 0x80008000u);
            if (kMask || partial) q &= mk[p];
            mx = p ? __builtin_elementwise_max(mx, as_us2(q)) : as_us2(q);
          }
          rmax = as_u32(__builtin_elementwise_max(as_us2(rmax), mx));
          mx = __builtin_elementwise_max(mx, as_us2(cap_th2));
          c = as_u32(mx) != cap_th2;
        }
        append(c, vi, buf[k], ab);
      }
    }
    if constexpr (kMode == 3 && count) lse_fold_block_max<false, kG, 8>(st, xf, cm);
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  auto run = [&](const u32x4(&buf)[kG], uint32_t sw, uint32_t chunk, auto count_c, auto capture_c)
                 __attribute__((always_inline)) {
    if (ragged && perm(chunk) == nchunks - 1) work(buf, sw, chunk, T_{}, count_c, capture_c);
    else work(buf, sw, chunk, F_{}, count_c, capture_c);
  };

  // ---- 3. pilot: count each wave's first chunk, pick theta from the counts
  if (ca < nchunks) run(qa, swa, ca, T_{}, F_{});
  __syncthreads();
  {
    const int64_t sampled = (int64_t)(nchunks < (uint32_t)kW ? nchunks : (uint32_t)kW) * kChunk * 8;
    const uint64_t sample = (uint64_t)(sampled < V ? sampled : V);
    const uint32_t ks =
        (uint32_t)(((uint64_t)(kPen ? kTargetPen : kTarget) * sample + (uint64_t)V - 1) / (uint64_t)V);
    uint32_t s = 0u;
    if (tid < kOwners) {
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int v = tid * kPer + rot(j);
        s += cnt(sm, 0u, v) + (kPen ? cnt(sm, kR2, v) : 0u);
      }
    }
    const uint32_t incl = wave_scan_u32(s);
    if (lane == kWave - 1) sm.red_u[wid][0] = incl;
    __syncthreads();
    uint32_t ex = incl - s;
#pragma unroll
    for (int i = 0; i < kW; ++i) ex += i < wid ? sm.red_u[i][0] : 0u;
    if (ex < ks && ks <= ex + s) {
      uint32_t run_c = ex;
      int vt = -1;
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        run_c += cnt(sm, 0u, tid * kPer + j) + (kPen ? cnt(sm, kR2, tid * kPer + j) : 0u);
        if (vt < 0 && run_c >= ks) vt = tid * kPer + j;
      }
      sm.theta = vb_bits(vt);
    }
    __syncthreads();
    const uint32_t th = sm.theta;
    if (th != kNone && !(th & 0x8000u)) {
      cap_signed = true;
      th_s = (int)th;
      cap_th2 = (th - 1u) * 0x10001u;
      rmax = 0x80008000u;
    } else {
      th_o = th == kNone ? 1u : ord16(th);
      cap_th2 = (th_o - 1u) * 0x10001u;
      rmax = 0u;
    }
  }
  if (ca < nchunks) run(qa, swa, ca, F_{}, T_{});

  // ---- 4. stream (chunk A of the pilot is done; B is in flight)
  while (true) {
    if (cb >= nchunks) break;
    ca = grab();
    if (ca < nchunks) issue(qa, swa, ca);
    run(qb, swb, cb, T_{}, T_{});
    if (ca >= nchunks) break;
    cb = grab();
    if (cb < nchunks) issue(qb, swb, cb);
    run(qa, swa, ca, T_{}, T_{});
  }
  // tail tokens (V not a multiple of 8): lane 0 of wave 0, one token at a
  // time; the tail is vector nvec (padded with -inf) in the pool
  if (wid == 0 && nvec * 8 < V && lane == 0) {
    float xt[1][8];
    uint32_t wt[4] = {0xFF80FF80u, 0xFF80FF80u, 0xFF80FF80u, 0xFF80FF80u};
    uint32_t abt = 0u, mo = 0u;
    for (int j = 0; j < 8; ++j) {
      const int64_t id = nvec * 8 + j;
      xt[0][j] = kNegInf;
      if (id >= V) continue;
      const uint32_t h = r.x[id];
      xt[0][j] = u2f(h << 16);
      wt[j >> 1] = (j & 1) ? (wt[j >> 1] & 0xFFFFu) | (h << 16) : (wt[j >> 1] & 0xFFFF0000u) | h;
      const bool on = r.allowed(id);
      const bool pn = kPen && ((sm.pen()[id >> 5] >> (id & 31)) & 1u);
      uint32_t wi = pair_words(h) & 0xFFFFu;
      if (kMode == 1 && pn) wi |= kR2;
      if (kMode == 2 && !on) wi |= kR2;
      if (kMode == 3) wi = on ? (wi | (pn ? kR2 : 0u)) : kSpill;
      lds_add(sm, wi, 1u + 0xFFFFu * ((h >> 15) & 1u));
      if (!on) continue;
      const uint32_t key = ord16(h);
      if (cap_signed) {
        const int hv = (int)(short)h;
        const int rv = (int)(short)(rmax & 0xFFFFu);
        if (hv > rv) rmax = (rmax & 0xFFFF0000u) | h;
      } else if (key > (rmax & 0xFFFFu)) {
        rmax = (rmax & 0xFFFF0000u) | key;
      }
      abt |= 1u << j;
      mo = key > mo ? key : mo;
    }
    if (kMode == 3) lse_fold_block_max<false, 1, 8>(st, xt, vec_max<8>(xt[0]));
    if (mo != 0u && mo >= th_o && (!cap_signed || (int)(short)unord16(mo) >= th_s)) {
      const uint32_t o = seg < kSegV ? 0u : atomicAdd(&sm.over_n, 1u);
      if (seg < kSegV || o < kOver) {  // (wave 0's segment, else the overflow area)
        const uint32_t e = seg < kSegV ? seg : kW * kSegV + o;
        sm.qd[e] = u32x4{wt[0], wt[1], wt[2], wt[3]};
        sm.qv[e] = (uint32_t)nvec | (abt << 16);
      } else {
        atomicMax(&sm.drop_ord, mo);
      }
      ++seg;
    }
  }
  if (lane == 0) sm.seg_n[wid] = seg < kSegV ? seg : kSegV;
  __syncthreads();  // the stream is complete

  // ---- 5. maxima, escapes; the row status
  sm.x.own.w[tid] = 0ull;
  sm.x.own.c[tid] = 0u;
  int topA = kNV, topB = kNV;  // penalty: smallest nonempty value bin of region A / P
  uint32_t tot = 0u;           // penalty: tokens in the value bins and the spill words
  uint32_t key = 0u;           // no penalty: ord16 key of the allowed maximum
  if (kPen) {
    if (tid < kOwners) {
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int v = tid * kPer + rot(j);
        const uint32_t c1 = cnt(sm, 0u, v), c2 = cnt(sm, kR2, v);
        if (c1) topA = v < topA ? v : topA;
        if (c2) topB = v < topB ? v : topB;
        tot += c1 + c2;
      }
    } else if (kMode == 3) {
      const int q = tid - kOwners;  // 0..15: the 64 spill words
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t s = sm.hist[kSpill + 4 * q + i];
        tot += (s & 0xFFFFu) + (s >> 16);
      }
    }
  } else if (cap_signed) {
    const int lo = (int)(short)(rmax & 0xFFFFu), hi = (int)(short)(rmax >> 16);
    const int mv = lo > hi ? lo : hi;
    key = mv >= 0 ? ((uint32_t)mv | 0x8000u) : 0u;  // (the maximum is >= theta >= 0)
  } else {
    key = (rmax & 0xFFFFu) > (rmax >> 16) ? (rmax & 0xFFFFu) : (rmax >> 16);
  }
  Lse3 rl{kNegInf, 0.0f, 0.0f};
  if (kMode == 3) rl = block_lse3_dpp<kB>(st, sm.red_f);
  {
    topA = (int)wave_min_u32((uint32_t)topA);  // (bins are >= 0)
    topB = (int)wave_min_u32((uint32_t)topB);
    key = wave_max_u32(key);
    tot = wave_total_u32(tot);
    __syncthreads();
    if (lane == 0) {
      sm.red_u[wid][0] = (uint32_t)topA;
      sm.red_u[wid][1] = (uint32_t)topB;
      sm.red_u[wid][2] = tot;
      sm.red_u[wid][3] = key;
    }
    __syncthreads();
    topA = topB = kNV;
    tot = key = 0u;
#pragma unroll
    for (int i = 0; i < kW; ++i) {
      topA = (int)sm.red_u[i][0] < topA ? (int)sm.red_u[i][0] : topA;
      topB = (int)sm.red_u[i][1] < topB ? (int)sm.red_u[i][1] : topB;
      tot += sm.red_u[i][2];
      key = sm.red_u[i][3] > key ? sm.red_u[i][3] : key;
    }
  }
  // escapes (values above the bins, infinities, NaN) and 16-bit count
  // overflows (the counts then miss tokens) go to the row-wise path
  {
    const uint32_t e1 = sm.hist[kNI], e2 = kMode ? sm.hist[kR2 + kNI] : 0u;
    if ((e1 | e2) != 0u) return false;
  }
  if (kPen && tot != (uint32_t)V) return false;
  if (!kPen && key != 0u) topA = vb_of(unord16(key));
  const float u = sm.u;
  int32_t status = GTP_ROW_OK;
  if (kMode == 3 && (rl.s != rl.s || rl.m == kPosInf)) status = GTP_ROW_NONFINITE;
  else if (sm.flags & 2u) status = GTP_ROW_BAD_HISTORY;
  else if (!(u >= 0.0f && u < 1.0f)) status = GTP_ROW_BAD_UNIFORM;
  if (status != GTP_ROW_OK) {
    if (tid == 0) write_row_f(a, b, sm.fin != 0u, status, -1, 0.f, 0.f, 0, 0.f, -1);
    return true;
  }
  float m = kNegInf;
  if (topA >= 0 && topA < kNV) m = r.ybin(topA);
  if (kPen && topB < kNV) {
    const float yp = r.ypen(topB);
    if (!(yp < kPosInf)) return false;  // the penalty overflowed: hand over
    m = yp > m ? yp : m;
  }
  if (m == kNegInf) {
    if (tid == 0) write_row_f(a, b, sm.fin != 0u, GTP_ROW_EMPTY, -1, 0.f, 0.f, 0, 0.f, -1);
    return true;
  }
  // The zero bins hold zeros and values below 2^-40 as the value 0: exact
  // when every such token weighs what a zero weighs (DETEXP_FIX is monotone:
  // the extremes decide) and the maximum is not among them.
  if (m == 0.0f) return false;
  if ((sm.hist[0] | (kPen ? sm.hist[kR2] : 0u)) != 0u) {
    const float xt = u2f((kBase - 1u) << 16);  // the largest magnitude below the bins
    float hi = r.y_of(xt), lo = r.y_of(-xt);
    if (kPen) {
      const float y3 = r.y_of(r.pen_v(xt)), y4 = r.y_of(r.pen_v(-xt));
      hi = y3 > hi ? y3 : hi;
      lo = y4 < lo ? y4 : lo;
    }
    if (!(hi < m) || detexp_fix(hi - m) != detexp_fix(lo - m)) return false;
  }

  // ---- 6. weights, the penalised values' owners, the block scan
  // The per-value work is spread over all waves: in layer j, lane l of wave w
  // takes value bin 1024 j + 64 w + l and adds its weight and count to
  // own.w / own.c of the thread that owns the bin (v / 16); penalised
  // values add to the thread whose bins hold their y.  Without the per-token
  // fold the raw log-sum-exp comes from the counts: around the known raw
  // maximum without a mask, online with one (the masked maximum is unknown).
  float lm = kNegInf, lsum = 0.0f;
  if (kMode == 0 || kMode == 1) {
    lm = topA < kNV ? vb_x(topA) : kNegInf;
    if (kMode == 1 && topB < kNV) lm = vb_x(topB) > lm ? vb_x(topB) : lm;
  }
  uint32_t n2 = 0u;  // region-2 tokens (no penalty: the masked tokens)
  bool unowned = false;
  auto lse_add = [&](float x, uint32_t c) {
    if (kMode != 2) {
      lsum += (float)c * __builtin_amdgcn_exp2f((x - lm) * kLog2e);
    } else if (x > lm) {
      lsum = lsum * __builtin_amdgcn_exp2f((lm - x) * kLog2e) + (float)c;
      lm = x;
    } else {
      lsum += (float)c * __builtin_amdgcn_exp2f((x - lm) * kLog2e);
    }
  };
  for (int j = 0; j < kPer; ++j) {
    const int v = 1024 * j + kWave * wid + lane;
    const bool in = v < kNV;
    const uint32_t c = in ? cnt(sm, 0u, v) : 0u;
    const uint32_t c2 = (kMode != 0 && in) ? cnt(sm, kR2, v) : 0u;
    if (!__ballot((c | c2) != 0u)) continue;
    unsigned long long wv = 0ull;
    if (c) {
      wv = (unsigned long long)c * detexp_fix(r.ybin(v) - m);
      if (kMode != 3) lse_add(vb_x(v), c);
    }
    if (kMode != 0 && c2) {
      if (kMode != 3) lse_add(vb_x(v), c2);
      if (!kPen) n2 += c2;
      if (kPen) {
        const float y = r.ypen(v);
        const int g = ceil_v(r, y);
        if (g < 0) {
          unowned = true;
        } else {
          atomicAdd(&sm.x.own.w[g / kPer], (unsigned long long)c2 * detexp_fix(y - m));
          atomicAdd(&sm.x.own.c[g / kPer], c2);
        }
      }
    }
    // the 16 lanes of a row of the wave share one owner (v >> 4): their sums
    // (DPP), then one LDS atomic per row instead of 16 on one address
    const unsigned long long rw = row_scan_u64(wv);
    const uint32_t rc = row_scan_u32(c);
    if ((lane & 15) == 15 && rc) {
      atomicAdd(&sm.x.own.w[v >> 4], rw);
      atomicAdd(&sm.x.own.c[v >> 4], rc);
    }
  }
  if (kPen && unowned) atomicOr(&sm.flags, 1u);
  __syncthreads();
  if (kPen && (sm.flags & 1u)) return false;
  const unsigned long long Wt = sm.x.own.w[tid];
  const uint32_t Nt = sm.x.own.c[tid];
  unsigned long long ew, W;
  uint32_t ec, N, N2;
  float lse_m, lse_s;
  weight_scan<kMode>(sm, Wt, Nt, n2, lm, lsum, ew, ec, W, N, N2, lse_m, lse_s);
  // no penalty: every token is in a value bin (the counts add up)
  if (!kPen && N + N2 != (uint32_t)V) return false;
  sm.x.ex.w[tid] = ew;
  sm.x.ex.c[tid] = ec;
  if (tid == 0) {
    sm.x.ex.w[kB] = W;
    sm.x.ex.c[kB] = N;
  }
  if (kMode == 3) {
    lse_m = rl.m;
    lse_s = rl.s;
  }
  const float lse_ln = __builtin_amdgcn_logf(lse_s) * kLn2;
  __syncthreads();

  // ---- 7. the cut and the draw (wave 0)
  if (wid == 0) {
    Level L0, L1;
    const unsigned long long F = floor_mul(a.P, W);
    bool ok = resolve<kMode>(sm, r, m, F, L0);
    if (ok) {
      const unsigned long long Wp = L0.s_before + (unsigned long long)(L0.k + 1u) * L0.w;
      ok = resolve<kMode>(sm, r, m, floor_mul(u, Wp), L1);
    }
    if (lane == 0) {
      sm.lv[0] = L0;
      sm.lv[1] = L1;
      sm.bad = ok ? 0 : 1;
    }
  }
  __syncthreads();
  if (sm.bad) return false;
  const Level L0 = sm.lv[0], L1 = sm.lv[1];
  const uint32_t R = L0.n_before + L0.k + 1u;
  const unsigned long long Wp = L0.s_before + (unsigned long long)(L0.k + 1u) * L0.w;

  // ---- 8. ids: from the pool when it holds both values, else a rescan
  const uint32_t th = sm.theta, drop = sm.drop_ord;
  const uint32_t th_ord = th == kNone ? 0u : ord16(th);
  auto pooled = [&](uint32_t h) { return h == kNone || (ord16(h) >= th_ord && ord16(h) > drop); };
  if (pooled(L0.hu) && pooled(L0.hp) && pooled(L1.hu) && pooled(L1.hp)) {
    const bool big0 = L0.n > (uint32_t)kSmall, big1 = L1.n > (uint32_t)kSmall;
    const int nwords = (int)((V + 31) / 32);
    // level l: a list at hist[l * 8192] (small) or an id bitmap there (big)
    if (big0)
      for (int i = tid; i < nwords; i += kB) sm.hist[i] = 0u;
    if (big1)
      for (int i = tid; i < nwords; i += kB) sm.hist[8192 + i] = 0u;
    if (big0 || big1) __syncthreads();

    auto add = [&](int l, bool big, uint32_t id) {
      uint32_t* base = sm.hist + l * 8192;
      if (big) {
        atomicOr(&base[id >> 5], 1u << (id & 31));
      } else {
        const uint32_t s = atomicAdd(&sm.list_n[l], 1u);
        if (s < (uint32_t)kSmall) base[s] = id;
      }
    };
    // the levels' values in both halves; a vector is looked at token by token
    // only when a half equals one of them (packed compares)
    auto pat = [](uint32_t h) { return h == kNone ? 0xFFFFFFFFu : h * 0x10001u; };
    const uint32_t pu0 = pat(L0.hu), pp0 = pat(L0.hp), pu1 = pat(L1.hu), pp1 = pat(L1.hp);
    auto zeq = [](uint32_t w, uint32_t pt) {
      const uint32_t x = w ^ pt;
      return as_u32(as_us2(x) - (us2)(unsigned short)1) & ~x & 0x80008000u;
    };
    const uint32_t n_over = sm.over_n < kOver ? sm.over_n : kOver;
    for (uint32_t s = tid; s < kCap; s += kB) {
      if (s < kW * kSegV ? s % kSegV >= sm.seg_n[s / kSegV] : s - kW * kSegV >= n_over) continue;
      const u32x4 q = sm.qd[s];
      const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
      uint32_t any = 0u;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        any |= zeq(wd[p], pu0) | zeq(wd[p], pu1);
        if (kPen) any |= zeq(wd[p], pp0) | zeq(wd[p], pp1);
      }
      if (!any) continue;
      const uint32_t vi = sm.qv[s] & 0xFFFFu, ab = sm.qv[s] >> 16;
      for (int j = 0; j < 8; ++j) {
        const uint32_t id = vi * 8u + (uint32_t)j;
        if (!((ab >> j) & 1u) || id >= (uint32_t)V) continue;
        const uint32_t h = (j & 1) ? wd[j >> 1] >> 16 : wd[j >> 1] & 0xFFFFu;
        const bool pn = kPen && ((sm.pen()[id >> 5] >> (id & 31)) & 1u);
        if (in_level(L0, pn, h)) add(0, big0, id);
        if (in_level(L1, pn, h)) add(1, big1, id);
      }
    }
    __syncthreads();
    // small levels: wave l ranks its list
    if (wid < 2) {
      const Level& L = wid ? L1 : L0;
      const bool big = wid ? big1 : big0;
      if (!big) {
        const uint32_t n = sm.list_n[wid];
        const uint32_t* lst = sm.hist + wid * 8192;
        if (n != L.n) {
          if (lane == 0) sm.bad = 1;
        } else {
          // rank of each listed id among the list, in registers
          const uint32_t my = (uint32_t)lane < n ? lst[lane] : 0xFFFFFFFFu;
          uint32_t rank = 0u;
#pragma unroll
          for (int j = 0; j < kWave; ++j)
            rank += (uint32_t)__builtin_amdgcn_readlane((int)my, j) < my ? 1u : 0u;
          if ((uint32_t)lane < n && rank == L.k) sm.id_out[wid] = (int32_t)my;
        }
      }
    }
    // big levels: popcounts of the bitmap words, one block scan
    if (big0 || big1) {
      uint32_t w0[8], w1[8], p0 = 0u, p1 = 0u;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int wi = 8 * tid + i;
        w0[i] = big0 && wi < nwords ? sm.hist[wi] : 0u;
        w1[i] = big1 && wi < nwords ? sm.hist[8192 + wi] : 0u;
        p0 += __builtin_popcount(w0[i]);
        p1 += __builtin_popcount(w1[i]);
      }
      unsigned long long e0, t0;
      uint32_t e1, t1;
      float f0;
      block_scan2(sm, p0, p1, 0.0f, e0, e1, t0, t1, f0);
      if ((big0 && t0 != L0.n) || (big1 && t1 != L1.n)) return false;
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
      if (big0 && e0 <= L0.k && L0.k < e0 + p0) sm.id_out[0] = find(w0, (uint32_t)(L0.k - e0));
      if (big1 && e1 <= L1.k && L1.k < e1 + p1) sm.id_out[1] = find(w1, L1.k - e1);
    }
    __syncthreads();
    if (sm.bad) return false;
  } else {
    rescan_ids<kMode>(sm, r, 0, nvec, true, 0, 0, false, L0.k, L1.k, false);
  }

  // ---- 9. outputs (both ids found, or the row goes to the row-wise path)
  if (sm.id_out[0] < 0 || sm.id_out[1] < 0) return false;
  if (tid == 0) {
    const int32_t id_thr = sm.id_out[0], id_draw = sm.id_out[1];
    const bool dp = kPen && ((sm.pen()[id_draw >> 5] >> (id_draw & 31)) & 1u);
    const uint32_t hd = dp ? L1.hp : L1.hu;
    const float x_draw = u2f(hd << 16);
    const float slp = __builtin_amdgcn_logf((float)((double)L1.w / (double)Wp)) * kLn2;
    write_row_f(a, b, sm.fin != 0u, GTP_ROW_OK, id_draw, raw_logprob(x_draw, lse_m, lse_ln), slp, (int32_t)R,
              L0.y, id_thr);
  }
  return true;
}

}  // namespace topp

// One row per workgroup.  A row outside the top-p path's bounds (topp_row
// returns false, the same in every thread, before any output is written)
// runs the row-wise path in the same workgroup, in the same LDS: a top-p
// call is one launch.  The row-wise path raises the kernel to 128 VGPRs and
// 240 bytes of scratch per lane (its own spills), which costs less than a
// second launch did.
// kMode bit 0: repetition penalty active; bit 1: allow mask.
template <int kMode>
__global__ __launch_bounds__(topp::kB) void sampler_topp_kernel(SamplerArgs a) {
  __shared__ union {
    topp::Smem t;
    SamplerSmem g;
  } smu;
  const int64_t b = blockIdx.x;
  if (!topp::topp_row<kMode>(a, b, smu.t)) {
    __syncthreads();  // every thread is done with the top-p state
    rowwise_row<uint16_t>(a, b, smu.g);
  }
}

}  // namespace gtp
