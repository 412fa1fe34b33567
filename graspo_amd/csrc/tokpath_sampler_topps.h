// tokpath_sampler_topps.h -- the top-p sampler for bf16 rows split over
// several workgroups per row (gfx950).
//
// Serves what sampler_topp_kernel serves (sampling rows with top-p active
// and no top-k, 16-byte aligned bf16 rows of 65536 <= V <= 2^18,
// 0 < T <= 1024: the decode step of the reference's
// _next_token_from_logits(logits, temperature, top_p),
// src/graspo/backends/graspoflow/tensor_utils.py:649-683) when the batch is
// small: with one workgroup per row a batch of 64 rows keeps 64 CUs busy and
// each row streams at one CU's bandwidth.  Here slice s of S contiguous
// slices of a row goes to workgroup (s, b); the answer is the same bit for
// bit.
//
// 1. Count.  Each workgroup counts its slice's tokens into the value bins
//    the one-workgroup kernel uses (region A: allowed unpenalised tokens;
//    region 2: allowed penalised tokens, or the masked ones without a
//    penalty; the spill words and a per-token raw log-sum-exp with both a
//    mask and a penalty), then stores the nonempty word range of each region
//    (and the spill words) in its workspace slot and a small header.
// 2. Merge.  The last workgroup of the row to arrive at the row's counter
//    adds the other slots' ranges to its own bins: they then hold the whole
//    row's counts, and the maximum, the weights, the cut and the draw are the
//    one-workgroup kernel's steps on them.
// 3. Ids.  The slots' counts of the cut's and the draw's values say which
//    slice holds each wanted token and its rank among the value's tokens
//    there; one more read of that slice (or of both) finds them.
// A row outside the bounds runs the row-wise path in its last workgroup, as
// in the one-workgroup kernel.
#pragma once

// The publication of slice counts below relies on gfx950's code generation
// (see the arrival step of topps_row).
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "tokpath_sampler_topps.h: the split top-p publication protocol is written for gfx950"
#endif

namespace gtp {
namespace topps {

using namespace topp;

constexpr int kMaxS = 8;            // slices per row
// per slice: ranges A and 2, the raw (m, s, t), the largest value's bin in
// regions A and 2, the tokens counted, the escapes
constexpr int kHdrWords = 16;
constexpr int kSlotWords = kHistWords;  // a slot mirrors the bins' word layout

// Workspace of a split call: the zero region (the per-row arrival counters
// at word kToppSplitCtrWord), the headers, the slots.
__device__ __forceinline__ uint32_t* split_headers(unsigned char* ws) {
  return reinterpret_cast<uint32_t*>(ws + kWsZeroBytes);
}
__device__ __forceinline__ uint32_t* split_slots(unsigned char* ws, int64_t B, int S) {
  const size_t hb = (((size_t)B * S * kHdrWords * 4) + 255) / 256 * 256;
  return reinterpret_cast<uint32_t*>(ws + kWsZeroBytes + hb);
}

struct Extra {
  uint32_t hd[kMaxS][kHdrWords];  // the row's slice headers (last workgroup)
  uint32_t last;                  // this workgroup is the row's last to arrive
  int32_t sl[2];                  // slice of each wanted token
  uint32_t jl[2];                 // its rank among its value's tokens there
  uint32_t pub[8];                // the slice's ranges, largest-value bins, tokens, escapes
};

// One workgroup's part of row b: slice s of S (vectors [s vps, (s+1) vps)).
// False: the row must be handed over (only the row's last workgroup decides;
// a block-uniform decision taken before any output of the row is written).
template <int kMode>
__device__ __forceinline__ bool topps_row(const SamplerArgs& a, int64_t b, int s, int S, int64_t vps,
                                          int64_t B, unsigned char* ws, topp::Smem& sm, Extra& ex) {
  constexpr bool kPen = (kMode & 1) != 0, kMask = (kMode & 2) != 0;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  topp::Row r;
  r.x = reinterpret_cast<const uint16_t*>(a.logits) + b * a.row_stride;
  r.mask = kMask ? a.mask + b * a.mask_stride : nullptr;
  r.V = a.V;
  r.nvec = a.V / 8;
  r.rho = a.rho;
  r.Tc = a.T > 1e-6f ? a.T : 1e-6f;
  const int64_t V = a.V, nvec = r.nvec;
  const int64_t s0 = (int64_t)s * vps;
  const int64_t s1 = s0 + vps < nvec ? s0 + vps : nvec;
  const uint32_t nch = (uint32_t)((s1 - s0 + kChunk - 1) / kChunk);
  const bool ragged = ((s1 - s0) % kChunk) != 0;  // the slice's last chunk is partial

  // ---- 0. the first two chunks of each wave in flight, then the clear
  const uint32_t last_word = (uint32_t)((V - 1) >> 5);
  const uint32_t s0u = (uint32_t)s0, s1u = (uint32_t)s1;  // (nvec < 2^15)
  auto issue = [&](u32x4(&buf)[kG], uint32_t& sw, uint32_t chunk) {
    const uint32_t base = s0u + chunk * (uint32_t)kChunk;
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      uint32_t vi = base + (uint32_t)(k * kWave + lane);
      vi = vi < s1u ? vi : s1u - 1u;
      buf[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(r.x) + vi);
    }
    if (kMask) {  // the chunk's 64 mask words, one per lane
      const uint32_t w = base / 4u + (uint32_t)lane;
      sw = r.mask[w < last_word ? w : last_word];
    }
  };
  u32x4 qa[kG], qb[kG];
  uint32_t swa = 0xFFFFFFFFu, swb = 0xFFFFFFFFu;
  uint32_t ca = (uint32_t)wid, cb = (uint32_t)(kW + wid);
  if (ca < nch) issue(qa, swa, ca);
  if (cb < nch) issue(qb, swb, cb);
  {
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int i = tid; i < kHistWords / 4; i += kB) reinterpret_cast<u32x4*>(sm.hist)[i] = z;
    if (kPen)
      for (int64_t i = tid; i < (V + 127) / 128; i += kB) reinterpret_cast<u32x4*>(sm.pen())[i] = z;
  }
  if (tid == 0) {
    sm.u = a.uniforms[b];
    sm.fin = a.finished && a.finished[b];
    sm.chunk_ctr = 2u * kW;
    sm.flags = 0u;
    sm.bad = 0;
    sm.id_out[0] = -1;
    sm.id_out[1] = -1;
  }
  __syncthreads();

  // ---- 1. the history bitmap (the whole row's: the ids step may read any
  // slice)
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
  __syncthreads();

  auto allow_byte = [&](uint32_t sw, int k) -> uint32_t {
    const uint32_t w = (uint32_t)__shfl((int)sw, k * (kWave / 4) + lane / 4, kWave);
    return (w >> ((lane & 3) * 8)) & 0xFFu;
  };
  auto grab = [&]() -> uint32_t {
    uint32_t c = 0;
    if (lane == 0) c = atomicAdd(&sm.chunk_ctr, 1u);
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)c);
  };

  // ---- 2. count the slice
  Lse3 st{kNegInf, 0.0f, 0.0f};  // raw log-sum-exp per token (mask and penalty)
  const uint32_t junk2 = kJunk * 0x10001u;
  const uint32_t spill2 = (kSpill + (uint32_t)lane) * 0x10001u;
  const uint32_t lastv = (uint32_t)(nvec - 1);
  auto work = [&](const u32x4(&buf)[kG], uint32_t sw, uint32_t chunk, auto partial_c)
                  __attribute__((always_inline)) {
    constexpr bool partial = decltype(partial_c)::value;
    const uint32_t base = s0u + chunk * (uint32_t)kChunk;
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      const uint32_t vi = base + (uint32_t)(k * kWave + lane);
      const bool valid = !partial || vi < s1u;
      uint32_t ab = kMask ? allow_byte(sw, k) : 0xFFu;
      if (partial && !valid) ab = 0u;
      const uint32_t pb =
          kPen ? (sm.pen()[(vi < lastv ? vi : lastv) >> 2] >> ((vi & 3) * 8)) & 0xFFu : 0u;
      const uint32_t wd[4] = {buf[k].x, buf[k].y, buf[k].z, buf[k].w};
      uint32_t mk[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) mk[p] = (kMask || partial) ? spread(ab, p) : 0xFFFFFFFFu;
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
        const uint32_t neg = as_u32(as_ss2(w) >> (ss2)(short)15);
        lds_add(sm, a2 & 0xFFFFu, (neg & 0xFFFFu) + 1u);
        lds_add(sm, a2 >> 16, (neg >> 16) + 1u);
      }
      if constexpr (kMode == 3) {  // (one vector at a time: 8 live floats, no spills)
        float xk[1][8];
        Vec<uint16_t>::cvt(buf[k], xk[0]);
        if (partial && !valid) {
#pragma unroll
          for (int j = 0; j < 8; ++j) xk[0][j] = kNegInf;
        }
        lse_fold_block_max<false, 1, 8>(st, xk, vec_max<8>(xk[0]));
      }
    }
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  auto run = [&](const u32x4(&buf)[kG], uint32_t sw, uint32_t chunk) __attribute__((always_inline)) {
    if (ragged && chunk == nch - 1) work(buf, sw, chunk, T_{});
    else work(buf, sw, chunk, F_{});
  };
  if (ca < nch) run(qa, swa, ca);
  while (true) {
    if (cb >= nch) break;
    ca = grab();
    if (ca < nch) issue(qa, swa, ca);
    run(qb, swb, cb);
    if (ca >= nch) break;
    cb = grab();
    if (cb < nch) issue(qb, swb, cb);
    run(qa, swa, ca);
  }
  // tail tokens (V not a multiple of 8): the last slice, lane 0 of wave 0
  if (s == S - 1 && wid == 0 && lane == 0 && nvec * 8 < V) {
    float xt[1][8];
    for (int j = 0; j < 8; ++j) {
      const int64_t id = nvec * 8 + j;
      xt[0][j] = kNegInf;
      if (id >= V) continue;
      const uint32_t h = r.x[id];
      xt[0][j] = u2f(h << 16);
      const bool on = r.allowed(id);
      const bool pn = kPen && ((sm.pen()[id >> 5] >> (id & 31)) & 1u);
      uint32_t wi = pair_words(h) & 0xFFFFu;
      if (kMode == 1 && pn) wi |= kR2;
      if (kMode == 2 && !on) wi |= kR2;
      if (kMode == 3) wi = on ? (wi | (pn ? kR2 : 0u)) : kSpill;
      lds_add(sm, wi, 1u + 0xFFFFu * ((h >> 15) & 1u));
    }
    if (kMode == 3) lse_fold_block_max<false, 1, 8>(st, xt, vec_max<8>(xt[0]));
  }
  Lse3 rl{kNegInf, 0.0f, 0.0f};
  if (kMode == 3) rl = block_lse3_dpp<kB>(st, sm.red_f);  // (its barrier ends the stream)
  else __syncthreads();

  // ---- 3. publish: the nonempty word range of each region (words 0..kNI
  // of region A, kR2..kR2 + kNI of region 2: the bins and the escape word),
  // rounded out to 16-byte units, the spill words, and in the header the
  // largest value's bin of each region, the tokens counted and the escapes.
  // Slot and header go out as agent-scope atomic stores, which write through
  // L2 (no L2 write-back is needed to publish them).
  {
    uint32_t* hdr = split_headers(ws) + ((size_t)b * S + s) * kHdrWords;
    uint32_t* slot = split_slots(ws, B, S) + ((size_t)b * S + s) * kSlotWords;
    // thread t looks at words 16t..16t+15: waves 0-7 region A, 8-15 region 2
    const uint32_t w0 = 16u * (uint32_t)tid;
    const uint32_t rbase = w0 < kR2 ? 0u : kR2;
    uint32_t lo = 0xFFFFFFFFu, hi = 0u, tot = 0u, esc = 0u;
    int pmax = -1, nmin = (int)kNI;  // largest word with a positive count, smallest with a negative one
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 v = reinterpret_cast<const u32x4*>(sm.hist)[4 * tid + q];
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = w0 + 4u * q + e, i = w - rbase;
        if (wv[e] != 0u && i <= kNI) {
          lo = w < lo ? w : lo;
          hi = w + 1u;
        }
        if (i < kNI) {
          tot += (wv[e] & 0xFFFFu) + (wv[e] >> 16);
          if (wv[e] & 0xFFFFu) pmax = (int)i;
          if ((wv[e] >> 16) && nmin == (int)kNI) nmin = (int)i;
        } else if (i == kNI) {
          esc |= wv[e];
        } else if (kMode == 3 && w >= kSpill) {
          tot += (wv[e] & 0xFFFFu) + (wv[e] >> 16);
        }
      }
    }
    lo = wave_min_u32(lo);
    hi = wave_max_u32(hi);
    pmax = (int)wave_max_u32((uint32_t)(pmax + 1)) - 1;  // (pmax >= -1)
    nmin = (int)wave_min_u32((uint32_t)nmin);            // (nmin >= 0)
    tot = wave_total_u32(tot);
    esc = __ballot(esc != 0u) ? 1u : 0u;
    __syncthreads();  // (red_u is free)
    if (lane == 0) {
      sm.red_u[wid][0] = lo;
      sm.red_u[wid][1] = hi;
      sm.red_u[wid][2] = tot;
      sm.red_u[wid][3] = (uint32_t)(pmax + 1) | ((uint32_t)nmin << 14) | (esc << 28);
    }
    __syncthreads();
    // wave 0 combines the 16 waves' partials (lanes 0-7 region A, 8-15
    // region 2) and hands the slice's summary to every thread
    if (wid == 0) {
      const bool in = lane < kW;
      uint32_t rlo = in ? sm.red_u[lane][0] : 0xFFFFFFFFu, rhi = in ? sm.red_u[lane][1] : 0u;
      uint32_t nt = in ? sm.red_u[lane][2] : 0u;
      const uint32_t pk = in ? sm.red_u[lane][3] : (kNI << 14);
      int pm = (int)(pk & 0x3FFFu) - 1, nm = (int)((pk >> 14) & 0x3FFFu);
      uint32_t es = pk >> 28;
      // within aligned groups of 8 lanes (DPP)
      auto step = [&](auto xr) __attribute__((always_inline)) {
        const uint32_t ol = xr(rlo), oh = xr(rhi);
        const int op = (int)xr((uint32_t)pm), on = (int)xr((uint32_t)nm);
        nt += xr(nt);
        es |= xr(es);
        rlo = ol < rlo ? ol : rlo;
        rhi = oh > rhi ? oh : rhi;
        pm = op > pm ? op : pm;
        nm = on < nm ? on : nm;
      };
      static_assert(kW / 2 == 8, "groups of 8 lanes");
      step([](uint32_t v) { return lane_xor<1>(v); });
      step([](uint32_t v) { return lane_xor<2>(v); });
      step([](uint32_t v) { return lane_xor<4>(v); });
      const uint32_t nt_all = (uint32_t)__builtin_amdgcn_readlane((int)nt, 0) +
                              (uint32_t)__builtin_amdgcn_readlane((int)nt, kW / 2);
      const uint32_t es_all = (uint32_t)__builtin_amdgcn_readlane((int)es, 0) |
                              (uint32_t)__builtin_amdgcn_readlane((int)es, kW / 2);
      if (lane == 0 || lane == kW / 2) {
        const int g = lane / (kW / 2);
        // smallest value bin: the largest positive value, else the negative
        // value nearest zero (bin v = kNI - 1 - i for the positive half of word
        // i, kNI + i for the negative half); an empty region: lo = hi = 0
        ex.pub[3 * g + 0] = rhi ? rlo & ~3u : 0u;
        ex.pub[3 * g + 1] = (rhi + 3u) & ~3u;
        ex.pub[3 * g + 2] =
            pm >= 0 ? kNI - 1u - (uint32_t)pm : (nm < (int)kNI ? kNI + (uint32_t)nm : (uint32_t)kNV);
      }
      if (lane == 0) {
        ex.pub[6] = nt_all;
        ex.pub[7] = es_all;
      }
    }
    __syncthreads();
    const uint32_t rg[2][2] = {{ex.pub[0], ex.pub[1]}, {ex.pub[3], ex.pub[4]}};
    const uint32_t top[2] = {ex.pub[2], ex.pub[5]}, ntok = ex.pub[6], nesc = ex.pub[7];
    auto put = [&](uint32_t q) {  // u32x4 q of the bins to the slot, written through
      const u32x4 v = reinterpret_cast<const u32x4*>(sm.hist)[q];
      unsigned long long* d = reinterpret_cast<unsigned long long*>(slot) + 2 * q;
      __hip_atomic_store(d, (unsigned long long)v.x | ((unsigned long long)v.y << 32), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(d + 1, (unsigned long long)v.z | ((unsigned long long)v.w << 32), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    };
    for (uint32_t q = rg[0][0] / 4 + tid; q < rg[0][1] / 4; q += kB) put(q);
    for (uint32_t q = rg[1][0] / 4 + tid; q < rg[1][1] / 4; q += kB) put(q);
    if (kMode == 3 && tid < 16) put(kSpill / 4 + tid);
    if (tid < kHdrWords) {
      const uint32_t hv[kHdrWords] = {rg[0][0], rg[0][1], rg[1][0], rg[1][1], f2u(rl.m), f2u(rl.s), f2u(rl.t),
                                      top[0], top[1], ntok, nesc, 0u, 0u, 0u, 0u, 0u};
      uint32_t v = hv[0];
#pragma unroll
      for (int i = 1; i < kHdrWords; ++i) v = tid == i ? hv[i] : v;
      __hip_atomic_store(hdr + tid, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // ---- 4. arrival.  Each wave waits until its written-through stores have
  // completed, the barrier joins the waves, and one relaxed agent-scope
  // increment of the row's counter announces the slice; the last workgroup
  // to arrive has seen every increment, and its acquire fence (an L1 and L2
  // invalidate) makes the other slots visible to its waves.
  //
  // This publication has no release operation, so the HIP/LLVM memory model
  // alone gives it no happens-before edge: it rests on gfx950's code
  // generation, where agent-scope stores write through to L2 and vmcnt(0)
  // waits for their completion, and on nothing being moved past the
  // barrier.  A release fence here would add an L2 write-back (buffer_wbl2)
  // per workgroup, 8-10 us per arrival with 32 workgroups per XCD.  The file
  // refuses to build for any other target (below), and the reader's loads
  // are relaxed agent-scope atomics of the same 64-bit words the writers
  // store.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stores are complete
  __syncthreads();
  if (tid == 0) {
    uint32_t* cnt = reinterpret_cast<uint32_t*>(ws) + kToppSplitCtrWord + b;
    const bool last = atomicAdd(cnt, 1u) + 1u == (uint32_t)S;
    if (last) {
      // every workgroup of the row has arrived: nothing else touches the
      // counter in this launch, so it goes back to zero for the next call
      __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    ex.last = last ? 1u : 0u;
  }
  __syncthreads();
  if (!ex.last) return true;

  // ---- 5. merge the other slices' counts into the bins
  const uint32_t* hrow = split_headers(ws) + (size_t)b * S * kHdrWords;
  const uint32_t* srow = split_slots(ws, B, S) + (size_t)b * S * kSlotWords;
  if (tid < S * kHdrWords)
    (&ex.hd[0][0])[tid] = __hip_atomic_load(hrow + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  {
    uint32_t uA = 0xFFFFFFFFu, vA = 0u, u2 = 0xFFFFFFFFu, v2 = 0u;  // the union of the ranges
    for (int j = 0; j < S; ++j) {
      if (j == s) continue;
      if (ex.hd[j][1] > ex.hd[j][0]) {
        uA = ex.hd[j][0] < uA ? ex.hd[j][0] : uA;
        vA = ex.hd[j][1] > vA ? ex.hd[j][1] : vA;
      }
      if (ex.hd[j][3] > ex.hd[j][2]) {
        u2 = ex.hd[j][2] < u2 ? ex.hd[j][2] : u2;
        v2 = ex.hd[j][3] > v2 ? ex.hd[j][3] : v2;
      }
    }
    // the merged counts are 16-bit halves too: a half whose sum passes 0xFFFF
    // (more than 65535 tokens of one value in the row) hands the row over
    bool over = false;
    auto merge = [&](uint32_t ulo, uint32_t uhi, int rw) {
      for (uint32_t q = ulo / 4 + tid; q < uhi / 4; q += kB) {
        const u32x4 own = reinterpret_cast<const u32x4*>(sm.hist)[q];
        u32x4 lo4 = own & 0xFFFFu, hi4 = own >> 16;
#pragma unroll
        for (int j = 0; j < kMaxS; ++j) {
          if (j < S && j != s && 4u * q >= ex.hd[j][rw] && 4u * q < ex.hd[j][rw + 1]) {
            // the two 64-bit words the slice's writer stored
            const unsigned long long* d =
                reinterpret_cast<const unsigned long long*>(srow + (size_t)j * kSlotWords) + 2 * q;
            const unsigned long long w0 = __hip_atomic_load(d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned long long w1 = __hip_atomic_load(d + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const u32x4 v = {(uint32_t)w0, (uint32_t)(w0 >> 32), (uint32_t)w1, (uint32_t)(w1 >> 32)};
            lo4 += v & 0xFFFFu;
            hi4 += v >> 16;
          }
        }
        const u32x4 hi_or = (lo4 | hi4) >> 16;
        over |= (hi_or.x | hi_or.y | hi_or.z | hi_or.w) != 0u;
        reinterpret_cast<u32x4*>(sm.hist)[q] = lo4 | (hi4 << 16);
      }
    };
    if (vA > 0u) merge(uA, vA, 0);
    if (v2 > 0u) merge(u2, v2, 2);
    if (over) atomicOr(&sm.flags, 1u);
    // (the spill words only count masked tokens: their halves stay far below
    // 0xFFFF)
    if (kMode == 3) {
      rl = Lse3{u2f(ex.hd[0][4]), u2f(ex.hd[0][5]), u2f(ex.hd[0][6])};
      for (int j = 1; j < S; ++j) rl = lse3_merge(rl, Lse3{u2f(ex.hd[j][4]), u2f(ex.hd[j][5]), u2f(ex.hd[j][6])});
    }
  }
  __syncthreads();

  // ---- 6. maxima, escapes, the token count (from the headers); the row
  // status
  sm.x.own.w[tid] = 0ull;
  sm.x.own.c[tid] = 0u;
  int topA = kNV, topB = kNV;  // smallest nonempty value bin of region A / of the penalised values
  uint32_t tot = 0u, esc = 0u;
  for (int j = 0; j < S; ++j) {
    topA = (int)ex.hd[j][7] < topA ? (int)ex.hd[j][7] : topA;
    topB = (int)ex.hd[j][8] < topB ? (int)ex.hd[j][8] : topB;
    tot += ex.hd[j][9];
    esc |= ex.hd[j][10];
  }
  if (!kPen) topB = kNV;
  // escapes (values above the bins, infinities, NaN) and 16-bit count
  // overflows (within a slice the counts then miss tokens) go to the
  // row-wise path
  if (esc || tot != (uint32_t)V || (sm.flags & 1u)) return false;
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
  // the zero bins hold zeros and values below 2^-40 as the value 0: exact
  // when every such token weighs what a zero weighs and the maximum is not
  // among them
  if (m == 0.0f) return false;
  if ((sm.hist[0] | (kPen ? sm.hist[kR2] : 0u)) != 0u) {
    const float xt = u2f((kBase - 1u) << 16);
    float hi = r.y_of(xt), lo = r.y_of(-xt);
    if (kPen) {
      const float y3 = r.y_of(r.pen_v(xt)), y4 = r.y_of(r.pen_v(-xt));
      hi = y3 > hi ? y3 : hi;
      lo = y4 < lo ? y4 : lo;
    }
    if (!(hi < m) || detexp_fix(hi - m) != detexp_fix(lo - m)) return false;
  }

  // ---- 7. weights, the penalised values' owners, the block scan (the
  // one-workgroup kernel's step on the merged bins)
  float lm = kNegInf, lsum = 0.0f;
  if (kMode == 0 || kMode == 1) {
    lm = topA < kNV ? vb_x(topA) : kNegInf;
    if (kMode == 1 && topB < kNV) lm = vb_x(topB) > lm ? vb_x(topB) : lm;
  }
  uint32_t n2 = 0u;
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
#pragma unroll 2
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
    const unsigned long long rw = row_scan_u64(wv);
    const uint32_t rc = row_scan_u32(c);
    if ((lane & 15) == 15 && rc) {
      atomicAdd(&sm.x.own.w[v >> 4], rw);
      atomicAdd(&sm.x.own.c[v >> 4], rc);
    }
  }
  if (kPen && unowned) atomicOr(&sm.flags, 4u);
  __syncthreads();
  if (kPen && (sm.flags & 4u)) return false;
  const unsigned long long Wt = sm.x.own.w[tid];
  const uint32_t Nt = sm.x.own.c[tid];
  unsigned long long exw, W;
  uint32_t exc, N, N2;
  float lse_m, lse_s;
  weight_scan<kMode>(sm, Wt, Nt, n2, lm, lsum, exw, exc, W, N, N2, lse_m, lse_s);
  if (!kPen && N + N2 != (uint32_t)V) return false;
  sm.x.ex.w[tid] = exw;
  sm.x.ex.c[tid] = exc;
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

  // ---- 8. the cut and the draw (wave 0), then the slice of each wanted
  // token from the slots' counts of its value
  if (wid == 0) {
    Level L0, L1;
    const unsigned long long F = floor_mul(a.P, W);
    bool ok = resolve<kMode>(sm, r, m, F, L0);
    if (ok) {
      const unsigned long long Wp = L0.s_before + (unsigned long long)(L0.k + 1u) * L0.w;
      ok = resolve<kMode>(sm, r, m, floor_mul(u, Wp), L1);
    }
    // lane j < S: slot j's tokens of each level (its unpenalised value in
    // region A, its penalised value in region 2)
    auto count_in = [&](int j, uint32_t h, uint32_t region, int rw) -> uint32_t {
      if (h == kNone) return 0u;
      const int v = vb_of(h);
      if (v < 0) return 0u;
      const uint32_t w = region + vb_word(v);
      if (w < ex.hd[j][rw] || w >= ex.hd[j][rw + 1]) return 0u;
      const unsigned long long d = __hip_atomic_load(
          reinterpret_cast<const unsigned long long*>(srow + (size_t)j * kSlotWords) + (w >> 1),
          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return ((uint32_t)(d >> (32 * (w & 1))) >> vb_shift(v)) & 0xFFFFu;
    };
    uint32_t c0 = 0u, c1 = 0u;
    if (ok && lane < S) {
      c0 = count_in(lane, L0.hu, 0u, 0) + (kPen ? count_in(lane, L0.hp, kR2, 2) : 0u);
      c1 = count_in(lane, L1.hu, 0u, 0) + (kPen ? count_in(lane, L1.hp, kR2, 2) : 0u);
    }
    const uint32_t i0 = wave_scan_u32(c0), i1 = wave_scan_u32(c1);
    if (ok && (lane63_u32(i0) != L0.n || lane63_u32(i1) != L1.n)) ok = false;
    if (ok) {
      const bool h0 = lane < S && i0 - c0 <= L0.k && L0.k < i0;
      const bool h1 = lane < S && i1 - c1 <= L1.k && L1.k < i1;
      if (!__ballot(h0) || !__ballot(h1)) ok = false;  // (the totals make each exactly one lane)
      if (h0) {
        ex.sl[0] = lane;
        ex.jl[0] = L0.k - (i0 - c0);
      }
      if (h1) {
        ex.sl[1] = lane;
        ex.jl[1] = L1.k - (i1 - c1);
      }
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

  // ---- 9. ids: one read of each slice that holds a wanted token
  {
    const int sa = ex.sl[0], sb = ex.sl[1];
    auto lo_of = [&](int j) -> int64_t { return (int64_t)j * vps; };
    auto hi_of = [&](int j) -> int64_t { return (int64_t)j * vps + vps < nvec ? (int64_t)j * vps + vps : nvec; };
    // one slice: all 16 waves on it; two: eight waves on each, at once
    rescan_ids<kMode>(sm, r, lo_of(sa), hi_of(sa), sa == S - 1, lo_of(sb), hi_of(sb), sb == S - 1, ex.jl[0],
                      ex.jl[1], sa != sb);
  }

  // ---- 10. outputs (both ids found, or the row goes to the row-wise path)
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

}  // namespace topps

// Workgroup (s, b) takes slice s of row b; the row's last workgroup to
// arrive finishes it.  A row outside the top-p path's bounds (only the last
// workgroup decides, the same in all its threads, before any output is
// written) runs the row-wise path in that workgroup and LDS, so the call is
// one launch.
// kMode bit 0: repetition penalty active; bit 1: allow mask.
template <int kMode>
__global__ __launch_bounds__(topp::kB) void sampler_topps_kernel(SamplerArgs a, unsigned char* __restrict__ ws,
                                                                 int64_t vps) {
  __shared__ union {
    struct {
      topp::Smem sm;
      topps::Extra ex;
    } t;
    SamplerSmem g;
  } smu;
  const int64_t b = blockIdx.y;
  if (!topps::topps_row<kMode>(a, b, (int)blockIdx.x, (int)gridDim.x, vps, (int64_t)gridDim.y, ws, smu.t.sm,
                               smu.t.ex)) {
    __syncthreads();  // every thread is done with the top-p state
    rowwise_row<uint16_t>(a, b, smu.g);
  }
}

}  // namespace gtp
