// tokpath_lmhead.hip -- the lm_head GEMM with the log-sum-exp in its epilogue (gfx950).
//
// logprob[n] = h_n . w_{t_n} - logsumexp_v(h_n . w_v) over bf16 hidden states
// h [N, K] and the bf16 lm_head weight w [V, K], without writing the [N, V]
// logits: each workgroup multiplies a 256-vocabulary x 256-token tile on the
// matrix cores (v_mfma_f32_32x32x16_bf16, fp32 accumulation, so every bf16
// product is exact and only the summation order differs from an fp32 GEMM)
// and folds the tile into a per-token (m, s, t) state in registers before
// the next tile.  Replaces the chunked F.linear + logsumexp + logaddexp loop
// of _selected_token_log_probs_from_hidden
// (src/graspo/backends/graspoflow/tensor_utils.py:167-186).
//
// Tile loop.  4 waves, 2 x 2 over the tile, each wave 128 x 128 (4 x 4 MFMA
// blocks of 32 x 32, 256 fp32 accumulators per lane).  K advances 64 at a
// time through two LDS stages of 32 KB per operand; the stage for step i+1
// is loaded straight from global memory into LDS (buffer_load_dwordx4 ...
// lds, no registers) while the matrix cores work on step i.  Each 128-byte
// LDS row holds its eight 16-byte chunks XOR-swizzled by bits 1-3 of the
// row index: an MFMA operand read takes one chunk from each of 16
// consecutive rows per 16 lanes, and (row & 1, chunk) then covers all 16
// 16-byte bank groups of the 64 banks once.
//
// The GEMM computes logits transposed, vocabulary x tokens: lane l of a
// 32 x 32 block holds token (l mod 32) and 16 vocabulary rows, so a token's
// 64 values per wave fold in registers and only the two lane halves and the
// vocabulary tiles merge afterwards.
//
// Order of work.  The workgroup for (vocabulary group g, token tile j) runs
// kTilesPerGroup vocabulary tiles in a row (its K loop runs on across the
// tile boundary), merging each tile into its running state, and writes one
// partial state per (g, wave half, token).  Workgroup b = g * n_tt + j runs
// on XCD b mod 8, so with 32 token tiles the 32 workgroups that share an
// XCD's L2 at a time cover 8 vocabulary groups x 4 token tiles: 12 operand
// tiles per K step come into that L2 (the fewest for 32 workgroups; a whole
// vocabulary group per XCD would bring in 33), and the window of 8 groups
// is read from HBM once (the hidden states stay in the last-level cache).
// A merge kernel folds the partials and the target logits (one fp32 dot
// product per token, the reference's own selected_logits) into logprob,
// entropy and lse.
#include "tokpath_stream.h"

namespace gtp {
namespace lmh {

constexpr int kBV = 256;                 // vocabulary rows per tile
constexpr int kBT = 256;                 // tokens per tile
constexpr int kBK = 64;                  // K per stage: 128 bytes of bf16 per row
// 2 x 2 waves of 128 x 128 (2 x 4 waves of 128 x 64, two per SIMD, measured
// the same: 13.33 against 13.26 ms)
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kWTn = kWaves / 2;          // waves along the tokens (2 along the vocabulary)
constexpr int kXB = 4;                    // 32-row vocabulary blocks per wave
constexpr int kYB = 256 / 32 / kWTn;      // 32-token blocks per wave
constexpr int kQ = 32 / kWaves;           // 1 KB loads per wave per operand and K step
constexpr int kChunks = kBK / 8;         // 16-byte chunks per tile row
constexpr int kStage = kBV * kChunks;    // 16-byte chunks per operand stage (32 KB)
constexpr int kTilesPerGroup = 2;        // vocabulary tiles per workgroup
constexpr int kMaxLd = (1 << 22) - 1;    // row strides (elements): 256 rows fit a buffer range
constexpr int kRsrcWord3 = 0x00020000;   // raw buffer: 32-bit data format, no swizzle

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

struct Args {
  const uint16_t* w;  // [V, K] bf16, row stride ldw
  const uint16_t* h;  // [N, K] bf16, row stride ldh
  int64_t V, N, K, ldw, ldh;
  int n_vfull, n_tt, n_vg;  // full vocabulary tiles, token tiles, groups of full tiles
  float4* partial;          // [2 * n_vg + 2][N]: (m, s, t, 0), t in base-2 units
  float* logits;            // [V, N] fp32, vocabulary-major, row stride ldl (kStore only)
  int64_t ldl;
};

// s_waitcnt vmcnt(0), the other counters untouched
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Merge of two (m, s, t) states (t in base-2 units) without branches: a
// side whose maximum is below the other's scales by 2^dl, dl clamped at
// -256 so that an empty side (m = -inf, s = t = 0) adds exactly zero.  NaN
// sums stay NaN.
__device__ __forceinline__ Lse3 merge_states(Lse3 a, Lse3 b) {
  const float m = fmaxf(a.m, b.m);
  const float da = a.m == m ? 0.0f : fmaxf((a.m - m) * kLog2e, -256.0f);
  const float db = b.m == m ? 0.0f : fmaxf((b.m - m) * kLog2e, -256.0f);
  const float fa = __builtin_amdgcn_exp2f(da), fb = __builtin_amdgcn_exp2f(db);
  return Lse3{m, a.s * fa + b.s * fb,
              fa * __builtin_fmaf(da, a.s, a.t) + fb * __builtin_fmaf(db, b.s, b.t)};
}

// An accumulator read straight from its AGPR (keeps the compiler from
// copying every accumulator to VGPRs at once before the epilogue).
__device__ __forceinline__ float acc_read(float a) {
  float v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}

// Lane l's value of lane l ^ 32.
__device__ __forceinline__ float swap_halves(float v) {
  return __int_as_float(__shfl_xor(__float_as_int(v), 32, kWave));
}

// kTail = false: the full vocabulary tiles, kTilesPerGroup per workgroup.
// kTail = true: the last, partial tile (V mod 256 rows), one per token tile,
// its rows past V masked in the epilogue; its partials follow the groups'.
// kStore: the epilogue also writes every logit of the tile to a.logits,
// vocabulary-major: one non-temporal dword store per value, whose 32 lanes of
// a lane half hold 32 consecutive tokens of one vocabulary row, so that each
// store instruction writes two whole 128-byte lines (rows past V and tokens
// past N are not written).  Token-major 16-byte stores (4 rows of a token
// per lane, 32 bytes per token row per instruction) cost 4.2 ms on top of
// the 13.5 ms GEMM at 8192 x 4096 x 248320.
template <bool kTail, bool kStore>
__global__ __launch_bounds__(kThreads, 1) void lm_head_lse_kernel(Args a) {
  __shared__ __attribute__((aligned(16))) uint4 sA0[kStage], sA1[kStage], sB0[kStage], sB1[kStage];

  // ---- which tiles: token tiles fastest
  const int b = blockIdx.x;
  int tt, vg, vt0, ntiles;
  if constexpr (kTail) {
    tt = b;
    vg = a.n_vg;
    vt0 = a.n_vfull;
    ntiles = 1;
  } else {
    tt = b % a.n_tt;
    vg = b / a.n_tt;
    vt0 = vg * kTilesPerGroup;
    ntiles = min(kTilesPerGroup, a.n_vfull - vt0);
  }

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wv = wave / kWTn, wt = wave % kWTn;  // the wave's vocabulary half and token part

  // ---- load addressing: wave w's instruction q fills the 1 KB of LDS that
  // holds tile rows (8w + q) * 8 + lane / 8, physical chunk lane & 7, so the
  // lane fetches logical chunk (lane & 7) ^ ((row >> 1) & 7); with row =
  // 8(8w + q) + lane / 8 that is (lane & 7) ^ ((4 (q & 1) + lane / 16) & 7).
  // Buffer resources cover exactly the tile's valid rows: a row past N or V
  // reads as out of range (no access) and its stale LDS values only reach
  // outputs that are masked or dropped.
  const int lrow = (wave * kQ) * 8 + (lane >> 3);
  const int lchunk0 = (lane & 7) ^ ((lane >> 4) & 7);        // even q
  const int lchunk1 = (lane & 7) ^ ((4 + (lane >> 4)) & 7);  // odd q
  const uint32_t voff_h0 = (uint32_t)((lrow * a.ldh + lchunk0 * 8) * 2);
  const uint32_t voff_h1 = (uint32_t)((lrow * a.ldh + lchunk1 * 8) * 2);
  const uint32_t voff_w0 = (uint32_t)((lrow * a.ldw + lchunk0 * 8) * 2);
  const uint32_t voff_w1 = (uint32_t)((lrow * a.ldw + lchunk1 * 8) * 2);
  const int64_t t_rows = min((int64_t)kBT, a.N - (int64_t)tt * kBT);
  const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.h + (int64_t)tt * kBT * a.ldh), (short)0, (int)(t_rows * a.ldh * 2), kRsrcWord3);
  const int kt = (int)(a.K / kBK);
  const int total = ntiles * kt;

  // Loads of K step `it` (its weight tile's buffer resource and the byte
  // offset of its K range): 16 buffer loads per wave, j even = weight rows,
  // j odd = hidden rows, issued one per 2 MFMAs, so that the vector-memory
  // queue never holds the wave back from the matrix cores.
  auto w_rsrc = [&](int it) {
    const int64_t vt = (int64_t)vt0 + it / kt;
    const int64_t v_rows = min((int64_t)kBV, a.V - vt * kBV);
    return __builtin_amdgcn_make_buffer_rsrc((void*)(a.w + vt * kBV * a.ldw), (short)0,
                                             (int)(v_rows * a.ldw * 2), kRsrcWord3);
  };
  auto k0b_of = [&](int it) { return (it % kt) * kBK * 2; };
  // the whole offset goes in the VGPR operand: the range check covers it
  auto issue_one = [&](int j, __amdgpu_buffer_rsrc_t rw, int k0b, uint4* sa, uint4* sb) {
    const int q = j >> 1;
    if (j & 1) {
      const uint32_t vh = (q & 1) ? voff_h1 : voff_h0;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rh, (lds_void*)(sb + (wave * kQ + q) * 64), 16,
                                               vh + (uint32_t)(q * 8 * a.ldh * 2 + k0b), 0, 0, 0);
    } else {
      const uint32_t vw = (q & 1) ? voff_w1 : voff_w0;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void*)(sa + (wave * kQ + q) * 64), 16,
                                               vw + (uint32_t)(q * 8 * a.ldw * 2 + k0b), 0, 0, 0);
    }
  };

  f32x16 acc[kXB][kYB];
#pragma unroll
  for (int x = 0; x < kXB; ++x)
#pragma unroll
    for (int y = 0; y < kYB; ++y) acc[x][y] = f32x16{};

  // running (m, s, t) of the wave's 4 tokens (t in base-2 units)
  float rm[kYB], rs[kYB], rt[kYB];
#pragma unroll
  for (int y = 0; y < kYB; ++y) {
    rm[y] = kNegInf;
    rs[y] = 0.0f;
    rt[y] = 0.0f;
  }

  // operand reads: row = 32-row block base + (lane & 31), logical chunk
  // 2kk + lane / 32 at physical chunk ^ ((row >> 1) & 7) = ^ ((lane >> 1) & 7).
  // The fragments of k16 step kk + 1 are read while the MFMAs of step kk run
  // (registers double-buffered).
  const int rd_row = lane & 31;
  auto read_frags = [&](const uint4* sa, const uint4* sb, int kk, bf16x8 (&fa)[kXB], bf16x8 (&fb)[kYB]) {
    const int ch = (2 * kk + (lane >> 5)) ^ ((lane >> 1) & 7);
#pragma unroll
    for (int x = 0; x < kXB; ++x)
      fa[x] = __builtin_bit_cast(bf16x8, sa[(wv * 128 + x * 32 + rd_row) * kChunks + ch]);
#pragma unroll
    for (int y = 0; y < kYB; ++y)
      fb[y] = __builtin_bit_cast(bf16x8, sb[(wt * kYB * 32 + y * 32 + rd_row) * kChunks + ch]);
  };

  // 16 MFMAs of one k16 step from fragment set c, with loads j0, j0 + 1, ...
  // (weight resource rw, K offset k0b, into (la, lb)) after every second
  // MFMA when `load` is set.
  bf16x8 fa[2][kXB], fb[2][kYB];
  auto mfma16 = [&](int c, bool load, int j0, __amdgpu_buffer_rsrc_t rw, int k0b, uint4* la,
                    uint4* lb) {
#pragma unroll
    for (int x = 0; x < kXB; ++x) {
#pragma unroll
      for (int y = 0; y < kYB; ++y) {
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[c][x], fb[c][y], acc[x][y], 0, 0, 0);
        if (load && (y & 1)) issue_one(j0 + x * (kYB / 2) + (y >> 1), rw, k0b, la, lb);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // K step `it` from LDS stage (cur_a, cur_b), whose first k16 fragments are
  // already in set 0.  Step it + 1 lives in (nxt_a, nxt_b): its loads 0-7
  // went out during the last k16 of step it - 1, its loads 8-15 go out
  // during the first k16 here.  The barrier that publishes it sits before
  // the last k16: every wave has read all of step it's fragments by then, so
  // the loads 0-7 of step it + 2 into (cur_a, cur_b) go out during that last
  // k16, while step it + 1's first fragments are read.
  auto stage = [&](int it, uint4* cur_a, uint4* cur_b, uint4* nxt_a, uint4* nxt_b) {
    const bool has1 = it + 1 < total, has2 = it + 2 < total;
    const int i1 = has1 ? it + 1 : it, i2 = has2 ? it + 2 : it;
    const __amdgpu_buffer_rsrc_t w1 = w_rsrc(i1), w2 = w_rsrc(i2);
    read_frags(cur_a, cur_b, 1, fa[1], fb[1]);
    __builtin_amdgcn_sched_barrier(0);
    mfma16(0, has1, kQ, w1, k0b_of(i1), nxt_a, nxt_b);
    read_frags(cur_a, cur_b, 2, fa[0], fb[0]);
    __builtin_amdgcn_sched_barrier(0);
    mfma16(1, false, 0, w1, 0, nxt_a, nxt_b);
    read_frags(cur_a, cur_b, 3, fa[1], fb[1]);
    __builtin_amdgcn_sched_barrier(0);
    mfma16(0, false, 0, w1, 0, nxt_a, nxt_b);
    wait_vm0();
    __syncthreads();
    if (has1) read_frags(nxt_a, nxt_b, 0, fa[0], fb[0]);
    __builtin_amdgcn_sched_barrier(0);
    mfma16(1, has2, 0, w2, k0b_of(i2), cur_a, cur_b);
  };

  // fold the finished tile into the running state and clear the accumulators;
  // in the tail kernel rows past V read as -inf.  A lane folds its 64 values
  // of a token one 16-value MFMA block at a time (online: a block with a new
  // maximum rescales (s, t) by 2^dl), so only 16 accumulators are held in
  // VGPRs at a time; then the two lane halves and the running state merge.
  // The loop over the 4 token blocks is not unrolled (the unrolled form runs
  // once per tile from a cold instruction cache): each trip folds block 0
  // and rotates the blocks (and the running states) down by one, so after 4
  // trips the accumulators are zero and the states are back in place.
  auto epilogue = [&](int tile) {
    // the accumulators are read by inline asm, which the compiler's hazard
    // checks do not see: no MFMA may be scheduled past this point, and 24
    // wait states after the last one cover its result latency (11 for an
    // 8-pass MFMA)
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    int lim = 128;  // valid row offsets of this lane half are < lim
    // first vocabulary row of this lane half's values: value i of block x is
    // row vb + 32 x + 8 (i >> 2) + (i & 3)
    const int64_t vb = (int64_t)(vt0 + tile) * kBV + wv * 128 + 4 * (lane >> 5);
    if constexpr (kTail) lim = (int)min((int64_t)128, max(a.V - vb, (int64_t)0));
#pragma unroll 1
    for (int r = 0; r < kYB; ++r) {
      float m = kNegInf, s = 0.0f, t = 0.0f;
#pragma unroll
      for (int x = 0; x < kXB; ++x) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = acc_read(acc[x][0][i]);
        if constexpr (kStore) {
          // this trip folds token block r: token (lane & 31) of it
          const int64_t n = (int64_t)tt * kBT + wt * (kYB * 32) + r * 32 + (lane & 31);
          if (n < a.N) {
            // one running address, stepped through rows 0-3, 8-11, 16-19,
            // 24-27 of the block (the empty asm keeps the compiler from
            // holding all 16 addresses in registers across the tile loop)
            const int64_t ld = a.ldl;
            float* p = a.logits + (vb + x * 32) * ld + n;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              if (!kTail || x * 32 + 8 * (i >> 2) + (i & 3) < lim) __builtin_nontemporal_store(v[i], p);
              p += (i & 3) == 3 ? 5 * ld : ld;
              asm volatile("" : "+v"(p));
            }
          }
        }
        if constexpr (kTail) {
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (x * 32 + 8 * (i >> 2) + (i & 3) >= lim) v[i] = kNegInf;
        }
        float cm = v[0];
#pragma unroll
        for (int i = 1; i < 16; i += 2) cm = max3raw(cm, v[i], i + 1 < 16 ? v[i + 1] : v[i]);
        const float mn = fmaxf(m, cm);
        // rescale the running sums to the new maximum (2^-256 flushes an
        // empty start to zero without an inf * 0)
        const float dl = m == mn ? 0.0f : fmaxf((m - mn) * kLog2e, -256.0f);
        const float f = __builtin_amdgcn_exp2f(dl);
        t = f * __builtin_fmaf(dl, s, t);
        s *= f;
        m = mn;
        const float mb = m == kNegInf ? 0.0f : m * kLog2e;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float d = __builtin_fmaf(v[i], kLog2e, -mb);
          const float p = __builtin_amdgcn_exp2f(d);
          s += p;
          t = __builtin_fmaf(p, fmaxf(d, -256.0f), t);
        }
      }
      Lse3 st = merge_states(Lse3{m, s, t}, Lse3{swap_halves(m), swap_halves(s), swap_halves(t)});
      st = merge_states(Lse3{rm[0], rs[0], rt[0]}, st);
#pragma unroll
      for (int y = 0; y < kYB - 1; ++y) {
        rm[y] = rm[y + 1];
        rs[y] = rs[y + 1];
        rt[y] = rt[y + 1];
#pragma unroll
        for (int x = 0; x < kXB; ++x) acc[x][y] = acc[x][y + 1];
      }
      rm[kYB - 1] = st.m;
      rs[kYB - 1] = st.s;
      rt[kYB - 1] = st.t;
#pragma unroll
      for (int x = 0; x < kXB; ++x) acc[x][kYB - 1] = f32x16{};
    }
  };

  // ---- main loop: K steps in pairs so that each LDS stage is a fixed array;
  // the last steps of a tile load the next tile's first steps
  {
#pragma unroll
    for (int j = 0; j < 2 * kQ; ++j) issue_one(j, w_rsrc(0), k0b_of(0), sA0, sB0);
    if (total > 1) {
#pragma unroll
      for (int j = 0; j < kQ; ++j) issue_one(j, w_rsrc(1), k0b_of(1), sA1, sB1);
    }
    wait_vm0();
    __syncthreads();
    read_frags(sA0, sB0, 0, fa[0], fb[0]);
  }
  for (int tile = 0; tile < ntiles; ++tile) {
    for (int k = 0; k < kt; k += 2) {
      const int it = tile * kt + k;
      stage(it, sA0, sB0, sA1, sB1);
      stage(it + 1, sA1, sB1, sA0, sB0);
    }
    epilogue(tile);
  }

  // ---- one partial state per (group, wave half, token), from lane half 0
  if (lane < 32) {
#pragma unroll
    for (int y = 0; y < kYB; ++y) {
      const int64_t n = (int64_t)tt * kBT + wt * kYB * 32 + y * 32 + lane;
      if (n < a.N) a.partial[(int64_t)(vg * 2 + wv) * a.N + n] = float4{rm[y], rs[y], rt[y], 0.0f};
    }
  }
}

// x_t = h_n . w_{t_n} in fp32 (bf16 products are exact), one wave per token.
__global__ __launch_bounds__(256) void lm_head_target_kernel(const uint16_t* __restrict__ w,
                                                             const uint16_t* __restrict__ h,
                                                             int64_t N, int64_t V, int64_t K,
                                                             int64_t ldw, int64_t ldh,
                                                             const void* __restrict__ targets,
                                                             int t64, float* __restrict__ xt) {
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;
  const int64_t t = t64 ? reinterpret_cast<const int64_t*>(targets)[n]
                        : (int64_t)reinterpret_cast<const int32_t*>(targets)[n];
  if (t < 0 || t >= V) {
    if (lane == 0) xt[n] = __builtin_nanf("");
    return;
  }
  const uint4* hr = reinterpret_cast<const uint4*>(h + n * ldh);
  const uint4* wr = reinterpret_cast<const uint4*>(w + t * ldw);
  float acc = 0.0f;
  for (int64_t c = lane; c < K / 8; c += kWave) {
    const uint4 x = hr[c], y = wr[c];
    const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ys[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = __builtin_fmaf(bf16_lo(xs[e]), bf16_lo(ys[e]), acc);
      acc = __builtin_fmaf(bf16_hi(xs[e]), bf16_hi(ys[e]), acc);
    }
  }
  acc = wave_sum_f(acc);
  if (lane == 0) xt[n] = acc;
}

// Folds the partial states of each token: 16 tokens per workgroup, 16
// groups of threads each merging every 16th partial (a group reads 256
// contiguous bytes per partial), then one merge in LDS.
constexpr int kMergeTok = 16, kMergeGrp = 16;
__global__ __launch_bounds__(256) void lm_head_merge_kernel(const float4* __restrict__ partial,
                                                            int nsub, int64_t N,
                                                            const float* __restrict__ xt,
                                                            float* __restrict__ out_lp,
                                                            float* __restrict__ out_H,
                                                            float* __restrict__ out_lse,
                                                            int32_t* __restrict__ out_status) {
  __shared__ float red[kMergeGrp][kMergeTok][3];
  const int lt = threadIdx.x % kMergeTok, g = threadIdx.x / kMergeTok;
  const int64_t n = (int64_t)blockIdx.x * kMergeTok + lt;
  Lse3 st{kNegInf, 0.0f, 0.0f};
  if (n < N) {
#pragma unroll 4
    for (int p = g; p < nsub; p += kMergeGrp) {
      const float4 v = partial[(int64_t)p * N + n];
      st = merge_states(st, Lse3{v.x, v.y, v.z});
    }
  }
  red[g][lt][0] = st.m;
  red[g][lt][1] = st.s;
  red[g][lt][2] = st.t;
  __syncthreads();
  if (g != 0 || n >= N) return;
#pragma unroll
  for (int q = 1; q < kMergeGrp; ++q)
    st = merge_states(st, Lse3{red[q][lt][0], red[q][lt][1], red[q][lt][2]});
  const float ln_s = __builtin_amdgcn_logf(st.s) * kLn2;
  const float x = xt[n];
  if (out_lp) out_lp[n] = raw_logprob(x, st.m, ln_s);
  if (out_H) out_H[n] = ln_s - kLn2 * st.t / st.s;
  if (out_lse) out_lse[n] = st.m + ln_s;
  if (out_status) out_status[n] = x == x ? GTP_ROW_OK : GTP_ROW_BAD_TARGET;
}

struct Plan {
  int n_vfull, n_tt, n_vg;
  bool tail;
  size_t partial_bytes, xt_bytes;
};

inline Plan plan(int64_t N, int64_t V) {
  Plan p;
  p.n_vfull = (int)(V / kBV);
  p.tail = V % kBV != 0;
  p.n_tt = (int)((N + kBT - 1) / kBT);
  p.n_vg = (p.n_vfull + kTilesPerGroup - 1) / kTilesPerGroup;
  p.partial_bytes = ((size_t)(2 * p.n_vg + 2) * (size_t)N * sizeof(float4) + 255) / 256 * 256;
  p.xt_bytes = ((size_t)N * sizeof(float) + 255) / 256 * 256;
  return p;
}

}  // namespace lmh
}  // namespace gtp

using namespace gtp;

extern "C" size_t gtp_lm_head_workspace_bytes(int64_t N, int64_t V) {
  if (N <= 0 || V <= 0 || N > 0x7FFFFFFFll || V > 0x7FFFFFFFll) return 0;
  const lmh::Plan p = lmh::plan(N, V);
  return p.partial_bytes + p.xt_bytes;
}

namespace {
// Both entry points: out_logits == nullptr runs the kernels that write no
// logits.
int lm_head_run(const uint16_t* hidden, int64_t N, int64_t K, int64_t hidden_stride,
                const uint16_t* weight, int64_t V, int64_t weight_stride, const void* targets,
                int targets_int64, float* out_logprob, float* out_entropy, float* out_lse,
                int32_t* out_status, float* out_logits, int64_t logits_stride, void* workspace,
                size_t workspace_bytes, void* stream) {
  if (N < 0 || V <= 0 || K <= 0 || hidden_stride < K || weight_stride < K ||
      (N > 0 && (!hidden || !weight || !targets || !out_logprob || !workspace)))
    return GTP_ERR_INVALID_ARGUMENT;
  if (N > 0x7FFFFFFFll || V > 0x7FFFFFFFll || K > ((int64_t)1 << 30)) return GTP_ERR_UNSUPPORTED;
  // the tile loop's shape: K in steps of 128 (two stages), 16-byte rows
  if (K % (2 * lmh::kBK) != 0 || (hidden_stride & 7) || (weight_stride & 7) ||
      hidden_stride > lmh::kMaxLd || weight_stride > lmh::kMaxLd ||
      (reinterpret_cast<uintptr_t>(hidden) & 15u) || (reinterpret_cast<uintptr_t>(weight) & 15u))
    return GTP_ERR_UNSUPPORTED;
  if (out_logits) {
    if (logits_stride < N) return GTP_ERR_INVALID_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(out_logits) & 3u) || logits_stride > ((int64_t)1 << 40) / V)
      return GTP_ERR_UNSUPPORTED;
  }
  if (N == 0) return GTP_OK;
  const lmh::Plan p = lmh::plan(N, V);
  if (workspace_bytes < p.partial_bytes + p.xt_bytes) return GTP_ERR_INVALID_ARGUMENT;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  lmh::Args a;
  a.w = weight;
  a.h = hidden;
  a.V = V;
  a.N = N;
  a.K = K;
  a.ldw = weight_stride;
  a.ldh = hidden_stride;
  a.n_vfull = p.n_vfull;
  a.n_tt = p.n_tt;
  a.n_vg = p.n_vg;
  a.partial = reinterpret_cast<float4*>(workspace);
  a.logits = out_logits;
  a.ldl = logits_stride;
  float* xt = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(workspace) + p.partial_bytes);
  const int64_t grid = (int64_t)p.n_vg * p.n_tt;
  if (grid > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  if (out_logits) {
    if (grid > 0)
      launch_timed(lmh::lm_head_lse_kernel<false, true>, dim3((unsigned)grid), dim3(lmh::kThreads), s, a);
    if (p.tail)
      hipLaunchKernelGGL((lmh::lm_head_lse_kernel<true, true>), dim3((unsigned)p.n_tt),
                         dim3(lmh::kThreads), 0, s, a);
  } else {
    if (grid > 0)
      launch_timed(lmh::lm_head_lse_kernel<false, false>, dim3((unsigned)grid), dim3(lmh::kThreads), s, a);
    if (p.tail)
      hipLaunchKernelGGL((lmh::lm_head_lse_kernel<true, false>), dim3((unsigned)p.n_tt),
                         dim3(lmh::kThreads), 0, s, a);
  }
  hipLaunchKernelGGL(lmh::lm_head_target_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, s,
                     weight, hidden, N, V, K, weight_stride, hidden_stride, targets, targets_int64,
                     xt);
  hipLaunchKernelGGL(lmh::lm_head_merge_kernel,
                     dim3((unsigned)((N + lmh::kMergeTok - 1) / lmh::kMergeTok)), dim3(256), 0, s,
                     a.partial, 2 * p.n_vg + (p.tail ? 2 : 0), N, xt, out_logprob, out_entropy,
                     out_lse, out_status);
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}
}  // namespace

extern "C" int gtp_lm_head_logprob_rows(const uint16_t* hidden, int64_t N, int64_t K,
                                        int64_t hidden_stride, const uint16_t* weight, int64_t V,
                                        int64_t weight_stride, const void* targets,
                                        int targets_int64, float* out_logprob, float* out_entropy,
                                        float* out_lse, int32_t* out_status, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  return lm_head_run(hidden, N, K, hidden_stride, weight, V, weight_stride, targets,
                     targets_int64, out_logprob, out_entropy, out_lse, out_status, nullptr, 0,
                     workspace, workspace_bytes, stream);
}

extern "C" int gtp_lm_head_logprob_save_rows(const uint16_t* hidden, int64_t N, int64_t K,
                                             int64_t hidden_stride, const uint16_t* weight,
                                             int64_t V, int64_t weight_stride,
                                             const void* targets, int targets_int64,
                                             float* out_logprob, float* out_entropy,
                                             float* out_lse, int32_t* out_status,
                                             float* out_logits, int64_t logits_stride,
                                             void* workspace, size_t workspace_bytes,
                                             void* stream) {
  if (N > 0 && !out_logits) return GTP_ERR_INVALID_ARGUMENT;
  return lm_head_run(hidden, N, K, hidden_stride, weight, V, weight_stride, targets,
                     targets_int64, out_logprob, out_entropy, out_lse, out_status,
                     N > 0 ? out_logits : nullptr, logits_stride, workspace, workspace_bytes,
                     stream);
}
