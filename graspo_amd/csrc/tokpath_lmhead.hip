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
// is loaded straight from global memory into LDS (global_load_lds_dwordx4,
// no registers) while the matrix cores work on step i.  Each 128-byte LDS
// row holds its eight 16-byte chunks XOR-swizzled by the row's low 3 bits,
// so the MFMA operand reads (32 rows x one chunk per half-wave) hit 8
// different chunk columns per 8 lanes.
//
// The GEMM computes logits transposed, vocabulary x tokens: lane l of a
// 32 x 32 block holds token (l mod 32) and 16 vocabulary rows, so a token's
// 64 values per wave fold in registers and only the two lane halves and the
// vocabulary tiles merge afterwards.
//
// Order of work.  The workgroup for (vocabulary group g, token tile j) runs
// kTilesPerGroup vocabulary tiles in a row (its K loop runs on across the
// tile boundary), merging each tile into its running state, and writes one
// partial state per (g, wave half, token).  Workgroup b runs on XCD b mod 8;
// the 32 workgroups that share an XCD's L2 at a time take the same
// vocabulary group and consecutive token tiles, so each weight tile is
// fetched into that L2 once and read by all of them.  A merge kernel folds
// the partials and the target logits (one fp32 dot product per token, the
// reference's own selected_logits) into logprob, entropy and lse.
#include "tokpath_stream.h"

namespace gtp {
namespace lmh {

constexpr int kBV = 256;                 // vocabulary rows per tile
constexpr int kBT = 256;                 // tokens per tile
constexpr int kBK = 64;                  // K per stage: 128 bytes of bf16 per row
constexpr int kThreads = 256;            // 4 waves
constexpr int kChunks = kBK / 8;         // 16-byte chunks per tile row
constexpr int kStage = kBV * kChunks;    // 16-byte chunks per operand stage (32 KB)
constexpr int kTilesPerGroup = 4;        // vocabulary tiles per workgroup
constexpr int kXcds = 8;
constexpr int kMaxLd = (1 << 22) - 1;    // row strides (elements): 256 rows fit a buffer range
constexpr int kRsrcWord3 = 0x00020000;   // raw buffer: 32-bit data format, no swizzle

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

struct Args {
  const uint16_t* w;  // [V, K] bf16, row stride ldw
  const uint16_t* h;  // [N, K] bf16, row stride ldh
  int64_t V, N, K, ldw, ldh;
  int n_vt, n_tt, n_vg;  // vocabulary tiles, token tiles, vocabulary groups
  float4* partial;       // [2 * n_vg][N]: (m, s, t, 0), t in base-2 units
};

// s_waitcnt vmcnt(0), the other counters untouched
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Lane l's value of lane l ^ 32.
__device__ __forceinline__ float swap_halves(float v) {
  return __int_as_float(__shfl_xor(__float_as_int(v), 32, kWave));
}

__global__ __launch_bounds__(kThreads, 1) void lm_head_lse_kernel(Args a) {
  __shared__ __attribute__((aligned(16))) uint4 sA0[kStage], sA1[kStage], sB0[kStage], sB1[kStage];

  // ---- which tile group: XCD-major, token tiles fastest within an XCD
  const int b = blockIdx.x;
  const int xcd = b % kXcds, j = b / kXcds;
  const int tt = j % a.n_tt;
  const int vg = (j / a.n_tt) * kXcds + xcd;
  if (vg >= a.n_vg) return;
  const int vt0 = vg * kTilesPerGroup;
  const int ntiles = min(kTilesPerGroup, a.n_vt - vt0);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wv = wave >> 1, wt = wave & 1;  // the wave's vocabulary and token halves

  // ---- load addressing: wave w's instruction q fills tile rows
  // (8w + q) * 8 + lane / 8, chunk (lane & 7) ^ (row & 7) -- the row's low
  // 3 bits are lane / 8 for every q.  Buffer resources cover exactly the
  // tile's valid rows: a row past N or V reads as out of range (no access)
  // and its stale LDS values only reach outputs that are masked or dropped.
  const int lrow = (wave * 8) * 8 + (lane >> 3);
  const int lchunk = (lane & 7) ^ ((lane >> 3) & 7);
  const uint32_t voff_h = (uint32_t)((lrow * a.ldh + lchunk * 8) * 2);
  const uint32_t voff_w = (uint32_t)((lrow * a.ldw + lchunk * 8) * 2);
  const int64_t t_rows = min((int64_t)kBT, a.N - (int64_t)tt * kBT);
  const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.h + (int64_t)tt * kBT * a.ldh), (short)0, (int)(t_rows * a.ldh * 2), kRsrcWord3);
  __amdgpu_buffer_rsrc_t rw;
  auto set_tile = [&](int vt) {
    const int64_t v_rows = min((int64_t)kBV, a.V - (int64_t)vt * kBV);
    rw = __builtin_amdgcn_make_buffer_rsrc((void*)(a.w + (int64_t)vt * kBV * a.ldw), (short)0,
                                           (int)(v_rows * a.ldw * 2), kRsrcWord3);
  };

  const int kt = (int)(a.K / kBK);
  const int total = ntiles * kt;
  int load_tile = 0;  // tile of the next stage to load
  set_tile(vt0);

  auto issue = [&](int it, uint4* sa, uint4* sb) {
    const int tile = it / kt;
    if (tile != load_tile) {
      load_tile = tile;
      set_tile(vt0 + tile);
    }
    const int k0b = (it - tile * kt) * kBK * 2;
    // the whole offset goes in the VGPR operand: the range check covers it
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void*)(sa + (wave * 8 + q) * 64), 16,
                                               voff_w + (uint32_t)(q * 8 * a.ldw * 2 + k0b), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rh, (lds_void*)(sb + (wave * 8 + q) * 64), 16,
                                               voff_h + (uint32_t)(q * 8 * a.ldh * 2 + k0b), 0, 0, 0);
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y) acc[x][y] = f32x16{};

  // running (m, s, t) of the wave's 4 tokens (t in base-2 units)
  float rm[4], rs[4], rt[4];
#pragma unroll
  for (int y = 0; y < 4; ++y) {
    rm[y] = kNegInf;
    rs[y] = 0.0f;
    rt[y] = 0.0f;
  }

  // operand reads: row = 32-row block base + (lane & 31), chunk 2kk + lane/32,
  // swizzled by the row's low 3 bits (= lane & 7)
  const int rd_row = lane & 31;
  auto compute = [&](const uint4* sa, const uint4* sb) {
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int ch = (2 * kk + (lane >> 5)) ^ (lane & 7);
      bf16x8 fa[4], fb[4];
#pragma unroll
      for (int x = 0; x < 4; ++x)
        fa[x] = __builtin_bit_cast(bf16x8, sa[(wv * 128 + x * 32 + rd_row) * kChunks + ch]);
#pragma unroll
      for (int y = 0; y < 4; ++y)
        fb[y] = __builtin_bit_cast(bf16x8, sb[(wt * 128 + y * 32 + rd_row) * kChunks + ch]);
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[x], fb[y], acc[x][y], 0, 0, 0);
    }
  };

  // fold the finished tile into the running state and clear the accumulators;
  // rows past V (the last tile only) read as -inf, without a branch
  auto epilogue = [&](int tile) {
    const int64_t vb = (int64_t)(vt0 + tile) * kBV + wv * 128 + 4 * (lane >> 5);
    const int lim = (int)min((int64_t)128, max(a.V - vb, (int64_t)0));  // valid row offsets < lim
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      float xv[64];
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int r = x * 32 + 8 * (i >> 2) + (i & 3);
          xv[x * 16 + i] = r < lim ? acc[x][y][i] : kNegInf;
        }
      float m = kNegInf;
#pragma unroll
      for (int e = 0; e < 64; e += 2) m = max3raw(m, xv[e], xv[e + 1]);
      m = fmaxf(m, swap_halves(m));
      // a wave whose rows are all past V folds nothing (m stays -inf)
      const float mb = m == kNegInf ? 0.0f : m * kLog2e;
      float s = 0.0f, t = 0.0f;
#pragma unroll
      for (int e = 0; e < 64; ++e) {
        const float d = __builtin_fmaf(xv[e], kLog2e, -mb);
        const float p = __builtin_amdgcn_exp2f(d);
        s += p;
        t = __builtin_fmaf(p, fmaxf(d, -256.0f), t);
      }
      s += swap_halves(s);
      t += swap_halves(t);
      const Lse3 mg = lse3_merge(Lse3{rm[y], rs[y], rt[y]}, Lse3{m, s, t});
      rm[y] = mg.m;
      rs[y] = mg.s;
      rt[y] = mg.t;
#pragma unroll
      for (int x = 0; x < 4; ++x) acc[x][y] = f32x16{};
    }
  };

  // ---- main loop: k steps in pairs so that each LDS stage is a fixed array;
  // the last pair of a tile prefetches the next tile's first stage
  issue(0, sA0, sB0);
  for (int tile = 0; tile < ntiles; ++tile) {
    for (int k = 0; k < kt; k += 2) {
      const int it = tile * kt + k;
      wait_vm0();
      __syncthreads();
      issue(it + 1, sA1, sB1);
      __builtin_amdgcn_sched_barrier(0);  // the loads go out before the stage's math
      compute(sA0, sB0);
      wait_vm0();
      __syncthreads();
      if (it + 2 < total) issue(it + 2, sA0, sB0);
      __builtin_amdgcn_sched_barrier(0);
      compute(sA1, sB1);
    }
    epilogue(tile);
  }

  // ---- one partial state per (group, wave half, token), from lane half 0
  if (lane < 32) {
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const int64_t n = (int64_t)tt * kBT + wt * 128 + y * 32 + lane;
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

// Folds the 2 * n_vg partial states of each token: 64 tokens per workgroup,
// 4 waves each merging a quarter of the partials, then one merge in LDS.
__global__ __launch_bounds__(256) void lm_head_merge_kernel(const float4* __restrict__ partial,
                                                            int nsub, int64_t N,
                                                            const float* __restrict__ xt,
                                                            float* __restrict__ out_lp,
                                                            float* __restrict__ out_H,
                                                            float* __restrict__ out_lse,
                                                            int32_t* __restrict__ out_status) {
  __shared__ float red[4][64][3];
  const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int64_t n = (int64_t)blockIdx.x * 64 + lane;
  Lse3 st{kNegInf, 0.0f, 0.0f};
  if (n < N)
    for (int p = g; p < nsub; p += 4) {
      const float4 v = partial[(int64_t)p * N + n];
      st = lse3_merge(st, Lse3{v.x, v.y, v.z});
    }
  red[g][lane][0] = st.m;
  red[g][lane][1] = st.s;
  red[g][lane][2] = st.t;
  __syncthreads();
  if (g != 0 || n >= N) return;
#pragma unroll
  for (int q = 1; q < 4; ++q) st = lse3_merge(st, Lse3{red[q][lane][0], red[q][lane][1], red[q][lane][2]});
  const float ln_s = __builtin_amdgcn_logf(st.s) * kLn2;
  const float x = xt[n];
  if (out_lp) out_lp[n] = raw_logprob(x, st.m, ln_s);
  if (out_H) out_H[n] = ln_s - kLn2 * st.t / st.s;
  if (out_lse) out_lse[n] = st.m + ln_s;
  if (out_status) out_status[n] = x == x ? GTP_ROW_OK : GTP_ROW_BAD_TARGET;
}

struct Plan {
  int n_vt, n_tt, n_vg;
  size_t partial_bytes, xt_bytes;
};

inline Plan plan(int64_t N, int64_t V) {
  Plan p;
  p.n_vt = (int)((V + kBV - 1) / kBV);
  p.n_tt = (int)((N + kBT - 1) / kBT);
  p.n_vg = (p.n_vt + kTilesPerGroup - 1) / kTilesPerGroup;
  p.partial_bytes = ((size_t)2 * p.n_vg * (size_t)N * sizeof(float4) + 255) / 256 * 256;
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

extern "C" int gtp_lm_head_logprob_rows(const uint16_t* hidden, int64_t N, int64_t K,
                                        int64_t hidden_stride, const uint16_t* weight, int64_t V,
                                        int64_t weight_stride, const void* targets,
                                        int targets_int64, float* out_logprob, float* out_entropy,
                                        float* out_lse, int32_t* out_status, void* workspace,
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
  a.n_vt = p.n_vt;
  a.n_tt = p.n_tt;
  a.n_vg = p.n_vg;
  a.partial = reinterpret_cast<float4*>(workspace);
  float* xt = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(workspace) + p.partial_bytes);
  const int64_t per_xcd = ((int64_t)p.n_vg + lmh::kXcds - 1) / lmh::kXcds;
  const int64_t grid = per_xcd * lmh::kXcds * p.n_tt;
  if (grid > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  launch_timed(lmh::lm_head_lse_kernel, dim3((unsigned)grid), dim3(lmh::kThreads), s, a);
  hipLaunchKernelGGL(lmh::lm_head_target_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, s,
                     weight, hidden, N, V, K, weight_stride, hidden_stride, targets, targets_int64,
                     xt);
  hipLaunchKernelGGL(lmh::lm_head_merge_kernel, dim3((unsigned)((N + 63) / 64)), dim3(256), 0, s,
                     a.partial, 2 * p.n_vg, N, xt, out_logprob, out_entropy, out_lse, out_status);
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}
