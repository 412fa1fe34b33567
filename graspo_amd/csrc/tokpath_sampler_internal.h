// tokpath_sampler_internal.h -- pieces shared by the sampler's two paths
// (tokpath_sampler.hip: one workgroup per row, any shape; tokpath_sampler_fast.hip:
// vocabulary split over workgroups with a last-arriving-workgroup merge).
#pragma once

#include "tokpath_common.h"

namespace gtp {

struct SamplerArgs {
  const void* logits;
  int64_t V;
  int64_t row_stride;
  const int32_t* hist;
  int64_t hist_len;
  int64_t hist_stride;
  const uint32_t* mask;
  int64_t mask_stride;
  const float* uniforms;
  float T;
  int32_t K;
  float P;
  float rho;
  const uint8_t* finished;
  int64_t pad_id;
  int64_t* out_ids;
  float* out_lp;
  float* out_slp;
  int32_t* out_kept;
  float* out_tv;
  int32_t* out_tid;
  int32_t* out_status;
};

// One workgroup of 1024 threads per row (any layout, V <= GTP_SAMPLER_MAX_V),
// or, for small batches of bf16 top-p rows, S workgroups per row that merge
// their counts through `workspace` (topp_workspace_bytes of it, zeroed once).
int launch_sampler_general(const SamplerArgs& a, int dtype, int64_t B, hipStream_t s,
                           void* workspace, size_t workspace_bytes);


// The first kWsZeroBytes of a sampler workspace are words that every call
// leaves zero: the split kernel's per-row arrival counters (words 0..B-1,
// B < CUs) and the split top-p kernel's (word kToppSplitCtrWord + b).
// The kernels' slot data lies after it, so a call never finds another call's
// slot data in its counters.
constexpr size_t kWsZeroBytes = 16384;
constexpr uint32_t kToppSplitCtrWord = 2048;
// rows a split top-p call may have (at 128 rows of 248320 the one-workgroup
// kernel is faster: 46 against 50 us)
constexpr int64_t kToppSplitMaxB = 64;

// Compute units of the current device (cached per device).
int64_t device_cus();

// The split top-p kernel's launch for these parameters: S slices of vps
// vectors per row and the workspace it needs, at most `cap` bytes (fewer
// slices when more would not fit); S = 0 when the call does not take it.
struct ToppSplit {
  int S;
  int64_t vps;
  size_t bytes;
};
ToppSplit plan_topp_split(int dtype, int64_t B, int64_t V, const gtp_sampler_params* p, size_t cap);

// Which kernel launch_sampler_general runs for a call (GTP_ROUTE_*, never
// GTP_ROUTE_SPLIT_TOPK), and the split top-p kernel's plan when it takes the
// call.  The one decision both the launch and gtp_sample_route use.
struct GeneralRoute {
  int route;
  ToppSplit split;
};
// aligned: 16-byte aligned logits and row stride; hist_len: history entries
// per row (0 without a history); has_ws: a workspace was passed.
GeneralRoute route_general(int dtype, int64_t B, int64_t V, bool aligned, int64_t hist_len,
                           bool has_mask, const gtp_sampler_params* p, bool has_ws,
                           size_t workspace_bytes);

// Workspace of the top-p path for these parameters within `cap` bytes: the
// split top-p kernel's counters, headers and slots (0 when the call takes
// another path, the one-workgroup top-p kernels included).
size_t topp_workspace_bytes(int dtype, int64_t B, int64_t V, const gtp_sampler_params* p, size_t cap);

// Greedy decoding (T <= 0) is the reference's logits.argmax(dim=-1)
// (src/graspo/backends/graspoflow/tensor_utils.py:658) over the allowed
// tokens' penalised logits y = pen(x): a NaN beats every value and +inf
// every finite one (torch's argmax propagates NaN), ties go to the lowest
// id, and a row whose allowed tokens are all -inf returns the first of them.
// The ordered paths of both kernels handle rows of finite values; a greedy
// row they report as non-finite or empty comes here instead, where one wave
// (all 64 lanes of the calling wave; the rest of the workgroup idle) scans
// the row in id order.  `pen` is an LDS bitmap of at least ceil(V/32) words
// that this wave rebuilds from the history when `rebuild_pen` is set (the
// caller's copy covers only its slice), or that already holds the row's
// penalised ids.  Lane 0 writes the row's outputs; logprob is NaN when the
// raw row holds a NaN or +inf (`raw_nonfinite`), as log_softmax gives.
template <typename T>
__device__ __forceinline__ void greedy_argmax_rescan(const SamplerArgs& a, int64_t b, uint32_t* pen,
                                                  bool rebuild_pen, bool raw_nonfinite,
                                                  float lse_m, float lse_ln) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t V = a.V;
  const bool use_pen = a.hist && a.hist_len > 0 && a.rho != 1.0f;
  if (use_pen && rebuild_pen) {
    const int64_t nw = (V + 31) / 32;
    for (int64_t w = lane; w < nw; w += kWave) pen[w] = 0u;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    const int32_t* h = a.hist + b * a.hist_stride;
    for (int64_t j = lane; j < a.hist_len; j += kWave) {
      const int32_t id = h[j];
      if (id >= 0 && id < V) atomicOr(&pen[id >> 5], 1u << (id & 31));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
  const T* row = reinterpret_cast<const T*>(a.logits) + b * a.row_stride;
  const uint32_t* mrow = a.mask ? a.mask + b * a.mask_stride : nullptr;
  // lane L takes tokens [8 (L + 64 k), + 8): ascending ids within the lane
  int64_t bid = -1;
  float by = 0.0f;
  for (int64_t i0 = (int64_t)lane * 8; i0 < V; i0 += (int64_t)kWave * 8) {
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = i0 + j < V ? Elem<T>::get(row, i0 + j) : 0.0f;
    const uint32_t mw = mrow ? (mrow[i0 >> 5] >> (i0 & 31)) : 0xFFu;  // i0 % 8 == 0
    const uint32_t pw = use_pen ? (pen[i0 >> 5] >> (i0 & 31)) : 0u;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (i0 + j >= V || !((mw >> j) & 1u)) continue;
      float y = x[j];
      if ((pw >> j) & 1u) y = (y < 0.0f) ? y * a.rho : y / a.rho;
      y = y + 0.0f;
      if (bid < 0 || (by == by && (y != y || y > by))) {
        bid = i0 + j;
        by = y;
      }
    }
  }
  // wave reduction: (valid, NaN first, larger y, lower id)
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int64_t oid = __shfl_xor(bid, o, kWave);
    const float oy = __shfl_xor(by, o, kWave);
    bool take;
    if (oid < 0) take = false;
    else if (bid < 0) take = true;
    else if ((oy != oy) != (by != by)) take = oy != oy;
    else if (oy != oy || oy == by) take = oid < bid;
    else take = oy > by;
    if (take) {
      bid = oid;
      by = oy;
    }
  }
  if (lane != 0) return;
  const bool fin = a.finished && a.finished[b];
  const bool ok = bid >= 0;
  a.out_ids[b] = fin ? a.pad_id : (ok ? bid : -1);
  const float lp = (!ok || raw_nonfinite)
                       ? __builtin_nanf("")
                       : raw_logprob(Elem<T>::get(row, ok ? bid : 0), lse_m, lse_ln);
  if (a.out_lp) a.out_lp[b] = lp;
  if (a.out_slp) a.out_slp[b] = ok ? 0.0f : __builtin_nanf("");
  if (a.out_kept) a.out_kept[b] = ok ? 1 : 0;
  if (a.out_tv) a.out_tv[b] = ok ? by : 0.0f;
  if (a.out_tid) a.out_tid[b] = ok ? (int32_t)bid : -1;
  if (a.out_status) a.out_status[b] = ok ? GTP_ROW_OK : GTP_ROW_EMPTY;
}

}  // namespace gtp
