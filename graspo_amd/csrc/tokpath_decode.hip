// tokpath_decode.hip -- the per-token bookkeeping of the generation loop,
// fused into one launch (gfx950).
//
// After the sampler has written a token per row (pad_token_id for rows that
// were already finished), the reference's loop body runs
//   sequences = torch.cat([sequences, next_token.unsqueeze(1)], dim=1)
//   finished |= next_token.eq(eos_token_id)
//   all_finished = bool(finished.all())          (a host sync every token)
//   attention_mask = sequences.ne(pad_token_id)
// (src/graspo/backends/graspoflow/models/qwen3/adapter.py:293-304,
//  models/qwen35_36/generation.py:259-270).  Here one workgroup writes the
// token into a preallocated sequence column and the attention-mask column,
// updates `finished` in place and writes two counters (rows still
// unfinished, rows whose sampler status is not OK) that the host reads
// asynchronously, a step later, instead of synchronising on every token.
// A row whose sampler status is not OK carries id -1; its id is replaced by
// pad_token_id here (in `ids` itself, in the sequence and in the attention
// mask) so that the next forward, queued before the host reads the counts
// and raises, never embeds an id outside [0, V).
#include "tokpath_common.h"

namespace gtp {

constexpr int kDuBlock = 1024;

__global__ __launch_bounds__(kDuBlock) void decode_update_kernel(
    int64_t* __restrict__ ids, const int32_t* __restrict__ status, int64_t B, int64_t eos,
    int64_t pad, uint8_t* __restrict__ finished, int64_t* __restrict__ seq, int64_t seq_stride,
    uint8_t* __restrict__ attn, int64_t attn_stride, int64_t col, int32_t* __restrict__ flags) {
  __shared__ int32_t red[2][kDuBlock / kWave];
  int32_t open = 0, bad = 0;
  for (int64_t b = threadIdx.x; b < B; b += kDuBlock) {
    const bool row_bad = status && status[b] != GTP_ROW_OK;
    int64_t id = ids[b];
    if (row_bad) {
      id = pad;
      ids[b] = pad;
    }
    const bool f = finished[b] != 0 || id == eos;
    finished[b] = f ? 1 : 0;
    if (seq) seq[b * seq_stride + col] = id;
    if (attn) attn[b * attn_stride + col] = id != pad ? 1 : 0;
    open += f ? 0 : 1;
    bad += row_bad ? 1 : 0;
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    open += __shfl_xor(open, o, kWave);
    bad += __shfl_xor(bad, o, kWave);
  }
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  if (lane == 0) {
    red[0][wid] = open;
    red[1][wid] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t o = 0, d = 0;
#pragma unroll
    for (int w = 0; w < kDuBlock / kWave; ++w) {
      o += red[0][w];
      d += red[1][w];
    }
    flags[0] = o;
    flags[1] = d;
  }
}

}  // namespace gtp

using namespace gtp;

extern "C" int gtp_decode_update_rows(int64_t* ids, const int32_t* status, int64_t B,
                                      int64_t eos_token_id, int64_t pad_token_id,
                                      uint8_t* finished, int64_t* seq, int64_t seq_stride,
                                      uint8_t* attn, int64_t attn_stride, int64_t col,
                                      int32_t* flags, void* stream) {
  if (B < 0 || col < 0 || !flags || (B > 0 && (!ids || !finished))) return GTP_ERR_INVALID_ARGUMENT;
  if ((seq && seq_stride <= col) || (attn && attn_stride <= col)) return GTP_ERR_INVALID_ARGUMENT;
  if (B > 0x7FFFFFFFll) return GTP_ERR_UNSUPPORTED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(decode_update_kernel, dim3(1), dim3(kDuBlock), 0, s, ids, status, B,
                     eos_token_id, pad_token_id, finished, seq, seq_stride, attn, attn_stride, col,
                     flags);
  return hipGetLastError() == hipSuccess ? GTP_OK : GTP_ERR_LAUNCH;
}
