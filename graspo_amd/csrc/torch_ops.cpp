// torch_ops.cpp -- thin PyTorch-ROCm binding of the C ABI (host-only C++).
//
// Registers torch.ops.graspo_tokpath.{sample, sample_route, logprob_entropy, logprob_backward, graspo_loss_*, lse_partial,
// lse_finalize, decode_update, to_bf16_exact, logprob_backward_split, time_next_launch,
// lm_head_logprob, lm_head_logprob_save, softmax_grad_bf16}.  Each op validates its tensors (TORCH_CHECK surfaces as a
// Python RuntimeError), allocates the outputs on the logits' device, and
// enqueues the HIP kernels on the stream handle passed in from Python
// (torch.cuda.current_stream().cuda_stream), so work orders with the
// caller's other torch work exactly as the reference's ATen ops did.
#include <ATen/ATen.h>
#include <torch/library.h>

#include <map>
#include <mutex>
#include <tuple>
#include <utility>

#include "graspo_tokpath.h"

namespace {

int dtype_code(const at::Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat:
      return GTP_DTYPE_F32;
    case at::kBFloat16:
      return GTP_DTYPE_BF16;
    case at::kHalf:
      return GTP_DTYPE_F16;
    default:
      TORCH_CHECK(false, "graspo_tokpath: logits must be float32, bfloat16 or float16, got ",
                  t.scalar_type());
  }
  return -1;
}

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == GTP_OK, "graspo_tokpath: ", what, " failed with code ", rc,
              rc == GTP_ERR_INVALID_ARGUMENT ? " (invalid argument)"
              : rc == GTP_ERR_UNSUPPORTED    ? " (unsupported shape)"
                                             : " (kernel launch error)");
}

void check_rows(const at::Tensor& logits, const char* name) {
  TORCH_CHECK(logits.is_cuda(), "graspo_tokpath: ", name, " must be a GPU tensor");
  TORCH_CHECK(logits.dim() == 2, "graspo_tokpath: ", name, " must be 2-D [rows, V], got ",
              logits.dim(), "-D");
  TORCH_CHECK(logits.size(1) == 0 || logits.stride(1) == 1, "graspo_tokpath: ", name,
              " rows must be contiguous (stride(-1) == 1)");
}

int64_t row_stride_of(const at::Tensor& logits) {
  return logits.size(0) > 1 ? logits.stride(0) : logits.size(1);
}

void check_same_device(const at::Tensor& a, const at::Tensor& b, const char* name) {
  TORCH_CHECK(b.device() == a.device(), "graspo_tokpath: ", name, " must be on ", a.device());
}

// Sampler workspace, one per (device, stream): zero-filled when allocated (the
// library keeps it reusable from call to call), grown when a call needs more.
// Calls on one stream are ordered, so they can share it.
void* sampler_workspace(const at::Tensor& like, size_t bytes, int64_t stream) {
  if (bytes == 0) return nullptr;
  static std::mutex mu;
  static std::map<std::pair<int, int64_t>, at::Tensor> cache;
  std::lock_guard<std::mutex> lock(mu);
  at::Tensor& ws = cache[{(int)like.get_device(), stream}];
  if (!ws.defined() || (size_t)ws.numel() < bytes) {
    const int64_t n = (int64_t)((bytes + 4095) / 4096 * 4096);
    ws = at::zeros({n}, like.options().dtype(at::kByte));
  }
  return ws.data_ptr();
}

using SampleOut =
    std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor>;

SampleOut sample(const at::Tensor& logits, double temperature, int64_t top_k, double top_p,
                 double repetition_penalty, const c10::optional<at::Tensor>& history,
                 const c10::optional<at::Tensor>& allow_mask,
                 const c10::optional<at::Tensor>& uniforms,
                 const c10::optional<at::Tensor>& finished, int64_t pad_token_id, int64_t stream) {
  check_rows(logits, "logits");
  const int64_t B = logits.size(0), V = logits.size(1);
  TORCH_CHECK(V > 0, "graspo_tokpath.sample: empty vocabulary");
  TORCH_CHECK(V <= GTP_SAMPLER_MAX_V, "graspo_tokpath.sample: V = ", V, " exceeds ",
              GTP_SAMPLER_MAX_V);
  TORCH_CHECK(repetition_penalty > 0.0, "graspo_tokpath.sample: repetition_penalty must be > 0");
  TORCH_CHECK(top_k >= 0 && top_k <= INT32_MAX, "graspo_tokpath.sample: top_k must be >= 0");
  const int32_t* hist = nullptr;
  int64_t hist_len = 0, hist_stride = 0;
  if (history.has_value() && history->numel() > 0) {
    const auto& h = *history;
    check_same_device(logits, h, "history");
    TORCH_CHECK(h.scalar_type() == at::kInt && h.dim() == 2 && h.size(0) == B && h.stride(1) == 1,
                "graspo_tokpath.sample: history must be int32 [B, L] with contiguous rows");
    hist = h.data_ptr<int32_t>();
    hist_len = h.size(1);
    hist_stride = B > 1 ? h.stride(0) : hist_len;
  }
  const uint32_t* mask = nullptr;
  int64_t mask_stride = 0;
  if (allow_mask.has_value()) {
    const auto& m = *allow_mask;
    check_same_device(logits, m, "allow_mask");
    TORCH_CHECK((m.scalar_type() == at::kInt || m.scalar_type() == at::kUInt32) && m.dim() == 2 &&
                    m.size(0) == B && m.size(1) >= (V + 31) / 32 && m.stride(1) == 1,
                "graspo_tokpath.sample: allow_mask must be int32/uint32 [B, >= ceil(V/32)]");
    mask = static_cast<const uint32_t*>(m.data_ptr());
    mask_stride = B > 1 ? m.stride(0) : m.size(1);
  }
  const bool greedy = !(temperature > 0.0);
  const float* u = nullptr;
  if (uniforms.has_value()) {
    const auto& uu = *uniforms;
    check_same_device(logits, uu, "uniforms");
    TORCH_CHECK(uu.scalar_type() == at::kFloat && uu.dim() == 1 && uu.size(0) == B &&
                    uu.is_contiguous(),
                "graspo_tokpath.sample: uniforms must be float32 [B]");
    u = uu.data_ptr<float>();
  }
  TORCH_CHECK(greedy || u != nullptr, "graspo_tokpath.sample: uniforms are required when T > 0");
  const uint8_t* fin = nullptr;
  if (finished.has_value()) {
    const auto& f = *finished;
    check_same_device(logits, f, "finished");
    TORCH_CHECK((f.scalar_type() == at::kBool || f.scalar_type() == at::kByte) && f.dim() == 1 &&
                    f.size(0) == B && f.is_contiguous(),
                "graspo_tokpath.sample: finished must be bool/uint8 [B]");
    fin = static_cast<const uint8_t*>(f.data_ptr());
  }
  auto opt = logits.options();
  at::Tensor ids = at::empty({B}, opt.dtype(at::kLong));
  at::Tensor lp = at::empty({B}, opt.dtype(at::kFloat));
  at::Tensor slp = at::empty({B}, opt.dtype(at::kFloat));
  at::Tensor kept = at::empty({B}, opt.dtype(at::kInt));
  at::Tensor tv = at::empty({B}, opt.dtype(at::kFloat));
  at::Tensor tid = at::empty({B}, opt.dtype(at::kInt));
  at::Tensor st = at::empty({B}, opt.dtype(at::kInt));
  gtp_sampler_params p;
  p.temperature = (float)temperature;
  p.top_k = (int32_t)top_k;
  p.top_p = (float)top_p;
  p.repetition_penalty = (float)repetition_penalty;
  const size_t ws_bytes = gtp_sample_workspace_bytes(dtype_code(logits), B, V, &p);
  void* ws = sampler_workspace(logits, ws_bytes, stream);
  const int rc = gtp_sample_rows(
      logits.data_ptr(), dtype_code(logits), B, V, row_stride_of(logits), hist, hist_len,
      hist_stride, mask, mask_stride, u, &p, fin, pad_token_id, ids.data_ptr<int64_t>(),
      lp.data_ptr<float>(), slp.data_ptr<float>(), kept.data_ptr<int32_t>(), tv.data_ptr<float>(),
      tid.data_ptr<int32_t>(), st.data_ptr<int32_t>(), ws, ws_bytes,
      reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_sample_rows");
  return {ids, lp, slp, kept, tv, tid, st};
}

// The kernel `sample` would run for these logits and parameters (with the
// workspace it would pass): (GTP_ROUTE_*, workgroups per row).
std::tuple<int64_t, int64_t> sample_route(const at::Tensor& logits, double temperature,
                                          int64_t top_k, double top_p, double repetition_penalty,
                                          int64_t hist_len, bool has_mask) {
  check_rows(logits, "logits");
  const int64_t B = logits.size(0), V = logits.size(1);
  TORCH_CHECK(B > 0 && V > 0 && V <= GTP_SAMPLER_MAX_V && top_k >= 0 && top_k <= INT32_MAX &&
                  hist_len >= 0,
              "graspo_tokpath.sample_route: bad shape or parameters");
  gtp_sampler_params p;
  p.temperature = (float)temperature;
  p.top_k = (int32_t)top_k;
  p.top_p = (float)top_p;
  p.repetition_penalty = (float)repetition_penalty;
  const int dt = dtype_code(logits);
  const size_t ws_bytes = gtp_sample_workspace_bytes(dt, B, V, &p);
  const int64_t es = logits.element_size();
  const bool aligned = (reinterpret_cast<uintptr_t>(logits.data_ptr()) & 15u) == 0 &&
                       ((uint64_t)(row_stride_of(logits) * es) & 15u) == 0;
  int32_t route = 0, slices = 0;
  check_rc(gtp_sample_route(dt, B, V, aligned ? 1 : 0, hist_len, has_mask ? 1 : 0, &p, ws_bytes,
                            &route, &slices),
           "gtp_sample_route");
  return {route, slices};
}

const void* targets_ptr(const at::Tensor& logits, const at::Tensor& targets, int64_t N,
                        int* is64) {
  check_same_device(logits, targets, "targets");
  TORCH_CHECK((targets.scalar_type() == at::kInt || targets.scalar_type() == at::kLong) &&
                  targets.dim() == 1 && targets.size(0) == N && targets.is_contiguous(),
              "graspo_tokpath: targets must be int32/int64 [N] contiguous");
  *is64 = targets.scalar_type() == at::kLong;
  return targets.data_ptr();
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> logprob_entropy(const at::Tensor& logits,
                                                               const at::Tensor& targets,
                                                               int64_t stream) {
  check_rows(logits, "logits");
  const int64_t N = logits.size(0), V = logits.size(1);
  TORCH_CHECK(V > 0, "graspo_tokpath.logprob_entropy: empty vocabulary");
  int t64 = 0;
  const void* tp = targets_ptr(logits, targets, N, &t64);
  auto opt = logits.options();
  at::Tensor lp = at::empty({N}, opt.dtype(at::kFloat));
  at::Tensor H = at::empty({N}, opt.dtype(at::kFloat));
  at::Tensor st = at::empty({N}, opt.dtype(at::kInt));
  const int rc = gtp_logprob_entropy_rows(logits.data_ptr(), dtype_code(logits), N, V,
                                          row_stride_of(logits), tp, t64, lp.data_ptr<float>(),
                                          H.data_ptr<float>(), st.data_ptr<int32_t>(),
                                          reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_logprob_entropy_rows");
  return {lp, H, st};
}

void lse_partial(const at::Tensor& logits, const c10::optional<at::Tensor>& targets,
                 int64_t col_offset, const at::Tensor& state, bool accumulate, int64_t stream) {
  check_rows(logits, "logits");
  const int64_t N = logits.size(0), Vc = logits.size(1);
  TORCH_CHECK(Vc > 0, "graspo_tokpath.lse_partial: empty chunk");
  check_same_device(logits, state, "state");
  TORCH_CHECK(state.scalar_type() == at::kFloat && state.dim() == 2 && state.size(0) == N &&
                  state.size(1) == 4 && state.is_contiguous(),
              "graspo_tokpath.lse_partial: state must be float32 [N, 4] contiguous");
  int t64 = 0;
  const void* tp = nullptr;
  if (targets.has_value()) tp = targets_ptr(logits, *targets, N, &t64);
  const int rc = gtp_lse_partial_rows(logits.data_ptr(), dtype_code(logits), N, Vc,
                                      row_stride_of(logits), col_offset, tp, t64,
                                      state.data_ptr<float>(), accumulate ? 1 : 0,
                                      reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_lse_partial_rows");
}

std::tuple<at::Tensor, at::Tensor> lse_finalize(const at::Tensor& state, int64_t stream) {
  TORCH_CHECK(state.is_cuda() && state.scalar_type() == at::kFloat && state.dim() == 2 &&
                  state.size(1) == 4 && state.is_contiguous(),
              "graspo_tokpath.lse_finalize: state must be a float32 [N, 4] GPU tensor");
  const int64_t N = state.size(0);
  at::Tensor lp = at::empty({N}, state.options());
  at::Tensor H = at::empty({N}, state.options());
  const int rc = gtp_lse_finalize_rows(state.data_ptr<float>(), N, lp.data_ptr<float>(),
                                       H.data_ptr<float>(), reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_lse_finalize_rows");
  return {lp, H};
}

at::Tensor logprob_backward(const at::Tensor& logits, const at::Tensor& targets,
                            const at::Tensor& grad_logprob, const at::Tensor& lse,
                            int64_t col_offset, const c10::optional<at::Tensor>& out,
                            int64_t stream) {
  check_rows(logits, "logits");
  const int64_t N = logits.size(0), V = logits.size(1);
  TORCH_CHECK(V > 0, "graspo_tokpath.logprob_backward: empty vocabulary");
  int t64 = 0;
  const void* tp = targets_ptr(logits, targets, N, &t64);
  for (const at::Tensor* t : {&grad_logprob, &lse}) {
    check_same_device(logits, *t, "grad_logprob / lse");
    TORCH_CHECK(t->scalar_type() == at::kFloat && t->dim() == 1 && t->size(0) == N &&
                    t->is_contiguous(),
                "graspo_tokpath.logprob_backward: grad_logprob and lse must be float32 [N] "
                "contiguous");
  }
  at::Tensor grad;
  if (out.has_value()) {
    grad = *out;
    check_same_device(logits, grad, "out");
    TORCH_CHECK(grad.scalar_type() == logits.scalar_type() && grad.dim() == 2 &&
                    grad.size(0) == N && grad.size(1) == V && (V == 1 || grad.stride(1) == 1) &&
                    grad.stride(0) >= V,
                "graspo_tokpath.logprob_backward: out must be [N, V] of the logits' dtype "
                "with unit column stride");
  } else {
    grad = at::empty({N, V}, logits.options());
  }
  const int64_t gstride = N > 1 ? grad.stride(0) : V;
  const int rc = gtp_logprob_backward_rows(
      logits.data_ptr(), dtype_code(logits), N, V, row_stride_of(logits), col_offset, tp, t64,
      grad_logprob.data_ptr<float>(), lse.data_ptr<float>(), grad.data_ptr(), gstride,
      reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_logprob_backward_rows");
  return grad;
}

void check_loss_input(const at::Tensor& t, const at::Tensor& ref, const char* name) {
  check_same_device(ref, t, name);
  TORCH_CHECK(t.scalar_type() == at::kFloat && t.is_contiguous() && t.sizes() == ref.sizes(),
              "graspo_tokpath.graspo_loss: ", name, " must be float32, contiguous, of the shape "
              "of log_probs");
}

// fp32 weights or bool / uint8 0-1 bytes, of the shape of log_probs
const void* loss_mask(const c10::optional<at::Tensor>& mask, const at::Tensor& logp, int* u8) {
  *u8 = 0;
  if (!mask.has_value()) return nullptr;
  const at::Tensor& m = *mask;
  check_same_device(logp, m, "action_mask");
  TORCH_CHECK((m.scalar_type() == at::kFloat || m.scalar_type() == at::kBool ||
               m.scalar_type() == at::kByte) &&
                  m.is_contiguous() && m.sizes() == logp.sizes(),
              "graspo_tokpath.graspo_loss: action_mask must be float32, bool or uint8, "
              "contiguous, of the shape of log_probs");
  *u8 = m.scalar_type() != at::kFloat;
  return m.data_ptr();
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> graspo_loss_forward(
    const at::Tensor& logp, const at::Tensor& old_logp, const at::Tensor& adv,
    const c10::optional<at::Tensor>& mask, double clip_lo, double clip_hi, int64_t stream) {
  TORCH_CHECK(logp.is_cuda() && logp.dim() == 2 && logp.size(0) > 0 && logp.size(1) > 0,
              "graspo_tokpath.graspo_loss: log_probs must be a non-empty [B, T] GPU tensor");
  check_loss_input(logp, logp, "log_probs");
  check_loss_input(old_logp, logp, "old_log_probs");
  check_loss_input(adv, logp, "advantages");
  int mu8 = 0;
  const void* mp = loss_mask(mask, logp, &mu8);
  const int64_t B = logp.size(0), T = logp.size(1);
  at::Tensor loss = at::empty({}, logp.options());
  at::Tensor per_seq = at::empty({B}, logp.options());
  at::Tensor inv_den = at::empty({B}, logp.options());
  const int rc = gtp_graspo_loss_forward(
      logp.data_ptr<float>(), old_logp.data_ptr<float>(), adv.data_ptr<float>(), mp, mu8, B, T,
      (float)clip_lo, (float)clip_hi, loss.data_ptr<float>(), per_seq.data_ptr<float>(),
      inv_den.data_ptr<float>(), reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_graspo_loss_forward");
  return {loss, per_seq, inv_den};
}

at::Tensor graspo_loss_backward(const at::Tensor& logp, const at::Tensor& old_logp,
                                const at::Tensor& adv, const c10::optional<at::Tensor>& mask,
                                const at::Tensor& inv_denom, const at::Tensor& grad_loss,
                                double clip_lo, double clip_hi, int64_t stream) {
  check_loss_input(old_logp, logp, "old_log_probs");
  check_loss_input(adv, logp, "advantages");
  int mu8 = 0;
  const void* mp = loss_mask(mask, logp, &mu8);
  const int64_t B = logp.size(0), T = logp.size(1);
  TORCH_CHECK(inv_denom.scalar_type() == at::kFloat && inv_denom.numel() == B &&
                  grad_loss.scalar_type() == at::kFloat && grad_loss.numel() == 1,
              "graspo_tokpath.graspo_loss_backward: bad inv_denom / grad_loss");
  at::Tensor grad = at::empty_like(logp);
  const int rc = gtp_graspo_loss_backward(
      logp.data_ptr<float>(), old_logp.data_ptr<float>(), adv.data_ptr<float>(), mp, mu8,
      inv_denom.data_ptr<float>(), grad_loss.data_ptr<float>(), B, T, (float)clip_lo,
      (float)clip_hi, grad.data_ptr<float>(), reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_graspo_loss_backward");
  return grad;
}

// one [B] byte flag tensor (bool or uint8) or a [B, >col] column target
uint8_t* byte_arg(const at::Tensor& t, const at::Tensor& ids, const char* name) {
  check_same_device(ids, t, name);
  TORCH_CHECK(t.scalar_type() == at::kBool || t.scalar_type() == at::kByte,
              "graspo_tokpath.decode_update: ", name, " must be bool or uint8");
  return static_cast<uint8_t*>(t.data_ptr());
}

void decode_update(const at::Tensor& ids, const c10::optional<at::Tensor>& status,
                   const at::Tensor& finished, int64_t eos_token_id, int64_t pad_token_id,
                   const c10::optional<at::Tensor>& seq, const c10::optional<at::Tensor>& attn,
                   int64_t col, const at::Tensor& flags, int64_t stream) {
  TORCH_CHECK(ids.is_cuda(), "graspo_tokpath.decode_update: ids must be a GPU tensor");
  TORCH_CHECK(ids.scalar_type() == at::kLong && ids.dim() == 1 && ids.is_contiguous(),
              "graspo_tokpath.decode_update: ids must be int64 [B]");
  const int64_t B = ids.size(0);
  TORCH_CHECK(finished.dim() == 1 && finished.size(0) == B && finished.is_contiguous(),
              "graspo_tokpath.decode_update: finished must be [B], contiguous");
  uint8_t* fin = byte_arg(finished, ids, "finished");
  const int32_t* st = nullptr;
  if (status.has_value()) {
    check_same_device(ids, *status, "status");
    TORCH_CHECK(status->scalar_type() == at::kInt && status->numel() == B && status->is_contiguous(),
                "graspo_tokpath.decode_update: status must be int32 [B]");
    st = status->data_ptr<int32_t>();
  }
  int64_t* sp = nullptr;
  int64_t s_stride = 0;
  if (seq.has_value()) {
    const auto& s = *seq;
    check_same_device(ids, s, "sequences");
    TORCH_CHECK(s.scalar_type() == at::kLong && s.dim() == 2 && s.size(0) == B &&
                    s.size(1) > col && (B <= 1 || s.stride(1) == 1),
                "graspo_tokpath.decode_update: sequences must be int64 [B, > col] with "
                "contiguous rows");
    sp = s.data_ptr<int64_t>();
    s_stride = B > 1 ? s.stride(0) : s.size(1);
  }
  uint8_t* ap = nullptr;
  int64_t a_stride = 0;
  if (attn.has_value()) {
    const auto& a = *attn;
    ap = byte_arg(a, ids, "attention_mask");
    TORCH_CHECK(a.dim() == 2 && a.size(0) == B && a.size(1) > col && (B <= 1 || a.stride(1) == 1),
                "graspo_tokpath.decode_update: attention_mask must be [B, > col] with contiguous "
                "rows");
    a_stride = B > 1 ? a.stride(0) : a.size(1);
  }
  check_same_device(ids, flags, "flags");
  TORCH_CHECK(flags.scalar_type() == at::kInt && flags.numel() >= 2 && flags.is_contiguous(),
              "graspo_tokpath.decode_update: flags must be int32 [2]");
  const int rc = gtp_decode_update_rows(ids.data_ptr<int64_t>(), st, B, eos_token_id,
                                        pad_token_id, fin, sp, s_stride, ap, a_stride, col,
                                        flags.data_ptr<int32_t>(), reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_decode_update_rows");
}

// (hi, lo) bf16 parts of the logprob gradient of fp32 logits [N, V]
std::tuple<at::Tensor, at::Tensor> logprob_backward_split(const at::Tensor& logits,
                                                          const at::Tensor& targets,
                                                          const at::Tensor& grad_logprob,
                                                          const at::Tensor& lse,
                                                          int64_t col_offset, int64_t stream) {
  check_rows(logits, "logits");
  TORCH_CHECK(logits.scalar_type() == at::kFloat,
              "graspo_tokpath.logprob_backward_split: logits must be float32");
  const int64_t N = logits.size(0), V = logits.size(1);
  check_same_device(logits, targets, "targets");
  check_same_device(logits, grad_logprob, "grad_logprob");
  check_same_device(logits, lse, "lse");
  TORCH_CHECK((targets.scalar_type() == at::kInt || targets.scalar_type() == at::kLong) &&
                  targets.numel() == N && targets.is_contiguous(),
              "graspo_tokpath.logprob_backward_split: targets must be int32/int64 [N]");
  TORCH_CHECK(grad_logprob.scalar_type() == at::kFloat && grad_logprob.numel() == N &&
                  grad_logprob.is_contiguous() && lse.scalar_type() == at::kFloat &&
                  lse.numel() == N && lse.is_contiguous(),
              "graspo_tokpath.logprob_backward_split: grad_logprob and lse must be float32 [N]");
  at::Tensor hi = at::empty({N, V}, logits.options().dtype(at::kBFloat16));
  at::Tensor lo = at::empty({N, V}, logits.options().dtype(at::kBFloat16));
  const int rc = gtp_logprob_backward_split_rows(
      logits.data_ptr<float>(), N, V, row_stride_of(logits), col_offset, targets.data_ptr(),
      targets.scalar_type() == at::kLong ? 1 : 0, grad_logprob.data_ptr<float>(),
      lse.data_ptr<float>(), static_cast<uint16_t*>(hi.data_ptr()),
      static_cast<uint16_t*>(lo.data_ptr()), V, reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_logprob_backward_split_rows");
  return {hi, lo};
}

// bf16 copy of a contiguous fp32 tensor, and whether any value was not a bf16
// value (a device flag the caller reads)
std::tuple<at::Tensor, at::Tensor> to_bf16_exact(const at::Tensor& src, int64_t stream) {
  TORCH_CHECK(src.is_cuda(), "graspo_tokpath.to_bf16_exact: src must be a GPU tensor");
  TORCH_CHECK(src.scalar_type() == at::kFloat && src.is_contiguous(),
              "graspo_tokpath.to_bf16_exact: src must be a contiguous float32 tensor");
  at::Tensor dst = at::empty(src.sizes(), src.options().dtype(at::kBFloat16));
  at::Tensor flag = at::zeros({1}, src.options().dtype(at::kInt));
  const int rc = gtp_f32_to_bf16_exact(src.data_ptr<float>(), src.numel(),
                                       static_cast<uint16_t*>(dst.data_ptr()),
                                       reinterpret_cast<uint32_t*>(flag.data_ptr<int32_t>()),
                                       reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_f32_to_bf16_exact");
  return {dst, flag};
}

}  // namespace

void time_next_launch(int64_t start_event, int64_t stop_event) {
  TORCH_CHECK(start_event != 0 && stop_event != 0,
              "graspo_tokpath.time_next_launch: both events must exist (record them once first)");
  check_rc(gtp_time_next_launch(reinterpret_cast<void*>(start_event),
                                reinterpret_cast<void*>(stop_event)),
           "gtp_time_next_launch");
}

// logprob / entropy / lse of h W^T rows without the [N, V] logits: bf16
// hidden [N, K] and weight [V, K] (rows contiguous, 16-byte aligned, K a
// multiple of 128), targets int32/int64 [N].
std::tuple<at::Tensor, at::Tensor, at::Tensor> lm_head_logprob(const at::Tensor& hidden,
                                                               const at::Tensor& weight,
                                                               const at::Tensor& targets,
                                                               int64_t stream) {
  for (const at::Tensor* t : {&hidden, &weight}) {
    TORCH_CHECK(t->is_cuda(), "graspo_tokpath.lm_head_logprob: hidden / weight must be GPU tensors");
    TORCH_CHECK(t->scalar_type() == at::kBFloat16 && t->dim() == 2 && t->stride(1) == 1,
                "graspo_tokpath.lm_head_logprob: hidden / weight must be bfloat16 2-D with "
                "contiguous rows");
  }
  check_same_device(hidden, weight, "weight");
  const int64_t N = hidden.size(0), K = hidden.size(1), V = weight.size(0);
  TORCH_CHECK(weight.size(1) == K, "graspo_tokpath.lm_head_logprob: hidden is [N, ", K,
              "] but weight is [V, ", weight.size(1), "]");
  int t64 = 0;
  const void* tp = targets_ptr(hidden, targets, N, &t64);
  at::Tensor lp = at::empty({N}, hidden.options().dtype(at::kFloat));
  at::Tensor H = at::empty({N}, lp.options());
  at::Tensor lse = at::empty({N}, lp.options());
  const size_t ws_bytes = gtp_lm_head_workspace_bytes(N, V);
  at::Tensor ws = at::empty({(int64_t)ws_bytes}, hidden.options().dtype(at::kByte));
  const int64_t ldh = N > 1 ? hidden.stride(0) : K, ldw = V > 1 ? weight.stride(0) : K;
  const int rc = gtp_lm_head_logprob_rows(
      reinterpret_cast<const uint16_t*>(hidden.data_ptr()), N, K, ldh,
      reinterpret_cast<const uint16_t*>(weight.data_ptr()), V, ldw, tp, t64, lp.data_ptr<float>(),
      H.data_ptr<float>(), lse.data_ptr<float>(), nullptr, ws.data_ptr(), ws_bytes,
      reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_lm_head_logprob_rows");
  return {lp, H, lse};
}

// lm_head_logprob that also keeps the fp32 logits, vocabulary-major [V, N],
// and returns the per-row status, for the backward.
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> lm_head_logprob_save(
    const at::Tensor& hidden, const at::Tensor& weight, const at::Tensor& targets,
    int64_t stream) {
  for (const at::Tensor* t : {&hidden, &weight}) {
    TORCH_CHECK(t->is_cuda(),
                "graspo_tokpath.lm_head_logprob_save: hidden / weight must be GPU tensors");
    TORCH_CHECK(t->scalar_type() == at::kBFloat16 && t->dim() == 2 && t->stride(1) == 1,
                "graspo_tokpath.lm_head_logprob_save: hidden / weight must be bfloat16 2-D "
                "with contiguous rows");
  }
  check_same_device(hidden, weight, "weight");
  const int64_t N = hidden.size(0), K = hidden.size(1), V = weight.size(0);
  TORCH_CHECK(weight.size(1) == K, "graspo_tokpath.lm_head_logprob_save: hidden is [N, ", K,
              "] but weight is [V, ", weight.size(1), "]");
  int t64 = 0;
  const void* tp = targets_ptr(hidden, targets, N, &t64);
  at::Tensor lp = at::empty({N}, hidden.options().dtype(at::kFloat));
  at::Tensor lse = at::empty({N}, lp.options());
  at::Tensor status = at::empty({N}, lp.options().dtype(at::kInt));
  at::Tensor logits_t = at::empty({V, N}, lp.options());
  const size_t ws_bytes = gtp_lm_head_workspace_bytes(N, V);
  at::Tensor ws = at::empty({(int64_t)ws_bytes}, hidden.options().dtype(at::kByte));
  const int64_t ldh = N > 1 ? hidden.stride(0) : K, ldw = V > 1 ? weight.stride(0) : K;
  const int rc = gtp_lm_head_logprob_save_rows(
      reinterpret_cast<const uint16_t*>(hidden.data_ptr()), N, K, ldh,
      reinterpret_cast<const uint16_t*>(weight.data_ptr()), V, ldw, tp, t64, lp.data_ptr<float>(),
      nullptr, lse.data_ptr<float>(), status.data_ptr<int32_t>(), logits_t.data_ptr<float>(),
      N, ws.data_ptr(), ws_bytes, reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_lm_head_logprob_save_rows");
  return {lp, lse, logits_t, status};
}

// bf16(-g * softmax) of vocabulary-major fp32 logits [V, N] (row stride
// free, unit column stride), g and lse fp32 [N]; returns ([V, N] bf16 or an
// empty tensor, [N, V] bf16 or an empty tensor) as `layouts` asks (1:
// vocabulary-major, 2: token-major, 3: both)
std::tuple<at::Tensor, at::Tensor> softmax_grad_bf16(const at::Tensor& logits_t,
                                                     const at::Tensor& grad_logprob,
                                                     const at::Tensor& lse, int64_t layouts,
                                                     int64_t stream) {
  TORCH_CHECK(logits_t.is_cuda() && logits_t.scalar_type() == at::kFloat && logits_t.dim() == 2 &&
                  (logits_t.size(1) <= 1 || logits_t.stride(1) == 1),
              "graspo_tokpath.softmax_grad_bf16: logits_t must be a float32 [V, N] GPU tensor "
              "with unit column stride");
  const int64_t V = logits_t.size(0), N = logits_t.size(1);
  check_same_device(logits_t, grad_logprob, "grad_logprob");
  check_same_device(logits_t, lse, "lse");
  TORCH_CHECK(grad_logprob.scalar_type() == at::kFloat && grad_logprob.numel() == N &&
                  grad_logprob.is_contiguous() && lse.scalar_type() == at::kFloat &&
                  lse.numel() == N && lse.is_contiguous(),
              "graspo_tokpath.softmax_grad_bf16: grad_logprob and lse must be float32 [N]");
  TORCH_CHECK(layouts >= 1 && layouts <= 3, "graspo_tokpath.softmax_grad_bf16: layouts must be 1, 2 or 3");
  const auto bf = logits_t.options().dtype(at::kBFloat16);
  at::Tensor out_t = (layouts & 1) ? at::empty({V, N}, bf) : at::empty({0}, bf);
  at::Tensor out_n = (layouts & 2) ? at::empty({N, V}, bf) : at::empty({0}, bf);
  if (V == 0 || N == 0) return {out_t, out_n};
  const int64_t ld = V > 1 ? logits_t.stride(0) : N;
  const int rc = gtp_softmax_grad_bf16_cols(
      logits_t.data_ptr<float>(), V, N, ld, grad_logprob.data_ptr<float>(),
      lse.data_ptr<float>(), (layouts & 1) ? static_cast<uint16_t*>(out_t.data_ptr()) : nullptr,
      N, (layouts & 2) ? static_cast<uint16_t*>(out_n.data_ptr()) : nullptr, V,
      reinterpret_cast<void*>(stream));
  check_rc(rc, "gtp_softmax_grad_bf16_cols");
  return {out_t, out_n};
}

TORCH_LIBRARY(graspo_tokpath, m) {
  m.def(
      "sample(Tensor logits, float temperature, int top_k, float top_p, float repetition_penalty, "
      "Tensor? history, Tensor? allow_mask, Tensor? uniforms, Tensor? finished, int pad_token_id, "
      "int stream) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
      &sample);
  m.def(
      "sample_route(Tensor logits, float temperature, int top_k, float top_p, "
      "float repetition_penalty, int hist_len, bool has_mask) -> (int, int)",
      &sample_route);
  m.def("logprob_entropy(Tensor logits, Tensor targets, int stream) -> (Tensor, Tensor, Tensor)",
        &logprob_entropy);
  m.def(
      "lse_partial(Tensor logits, Tensor? targets, int col_offset, Tensor(a!) state, "
      "bool accumulate, int stream) -> ()",
      &lse_partial);
  m.def("lse_finalize(Tensor state, int stream) -> (Tensor, Tensor)", &lse_finalize);
  m.def(
      "logprob_backward(Tensor logits, Tensor targets, Tensor grad_logprob, Tensor lse, "
      "int col_offset, Tensor(a!)? out, int stream) -> Tensor",
      &logprob_backward);
  m.def(
      "graspo_loss_forward(Tensor log_probs, Tensor old_log_probs, Tensor advantages, "
      "Tensor? action_mask, float clip_lo, float clip_hi, int stream) -> (Tensor, Tensor, Tensor)",
      &graspo_loss_forward);
  m.def(
      "graspo_loss_backward(Tensor log_probs, Tensor old_log_probs, Tensor advantages, "
      "Tensor? action_mask, Tensor inv_denom, Tensor grad_loss, float clip_lo, float clip_hi, "
      "int stream) -> Tensor",
      &graspo_loss_backward);
  m.def(
      "decode_update(Tensor(e!) ids, Tensor? status, Tensor(a!) finished, int eos_token_id, "
      "int pad_token_id, Tensor(b!)? sequences, Tensor(c!)? attention_mask, int col, "
      "Tensor(d!) flags, int stream) -> ()",
      &decode_update);
  m.def("to_bf16_exact(Tensor src, int stream) -> (Tensor, Tensor)", &to_bf16_exact);
  m.def("time_next_launch(int start_event, int stop_event) -> ()", &time_next_launch);
  m.def(
      "logprob_backward_split(Tensor logits, Tensor targets, Tensor grad_logprob, Tensor lse, "
      "int col_offset, int stream) -> (Tensor, Tensor)",
      &logprob_backward_split);
  m.def("lm_head_logprob(Tensor hidden, Tensor weight, Tensor targets, int stream) -> "
        "(Tensor, Tensor, Tensor)",
        &lm_head_logprob);
  m.def("lm_head_logprob_save(Tensor hidden, Tensor weight, Tensor targets, int stream) -> "
        "(Tensor, Tensor, Tensor, Tensor)",
        &lm_head_logprob_save);
  m.def("softmax_grad_bf16(Tensor logits_t, Tensor grad_logprob, Tensor lse, int layouts, int stream) -> (Tensor, Tensor)",
        &softmax_grad_bf16);
}
