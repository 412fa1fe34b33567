"""Tensor-level entry points of the gfx950 token path.

Each function validates nothing beyond what the native op checks, enqueues
the HIP kernels on the caller's current stream and returns device tensors;
none of them synchronises the host.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from . import load

ROW_OK, ROW_NONFINITE, ROW_EMPTY, ROW_BAD_HISTORY, ROW_BAD_UNIFORM, ROW_BAD_TARGET = range(6)
STATUS_NAMES = {
    ROW_OK: "ok",
    ROW_NONFINITE: "non-finite logits",
    ROW_EMPTY: "no allowed token",
    ROW_BAD_HISTORY: "history id >= V",
    ROW_BAD_UNIFORM: "uniform outside [0, 1)",
    ROW_BAD_TARGET: "target outside [0, V)",
}


class SampleOutput(NamedTuple):
    ids: torch.Tensor              # int64 [B]
    logprob: torch.Tensor          # fp32 [B], log_softmax(raw row)[id]
    sampled_logprob: torch.Tensor  # fp32 [B], log of the final sampling probability
    kept: torch.Tensor             # int32 [B], size of the kept (top-k/top-p) set
    thresh_value: torch.Tensor     # fp32 [B], processed logit of the last kept rank
    thresh_id: torch.Tensor        # int32 [B], id of the last kept rank
    status: torch.Tensor           # int32 [B], 0 = ok


def _stream(t: torch.Tensor) -> int:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"graspo_tokpath: tensors must be on a GPU (got {t.device}); there is no CPU path")
    return torch.cuda.current_stream(t.device).cuda_stream


def _as_rows(logits: torch.Tensor) -> torch.Tensor:
    if logits.dim() == 1:
        logits = logits.unsqueeze(0)
    if logits.dim() != 2:
        raise ValueError(f"expected [rows, V] logits, got shape {tuple(logits.shape)}")
    if logits.size(1) > 0 and logits.stride(1) != 1:
        logits = logits.contiguous()
    return logits


def draw_uniforms(batch: int, device, generator: torch.Generator | None = None) -> torch.Tensor:
    """U(0,1) draws on the 2^-24 grid from torch's generator (the same RNG
    stream the reference's torch.multinomial consumes, so a restored RNG state
    reproduces the draws)."""
    # randint's values do not depend on its dtype; fp32 holds k < 2^24
    # exactly, so this is (int32 k) * 2^-24 in two launches instead of three
    k = torch.randint(0, 1 << 24, (batch,), device=device, generator=generator,
                      dtype=torch.float32)
    return k.mul_(2.0 ** -24)


def sample(
    logits: torch.Tensor,
    *,
    temperature: float,
    top_k: int = 0,
    top_p: float = 1.0,
    repetition_penalty: float = 1.0,
    history: torch.Tensor | None = None,
    allow_mask: torch.Tensor | None = None,
    uniforms: torch.Tensor | None = None,
    finished: torch.Tensor | None = None,
    pad_token_id: int = 0,
    generator: torch.Generator | None = None,
) -> SampleOutput:
    """One token per row of ``logits`` [B, V] (bf16 / fp16 / fp32; rows may be
    strided, e.g. ``logits[:, -1, :]``).  See include/graspo_tokpath.h for the
    exact contract.  ``uniforms`` default to draws from torch's generator."""
    ops = load()
    logits = _as_rows(logits)
    B = logits.size(0)
    if temperature > 0 and uniforms is None:
        uniforms = draw_uniforms(B, logits.device, generator)
    if history is not None and history.dtype != torch.int32:
        history = history.to(torch.int32)
    if finished is not None and finished.dtype not in (torch.bool, torch.uint8):
        finished = finished.to(torch.bool)
    out = ops.sample(
        logits, float(temperature), int(top_k), float(top_p), float(repetition_penalty),
        history, allow_mask, uniforms, finished, int(pad_token_id), _stream(logits),
    )
    return SampleOutput(*out)


ROUTES = {1: "split top-k", 2: "split top-p", 3: "top-p", 4: "fp32 top-p",
          5: "value histogram", 6: "row-wise"}
ROUTE_SPLIT_TOPK, ROUTE_TOPP_SPLIT, ROUTE_TOPP, ROUTE_TOPP32, ROUTE_HIST, ROUTE_ROWWISE = range(1, 7)


def sample_route(logits: torch.Tensor, *, temperature: float, top_k: int = 0,
                 top_p: float = 1.0, repetition_penalty: float = 1.0, hist_len: int = 0,
                 has_mask: bool = False) -> tuple[int, int]:
    """(ROUTE_*, workgroups per row) of the kernel :func:`sample` would run for
    these logits and parameters (gtp_sample_route, with the workspace the op
    passes).  Host-only: launches nothing."""
    ops = load()
    logits = _as_rows(logits)
    return tuple(ops.sample_route(logits, float(temperature), int(top_k), float(top_p),
                                  float(repetition_penalty), int(hist_len), bool(has_mask)))


def logprob_entropy(logits: torch.Tensor, targets: torch.Tensor):
    """(logprob, entropy, status) per row of ``logits`` [N, V]; one HBM read."""
    ops = load()
    logits = _as_rows(logits)
    targets = targets.reshape(-1)
    if targets.dtype not in (torch.int32, torch.int64):
        targets = targets.to(torch.int64)
    return ops.logprob_entropy(logits, targets.contiguous(), _stream(logits))


def logprob_backward(logits: torch.Tensor, targets: torch.Tensor, grad_logprob: torch.Tensor,
                     lse: torch.Tensor, col_offset: int = 0,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """d/dlogits of sum_n grad_logprob[n] * log_softmax(logits[n])[targets[n]]:
    g * (onehot - softmax) in the logits' dtype, [N, V] (written into ``out``
    when given: [N, V], unit column stride).  ``lse`` is each row's
    log-sum-exp over the whole vocabulary; for a vocabulary chunk pass its
    first column as ``col_offset``.  Rows with g == 0 are zeros (not read)."""
    ops = load()
    logits = _as_rows(logits)
    targets = targets.reshape(-1)
    if targets.dtype not in (torch.int32, torch.int64):
        targets = targets.to(torch.int64)
    return ops.logprob_backward(
        logits, targets.contiguous(), grad_logprob.reshape(-1).to(torch.float32).contiguous(),
        lse.reshape(-1).to(torch.float32).contiguous(), int(col_offset), out, _stream(logits))


def logprob_backward_split(logits: torch.Tensor, targets: torch.Tensor,
                           grad_logprob: torch.Tensor, lse: torch.Tensor, col_offset: int = 0):
    """The logprob gradient of fp32 ``logits`` [N, V] as two bf16 [N, V]
    tensors (hi, lo) with |grad - hi - lo| <= 2^-16 |grad|."""
    ops = load()
    logits = _as_rows(logits)
    targets = targets.reshape(-1)
    if targets.dtype not in (torch.int32, torch.int64):
        targets = targets.to(torch.int64)
    return ops.logprob_backward_split(
        logits, targets.contiguous(), grad_logprob.reshape(-1).to(torch.float32).contiguous(),
        lse.reshape(-1).to(torch.float32).contiguous(), int(col_offset), _stream(logits))


def graspo_loss_forward(log_probs: torch.Tensor, old_log_probs: torch.Tensor,
                        advantages: torch.Tensor, action_mask: torch.Tensor | None,
                        clip_lo: float, clip_hi: float):
    """(loss, per-sequence masked means, 1 / max(1, mask sums)) of the
    GRASPO PPO-clip surrogate over fp32 [B, T] inputs."""
    ops = load()
    return ops.graspo_loss_forward(log_probs, old_log_probs, advantages, action_mask,
                                   float(clip_lo), float(clip_hi), _stream(log_probs))


def graspo_loss_backward(log_probs, old_log_probs, advantages, action_mask, inv_denom,
                         grad_loss, clip_lo: float, clip_hi: float) -> torch.Tensor:
    """d(loss)/d(log_probs) scaled by ``grad_loss`` (a 1-element fp32 tensor)."""
    ops = load()
    return ops.graspo_loss_backward(log_probs, old_log_probs, advantages, action_mask, inv_denom,
                                    grad_loss, float(clip_lo), float(clip_hi),
                                    _stream(log_probs))


def lse_partial(logits_chunk: torch.Tensor, targets: torch.Tensor | None, col_offset: int,
                state: torch.Tensor, accumulate: bool) -> None:
    """Fold a vocabulary chunk into the running (m, s, t, x_target) row state."""
    ops = load()
    logits_chunk = _as_rows(logits_chunk)
    if targets is not None:
        targets = targets.reshape(-1).contiguous()
    ops.lse_partial(logits_chunk, targets, int(col_offset), state, bool(accumulate),
                    _stream(logits_chunk))


def lse_finalize(state: torch.Tensor):
    """(logprob, entropy) from a chunk state."""
    ops = load()
    return ops.lse_finalize(state, _stream(state))


def lm_head_supported(hidden: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether lm_head_logprob takes these bf16 operands: 2-D with contiguous,
    16-byte aligned rows, K a multiple of 128 and row strides below 2^22."""
    ok = (hidden.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and hidden.dim() == 2
          and weight.dim() == 2 and hidden.size(1) == weight.size(1) and hidden.size(1) % 128 == 0
          and hidden.size(1) > 0 and weight.size(0) > 0)
    for t in (hidden, weight):
        ok = ok and t.stride(1) == 1 and t.data_ptr() % 16 == 0
        ok = ok and (t.size(0) <= 1 or (t.stride(0) % 8 == 0 and t.stride(0) < (1 << 22)))
    return bool(ok)


def lm_head_logprob(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor):
    """(logprob, entropy, lse) [N] fp32 of the logits ``hidden @ weight.T``
    without writing them: the bf16 GEMM on the matrix cores with the
    log-sum-exp in its epilogue (bf16 ``hidden`` [N, K], ``weight`` [V, K],
    ``lm_head_supported`` true)."""
    ops = load()
    targets = targets.reshape(-1).contiguous()
    return ops.lm_head_logprob(hidden, weight, targets, _stream(hidden))


def lm_head_logprob_save(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor):
    """(logprob, lse, logits_t, status) of ``hidden @ weight.T``: the fused
    kernel of :func:`lm_head_logprob` that also writes the fp32 logits,
    vocabulary-major (``logits_t`` [V, N] = the logits transposed), for the
    backward, and the per-row status (a target outside [0, V) is
    ``ROW_BAD_TARGET``)."""
    ops = load()
    targets = targets.reshape(-1).contiguous()
    return ops.lm_head_logprob_save(hidden, weight, targets, _stream(hidden))


def softmax_grad_bf16(logits_t: torch.Tensor, grad_logprob: torch.Tensor, lse: torch.Tensor,
                      *, vocab_major: bool = True, token_major: bool = False):
    """bf16 -g_n * softmax(logits[n]) for vocabulary-major fp32 ``logits_t``
    [V, N] (unit column stride; ``lse`` each token's log-sum-exp): the
    gradient of g * log_softmax(logits)[t] without its one-hot term
    g * [v == t].  Returns ``(grad_t [V, N], grad [N, V])``, each written
    when asked for (None otherwise), both from one read of the logits."""
    if not (vocab_major or token_major):
        raise ValueError("softmax_grad_bf16: ask for at least one layout")
    ops = load()
    gt, gn = ops.softmax_grad_bf16(
        logits_t, grad_logprob.reshape(-1).to(torch.float32).contiguous(),
        lse.reshape(-1).to(torch.float32).contiguous(),
        (1 if vocab_major else 0) | (2 if token_major else 0), _stream(logits_t))
    return (gt if vocab_major else None), (gn if token_major else None)


def decode_update(ids: torch.Tensor, status: torch.Tensor | None, finished: torch.Tensor,
                  eos_token_id: int, pad_token_id: int, sequences: torch.Tensor | None,
                  attention_mask: torch.Tensor | None, col: int, flags: torch.Tensor) -> None:
    """After a sampler step: ``sequences[:, col] = ids``,
    ``attention_mask[:, col] = ids != pad``, ``finished |= ids == eos`` (in
    place) and ``flags = [rows still unfinished, rows with a bad status]``
    (int32 [2]), in one launch.  Rows with a bad status get ``pad_token_id``
    in ``ids`` (in place) as well as in the two columns."""
    ops = load()
    ops.decode_update(ids, status, finished, int(eos_token_id), int(pad_token_id), sequences,
                      attention_mask, int(col), flags, _stream(ids))


def to_bf16_exact(src: torch.Tensor):
    """(bf16 copy, inexact) of a contiguous fp32 GPU tensor: the copy holds the
    upper 16 bits of each value, and ``inexact`` (int32 [1], on the device) is
    nonzero when some value is not a bf16 value."""
    ops = load()
    return ops.to_bf16_exact(src.contiguous(), _stream(src))


def time_next_launch(start: torch.cuda.Event, stop: torch.cuda.Event) -> None:
    """Measurement hook: the next sampler, logprob or logprob-gradient kernel
    launched from this thread records ``start`` and ``stop`` (timing events
    that have been recorded once, so that they exist) at its own dispatch's
    start and end."""
    ops = load()
    ops.time_next_launch(int(start.cuda_event), int(stop.cuda_event))


def new_lse_state(rows: int, device) -> torch.Tensor:
    return torch.empty((rows, 4), dtype=torch.float32, device=device)


def raise_on_bad_status(status: torch.Tensor, what: str) -> None:
    """Host check (one device sync) mirroring the reference's errors on
    invalid rows (torch.multinomial rejects NaN/inf probabilities)."""
    bad = status.ne(ROW_OK)
    if bool(bad.any()):
        codes = sorted({int(c) for c in status[bad].tolist()})
        rows = bad.nonzero().flatten()[:8].tolist()
        names = ", ".join(STATUS_NAMES.get(c, str(c)) for c in codes)
        raise RuntimeError(f"{what}: invalid rows {rows} ({names})")
