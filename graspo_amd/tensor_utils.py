"""Drop-ins for the hot-path helpers of
``src/graspo/backends/graspoflow/tensor_utils.py``.

Same names, same keyword-only signatures and the same return types as the
reference; the extra keywords default to "off", so existing call sites need
no edit.  All arithmetic runs in the gfx950 kernels of
``libgraspo_tokpath.so``; torch is used for allocation, the vocabulary-chunk
GEMMs of the hidden-state path, and the backward passes.
"""

from __future__ import annotations

import torch
import torch.distributed as dist
from torch.nn import functional as F  # noqa: N812

from . import ops


def _next_token_from_logits(
    logits: torch.Tensor,
    *,
    temperature: float,
    top_p: float,
    top_k: int = 0,
    repetition_penalty: float = 1.0,
    history: torch.Tensor | None = None,
    allow_mask: torch.Tensor | None = None,
    uniforms: torch.Tensor | None = None,
    generator: torch.Generator | None = None,
    check_status: bool = True,
) -> torch.Tensor:
    """Next token per row (reference: tensor_utils.py:649-658).

    ``temperature <= 0`` is greedy (argmax, lowest id on ties); otherwise the
    row is divided by ``max(temperature, 1e-6)`` and sampled under top-k /
    top-p from ``uniforms`` (drawn from torch's generator when omitted, as the
    reference's ``torch.multinomial`` does).  Returns int64 [B]."""
    out = ops.sample(
        logits,
        temperature=float(temperature),
        top_k=top_k,
        top_p=float(top_p),
        repetition_penalty=repetition_penalty,
        history=history,
        allow_mask=allow_mask,
        uniforms=uniforms,
        generator=generator,
    )
    if check_status:
        ops.raise_on_bad_status(out.status, "_next_token_from_logits")
    return out.ids


def _sample_next_token(
    logits: torch.Tensor,
    *,
    top_p: float,
    top_k: int = 0,
    uniforms: torch.Tensor | None = None,
    generator: torch.Generator | None = None,
    check_status: bool = True,
) -> torch.Tensor:
    """Sample from already temperature-scaled logits (reference:
    tensor_utils.py:671-683): softmax, top-p cut with the first token always
    kept, renormalise, draw.  Division by 1.0 is exact, so this is the
    sampler at temperature 1."""
    return _next_token_from_logits(
        logits, temperature=1.0, top_p=top_p, top_k=top_k, uniforms=uniforms,
        generator=generator, check_status=check_status,
    )


def _broadcast_and_pad_finished(
    next_token: torch.Tensor,
    finished: torch.Tensor,
    pad_token_id: int,
) -> torch.Tensor:
    """Rank 0's ids to every rank, then ``pad_token_id`` for finished rows
    (reference: tensor_utils.py:661-668).  On one GPU there is no broadcast;
    the sampler can also fold the padding itself (``finished=`` of
    :func:`graspo_amd.ops.sample`)."""
    if dist.is_available() and dist.is_initialized():
        dist.broadcast(next_token, src=0)
    return next_token.masked_fill(finished, pad_token_id)


# ------------------------------------------------------------- logprobs

class _SelectedLogProbsFromHidden(torch.autograd.Function):
    """log_softmax(h W^T)[target] without materialising [N, V] logits:
    vocabulary chunks of the GEMM are folded into a running (m, s) state by
    the lse kernel; the backward recomputes each chunk's softmax."""

    @staticmethod
    def forward(ctx, hidden, weight, output_ids, chunk):
        H = hidden.shape[-1]
        h2 = hidden.reshape(-1, H)
        t = output_ids.reshape(-1)
        N, V = h2.shape[0], weight.shape[0]
        state = ops.new_lse_state(N, hidden.device)
        for c, start in enumerate(range(0, V, chunk)):
            logits = F.linear(h2, weight[start : start + chunk])
            ops.lse_partial(logits, t, start, state, accumulate=c > 0)
        lp, _ = ops.lse_finalize(state)
        lse = state[:, 0] + torch.log(state[:, 1])
        ctx.save_for_backward(h2, weight, t, lse)
        ctx.chunk = chunk
        ctx.out_shape = output_ids.shape
        return lp.view(output_ids.shape)

    @staticmethod
    def backward(ctx, grad_out):
        h2, weight, t, lse = ctx.saved_tensors
        g = grad_out.reshape(-1).to(torch.float32)
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        grad_h = torch.zeros_like(h2) if need_h else None
        grad_w = torch.empty_like(weight) if need_w else None
        for start in range(0, weight.shape[0], ctx.chunk):
            w_c = weight[start : start + ctx.chunk]
            # g * (onehot - softmax) of this chunk's logits, one kernel pass
            gc = ops.logprob_backward(F.linear(h2, w_c), t, g, lse, col_offset=start)
            if need_h:
                grad_h += gc.to(h2.dtype) @ w_c.to(h2.dtype)
            if need_w:
                grad_w[start : start + ctx.chunk] = (gc.t() @ h2.to(gc.dtype)).to(weight.dtype)
        if grad_h is not None:
            grad_h = grad_h.view(*ctx.out_shape, h2.shape[-1])
        return grad_h, grad_w, None, None


def _selected_token_log_probs_from_hidden(
    hidden_states: torch.Tensor,
    lm_head_weight: torch.Tensor,
    output_ids: torch.Tensor,
    *,
    vocab_chunk_size: int = 32768,
) -> torch.Tensor:
    """logit[target] - logsumexp over the vocabulary, fp32 [*output_ids.shape]
    (reference: tensor_utils.py:167-186).  The chunk loop keeps the
    reference's ``vocab_chunk_size`` GEMMs; the logsumexp / logaddexp fold is
    the lse kernel.  Differentiable in ``hidden_states`` and
    ``lm_head_weight``."""
    return _SelectedLogProbsFromHidden.apply(
        hidden_states, lm_head_weight, output_ids, int(vocab_chunk_size)
    )
