"""Drop-ins for ``src/graspo/core/graspo_loss.py``.

``sequence_log_probs_from_logits`` runs the logprob kernel (one read of the
logits, no [N, V] log-softmax written); ``masked_mean`` and ``GRASPOLoss``
are the consumers of its output, kept as small torch expressions.
"""

from __future__ import annotations

import numpy as np
import torch
from torch import nn

from . import ops


def _rows_logprob_entropy_status(logits: torch.Tensor, output_ids: torch.Tensor):
    """(logprob, entropy, status) over the last dim of ``logits`` [..., V];
    views whose leading dims cannot be flattened without a copy are walked
    per slice."""
    V = logits.shape[-1]
    lead = logits.shape[:-1]
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    try:
        rows = logits.view(-1, V)
    except RuntimeError:
        rows = None
    if rows is not None:
        lp, H, st = ops.logprob_entropy(rows, output_ids.reshape(-1))
        return lp.view(lead), H.view(lead), st.view(lead)
    parts = [_rows_logprob_entropy_status(logits[i], output_ids[i])
             for i in range(logits.shape[0])]
    return tuple(torch.stack(p) for p in zip(*parts))


def _rows_logprob_entropy(logits: torch.Tensor, output_ids: torch.Tensor):
    """(logprob, entropy); a target outside [0, V) raises ``RuntimeError``, as
    the reference's ``gather`` rejects such an index (one host
    synchronisation on the per-row status)."""
    lp, H, st = _rows_logprob_entropy_status(logits, output_ids)
    ops.raise_on_bad_status(st.reshape(-1), "sequence_log_probs_from_logits")
    return lp, H


class _SequenceLogProbs(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, output_ids):
        lp, _ = _rows_logprob_entropy(logits, output_ids)
        ctx.save_for_backward(logits, output_ids, lp)
        return lp

    @staticmethod
    def backward(ctx, grad_out):
        logits, output_ids, lp = ctx.saved_tensors
        # d logprob_t / d x = onehot(t) - softmax(x), with softmax from the
        # saved lse = x_t - logprob_t: one read of the logits, one write
        V = logits.shape[-1]
        rows = logits.reshape(-1, V)
        t = output_ids.reshape(-1).to(torch.int64)
        lse = rows.gather(1, t.unsqueeze(1)).squeeze(1).float() - lp.reshape(-1)
        grad = ops.logprob_backward(rows, t, grad_out.reshape(-1), lse)
        return grad.view(logits.shape), None


def sequence_log_probs_from_logits(logits: torch.Tensor, output_ids: torch.Tensor) -> torch.Tensor:
    """log_softmax(logits)[output_ids] in fp32 (reference: graspo_loss.py:19-21).
    Accepts fp32, bf16 or fp16 logits of shape [..., V]; differentiable."""
    if logits.requires_grad and torch.is_grad_enabled():
        return _SequenceLogProbs.apply(logits, output_ids)
    lp, _ = _rows_logprob_entropy(logits, output_ids)
    return lp


def sequence_log_probs_and_entropy_from_logits(
    logits: torch.Tensor, output_ids: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """(logprob, entropy) from the same single read of the logits (no grad)."""
    return _rows_logprob_entropy(logits, output_ids)


def masked_mean(
    tensor: torch.Tensor, mask: torch.Tensor | None, dim: int | None = None
) -> torch.Tensor:
    """Mean of ``tensor`` over positions where ``mask`` holds, at least one
    position counted per reduction (reference: graspo_loss.py:10-16)."""
    if mask is None:
        return tensor.mean(dim=dim)
    weights = mask.to(tensor.dtype)
    return (tensor * weights).sum(dim=dim) / mask.sum(dim=dim).clamp_min(1)


class _GRASPOLossFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, log_probs, old_log_probs, advantages, action_mask, clip_lo, clip_hi):
        loss, _, inv_denom = ops.graspo_loss_forward(
            log_probs, old_log_probs, advantages, action_mask, clip_lo, clip_hi)
        ctx.save_for_backward(log_probs, old_log_probs, advantages, action_mask, inv_denom)
        ctx.clip = (clip_lo, clip_hi)
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        log_probs, old_log_probs, advantages, action_mask, inv_denom = ctx.saved_tensors
        grad = None
        if ctx.needs_input_grad[0]:
            grad = ops.graspo_loss_backward(
                log_probs, old_log_probs, advantages, action_mask, inv_denom,
                grad_loss.reshape(1).float().contiguous(), *ctx.clip)
        return grad, None, None, None, None, None


class GRASPOLoss(nn.Module):
    """PPO-clip surrogate over token logprobs (reference: graspo_loss.py:45-63):
    -min(r A, clip(r, 1-eps, 1+eps) A) with r = exp(logp - logp_old), averaged
    per sequence over the action mask (masked_mean, graspo_loss.py:10-16),
    then over sequences.  Two fused kernels forward, one backward (d/dlogp
    only: the old logprobs, advantages and mask are data, as in every
    reference call site)."""

    def __init__(self, policy_ratio_clip_eps: float = 0.2) -> None:
        super().__init__()
        self.policy_ratio_clip_eps = policy_ratio_clip_eps

    def forward(
        self,
        log_probs: torch.Tensor,
        old_log_probs: torch.Tensor,
        advantages: torch.Tensor,
        action_mask: torch.Tensor | None,
    ) -> torch.Tensor:
        eps = self.policy_ratio_clip_eps
        # torch rounds the Python bounds 1 -/+ eps to fp32 the same way
        lo, hi = float(np.float32(1.0 - eps)), float(np.float32(1.0 + eps))
        T = log_probs.shape[-1]
        shape = log_probs.shape
        lp = log_probs.reshape(-1, T)
        dt = lp.dtype

        def rows(t, keep_dtype=False):
            t = torch.broadcast_to(t, shape).reshape(-1, T)
            return (t if keep_dtype else t.float()).contiguous()

        mask = None
        if action_mask is not None:
            mask = rows(action_mask, keep_dtype=action_mask.dtype in (torch.bool, torch.uint8))
        loss = _GRASPOLossFn.apply(lp.float().contiguous(), rows(old_log_probs.detach()),
                                   rows(advantages.detach()), mask, lo, hi)
        return loss.to(dt)
