"""Drop-ins for ``src/graspo/core/graspo_loss.py``.

``sequence_log_probs_from_logits`` runs the logprob kernel (one read of the
logits, no [N, V] log-softmax written); ``masked_mean`` and ``GRASPOLoss``
are the consumers of its output, kept as small torch expressions.
"""

from __future__ import annotations

import torch
from torch import nn

from . import ops


def _rows_logprob_entropy(logits: torch.Tensor, output_ids: torch.Tensor):
    """(logprob, entropy) over the last dim of ``logits`` [..., V]; views whose
    leading dims cannot be flattened without a copy are walked per slice."""
    V = logits.shape[-1]
    lead = logits.shape[:-1]
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    try:
        rows = logits.view(-1, V)
    except RuntimeError:
        rows = None
    if rows is not None:
        lp, H, _ = ops.logprob_entropy(rows, output_ids.reshape(-1))
        return lp.view(lead), H.view(lead)
    lps, Hs = [], []
    for i in range(logits.shape[0]):
        lp_i, H_i = _rows_logprob_entropy(logits[i], output_ids[i])
        lps.append(lp_i)
        Hs.append(H_i)
    return torch.stack(lps), torch.stack(Hs)


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


class GRASPOLoss(nn.Module):
    """PPO-clip surrogate over token logprobs (reference: graspo_loss.py:45-63):
    -min(r A, clip(r, 1-eps, 1+eps) A) with r = exp(logp - logp_old), averaged
    per sequence over the action mask, then over sequences."""

    def __init__(self, policy_ratio_clip_eps: float = 0.2) -> None:
        super().__init__()
        self.policy_ratio_clip_eps = policy_ratio_clip_eps

    def forward(
        self,
        log_probs: torch.Tensor,
        old_log_probs: torch.Tensor,
        advantages: torch.Tensor,
        action_mask: torch.Tensor,
    ) -> torch.Tensor:
        eps = self.policy_ratio_clip_eps
        ratio = torch.exp(log_probs - old_log_probs)
        unclipped = ratio * advantages
        clipped = torch.clamp(ratio, 1.0 - eps, 1.0 + eps) * advantages
        per_token = -torch.minimum(unclipped, clipped)
        return masked_mean(per_token, action_mask, dim=-1).mean()
