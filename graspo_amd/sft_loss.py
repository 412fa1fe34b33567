"""Drop-in for ``src/graspo/core/sft_loss.py``.

``sft_cross_entropy_loss`` is the mean token cross-entropy of the shifted
logits over the labels that are not ``ignore_index``, as
``F.cross_entropy(..., ignore_index=...)`` computes it in the reference
(sft_loss.py:12-34), without materialising the shifted copy or the [N, V]
softmax: the forward is the logprob kernel (one read of the logits), the
backward the logprob-gradient kernel (one read, one write).
"""

from __future__ import annotations

import torch

from . import ops


class _SFTCrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, labels, ignore_index):
        B, S, V = logits.shape
        tgt = labels[:, 1:]
        valid = tgt.ne(ignore_index)
        safe = torch.where(valid, tgt, torch.zeros_like(tgt)).to(torch.int64)
        lp = torch.empty((B, S - 1), dtype=torch.float32, device=logits.device)
        bad = torch.zeros((), dtype=torch.bool, device=logits.device)
        for b in range(B):  # the S - 1 rows of one sequence share one row stride
            lp_b, _, st_b = ops.logprob_entropy(logits[b, : S - 1], safe[b])
            lp[b] = lp_b
            bad |= st_b.ne(ops.ROW_OK).any()
        if bool(bad):  # F.cross_entropy rejects a label outside [0, V)
            raise RuntimeError("sft_cross_entropy_loss: a label is outside [0, vocab_size)")
        count = valid.sum()
        loss = -(lp * valid).sum() / count
        ctx.save_for_backward(logits, safe, valid, lp, count)
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        logits, safe, valid, lp, count = ctx.saved_tensors
        B, S, V = logits.shape
        g = torch.where(valid, -grad_loss.float() / count, torch.zeros_like(lp))
        grad = torch.empty_like(logits, memory_format=torch.contiguous_format)
        grad[:, S - 1].zero_()
        for b in range(B):
            rows = logits[b, : S - 1]
            lse = rows.gather(1, safe[b].unsqueeze(1)).squeeze(1).float() - lp[b]
            ops.logprob_backward(rows, safe[b], g[b], lse, out=grad[b, : S - 1])
        return grad, None, None


def sft_cross_entropy_loss(
    logits: torch.Tensor,
    labels: torch.Tensor,
    *,
    ignore_index: int = -100,
) -> torch.Tensor:
    """Mean cross-entropy of ``logits[:, :-1]`` against ``labels[:, 1:]``,
    skipping ``ignore_index`` (reference: sft_loss.py:12-34).  ``logits`` is
    [B, S, V] in fp32, bf16 or fp16; the loss is an fp32 scalar."""
    if logits.dim() != 3 or labels.shape != logits.shape[:2]:
        raise ValueError(
            f"expected logits [B, S, V] and labels [B, S], got {tuple(logits.shape)} and "
            f"{tuple(labels.shape)}")
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    return _SFTCrossEntropy.apply(logits, labels, int(ignore_index))
