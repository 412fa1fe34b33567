"""The reference's CPU path, batched, for the bench's cpu_baseline leg --
TEST / MEASUREMENT INFRASTRUCTURE ONLY (never imported by graspo_amd).

A literal torch restatement of what the reference runs per decode step and
per loss step, on CPU tensors:

* sampler: tensor_utils.py:649-683 (``logits / max(T, 1e-6)``, softmax,
  descending sort, cumsum, shifted ``cum > top_p`` cut, renormalise, draw),
  with the contract's extensions applied first (HF-style repetition penalty,
  allow mask, top-k) and ``torch.multinomial`` replaced by the inverse CDF of
  the supplied uniform;
* logprob: graspo_loss.py:19-21 (``log_softmax`` then ``gather``) plus the
  entropy of the same log-softmax.
"""

from __future__ import annotations

import torch


def sample_rows(logits, *, temperature, top_k=0, top_p=1.0, repetition_penalty=1.0,
                history=None, allow_mask_bits=None, uniforms=None):
    x = logits.float()
    if history is not None and repetition_penalty != 1.0:
        h = history.long().clamp_min(0)
        vals = x.gather(1, h)
        vals = torch.where(vals < 0, vals * repetition_penalty, vals / repetition_penalty)
        x = x.scatter(1, h, vals)
    if allow_mask_bits is not None:
        x = x.masked_fill(~allow_mask_bits, float("-inf"))
    if temperature <= 0:
        return x.argmax(dim=-1)
    x = x / max(float(temperature), 1e-6)
    if top_k > 0:
        kth = torch.topk(x, top_k, dim=-1).values[:, -1:]
        x = x.masked_fill(x < kth, float("-inf"))
    probs = torch.softmax(x, dim=-1)
    sorted_probs, sorted_idx = torch.sort(probs, descending=True, dim=-1)
    if 0.0 < top_p < 1.0:
        cum = torch.cumsum(sorted_probs, dim=-1)
        remove = cum > top_p
        remove[..., 1:] = remove[..., :-1].clone()
        remove[..., 0] = False
        sorted_probs = sorted_probs.masked_fill(remove, 0.0)
    sorted_probs = sorted_probs / sorted_probs.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    cdf = torch.cumsum(sorted_probs, dim=-1)
    r = torch.searchsorted(cdf, uniforms.float().unsqueeze(1), right=True).clamp_max(
        cdf.shape[1] - 1)
    return sorted_idx.gather(1, r).squeeze(1)


def logprob_entropy_rows(logits, targets):
    ls = torch.log_softmax(logits.float(), dim=-1)
    lp = ls.gather(-1, targets.long().unsqueeze(-1)).squeeze(-1)
    ent = -(ls.exp() * ls).sum(-1)
    return lp, ent
