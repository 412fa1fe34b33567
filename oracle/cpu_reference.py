"""The reference's CPU path, batched, for the bench's cpu_baseline leg --
TEST / MEASUREMENT INFRASTRUCTURE ONLY (never imported by graspo_amd).

A literal torch restatement of what the reference runs per decode step and
per loss step, on CPU tensors, in the reference's fp32:

* sampler: tensor_utils.py:649-683 (``logits / max(T, 1e-6)``, softmax,
  descending sort, cumsum, shifted ``cum > top_p`` cut, renormalise, draw),
  with the contract's extensions applied first (HF-style repetition penalty
  over the row's history ids, negative ids being padding; allow mask; top-k
  keeping exactly k tokens in (y desc, id asc) order) and
  ``torch.multinomial`` replaced by the inverse CDF of the supplied uniform;
* logprob: graspo_loss.py:19-21 (``log_softmax`` then ``gather``) plus the
  entropy of the same log-softmax.

The one sort of a row is stable and descending, so ties are ordered by
ascending id as the contract orders them; the reference's sort of the
softmax probabilities leaves equal probabilities in an unspecified order,
which only changes which of two equally likely tokens a uniform lands on.
"""

from __future__ import annotations

import torch


def penalised(x, history, repetition_penalty):
    """HF's ``RepetitionPenaltyLogitsProcessor`` rule (x < 0 ? x*rho : x/rho)
    once per distinct history id of each row; ids < 0 are padding and
    penalise nothing.  Every copy of a repeated id writes the same value,
    computed from the unpenalised logit."""
    h = history.long()
    valid = (h >= 0) & (h < x.shape[1])
    vals = x.gather(1, torch.where(valid, h, 0))
    pen = torch.where(vals < 0, vals * repetition_penalty, vals / repetition_penalty)
    rows = torch.arange(x.shape[0]).unsqueeze(1).expand_as(h)
    out = x.clone()
    out[rows[valid], h[valid]] = pen[valid]
    return out


def sample_rows(logits, *, temperature, top_k=0, top_p=1.0, repetition_penalty=1.0,
                history=None, allow_mask_bits=None, uniforms=None):
    x = logits.float()
    if history is not None and repetition_penalty != 1.0:
        x = penalised(x, history, repetition_penalty)
    if allow_mask_bits is not None:
        x = x.masked_fill(~allow_mask_bits, float("-inf"))
    if temperature <= 0:
        return x.argmax(dim=-1)
    x = x / max(float(temperature), 1e-6)
    if 0 < top_k < x.shape[1]:
        # exactly k tokens: every one above the k-th value, then the tokens
        # equal to it by ascending id; only those k are sorted.  torch.topk
        # keeps an arbitrary subset of a tie at the k-th value, so a row
        # whose tie is split takes its lowest ids instead.
        vals, cand = torch.topk(x, top_k, dim=-1)
        kth = vals[:, -1:]
        split = (x == kth).sum(dim=-1) != (vals == kth).sum(dim=-1)
        for b in split.nonzero().flatten().tolist():
            above = (x[b] > kth[b]).nonzero().flatten()
            ties = (x[b] == kth[b]).nonzero().flatten()[: top_k - above.numel()]
            cand[b] = torch.cat([above, ties])
        cand, _ = torch.sort(cand, dim=-1)  # ascending ids: the stable sort's tie order
        ys, order = torch.sort(x.gather(1, cand), dim=-1, descending=True, stable=True)
        sorted_idx = cand.gather(1, order)
    else:
        ys, sorted_idx = torch.sort(x, dim=-1, descending=True, stable=True)
    sorted_probs = torch.softmax(ys, dim=-1)
    if 0.0 < top_p < 1.0:
        cum = torch.cumsum(sorted_probs, dim=-1)
        remove = cum > top_p
        remove[..., 1:] = remove[..., :-1].clone()
        remove[..., 0] = False
        sorted_probs = sorted_probs.masked_fill(remove, 0.0)
    sorted_probs = sorted_probs / sorted_probs.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    cdf = torch.cumsum(sorted_probs, dim=-1)
    r = torch.searchsorted(cdf, uniforms.float().unsqueeze(1), right=True)
    # the last kept rank takes a uniform beyond the rounded cdf total
    kept = (sorted_probs > 0).sum(dim=-1, keepdim=True)
    r = torch.minimum(r, kept - 1)
    return sorted_idx.gather(1, r).squeeze(1)


def logprob_entropy_rows(logits, targets):
    ls = torch.log_softmax(logits.float(), dim=-1)
    lp = ls.gather(-1, targets.long().unsqueeze(-1)).squeeze(-1)
    ent = -(ls.exp() * ls).sum(-1)
    return lp, ent
