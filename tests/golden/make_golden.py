"""Write the golden fixtures of the token path (run once, offline, on CPU):

    python tests/golden/make_golden.py

Expected outputs come from library routines and the reference's own rule,
not from this repository's oracle:

* repetition penalty: transformers' ``RepetitionPenaltyLogitsProcessor``
  (transformers/generation/logits_process.py, the rule the sampler contract
  extends the reference with), applied per row over the row's history ids;
* ordering and top-k: ``torch.sort(descending=True, stable=True)`` of the
  fp32 processed logits (ties by ascending id, ``torch.argmax``'s first-index
  rule for greedy rows, as in src/graspo/backends/graspoflow/tensor_utils.py:658);
* top-p cut: the reference's rule (tensor_utils.py:671-683: softmax, descending
  sort, cumsum, remove ``cum > top_p`` shifted right by one) evaluated in fp64;
* draw: inverse CDF of the supplied uniform over the renormalised kept set in
  fp64 (the reference calls ``torch.multinomial``; the contract replaces its
  global-RNG draw by a supplied uniform);
* sampled logprob: ``log`` of the drawn token's fp64 probability in that
  renormalised kept set (tensor_utils.py:679-683), 0 for greedy rows;
* logprob / entropy: ``torch.log_softmax`` in fp64.

Uniforms are moved, and top-p values chosen, so that every fp64 cumulative
boundary is at least 1e-6 away (any exact evaluation then agrees).  Each
fixture is an ``.npz`` (no pickles) holding the inputs and expected outputs.
"""

from __future__ import annotations

import os

import numpy as np
import torch
from transformers.generation.logits_process import RepetitionPenaltyLogitsProcessor

HERE = os.path.dirname(os.path.abspath(__file__))
MARGIN = 1e-6


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()


def bf16_values(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy((bits.astype(np.uint32) << 16).view(np.float32).copy())


def pack_bits(bits: np.ndarray) -> np.ndarray:
    B, V = bits.shape
    W = (V + 31) // 32
    out = np.zeros((B, W), np.uint32)
    for i in range(32):
        col = bits[:, i::32].astype(np.uint32)
        out[:, : col.shape[1]] |= col << np.uint32(i)
    return out.view(np.int32)


def expected_row(x: torch.Tensor, hist, rho, allowed, T, k, P, u):
    """(id, kept, thresh_value, thresh_id, logprob, sampled_logprob, u_used)
    of one row, or None when a top-p boundary lies within MARGIN of P."""
    V = x.numel()
    xp = x.clone()
    if hist is not None and rho != 1.0:
        ids = torch.from_numpy(hist[hist >= 0].astype(np.int64)).view(1, -1)
        if ids.numel():
            xp = RepetitionPenaltyLogitsProcessor(penalty=rho)(ids, xp.view(1, -1)).view(-1)
    if allowed is not None:
        xp = torch.where(torch.from_numpy(allowed), xp, torch.tensor(float("-inf")))
    lsm = torch.log_softmax(x.double(), 0)
    if not (T > 0):
        i = int(torch.argmax(xp))
        return i, 1, float(xp[i]), i, float(lsm[i]), 0.0, u
    y = xp / max(T, 1e-6)  # one IEEE fp32 division
    ys, order = torch.sort(y, descending=True, stable=True)
    n_valid = int(torch.isfinite(ys).sum())
    ys, order = ys[:n_valid], order[:n_valid]
    if 0 < k < n_valid:
        ys, order = ys[:k], order[:k]
    p = torch.exp(ys.double() - ys[0].double())
    p = p / p.sum()
    if 0.0 < P < 1.0:
        before = torch.cumsum(p, 0) - p
        if float((before - P).abs().min()) < MARGIN:
            return None
        keep = int((before <= P).sum())
        ys, order, p = ys[:keep], order[:keep], p[:keep]
        p = p / p.sum()
    cum = torch.cumsum(p, 0)
    cum[-1] = 1.0
    while float((cum - u).abs().min()) < MARGIN:
        u = float(np.float32(u + 2.0 ** -12)) % 1.0
    r = int((cum <= u).sum())
    i = int(order[r])
    return (i, int(order.numel()), float(ys[-1]), int(order[-1]), float(lsm[i]),
            float(torch.log(p[r])), u)


def sampler_case(name, seed, B, V, *, scale, T, k, P, rho=1.0, hist_len=0, density=None,
                 ties=False):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    x = torch.randn(B, V, generator=g) * scale
    if ties:
        x[: B // 2] = torch.round(x[: B // 2] * 2) / 2  # exact ties in half the rows
    bits = bf16_bits(x)
    xv = bf16_values(bits)
    hist = rng.integers(-1, V, (B, hist_len)).astype(np.int32) if hist_len else None
    allowed = None
    if density is not None:
        allowed = rng.random((B, V)) < density
        allowed[:, rng.integers(0, V, 20)] = True
        allowed[-1] = False
        allowed[-1, int(rng.integers(0, V))] = True  # one row with a single allowed token
    u = (rng.integers(0, 1 << 24, B) * 2.0 ** -24).astype(np.float32)
    exp = {n: [] for n in ("ids", "kept", "thresh_value", "thresh_id", "logprob",
                           "sampled_logprob")}
    for b in range(B):
        r = None
        while r is None:
            r = expected_row(xv[b], None if hist is None else hist[b], rho,
                             None if allowed is None else allowed[b], T, k, P, float(u[b]))
            if r is None:  # move the row's largest logit one bf16 step: new boundaries
                j = int(torch.argmax(xv[b]))
                bits[b, j] += 1
                xv[b] = bf16_values(bits[b : b + 1])[0]
        i, kept, tv, tid, lp, slp, u_used = r
        u[b] = u_used
        for n, v in zip(exp, (i, kept, tv, tid, lp, slp)):
            exp[n].append(v)
    arrays = dict(
        logits_bf16=bits, V=np.int64(V), temperature=np.float32(T), top_k=np.int32(k),
        top_p=np.float32(P), repetition_penalty=np.float32(rho), uniforms=u,
        exp_ids=np.array(exp["ids"], np.int64), exp_kept=np.array(exp["kept"], np.int32),
        exp_thresh_value=np.array(exp["thresh_value"], np.float32),
        exp_thresh_id=np.array(exp["thresh_id"], np.int32),
        exp_logprob=np.array(exp["logprob"], np.float64),
        exp_sampled_logprob=np.array(exp["sampled_logprob"], np.float64),
    )
    if hist is not None:
        arrays["history"] = hist
    if allowed is not None:
        arrays["allow_mask"] = pack_bits(allowed)
    np.savez_compressed(os.path.join(HERE, f"sampler_{name}.npz"), **arrays)


def logprob_case(name, seed, N, V, dtype):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, V, generator=g) * 3.0
    x[0] = 0.25                       # uniform row: lp = -ln V, H = ln V
    x[1, 7] = 60.0                    # one-hot spike: H ~ 0
    t = torch.randint(0, V, (N,), generator=g, dtype=torch.int32)
    t[1] = 7
    if dtype == "bf16":
        bits = bf16_bits(x)
        xv = bf16_values(bits)
        data = dict(logits_bf16=bits)
    else:
        xv = x.float()
        data = dict(logits_f32=xv.numpy().copy())
    lsm = torch.log_softmax(xv.double(), -1)
    lp = lsm.gather(1, t.long().view(-1, 1)).view(-1)
    H = -(lsm.exp() * lsm).sum(-1)
    np.savez_compressed(os.path.join(HERE, f"logprob_{name}.npz"), V=np.int64(V),
                        targets=t.numpy(), exp_logprob=lp.numpy(), exp_entropy=H.numpy(), **data)


def main():
    sampler_case("greedy_penalty_mask", 11, 8, 2048, scale=2.0, T=0.0, k=0, P=1.0, rho=1.3,
                 hist_len=40, density=0.2, ties=True)
    sampler_case("greedy_penalty_below_one", 12, 6, 3001, scale=2.0, T=0.0, k=0, P=1.0,
                 rho=0.5, hist_len=300)
    sampler_case("top_k", 13, 8, 3001, scale=2.5, T=0.7, k=50, P=1.0, ties=True)
    sampler_case("top_k_small_aligned", 14, 8, 4096, scale=3.0, T=1.3, k=5, P=1.0,
                 rho=1.1, hist_len=100)
    sampler_case("top_p", 15, 12, 2048, scale=2.0, T=1.0, k=0, P=0.9)
    sampler_case("top_p_masked", 16, 8, 4099, scale=2.5, T=0.8, k=0, P=0.9, density=0.08)
    sampler_case("top_k_top_p_all", 17, 8, 4096, scale=3.0, T=0.7, k=64, P=0.9, rho=1.05,
                 hist_len=200, density=0.08)
    logprob_case("bf16", 21, 6, 4099, "bf16")
    logprob_case("f32", 22, 4, 2053, "f32")


if __name__ == "__main__":
    main()
