"""Seeded synthetic inputs for the five token-path workloads.

Every tensor comes from its own ``torch.Generator`` seeded ``1000*cfg + k``,
on the requested device (CPU for parity tests, the GPU for benchmarks, where
generating 4 GB of logits on the host would dominate).  ``rows`` / ``vocab``
shrink a workload for quick tests; the full shapes are the defaults.

1. fp32 [8, 151936] ~ N(0, 3); two rows get +15 on one token; 64-token
   history, penalty 1.05; T 0.7, top-k 50, top-p 0.9.
2. bf16 [64, 151936] ~ N(0, 2.5) plus a Zipf(1.1)-ranked bias per row
   (bias of rank r is -1.1 ln r over a seeded permutation); 2048-token history,
   penalty 1.1; T 1.0, top-p 0.95, no top-k.
3. bf16 [64, 151936] ~ N(0, 2.5); allow mask with ~8% of bits set plus a fixed
   300-token structural subset; two rows allow exactly one token; T 0.8,
   top-p 0.9.
4. logprob/entropy over bf16 [32768, 151936] ~ N(0, 2.5), int32 targets, in 4
   chunks of 8192 rows, for two logits seeds (policy / old policy).
5. bf16 [256, 248320] ~ N(0, 3); 10% of rows get +12 on 1-4 tokens;
   4096-token history, penalty 1.05; the 8% mask scheme; T 0.7, top-k 64,
   top-p 0.9.  Plus logprob/entropy over bf16 [8192, 248320] ~ N(0, 3).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

VOCAB = {1: 151936, 2: 151936, 3: 151936, 4: 151936, 5: 248320}
ROWS = {1: 8, 2: 64, 3: 64, 4: 32768, 5: 256}
LOGPROB_ROWS = {4: 32768, 5: 8192}
LOGPROB_CHUNK = {4: 8192, 5: 8192}


def _gen(cfg: int, k: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(1000 * cfg + k)
    return g


def pack_mask(bits: torch.Tensor) -> torch.Tensor:
    """[B, V] bool -> [B, ceil(V/32)] int32 words, bit (i & 31) of word i >> 5."""
    B, V = bits.shape
    W = (V + 31) // 32
    pad = W * 32 - V
    if pad:
        bits = torch.nn.functional.pad(bits, (0, pad))
    w = bits.view(B, W, 32).to(torch.int64) << torch.arange(32, device=bits.device)
    w = w.sum(-1)
    w = torch.where(w >= 2**31, w - 2**32, w)
    return w.to(torch.int32).contiguous()


def unpack_mask(words: torch.Tensor, V: int) -> torch.Tensor:
    """Inverse of :func:`pack_mask`."""
    w = words.to(torch.int64) & 0xFFFFFFFF
    bits = (w.unsqueeze(-1) >> torch.arange(32, device=words.device)) & 1
    return bits.view(words.shape[0], -1)[:, :V].bool()


def uniforms_24(n: int, g: torch.Generator, device) -> torch.Tensor:
    k = torch.randint(0, 1 << 24, (n,), generator=g, device=device, dtype=torch.int64)
    return (k.to(torch.float64) * 2.0**-24).to(torch.float32)


@dataclass
class SamplerWorkload:
    cfg: int
    logits: torch.Tensor
    temperature: float
    top_k: int
    top_p: float
    repetition_penalty: float
    history: torch.Tensor | None
    allow_mask: torch.Tensor | None
    uniforms: torch.Tensor
    single_rows: dict  # row -> the only allowed token (cfg 3)

    @property
    def shape(self):
        return tuple(self.logits.shape)

    def kwargs(self) -> dict:
        return dict(
            temperature=self.temperature, top_k=self.top_k, top_p=self.top_p,
            repetition_penalty=self.repetition_penalty, history=self.history,
            allow_mask=self.allow_mask, uniforms=self.uniforms,
        )

    def algorithmic_bytes(self) -> int:
        """One read of logits/mask/history/uniforms + the 12 output bytes per row."""
        B, V = self.logits.shape
        n = B * V * self.logits.element_size() + B * (4 + 12)
        if self.allow_mask is not None:
            n += B * 4 * ((V + 31) // 32)
        if self.history is not None:
            n += self.history.numel() * 4
        return n


def _mask_bits(cfg: int, B: int, V: int, device, k0: int) -> torch.Tensor:
    bern = torch.rand((B, V), generator=_gen(cfg, k0, device), device=device) < 0.08
    struct = torch.randperm(V, generator=_gen(cfg, k0 + 1, device), device=device)[:300]
    bern[:, struct] = True
    return bern


def sampler_workload(cfg: int, device="cpu", rows: int | None = None,
                     vocab: int | None = None) -> SamplerWorkload:
    if cfg not in (1, 2, 3, 5):
        raise ValueError(f"no sampler workload {cfg}")
    B = rows or ROWS[cfg]
    V = vocab or VOCAB[cfg]
    single: dict = {}
    if cfg == 1:
        x = torch.randn((B, V), generator=_gen(1, 1, device), device=device) * 3.0
        g = _gen(1, 2, device)
        spike_rows = torch.randperm(B, generator=g, device=device)[: min(2, B)]
        spike_tok = torch.randint(0, V, (spike_rows.numel(),), generator=g, device=device)
        x[spike_rows, spike_tok] += 15.0
        hist = torch.randint(0, V, (B, 64), generator=_gen(1, 3, device), device=device,
                             dtype=torch.int32)
        return SamplerWorkload(1, x.float().contiguous(), 0.7, 50, 0.9, 1.05, hist, None,
                               uniforms_24(B, _gen(1, 4, device), device), single)
    if cfg == 2:
        x = torch.randn((B, V), generator=_gen(2, 1, device), device=device) * 2.5
        perm = torch.rand((B, V), generator=_gen(2, 2, device), device=device).argsort(dim=1)
        base = -1.1 * torch.log(torch.arange(1, V + 1, device=device, dtype=torch.float32))
        bias = torch.empty_like(x)
        bias.scatter_(1, perm, base.expand(B, V))
        x = (x + bias).to(torch.bfloat16)
        hist = torch.randint(0, V, (B, 2048), generator=_gen(2, 3, device), device=device,
                             dtype=torch.int32)
        return SamplerWorkload(2, x.contiguous(), 1.0, 0, 0.95, 1.1, hist, None,
                               uniforms_24(B, _gen(2, 4, device), device), single)
    if cfg == 3:
        x = (torch.randn((B, V), generator=_gen(3, 1, device), device=device) * 2.5).to(
            torch.bfloat16)
        bits = _mask_bits(3, B, V, device, 2)
        g = _gen(3, 4, device)
        srows = torch.randperm(B, generator=g, device=device)[: min(2, B)]
        stoks = torch.randint(0, V, (srows.numel(),), generator=g, device=device)
        for r_, t_ in zip(srows.tolist(), stoks.tolist()):
            bits[r_] = False
            bits[r_, t_] = True
            single[r_] = t_
        return SamplerWorkload(3, x.contiguous(), 0.8, 0, 0.9, 1.0, None, pack_mask(bits),
                               uniforms_24(B, _gen(3, 5, device), device), single)
    # cfg 5
    x = torch.randn((B, V), generator=_gen(5, 1, device), device=device) * 3.0
    g = _gen(5, 2, device)
    n_spike = max(1, math.floor(0.1 * B)) if B >= 10 else min(1, B)
    srows = torch.randperm(B, generator=g, device=device)[:n_spike]
    counts = torch.randint(1, 5, (n_spike,), generator=g, device=device)
    for r_, c_ in zip(srows.tolist(), counts.tolist()):
        toks = torch.randint(0, V, (c_,), generator=g, device=device)
        x[r_, toks] += 12.0
    x = x.to(torch.bfloat16)
    hist = torch.randint(0, V, (B, 4096), generator=_gen(5, 3, device), device=device,
                         dtype=torch.int32)
    bits = _mask_bits(5, B, V, device, 4)
    return SamplerWorkload(5, x.contiguous(), 0.7, 64, 0.9, 1.05, hist, pack_mask(bits),
                           uniforms_24(B, _gen(5, 6, device), device), single)


def logprob_workload(cfg: int, device="cpu", rows: int | None = None, vocab: int | None = None,
                     pass_index: int = 0):
    """(logits bf16 [N, V], targets int32 [N]) for workload 4 (pass 0 = policy,
    1 = old policy: different logits seeds) or 5."""
    if cfg not in (4, 5):
        raise ValueError(f"no logprob workload {cfg}")
    N = rows or LOGPROB_ROWS[cfg]
    V = vocab or VOCAB[cfg]
    sigma = 2.5 if cfg == 4 else 3.0
    g = _gen(cfg, 10 + pass_index, device)
    x = torch.empty((N, V), dtype=torch.bfloat16, device=device)
    step = 1024  # generate in slabs to bound the fp32 temporary
    for s in range(0, N, step):
        x[s : s + step] = (torch.randn((min(step, N - s), V), generator=g, device=device)
                           * sigma).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), generator=_gen(cfg, 20, device), device=device,
                      dtype=torch.int32)
    return x, t


def logprob_algorithmic_bytes(N: int, V: int, elem: int = 2) -> int:
    """One read of the logits and targets + the 8 output bytes per row."""
    return N * (V * elem + 4 + 8)
