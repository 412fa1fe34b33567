"""GPU parity of the value-histogram sampler (bf16 sampling rows outside the
split kernel's top-k range: top-p only, plain sampling, top-k above 128)
against the exact CPU oracle.

Covers value bins holding many tokens (the drawn or last kept token found by
its rank among equal values, in id order), penalised and out-of-range
tokens kept one by one, the rows that leave the histogram for the row-wise
path (too many out-of-range tokens, an exact tie between a penalised token
and a value bin, crowded value segments), vocabularies with a tail,
extreme temperatures and the per-row statuses."""

import numpy as np
import pytest
import torch

from graspo_amd import workloads as W
from tests._util import oracle_sample
from tests.test_gpu_sampler import assert_parity, gpu_sample

pytestmark = pytest.mark.gpu
V_LARGE = 248320


def _rows(seed, B, V, scale=3.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, V, generator=g) * scale), g


def _edge_uniforms(B, g):
    u = W.uniforms_24(B, g, "cpu")
    u[0] = 0.0
    if B > 1:
        u[1] = 1.0 - 2.0 ** -24
    return u


@pytest.mark.parametrize("top_p,top_k", [(0.9, 0), (1.0, 0), (0.95, 1000), (0.5, 129)])
def test_dense_value_bins(top_p, top_k):
    """Rows whose values repeat (multiples of 1/4, 1/64, a handful of
    values): the cut and the draw land inside bins of many tokens."""
    x, g = _rows(31, 8, V_LARGE)
    x[2] = torch.round(x[2] * 4) / 4
    x[3] = torch.round(x[3] * 64) / 64
    x[4] = (torch.arange(V_LARGE) % 5).float() + 1.0
    x[5] = 1.5  # one bin holds the whole row
    x = x.to(torch.bfloat16)
    u = _edge_uniforms(8, g)
    for T in (0.7, 1.0):
        kw = dict(temperature=T, top_k=top_k, top_p=top_p, uniforms=u)
        print("dense", top_p, top_k, T, flush=True)
        assert_parity(gpu_sample(x, **kw), oracle_sample(x, **kw), f"p{top_p} k{top_k} T{T}")


@pytest.mark.parametrize("rho", [1.3, 0.7])
def test_penalty_and_mask(rho):
    x, g = _rows(32, 8, V_LARGE, 2.5)
    x[1] = torch.round(x[1] * 8) / 8
    # one or two values: a wave of the id pass holds thousands of members of
    # a bin, past its 512-entry list, with the mask and the penalty applied
    x[2] = 1.0
    x[3] = (torch.arange(V_LARGE) % 2).float() * 0.5 + 1.0
    x = x.to(torch.bfloat16)
    hist = torch.randint(-1, V_LARGE, (8, 300), generator=g, dtype=torch.int32)
    bits = torch.rand(8, V_LARGE, generator=g) < 0.3
    bits[:, hist[:, :100].clamp(min=0).long()] = True
    u = _edge_uniforms(8, g)
    for mask in (None, W.pack_mask(bits)):
        kw = dict(temperature=0.9, top_p=0.9, repetition_penalty=rho, history=hist,
                  allow_mask=mask, uniforms=u)
        print("penalty", rho, mask is not None, flush=True)
        assert_parity(gpu_sample(x, **kw), oracle_sample(x, **kw), f"rho{rho}")


def test_rows_leaving_the_histogram():
    """Each row exceeds one bound of the histogram path; results must not
    change."""
    B, V = 4, 65536
    x, g = _rows(33, B, V, 2.0)
    x[0, : V // 2] = 0.0                       # zeros are kept one by one: too many
    x[1] = torch.round(x[1] * 2) / 2           # rho = 2 maps x onto x / 2: exact ties
    x[2, :4000] = 3.0 + torch.arange(4000) * 1e-3   # crowded penalised values
    x[3, ::2] = -1e30                          # out-of-range values in half the row
    x = x.to(torch.bfloat16)
    hist = torch.arange(2000, dtype=torch.int32).repeat(B, 1)
    u = torch.tensor([0.3, 0.6, 0.05, 0.9])
    for rho, p in ((2.0, 0.8), (1.1, 0.999), (1.1, 0.3)):
        kw = dict(temperature=1.0, top_p=p, repetition_penalty=rho, history=hist, uniforms=u)
        print("leave", rho, p, flush=True)
        assert_parity(gpu_sample(x, **kw), oracle_sample(x, **kw), f"rho{rho} p{p}")


@pytest.mark.parametrize("V", [248323, 4101, 1000, 69, 8, 7])
def test_vocab_tail(V):
    """Aligned rows (stride a multiple of 8) whose length is not.  V = 69
    leaves one wave of the id pass only the partial last vector, V = 7 has
    no full vector at all."""
    stride = (V + 7) // 8 * 8
    full, g = _rows(34, 6, stride)
    full[3] = torch.round(full[3] * 4) / 4
    full = full.to(torch.bfloat16)
    x = full[:, :V]
    hist = torch.randint(0, V, (6, 50), generator=g, dtype=torch.int32)
    hist[:, 0] = V - 1
    u = _edge_uniforms(6, g)
    kw = dict(temperature=0.8, top_p=0.95, repetition_penalty=1.2, history=hist, uniforms=u)
    dev = torch.device("cuda:0")
    out = gpu_sample(full.to(dev)[:, :V], **kw)
    assert_parity(out, oracle_sample(x.contiguous(), **kw), f"V{V}")


@pytest.mark.parametrize("T", [1e-3, 0.05, 3.0, 900.0, 5000.0])
def test_extreme_temperature(T):
    x, g = _rows(35, 6, 32768)
    x[2] = torch.round(x[2] * 16) / 16
    x = x.to(torch.bfloat16)
    u = _edge_uniforms(6, g)
    kw = dict(temperature=T, top_p=0.9, uniforms=u)
    assert_parity(gpu_sample(x, **kw), oracle_sample(x, **kw), f"T{T}")


def test_status_rows_bf16():
    V = 40000
    x, g = _rows(36, 8, V)
    x[0, 3] = float("nan")
    x[1, 4] = float("inf")
    x[6] = float("-inf")
    x = x.to(torch.bfloat16)
    bits = torch.ones(8, V, dtype=torch.bool)
    bits[2] = False
    bits[3] = False
    bits[3, 39] = True
    hist = torch.full((8, 2), -1, dtype=torch.int32)
    hist[4, 1] = V
    u = torch.full((8,), 0.5)
    u[5] = 1.0
    fin = torch.zeros(8, dtype=torch.bool)
    fin[7] = True
    kw = dict(temperature=1.0, top_p=0.9, repetition_penalty=1.2, history=hist,
              allow_mask=W.pack_mask(bits), uniforms=u, finished=fin, pad_token_id=-5)
    assert_parity(gpu_sample(x, **kw), oracle_sample(x, **kw))
