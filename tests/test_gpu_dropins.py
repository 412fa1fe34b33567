"""The reference's helpers as the reference calls them, on the GPU:

* ``_sample_next_token(logits / T, top_p=P)`` (tensor_utils.py:671-683, fed
  already temperature-scaled rows by tensor_utils.py:655-656) against the
  exact oracle at T = 1 on the same scaled rows: ids, bit for bit;
* ``_broadcast_and_pad_finished`` (tensor_utils.py:661-668) against the
  reference's own expression ``torch.where(finished, full_like(pad), ids)``;
* the loss-side logprobs of configuration 4 (graspo_loss.py:19-21) on both
  passes (policy and old-policy logits from different seeds), every one of
  the four 8192-row chunks: torch fp32 on the GPU and bounds on all rows, the
  fp64 oracle on rows sampled from each chunk, and the old-policy pass's
  CPU-generated rows against the oracle."""

import math

import numpy as np
import pytest
import torch

from graspo_amd import tensor_utils as TU
from graspo_amd import workloads as W
from tests._util import oracle_logprob, oracle_sample

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-3


def _u(B, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 1 << 24, (B,), generator=g).float() * 2.0 ** -24


@pytest.mark.parametrize("case", ["bf16_64x151936", "fp32_8x151936", "bf16_256x248320",
                                  "fp32_scaled_256x248320", "small_vocab"])
def test_sample_next_token_on_scaled_rows(case):
    if case == "bf16_64x151936":
        x = W.sampler_workload(3, device=DEV).logits         # bf16 N(0, 2.5)
        T, P = 1.0, 0.9
    elif case == "fp32_8x151936":
        x = W.sampler_workload(1, device=DEV).logits         # fp32 N(0, 3) + spikes
        T, P = 0.7, 0.9
    elif case == "bf16_256x248320":
        x = W.sampler_workload(5, device=DEV).logits         # bf16 N(0, 3) + spikes
        T, P = 1.0, 0.95
    elif case == "fp32_scaled_256x248320":
        x = W.sampler_workload(5, device=DEV).logits.float()
        T, P = 0.7, 0.9                                      # scaled rows: not bf16 values
    else:
        g = torch.Generator().manual_seed(5)
        x = (torch.randn(16, 3001, generator=g) * 2).to(DEV)
        T, P = 0.8, 0.5
    B = x.shape[0]
    u = _u(B, B)
    scaled = x / max(float(T), 1e-6)                          # tensor_utils.py:656
    print("sample_next_token", case, tuple(x.shape), scaled.dtype, flush=True)
    ids = TU._sample_next_token(scaled, top_p=P, uniforms=u.to(DEV))
    torch.cuda.synchronize()
    ex = oracle_sample(scaled, temperature=1.0, top_p=P, uniforms=u)
    assert (ex.status == 0).all()
    assert ids.dtype == torch.int64 and tuple(ids.shape) == (B,)
    assert np.array_equal(ids.cpu().numpy(), ex.ids)


def test_sample_next_token_top_p_off_samples_the_softmax():
    """top_p outside (0, 1) samples the full softmax (tensor_utils.py:683)."""
    g = torch.Generator().manual_seed(8)
    x = (torch.randn(32, 70000, generator=g) * 2).to(torch.bfloat16)
    u = _u(32, 9)
    for P in (1.0, 0.0):
        ids = TU._sample_next_token(x.to(DEV), top_p=P, uniforms=u.to(DEV))
        ex = oracle_sample(x, temperature=1.0, top_p=1.0, uniforms=u)
        assert np.array_equal(ids.cpu().numpy(), ex.ids)
        assert (ex.kept == 70000).all()


@pytest.mark.parametrize("B,pad", [(1, 0), (256, 151643), (1000, -1)])
def test_broadcast_and_pad_finished_is_the_reference_expression(B, pad):
    g = torch.Generator().manual_seed(B)
    ids = torch.randint(0, 248320, (B,), generator=g).to(DEV)
    finished = (torch.rand(B, generator=g) < 0.3).to(DEV)
    want = torch.where(finished, torch.full_like(ids, pad), ids)  # tensor_utils.py:668
    got = TU._broadcast_and_pad_finished(ids.clone(), finished, pad)
    assert got.dtype == ids.dtype and torch.equal(got, want)
    none = TU._broadcast_and_pad_finished(ids.clone(), torch.zeros_like(finished), pad)
    assert torch.equal(none, ids)
    every = TU._broadcast_and_pad_finished(ids.clone(), torch.ones_like(finished), pad)
    assert bool((every == pad).all())


def test_workload4_old_policy_pass_rows_vs_oracle():
    x, t = W.logprob_workload(4, rows=1024, pass_index=1)
    x0, _ = W.logprob_workload(4, rows=8, pass_index=0)
    assert not torch.equal(x[:8], x0)  # a different seed from the policy pass
    print("workload 4 pass 1 rows 1024", flush=True)
    lp, H, st = TU.ops.logprob_entropy(x.to(DEV), t.to(DEV))
    rlp, rH, rst = oracle_logprob(x, t)
    assert np.abs(lp.cpu().numpy() - rlp).max() <= TOL
    assert np.abs(H.cpu().numpy() - rH).max() <= TOL
    assert np.array_equal(st.cpu().numpy(), rst)


@pytest.mark.parametrize("pass_index", [0, 1])
def test_workload4_every_chunk_of_both_passes(pass_index):
    """The full [32768, 151936] pass in its four 8192-row chunks, as the loss
    step runs it: every row against torch fp32 log_softmax on the GPU, the
    size-independent bounds lp <= 0 and 0 <= H <= ln V on every row, and 32
    rows of each chunk against the fp64 oracle."""
    x, t = W.logprob_workload(4, device=DEV, pass_index=pass_index)
    N, V = x.shape
    chunk = W.LOGPROB_CHUNK[4]
    assert N == 32768 and N // chunk == 4
    sample = torch.arange(0, chunk, chunk // 32, device=DEV)
    for c in range(N // chunk):
        xc, tc = x[c * chunk:(c + 1) * chunk], t[c * chunk:(c + 1) * chunk]
        print(f"workload 4 pass {pass_index} chunk {c}", flush=True)
        lp, H, st = TU.ops.logprob_entropy(xc, tc)
        assert bool((st == 0).all())
        worst_lp = worst_h = 0.0
        for s in range(0, chunk, 1024):
            ls = torch.log_softmax(xc[s:s + 1024].float(), -1)
            ref = ls.gather(-1, tc[s:s + 1024].long().unsqueeze(-1)).squeeze(-1)
            ent = -(ls.exp() * ls).sum(-1)
            worst_lp = max(worst_lp, float((lp[s:s + 1024] - ref).abs().max()))
            worst_h = max(worst_h, float((H[s:s + 1024] - ent).abs().max()))
            del ls
        assert worst_lp <= TOL and worst_h <= TOL, (c, worst_lp, worst_h)
        assert bool((lp <= TOL).all())
        assert bool((H >= -TOL).all()) and bool((H <= math.log(V) + TOL).all())
        rlp, rH, rst = oracle_logprob(xc[sample].cpu(), tc[sample].cpu())
        assert np.abs(lp[sample].cpu().numpy() - rlp).max() <= TOL
        assert np.abs(H[sample].cpu().numpy() - rH).max() <= TOL
