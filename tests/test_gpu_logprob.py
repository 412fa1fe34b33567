"""GPU parity of the logprob / entropy kernels (tolerance 1e-3 absolute,
fp32 accumulation) against the fp64 CPU oracle on row subsets, and against a
torch fp32 log_softmax on the GPU at full workload size."""

import math

import numpy as np
import pytest
import torch

from graspo_amd import graspo_loss as GL
from graspo_amd import ops
from graspo_amd import tensor_utils as TU
from graspo_amd import workloads as W
from tests._util import oracle_logprob

pytestmark = pytest.mark.gpu
TOL = 1e-3
DEV = "cuda:0"


@pytest.mark.parametrize("cfg,rows", [(4, 1024), (5, 512)])
def test_workload_rows_vs_oracle(cfg, rows):
    x, t = W.logprob_workload(cfg, rows=rows)
    print(f"workload {cfg} rows {rows}", flush=True)
    lp, H, st = ops.logprob_entropy(x.to(DEV), t.to(DEV))
    rlp, rH, rst = oracle_logprob(x, t)
    assert np.abs(lp.cpu().numpy() - rlp).max() <= TOL
    assert np.abs(H.cpu().numpy() - rH).max() <= TOL
    assert np.array_equal(st.cpu().numpy(), rst)


@pytest.mark.parametrize("cfg", [4, 5])
def test_full_chunk_vs_torch_fp32(cfg):
    """One full 8192-row chunk generated on the GPU, against torch's fp32
    log_softmax on the GPU (in slabs), plus size-independent bounds."""
    x, t = W.logprob_workload(cfg, device=DEV, rows=8192)
    lp, H, st = ops.logprob_entropy(x, t)
    worst_lp = worst_h = 0.0
    for s in range(0, 8192, 1024):
        ls = torch.log_softmax(x[s : s + 1024].float(), -1)
        ref = ls.gather(-1, t[s : s + 1024].long().unsqueeze(-1)).squeeze(-1)
        ent = -(ls.exp() * ls).sum(-1)
        worst_lp = max(worst_lp, float((lp[s : s + 1024] - ref).abs().max()))
        worst_h = max(worst_h, float((H[s : s + 1024] - ent).abs().max()))
    assert worst_lp <= TOL and worst_h <= TOL, (worst_lp, worst_h)
    assert bool((st == 0).all())
    V = x.shape[1]
    assert bool((H >= -TOL).all()) and bool((H <= math.log(V) + TOL).all())
    assert bool((lp <= TOL).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("V", [7, 1000, 4099, 151936])
def test_dtypes_odd_vocab_and_specials(dtype, V):
    g = torch.Generator().manual_seed(V)
    x = (torch.randn(8, V, generator=g) * 3).to(dtype)
    x[1] = 0  # uniform
    x[2, :] = -float("inf")
    x[2, V // 2] = 1.0  # single finite logit
    x[3, 0] = float("nan")
    t = torch.randint(0, V, (8,), generator=g)
    t[2] = V // 2
    t[5] = V  # out of range
    lp, H, st = ops.logprob_entropy(x.to(DEV), t.to(DEV))
    rlp, rH, rst = oracle_logprob(x, t)
    lp, H = lp.cpu().numpy(), H.cpu().numpy()
    assert np.array_equal(st.cpu().numpy(), rst)
    assert np.array_equal(np.isnan(lp), np.isnan(rlp))
    fin = ~np.isnan(rlp)
    assert np.abs(lp[fin] - rlp[fin]).max() <= TOL
    finH = ~np.isnan(rH)
    assert np.abs(H[finH] - rH[finH]).max() <= TOL
    assert abs(lp[1] + math.log(V)) <= TOL and abs(H[1] - math.log(V)) <= TOL
    assert abs(lp[2]) <= TOL and abs(H[2]) <= TOL


def test_partial_chunks_equal_full_row():
    x, t = W.logprob_workload(5, rows=64)
    xd, td = x.to(DEV), t.to(DEV)
    lp, H, _ = ops.logprob_entropy(xd, td)
    state = ops.new_lse_state(64, DEV)
    V = x.shape[1]
    for c, s in enumerate(range(0, V, 32768)):
        ops.lse_partial(xd[:, s : s + 32768], td, s, state, accumulate=c > 0)
    lp2, H2 = ops.lse_finalize(state)
    assert float((lp - lp2).abs().max()) <= 1e-4 and float((H - H2).abs().max()) <= 1e-4


def test_hidden_path_dropin_forward_backward():
    """_selected_token_log_probs_from_hidden vs a direct fp32 torch statement
    (logit - logsumexp), including gradients."""
    g = torch.Generator().manual_seed(3)
    B, S, Hd, V = 2, 9, 64, 5000
    h = torch.randn(B, S, Hd, generator=g).to(DEV).requires_grad_(True)
    w = (torch.randn(V, Hd, generator=g) * 0.2).to(DEV).requires_grad_(True)
    ids = torch.randint(0, V, (B, S), generator=g).to(DEV)
    out = TU._selected_token_log_probs_from_hidden(h, w, ids, vocab_chunk_size=1024)
    h2 = h.detach().clone().requires_grad_(True)
    w2 = w.detach().clone().requires_grad_(True)
    logits = h2 @ w2.t()
    ref = logits.gather(-1, ids.unsqueeze(-1)).squeeze(-1) - torch.logsumexp(logits, -1)
    assert float((out - ref).abs().max()) <= TOL
    gout = torch.randn(B, S, generator=g).to(DEV)
    (out * gout).sum().backward()
    (ref * gout).sum().backward()
    assert float((h.grad - h2.grad).abs().max()) <= 1e-3
    assert float((w.grad - w2.grad).abs().max()) <= 1e-3


def test_sequence_logprob_dropin_3d_views_and_grad():
    g = torch.Generator().manual_seed(4)
    logits = (torch.randn(3, 7, 1000, generator=g) * 2).to(DEV)
    ids = torch.randint(0, 1000, (3, 7), generator=g).to(DEV)
    view = logits[:, :-1]  # the call-site slice: not flattenable without a copy
    out = GL.sequence_log_probs_from_logits(view, ids[:, 1:])
    ref = torch.log_softmax(view.double(), -1).gather(-1, ids[:, 1:].unsqueeze(-1)).squeeze(-1)
    assert float((out.double() - ref).abs().max()) <= TOL
    lg = logits.detach().clone().requires_grad_(True)
    out = GL.sequence_log_probs_from_logits(lg, ids)
    out.sum().backward()
    lg2 = logits.detach().clone().requires_grad_(True)
    torch.log_softmax(lg2, -1).gather(-1, ids.unsqueeze(-1)).sum().backward()
    assert float((lg.grad - lg2.grad).abs().max()) <= 1e-4


def test_out_of_range_target_raises_like_gather():
    """A target outside [0, V) raises RuntimeError, as the reference's
    log_softmax(...).gather(...) (graspo_loss.py:19-21) and index_select
    (tensor_utils.py:167-186) reject such an index, instead of a silent NaN."""
    from graspo_amd.graspo_loss import sequence_log_probs_from_logits
    from graspo_amd.tensor_utils import _selected_token_log_probs_from_hidden

    dev = torch.device("cuda:0")
    x = torch.randn(2, 5, 300, device=dev)
    for bad in (300, -1):
        t = torch.randint(0, 300, (2, 5), device=dev)
        t[1, 3] = bad
        print("out-of-range target", bad, flush=True)
        with pytest.raises(RuntimeError, match="outside"):
            sequence_log_probs_from_logits(x, t)
        with pytest.raises(RuntimeError, match="outside"):
            sequence_log_probs_from_logits(x.clone().requires_grad_(True), t)
        h = torch.randn(2, 5, 64, device=dev)
        w = torch.randn(300, 64, device=dev)
        with pytest.raises(RuntimeError, match="outside"):
            _selected_token_log_probs_from_hidden(h, w, t)
