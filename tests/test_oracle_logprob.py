"""Pins of the logprob / entropy oracle against torch.log_softmax (fp64) and
closed forms (uniform rows, one-hot spikes, bounds)."""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from graspo_amd import workloads as W
from tests._util import logits_to_oracle


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_logprob_entropy_matches_torch_fp64(dtype):
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(32, 4099, generator=g) * 3).to(dtype)
    t = torch.randint(0, 4099, (32,), generator=g, dtype=torch.int32)
    a, dt = logits_to_oracle(x)
    lp, H, st = O.logprob_entropy_rows(a, dt, t.numpy())
    ref_lp, ref_H = O.logprob_entropy_semantic(x.double().numpy(), t.numpy())
    ls = torch.log_softmax(x.double(), -1)
    assert np.allclose(lp, ls.gather(-1, t.long()[:, None]).squeeze(-1).numpy(), atol=1e-5)
    assert np.allclose(lp, ref_lp, atol=1e-5) and np.allclose(H, ref_H, atol=1e-5)
    assert (st == 0).all()


def test_workload4_rows_match_torch():
    x, t = W.logprob_workload(4, rows=8)
    a, dt = logits_to_oracle(x)
    lp, H, _ = O.logprob_entropy_rows(a, dt, t.numpy())
    ls = torch.log_softmax(x.double(), -1)
    ref = ls.gather(-1, t.long()[:, None]).squeeze(-1).numpy()
    ent = -(ls.exp() * ls).sum(-1).numpy()
    assert np.abs(lp - ref).max() < 1e-5 and np.abs(H - ent).max() < 1e-4


def test_closed_forms():
    V = 1000
    x = np.zeros((3, V), np.float32)
    x[1, 17] = 200.0  # one-hot spike: entropy 0, logprob of the spike 0
    x[2, :10] = -np.inf  # ten impossible tokens
    t = np.array([5, 17, 3], np.int32)
    lp, H, st = O.logprob_entropy_rows(x, O.DTYPE_F32, t)
    assert abs(lp[0] + math.log(V)) < 1e-6 and abs(H[0] - math.log(V)) < 1e-6
    assert abs(lp[1]) < 1e-6 and abs(H[1]) < 1e-6
    assert lp[2] == -np.inf and abs(H[2] - math.log(V - 10)) < 1e-6
    assert (st == 0).all()


def test_bad_target_and_nan_rows():
    x = np.random.default_rng(0).standard_normal((3, 64)).astype(np.float32)
    x[2, 5] = np.nan
    t = np.array([64, -1, 0], np.int32)
    lp, H, st = O.logprob_entropy_rows(x, O.DTYPE_F32, t)
    assert np.isnan(lp[0]) and np.isnan(lp[1]) and np.isnan(lp[2]) and np.isnan(H[2])
    assert st.tolist() == [O.ROW_BAD_TARGET, O.ROW_BAD_TARGET, O.ROW_OK]


def test_entropy_bounds():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((20, 500)) * rng.uniform(0.1, 20, (20, 1))).astype(np.float32)
    _, H, _ = O.logprob_entropy_rows(x, O.DTYPE_F32, np.zeros(20, np.int32))
    assert (H >= -1e-6).all() and (H <= math.log(500) + 1e-6).all()
