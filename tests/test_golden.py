"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from transformers' repetition-penalty processor, torch's stable sort, the
reference's top-p rule in fp64 and torch.log_softmax in fp64) against the CPU
oracle and against the gfx950 kernels.  Each sampler fixture also holds the
fp64 log of the drawn token's renormalised probability, which pins the
contract's sampled_logprob = log(w / W') independently of the oracle."""

import glob
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SAMPLER = sorted(glob.glob(os.path.join(GOLDEN, "sampler_*.npz")))
LOGPROB = sorted(glob.glob(os.path.join(GOLDEN, "logprob_*.npz")))
LP_TOL = 1e-3


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _sampler_kwargs(f):
    return dict(temperature=float(f["temperature"]), top_k=int(f["top_k"]),
                top_p=float(f["top_p"]), repetition_penalty=float(f["repetition_penalty"]),
                history=f.get("history"), allow_mask=f.get("allow_mask"),
                uniforms=f["uniforms"])


def _check_sampler(name, f, ids, kept, tv, tid, lp, slp, status):
    assert (status == 0).all(), f"{name}: status {status}"
    np.testing.assert_array_equal(ids, f["exp_ids"], err_msg=f"{name}: ids")
    np.testing.assert_array_equal(kept, f["exp_kept"], err_msg=f"{name}: kept")
    np.testing.assert_array_equal(tid, f["exp_thresh_id"], err_msg=f"{name}: threshold id")
    np.testing.assert_array_equal(tv.view(np.uint32), f["exp_thresh_value"].view(np.uint32),
                                  err_msg=f"{name}: threshold value")
    assert np.abs(lp.astype(np.float64) - f["exp_logprob"]).max() <= LP_TOL, f"{name}: logprob"
    assert np.abs(slp.astype(np.float64) - f["exp_sampled_logprob"]).max() <= LP_TOL, (
        f"{name}: sampled logprob")


def test_fixtures_present():
    assert len(SAMPLER) >= 7 and len(LOGPROB) >= 2


@pytest.mark.parametrize("path", SAMPLER, ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_matches_sampler_fixture(path):
    f = _load(path)
    r = O.sample_rows(f["logits_bf16"], O.DTYPE_BF16, **_sampler_kwargs(f))
    _check_sampler(os.path.basename(path), f, r.ids, r.kept, r.thresh_value, r.thresh_id,
                   r.logprob, r.sampled_logprob, r.status)


@pytest.mark.parametrize("path", LOGPROB, ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_matches_logprob_fixture(path):
    f = _load(path)
    x, dt = (f["logits_bf16"], O.DTYPE_BF16) if "logits_bf16" in f else (f["logits_f32"], O.DTYPE_F32)
    lp, H, st = O.logprob_entropy_rows(x, dt, f["targets"])
    assert (st == 0).all()
    assert np.abs(lp - f["exp_logprob"]).max() <= 1e-5
    assert np.abs(H - f["exp_entropy"]).max() <= 1e-5


def _to_gpu_logits(f):
    dev = torch.device("cuda:0")
    if "logits_bf16" in f:
        return torch.from_numpy(f["logits_bf16"].view(np.int16)).view(torch.bfloat16).to(dev)
    return torch.from_numpy(f["logits_f32"]).to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("path", SAMPLER, ids=lambda p: os.path.basename(p)[:-4])
def test_gpu_matches_sampler_fixture(path):
    from graspo_amd import ops

    f = _load(path)
    dev = torch.device("cuda:0")
    kw = _sampler_kwargs(f)
    for n in ("history", "allow_mask", "uniforms"):
        if kw[n] is not None:
            kw[n] = torch.from_numpy(np.ascontiguousarray(kw[n])).to(dev)
    print("golden", os.path.basename(path), flush=True)
    out = ops.sample(_to_gpu_logits(f), **kw)
    torch.cuda.synchronize()
    _check_sampler(os.path.basename(path), f, out.ids.cpu().numpy(), out.kept.cpu().numpy(),
                   out.thresh_value.cpu().numpy(), out.thresh_id.cpu().numpy(),
                   out.logprob.cpu().numpy(), out.sampled_logprob.cpu().numpy(),
                   out.status.cpu().numpy())


@pytest.mark.gpu
@pytest.mark.parametrize("path", LOGPROB, ids=lambda p: os.path.basename(p)[:-4])
def test_gpu_matches_logprob_fixture(path):
    from graspo_amd import ops

    f = _load(path)
    print("golden", os.path.basename(path), flush=True)
    t = torch.from_numpy(f["targets"]).to("cuda:0")
    lp, H, st = ops.logprob_entropy(_to_gpu_logits(f), t)
    torch.cuda.synchronize()
    assert (st.cpu().numpy() == 0).all()
    assert np.abs(lp.cpu().numpy().astype(np.float64) - f["exp_logprob"]).max() <= LP_TOL
    assert np.abs(H.cpu().numpy().astype(np.float64) - f["exp_entropy"]).max() <= LP_TOL
