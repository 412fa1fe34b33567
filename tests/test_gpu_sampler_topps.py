"""GPU parity of the split top-p kernel (bf16 top-p rows of batches up to 64,
each row split over several workgroups) against the exact CPU oracle: ids,
kept sizes, thresholds and statuses bit for bit, logprobs within 1e-3.

Covers every (penalty, mask) variant on small batches and vocabulary tails
(the tail lies in the last slice), values held by hundreds of tokens in
several slices (the wanted token's slice and its rank there come from the
slices' counts), the cut and the draw in different slices, a value held by
more than 65535 tokens of a row but fewer in each slice (the merged 16-bit
count overflows: the row is handed over) or 65536 times in one slice (that
slice's count wraps: its token total gives it away), a value outside the bins in one
slice only, status rows, and the no-allocation entry point, whose 8 MiB
array holds fewer slices."""

import ctypes

import numpy as np
import pytest
import torch

from graspo_amd import workloads as W
from tests import _capi
from tests._util import oracle_sample
from tests.test_gpu_sampler import assert_parity, gpu_sample
from tests.test_gpu_sampler_topp import aligned_rows, one_workgroup_sample

pytestmark = pytest.mark.gpu


def _u(B, g):
    return torch.randint(0, 1 << 24, (B,), generator=g).float() * 2.0 ** -24


def _check(x, what, **kw):
    print("topps:", what, tuple(x.shape), {k: v for k, v in kw.items()
                                           if not isinstance(v, torch.Tensor)}, flush=True)
    g = gpu_sample(x, **kw)
    ref = oracle_sample(x, **kw)
    assert_parity(g, ref, what)
    return g, ref


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("B,V", [(1, 65536), (5, 65541), (32, 151936), (3, 248320), (2, 262144)])
def test_modes_and_shapes(mode, B, V):
    """Every variant; V = 65541 puts a 5-token tail in the last slice."""
    g = torch.Generator().manual_seed(mode * 100 + B)
    x = aligned_rows((torch.randn(B, V, generator=g) * 3).to(torch.bfloat16))
    kw = dict(temperature=0.8, top_p=0.9, uniforms=_u(B, g))
    if mode & 1:
        kw["history"] = torch.randint(-1, V, (B, 1500), generator=g, dtype=torch.int32)
        kw["repetition_penalty"] = 1.2
    if mode & 2:
        kw["allow_mask"] = W.pack_mask(torch.rand(B, V, generator=g) < 0.3)
    _check(x, f"mode {mode}", **kw)


def test_values_across_slices():
    """Values on a grid of 1/4: hundreds of tokens per value in every slice,
    the cut and the draw inside such values."""
    B, V = 16, 151936
    g = torch.Generator().manual_seed(3)
    x = (torch.round(torch.randn(B, V, generator=g) * 8) / 4).to(torch.bfloat16)
    for T, P in ((0.7, 0.9), (1.0, 0.5), (2.0, 0.99)):
        got, ref = _check(x, f"grid {T} {P}", temperature=T, top_p=P, uniforms=_u(B, g))
        assert (ref.kept > 100).all()


def test_merged_count_overflow_and_escape():
    """Row 0: 70000 tokens of one value (fewer than 65536 in each slice): the
    merged count overflows and the row is handed over.  Row 1: a value above
    the bins in one slice.  Both still bit-exact."""
    B, V = 2, 248320
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, V, generator=g) * 2
    idx = torch.randperm(V, generator=g)[:70000]
    x[0, idx] = 0.75
    x[1, 200000] = 3.0e7
    x = x.to(torch.bfloat16)
    _check(x, "overflow and escape", temperature=1.0, top_p=0.95, uniforms=_u(B, g))


def test_status_rows():
    B, V = 8, 100003
    g = torch.Generator().manual_seed(5)
    x = aligned_rows((torch.randn(B, V, generator=g) * 2).to(torch.bfloat16))
    u = _u(B, g)
    u[1] = 1.5                      # bad uniform
    hist = torch.zeros((B, 6), dtype=torch.int32)
    hist[2, 3] = V                  # bad history id
    fin = torch.zeros(B, dtype=torch.bool)
    fin[3] = True
    bits = torch.ones(B, V, dtype=torch.bool)
    bits[4] = False                 # no allowed token
    bits[5] = False
    bits[5, 77777] = True           # one allowed token
    got, ref = _check(x, "status rows", temperature=0.9, top_p=0.9, uniforms=u, history=hist,
                      repetition_penalty=1.1, finished=fin, pad_token_id=-3,
                      allow_mask=W.pack_mask(bits))
    assert int(got.status[1]) == 4 and int(got.status[2]) == 3 and int(got.status[4]) == 2
    assert int(got.ids[3]) == -3 and int(got.ids[5]) == 77777


def test_matches_the_one_workgroup_kernel():
    """Same rows through both kernels: configuration 2's rows (penalty) and
    decode rows of 248320 tokens."""
    wl = W.sampler_workload(2, rows=24)
    kw = wl.kwargs()
    got, ref = _check(wl.logits, "cfg2 rows", **kw)
    one = one_workgroup_sample(wl.logits, **kw)
    assert_parity(one, ref, "cfg2 rows (one workgroup)")
    wl5 = W.sampler_workload(5, rows=16)
    kw5 = dict(temperature=0.7, top_p=0.9, uniforms=wl5.uniforms)
    got, ref = _check(wl5.logits, "decode rows", **kw5)
    assert_parity(one_workgroup_sample(wl5.logits, **kw5), ref, "decode rows (one workgroup)")


def test_noalloc_entry_point_uses_fewer_slices():
    """gtp_sample_rows_noalloc on 16 decode rows: its 8 MiB array holds 7
    slices per row instead of 8; the answer is the same."""
    L = _capi.lib()
    dev = torch.device("cuda:0")
    wl = W.sampler_workload(5, rows=16)
    x = wl.logits.to(dev)
    kw = dict(temperature=0.7, top_p=0.9, uniforms=wl.uniforms.to(dev))
    args, p, B = _capi.sample_args(x, **kw)
    assert L.gtp_sample_workspace_bytes(1, B, x.shape[1], ctypes.byref(p)) > 8 << 20
    # the plan of this call: the split top-p kernel, 7 workgroups per row
    assert _capi.route(L, 1, B, x.shape[1], T=0.7, P=0.9,
                       workspace=_capi.NOALLOC_SCRATCH_BYTES) == (_capi.ROUTE_TOPP_SPLIT, 7)
    out = _capi.SampleBuffers(B, dev)
    assert L.gtp_sample_rows_noalloc(*args, *out.out_args(), _capi.stream_handle()) == 0
    torch.cuda.synchronize()
    got = out.cpu()
    ref = oracle_sample(wl.logits, temperature=0.7, top_p=0.9, uniforms=wl.uniforms)
    assert np.array_equal(got["ids"].numpy(), ref.ids)
    assert np.array_equal(got["kept"].numpy(), ref.kept)
    assert np.array_equal(got["thresh_id"].numpy(), ref.thresh_id)


def test_slice_count_overflow():
    """[64, 262144]: 4 slices of 65536 tokens.  Row 0's first slice holds one
    value 65536 times, so that slice's 16-bit count wraps; the slice's token
    total no longer adds up and the row is handed over.  Row 1 holds the
    value 40000 times in each of two slices (80000 in the row)."""
    B, V = 64, 262144
    g = torch.Generator().manual_seed(9)
    x = torch.randn(B, V, generator=g) * 2
    x[0, :65536] = 1.5
    x[1, 10000:50000] = 1.5
    x[1, 70000:110000] = 1.5
    x = x.to(torch.bfloat16)
    _check(x, "slice count overflow", temperature=1.0, top_p=0.9, uniforms=_u(B, g))


def test_repeated_calls_agree_with_the_one_workgroup_kernel():
    """40 back-to-back calls on fresh rows of one shape (the workspace's
    slots hold the previous call's counts): every split result equals the
    one-workgroup kernel's bit for bit, so no merge read a stale slot."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(11)
    B, V = 48, 151936
    hist = torch.randint(0, V, (B, 512), generator=g, device=dev, dtype=torch.int32)
    for it in range(40):
        x = (torch.randn(B, V, generator=g, device=dev) * (1.5 + (it % 5))).to(torch.bfloat16)
        u = torch.randint(0, 1 << 24, (B,), generator=g, device=dev).float() * 2.0 ** -24
        kw = dict(temperature=0.6 + 0.1 * (it % 7), top_p=0.8 + 0.04 * (it % 5), uniforms=u)
        if it % 2:
            kw.update(history=hist, repetition_penalty=1.15)
        got = gpu_sample(x, **kw)
        one = one_workgroup_sample(x, **kw)
        for f in ("ids", "kept", "thresh_id", "status"):
            assert torch.equal(getattr(got, f), getattr(one, f)), (it, f)
        assert torch.equal(got.thresh_value.view(torch.int32), one.thresh_value.view(torch.int32)), it
        assert torch.equal(got.sampled_logprob.view(torch.int32), one.sampled_logprob.view(torch.int32)), it
