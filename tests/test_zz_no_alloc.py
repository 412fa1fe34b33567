"""gtp_sample_rows_noalloc, the sampler entry point that allocates nothing
(its workspace is the library's own per-GPU device array), against
gtp_sample_rows with a caller-owned workspace: the same kernels, so ids,
kept sizes, thresholds and statuses must be identical bit for bit, and the
logprobs agree within 1e-3.  Two calls in a row, the second with a
smaller input (fewer rows, a shorter vocabulary, another top-k), so the
second call runs on what the first one left in the array."""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(B, V, dtype, params, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, V, generator=g) * 2.5).to(dtype)
    x[0, V // 3] = 11.0  # a spike
    u = torch.randint(0, 1 << 24, (B,), generator=g).float() * 2.0 ** -24
    hist = torch.randint(0, V, (B, 64), generator=g, dtype=torch.int32)
    kw = dict(params, uniforms=u.to(dev), history=hist.to(dev), repetition_penalty=1.1)
    return x.to(dev), kw


def _run(L, fn, x, kw, ws=None, ws_bytes=0):
    from tests import _capi

    args, _, B = _capi.sample_args(x, **kw)
    out = _capi.SampleBuffers(B, x.device)
    if fn == "noalloc":
        rc = L.gtp_sample_rows_noalloc(*args, *out.out_args(), _capi.stream_handle())
    else:
        rc = L.gtp_sample_rows(*args, *out.out_args(), ws, ws_bytes, _capi.stream_handle())
    torch.cuda.synchronize()
    return rc, out.cpu()


def _same(a, b, what):
    """Ids, kept sizes, thresholds and statuses bit for bit; the two
    logprobs within 1e-3 (the split kernel's log-sum-exp partials follow its
    dynamic chunk schedule, so their fp32 sum can differ by an ulp from one
    launch to the next)."""
    for k in a:
        va, vb = a[k].numpy(), b[k].numpy()
        if k in ("logprob", "sampled_logprob"):
            assert np.abs(va - vb).max() <= 1e-3, (what, k)
            continue
        if va.dtype == np.float32:
            va, vb = va.view(np.uint32), vb.view(np.uint32)
        assert np.array_equal(va, vb), (what, k)


def test_noalloc_matches_the_workspace_entry_point():
    from tests import _capi

    L = _capi.lib()
    dev = torch.device("cuda:0")
    # split rows (several workgroups per row merge through the workspace),
    # then a smaller call on the same array, then a one-slice greedy call
    cases = [
        (64, 151936, torch.bfloat16, dict(temperature=0.8, top_k=50, top_p=0.9), 1),
        (16, 32768, torch.bfloat16, dict(temperature=1.0, top_k=20), 2),
        (5, 4096, torch.float32, dict(temperature=0.0), 3),
    ]
    for i, (B, V, dtype, params, seed) in enumerate(cases):
        x, kw = _case(B, V, dtype, params, seed, dev)
        _, p, _ = _capi.sample_args(x, **kw)
        need = L.gtp_sample_workspace_bytes(_capi.DTYPE[dtype], B, V, ctypes.byref(p))
        if i < 2:
            assert need > 0  # these calls do use the workspace
        ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=dev)
        print(f"noalloc call {i}: B={B} V={V} {dtype} {params} workspace {need} B", flush=True)
        rc_w, want = _run(L, "workspace", x, kw, ws.data_ptr(), need)
        rc_n, got = _run(L, "noalloc", x, kw)
        assert rc_w == 0 and rc_n == 0
        _same(got, want, f"call {i}")
        assert (got["status"].numpy() == 0).all()


def test_noalloc_rejects_a_call_beyond_its_array():
    """More workspace than the array holds is refused on the host, before
    anything is launched (GTP_ERR_UNSUPPORTED)."""
    from tests import _capi

    L = _capi.lib()
    p = _capi.SamplerParams(1.0, 128, 1.0, 1.0)
    B, V = 8192, 1 << 18
    need = L.gtp_sample_workspace_bytes(0, B, V, ctypes.byref(p))
    assert need > 8 << 20
    dev = torch.device("cuda:0")
    ids = torch.empty(1, dtype=torch.int64, device=dev)
    u = torch.empty(1, dtype=torch.float32, device=dev)
    x = torch.empty(1, dtype=torch.float32, device=dev)
    rc = L.gtp_sample_rows_noalloc(x.data_ptr(), 0, B, V, V, None, 0, 0, None, 0, u.data_ptr(),
                                   ctypes.byref(p), None, 0, ids.data_ptr(), None, None, None,
                                   None, None, None, _capi.stream_handle())
    assert rc == 2


def test_noalloc_top_p_calls_that_need_no_workspace():
    """Top-p calls on the one-workgroup kernels need no workspace (a row
    outside their bounds runs the row-wise path inside the same launch): the
    allocation-free entry point passes none, and its answers equal those of
    gtp_sample_rows called without one, a row that takes the in-kernel
    fallback included."""
    from tests import _capi

    L = _capi.lib()
    dev = torch.device("cuda:0")
    cases = [
        (96, 70000, torch.bfloat16, dict(temperature=0.8, top_p=0.9), 4),  # > 64 rows: one workgroup per row
        (8, 70000, torch.float32, dict(temperature=0.7, top_p=0.9), 5),    # fp32 top-p kernel
    ]
    for i, (B, V, dtype, params, seed) in enumerate(cases):
        x, kw = _case(B, V, dtype, params, seed, dev)
        x[1, 7] = float("-inf") if dtype == torch.bfloat16 else 3.0e4  # the in-kernel fallback
        _, p, _ = _capi.sample_args(x, **kw)
        assert L.gtp_sample_workspace_bytes(_capi.DTYPE[dtype], B, V, ctypes.byref(p)) == 0
        print(f"noalloc top-p call {i}: B={B} V={V} {dtype} {params}", flush=True)
        rc_w, want = _run(L, "workspace", x, kw, None, 0)
        rc_n, got = _run(L, "noalloc", x, kw)
        assert rc_w == 0 and rc_n == 0
        _same(got, want, f"top-p call {i}")
        assert (got["status"].numpy() == 0).all()
