"""The C ABI library loads and exports every entry point the public header
declares; the torch extension registers its ops and rejects bad tensors on
the host.  No kernel is launched (CPU-only)."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

import graspo_amd
from graspo_amd import integration

HEADER = os.path.join(os.path.dirname(graspo_amd.HERE), "include", "graspo_tokpath.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gtp_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("gtp_sample_rows", "gtp_logprob_entropy_rows", "gtp_lse_partial_rows",
              "gtp_lse_finalize_rows", "gtp_version"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(graspo_amd.LIB_PATH)
    for s in declared_symbols():
        assert hasattr(lib, s), f"{s} not exported by libgraspo_tokpath.so"
    lib.gtp_version.restype = ctypes.c_char_p
    assert b"gfx950" in lib.gtp_version()


def test_sample_route_on_the_host():
    """gtp_sample_route (host-only; without a GPU the library plans for 256
    compute units) names the kernel each call shape takes: the split top-k
    sampler, the split and one-workgroup bf16 top-p kernels, the fp32 top-p
    kernel, the value-histogram kernel and the row-wise kernel."""
    from tests import _capi

    L = _capi.lib()
    F32, BF16, F16 = 0, 1, 2
    R = _capi
    assert R.route(L, BF16, 256, 248320, T=0.7, k=64, P=0.9, rho=1.05, hist_len=4096,
                   mask=True) == (R.ROUTE_SPLIT_TOPK, 1)
    assert R.route(L, F32, 8, 151936, T=0.7, k=50, P=0.9) == (R.ROUTE_SPLIT_TOPK, 8)
    assert R.route(L, BF16, 64, 151936, T=1.0, P=0.95, rho=1.1,
                   hist_len=2048) == (R.ROUTE_TOPP_SPLIT, 4)
    assert R.route(L, BF16, 64, 151936, T=0.8, P=0.9, mask=True) == (R.ROUTE_TOPP, 1)
    assert R.route(L, BF16, 256, 248320, T=0.7, P=0.9) == (R.ROUTE_TOPP, 1)
    assert R.route(L, F32, 256, 248320, T=0.7, P=0.9) == (R.ROUTE_TOPP32, 1)
    # the one-workgroup top-p kernels need no workspace; the split one does
    assert R.route(L, F32, 256, 248320, T=0.7, P=0.9, workspace=0) == (R.ROUTE_TOPP32, 1)
    assert R.route(L, BF16, 256, 248320, T=0.7, P=0.9, workspace=0) == (R.ROUTE_TOPP, 1)
    assert R.route(L, BF16, 16, 248320, T=0.7, P=0.9, workspace=0) == (R.ROUTE_TOPP, 1)
    assert R.route(L, BF16, 4, 70000, T=1.0, P=0.9, workspace=0, aligned=False)[0] == R.ROUTE_ROWWISE
    # the allocation-free entry point's 8 MiB array: 7 slices for 16 decode rows
    assert R.route(L, BF16, 16, 248320, T=0.7, P=0.9)[0] == R.ROUTE_TOPP_SPLIT
    assert R.route(L, BF16, 16, 248320, T=0.7, P=0.9,
                   workspace=R.NOALLOC_SCRATCH_BYTES) == (R.ROUTE_TOPP_SPLIT, 7)
    assert R.route(L, BF16, 4, 60000, T=1.0, P=0.9) == (R.ROUTE_HIST, 1)   # V < 65536
    assert R.route(L, BF16, 4, 70000, T=1.0, k=300) == (R.ROUTE_HIST, 1)   # top-k > 128
    assert R.route(L, F16, 4, 70000, T=1.0, P=0.9) == (R.ROUTE_ROWWISE, 1)
    assert R.route(L, BF16, 4, 70000, T=1.0, k=5, aligned=False)[0] == R.ROUTE_ROWWISE
    assert R.route(L, BF16, 4, 70000, T=0.0, aligned=True)[0] == R.ROUTE_SPLIT_TOPK


def test_invalid_arguments_rejected_before_launch():
    lib = ctypes.CDLL(graspo_amd.LIB_PATH)
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.gtp_logprob_entropy_rows.argtypes = [vp, ctypes.c_int, i64, i64, i64, vp, ctypes.c_int,
                                             vp, vp, vp, vp]
    # V = 0, row_stride < V, bad dtype: all rejected on the host
    assert lib.gtp_logprob_entropy_rows(None, 1, 4, 0, 0, None, 0, None, None, None, None) == 1
    assert lib.gtp_logprob_entropy_rows(1, 1, 4, 10, 5, 1, 0, 1, None, None, None) == 1
    assert lib.gtp_logprob_entropy_rows(1, 9, 4, 10, 10, 1, 0, 1, None, None, None) == 1
    # zero rows is a no-op success
    assert lib.gtp_logprob_entropy_rows(None, 1, 0, 10, 10, None, 0, None, None, None, None) == 0


def test_torch_ops_registered_and_reject_cpu_tensors():
    ops = graspo_amd.load()
    for name in ("sample", "logprob_entropy", "lse_partial", "lse_finalize"):
        assert hasattr(ops, name)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        ops.logprob_entropy(torch.zeros(2, 8), torch.zeros(2, dtype=torch.int64), 0)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        ops.sample(torch.zeros(2, 8), 0.0, 0, 1.0, 1.0, None, None, None, None, 0, 0)


def test_integration_rebinds_and_restores(monkeypatch):
    """install() rebinds the hot-path names in modules laid out like the
    reference package and uninstall() restores them."""
    import sys
    import types

    names = {
        "graspo": None,
        "graspo.backends": None,
        "graspo.backends.graspoflow": None,
        "graspo.backends.graspoflow.tensor_utils": integration._SAMPLER_NAMES
        + integration._LOGPROB_NAMES,
        "graspo.backends.graspoflow.models": None,
        "graspo.backends.graspoflow.models.qwen3": None,
        "graspo.backends.graspoflow.models.qwen3.adapter": integration._SAMPLER_NAMES,
        "graspo.core": None,
        "graspo.core.graspo_loss": ("sequence_log_probs_from_logits",),
    }
    originals = {}
    for mod_name, attrs in names.items():
        m = types.ModuleType(mod_name)
        for a in attrs or ():
            f = lambda *args, **kw: "reference"  # noqa: E731
            setattr(m, a, f)
            originals[(mod_name, a)] = f
        monkeypatch.setitem(sys.modules, mod_name, m)
    done = integration.install()
    assert ("graspo.backends.graspoflow.models.qwen3.adapter", "_next_token_from_logits") in done
    tu = sys.modules["graspo.backends.graspoflow.tensor_utils"]
    assert tu._next_token_from_logits is integration.REPLACEMENTS["_next_token_from_logits"]
    gl = sys.modules["graspo.core.graspo_loss"]
    assert gl.sequence_log_probs_from_logits is integration.REPLACEMENTS[
        "sequence_log_probs_from_logits"]
    integration.uninstall()
    for (mod_name, a), f in originals.items():
        assert getattr(sys.modules[mod_name], a) is f


def test_graspo_loss_has_no_cpu_path():
    """The fused loss runs on the GPU only; CPU tensors are rejected."""
    from graspo_amd.graspo_loss import GRASPOLoss

    x = torch.zeros(2, 3)
    with pytest.raises(RuntimeError):
        GRASPOLoss(policy_ratio_clip_eps=0.2)(x, x, x, torch.ones(2, 3, dtype=torch.bool))


@pytest.mark.gpu
def test_graspo_loss_known_answer():
    """The reference's own known-answer case (tests/core/test_graspo_loss.py:8-24)."""
    from graspo_amd.graspo_loss import GRASPOLoss

    dev = torch.device("cuda:0")
    log_probs = torch.tensor([[0.0, 0.2, -0.1], [0.1, -0.3, 0.4]])
    old = torch.tensor([[-0.1, 0.1, -0.1], [0.0, -0.1, 0.2]])
    adv = torch.tensor([[1.0, 1.0, 1.0], [-0.5, -0.5, -0.5]])
    mask = torch.tensor([[True, True, False], [True, False, True]])
    r = torch.exp(log_probs - old)
    per = -torch.min(r * adv, r.clamp(0.8, 1.2) * adv)
    want = ((per * mask).sum(-1) / mask.sum(-1)).mean()
    got = GRASPOLoss(policy_ratio_clip_eps=0.2)(log_probs.to(dev), old.to(dev), adv.to(dev),
                                                mask.to(dev)).cpu()
    assert torch.allclose(got, want)
    # the same case worked by hand: row 0 keeps ratios e^0.1 (inside the clip)
    # on two tokens; row 1 (advantage -0.5) keeps the unclipped e^0.2 term
    import math

    row0 = -math.exp(0.1)
    row1 = (0.5 * math.exp(0.1) + 0.5 * math.exp(0.2)) / 2
    assert abs(float(got) - (row0 + row1) / 2) < 1e-6


def test_integration_rebinds_decode_loop_methods(monkeypatch):
    """install() replaces the adapters' decode-loop methods on their classes
    (subclasses inherit them) and uninstall() restores the originals."""
    import sys
    import types

    from graspo_amd import decode_loop

    mods = {}
    for mod_name, classes in integration.METHOD_TARGETS.items():
        m = types.ModuleType(mod_name)
        for cls_name, names in classes.items():
            cls = type(cls_name, (), {n: (lambda self, **kw: "reference") for n in names})
            setattr(m, cls_name, cls)
        monkeypatch.setitem(sys.modules, mod_name, m)
        mods[mod_name] = m
    done = integration.install(targets={})
    adapter_cls = mods["graspo.backends.graspoflow.models.qwen3.adapter"].Qwen3Adapter
    assert adapter_cls._generate_group_with_kv_cache is decode_loop.generate_group_with_kv_cache
    mixin = mods["graspo.backends.graspoflow.models.qwen35_36.generation"]._Qwen35GenerationMethods
    sub = type("Qwen35Adapter", (mixin,), {})
    assert sub._generate_multimodal_full_forward is decode_loop.generate_multimodal_full_forward
    assert len(done) == 6
    integration.uninstall()
    assert adapter_cls._generate_group_with_kv_cache(None) == "reference"
    assert sub._generate_multimodal_full_forward(None) == "reference"


def test_decode_loop_has_no_cpu_path():
    from graspo_amd.decode_loop import DecodeState

    with pytest.raises(RuntimeError, match="no CPU path"):
        DecodeState(torch.zeros(2, 3, dtype=torch.int64), torch.zeros(2, dtype=torch.bool), 1, 0, 4)
    with pytest.raises(RuntimeError, match="GPU"):
        graspo_amd.load().decode_update(torch.zeros(2, dtype=torch.int64), None,
                                        torch.zeros(2, dtype=torch.bool), 1, 0, None, None, 0,
                                        torch.zeros(2, dtype=torch.int32), 0)


def _device_case(case, dev):
    """(logits, kwargs) of one raw-ABI sampler case, on the device."""
    from graspo_amd import workloads as W

    kind = case[0]
    if kind == "workload":
        wl = W.sampler_workload(case[1], rows=case[2])
        kw = wl.kwargs()
        kw.update(case[3])
        return wl.logits.to(dev), {k: (v.to(dev) if isinstance(v, torch.Tensor) else v)
                                   for k, v in kw.items()}
    _, B, V, dtype, params, seed = case
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, V, generator=g) * 2.5).to(dtype)
    u = ((torch.randint(0, 1 << 24, (B,), generator=g).float()) * 2.0 ** -24)
    return x.to(dev), dict(params, uniforms=u.to(dev))


# Calls in a row on one caller-owned workspace: B, V, dtype and top-k all
# change from call to call (split rows with S > 1, one-slice rows, greedy,
# and the one-workgroup paths that need no workspace).
RAW_CASES = [
    ("workload", 2, 64, dict(top_k=50)),                            # bf16, S = 4
    ("workload", 1, 8, {}),                                         # fp32 [8, 151936], k 50
    ("rand", 3, 40000, torch.bfloat16, dict(temperature=0.0), 1),   # greedy
    ("workload", 5, 256, {}),                                       # the large batch, S = 1
    ("rand", 17, 151936, torch.bfloat16, dict(temperature=0.8, top_k=128), 2),
    ("workload", 3, 64, {}),                                        # top-p, S = 4 per row
    ("rand", 64, 151936, torch.float32, dict(temperature=1.0, top_k=9, top_p=0.5), 3),
    # a split call with more rows than the earlier ones: its arrival counters
    # reach past where a 64-row call's slots would start
    ("rand", 100, 151936, torch.bfloat16, dict(temperature=0.9, top_k=20), 4),
    ("rand", 40, 151936, torch.float32, dict(temperature=0.7, top_p=0.9), 5),  # fp32 top-p
    ("rand", 100, 151936, torch.bfloat16, dict(temperature=0.9, top_k=20), 6),
    ("rand", 100, 151936, torch.bfloat16, dict(temperature=0.8, top_p=0.9), 7),  # one workgroup
    ("rand", 5, 248320, torch.bfloat16, dict(temperature=0.7, top_p=0.95), 8),   # top-p, S = 8
    ("rand", 64, 151936, torch.bfloat16, dict(temperature=0.9, top_k=40), 9),
]


@pytest.mark.gpu
def test_raw_abi_sampler_calls_share_one_workspace():
    """gtp_sample_rows through ctypes on caller-owned device buffers, as a
    non-torch caller binds it: one workspace sized by
    gtp_sample_workspace_bytes over every call, zero-filled once, then
    reused by calls whose B, V, dtype and top-k change.  Each call is
    bit-exact against the oracle (ids, kept, threshold, status)."""
    from tests import _capi
    from tests._util import oracle_sample

    L = _capi.lib()
    dev = torch.device("cuda:0")
    cases = [_device_case(c, dev) for c in RAW_CASES]
    need = 0
    for x, kw in cases:
        _, p, B = _capi.sample_args(x, **kw)
        need = max(need, L.gtp_sample_workspace_bytes(_capi.DTYPE[x.dtype], B, x.shape[1],
                                                      ctypes.byref(p)))
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)  # zero-filled once
    for i, (x, kw) in enumerate(cases):
        print("raw abi sampler call", i, RAW_CASES[i][:3], flush=True)
        args, p, B = _capi.sample_args(x, **kw)
        out = _capi.SampleBuffers(B, dev)
        rc = L.gtp_sample_rows(*args, *out.out_args(), ws.data_ptr(), need,
                               _capi.stream_handle())
        assert rc == 0
        torch.cuda.synchronize()
        got = out.cpu()
        ref = oracle_sample(x.cpu(), **{k: (v.cpu() if isinstance(v, torch.Tensor) else v)
                                        for k, v in kw.items()})
        assert np.array_equal(got["status"].numpy(), ref.status), i
        assert np.array_equal(got["ids"].numpy(), ref.ids), i
        ok = ref.status == 0
        assert np.array_equal(got["kept"].numpy()[ok], ref.kept[ok]), i
        assert np.array_equal(got["thresh_id"].numpy()[ok], ref.thresh_id[ok]), i
        assert np.array_equal(got["thresh_value"].numpy()[ok].view(np.uint32),
                              ref.thresh_value[ok].view(np.uint32)), i
        assert np.abs(got["logprob"].numpy()[ok] - ref.logprob[ok]).max() <= 1e-3, i


@pytest.mark.gpu
def test_raw_abi_logprob_and_decode_update():
    """gtp_logprob_entropy_rows and gtp_decode_update_rows through ctypes on
    caller-owned buffers: logprob / entropy against the oracle within 1e-3,
    the decode bookkeeping against its definition."""
    from graspo_amd import workloads as W
    from tests import _capi
    from tests._util import oracle_logprob

    L = _capi.lib()
    dev = torch.device("cuda:0")
    for N, kind in ((300, "int32"), (77, "int64")):
        x, t = W.logprob_workload(5, rows=N)
        t = t.to(torch.int64) if kind == "int64" else t
        xd, td = x.to(dev), t.to(dev)
        lp = torch.empty(N, dtype=torch.float32, device=dev)
        H = torch.empty(N, dtype=torch.float32, device=dev)
        st = torch.full((N,), -7, dtype=torch.int32, device=dev)
        print("raw abi logprob", N, kind, flush=True)
        rc = L.gtp_logprob_entropy_rows(xd.data_ptr(), 1, N, x.shape[1], x.shape[1],
                                        td.data_ptr(), int(kind == "int64"), lp.data_ptr(),
                                        H.data_ptr(), st.data_ptr(), _capi.stream_handle())
        assert rc == 0
        torch.cuda.synchronize()
        rlp, rH, rst = oracle_logprob(x, t)
        assert (st.cpu().numpy() == 0).all()
        assert np.abs(lp.cpu().numpy() - rlp).max() <= 1e-3
        assert np.abs(H.cpu().numpy() - rH).max() <= 1e-3

    B, pad, eos, col = 37, 0, 5, 3
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, 9, (B,), generator=g)
    status = (torch.rand(B, generator=g) < 0.1).to(torch.int32)
    ids[status.bool()] = -1
    fin = torch.rand(B, generator=g) < 0.2
    want_ids = torch.where(status.bool(), torch.full_like(ids, pad), ids)
    want_fin = fin | want_ids.eq(eos)
    ids_d, st_d, fin_d = ids.to(dev), status.to(dev), fin.to(torch.uint8).to(dev)
    seq = torch.full((B, 8), -3, dtype=torch.int64, device=dev)
    attn = torch.zeros((B, 8), dtype=torch.uint8, device=dev)
    flags = torch.zeros(2, dtype=torch.int32, device=dev)
    print("raw abi decode update", flush=True)
    rc = L.gtp_decode_update_rows(ids_d.data_ptr(), st_d.data_ptr(), B, eos, pad,
                                  fin_d.data_ptr(), seq.data_ptr(), 8, attn.data_ptr(), 8, col,
                                  flags.data_ptr(), _capi.stream_handle())
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(ids_d.cpu(), want_ids)
    assert torch.equal(fin_d.cpu().bool(), want_fin)
    assert torch.equal(seq[:, col].cpu(), want_ids)
    assert torch.equal(attn[:, col].cpu().bool(), want_ids.ne(pad))
    assert flags.cpu().tolist() == [int((~want_fin).sum()), int(status.ne(0).sum())]
