"""The C ABI library loads and exports every entry point the public header
declares; the torch extension registers its ops and rejects bad tensors on
the host.  No kernel is launched (CPU-only)."""

import ctypes
import os
import re

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
