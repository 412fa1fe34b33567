"""Install the gfx950 drop-ins into an imported ``graspo`` package.

The reference's adapters import the hot-path helpers *by name* at module
level (e.g. ``src/graspo/backends/graspoflow/models/qwen35_36/generation.py:20-24``,
``models/qwen3/adapter.py:25-32``), and Python resolves such names through
each importing module's globals at call time.  Rebinding those globals is
therefore enough: no reference call site is edited.

    import graspo_amd.integration as gi
    patched = gi.install()      # after graspo is importable
    ...
    gi.uninstall()
"""

from __future__ import annotations

import importlib

from . import decode_loop as _dl
from . import graspo_loss as _loss
from . import sft_loss as _sft
from . import tensor_utils as _tu

_TU = "graspo.backends.graspoflow.tensor_utils"
_SAMPLER_NAMES = ("_next_token_from_logits", "_sample_next_token", "_broadcast_and_pad_finished")
_LOGPROB_NAMES = ("_selected_token_log_probs_from_hidden",)

# module -> names it binds (from the reference's import lists)
TARGETS: dict[str, tuple[str, ...]] = {
    _TU: _SAMPLER_NAMES + _LOGPROB_NAMES,
    "graspo.backends.graspoflow.models.qwen35_36.generation": _SAMPLER_NAMES,
    "graspo.backends.graspoflow.models.qwen3.adapter": _SAMPLER_NAMES,
    "graspo.backends.graspoflow.models.qwen3.model": _LOGPROB_NAMES,
    "graspo.backends.graspoflow.models.qwen35_36.model": _LOGPROB_NAMES,
    "graspo.backends.graspoflow.models.qwen35_36.logprobs": _LOGPROB_NAMES,
    "graspo.backends.graspoflow.models.qwen35_36.training": _LOGPROB_NAMES,
    "graspo.backends.graspoflow.transformer_adapter": _LOGPROB_NAMES,
    # GRASPOLoss is imported inside the adapters' __init__ (transformer_adapter.py:118),
    # so install() must run before the adapter is built
    "graspo.core.graspo_loss": ("sequence_log_probs_from_logits", "GRASPOLoss"),
    # imported inside transformer_adapter.compute_loss (transformer_adapter.py:467),
    # so the module attribute is what that call resolves
    "graspo.core.sft_loss": ("sft_cross_entropy_loss",),
}

REPLACEMENTS = {
    "_next_token_from_logits": _tu._next_token_from_logits,
    "_sample_next_token": _tu._sample_next_token,
    "_broadcast_and_pad_finished": _tu._broadcast_and_pad_finished,
    "_selected_token_log_probs_from_hidden": _tu._selected_token_log_probs_from_hidden,
    "sequence_log_probs_from_logits": _loss.sequence_log_probs_from_logits,
    "sft_cross_entropy_loss": _sft.sft_cross_entropy_loss,
    "GRASPOLoss": _loss.GRASPOLoss,
}

# module -> class -> decode-loop methods replaced on that class (the loops
# call the sampler, pad, track EOS and test all-finished each token)
_TEXT_LOOPS = ("_generate_group_with_kv_cache", "_generate_group_full_forward")
METHOD_TARGETS: dict[str, dict[str, tuple[str, ...]]] = {
    "graspo.backends.graspoflow.models.qwen3.adapter": {"Qwen3Adapter": _TEXT_LOOPS},
    "graspo.backends.graspoflow.models.qwen35_36.generation": {
        "_Qwen35GenerationMethods": _TEXT_LOOPS
        + ("_generate_multimodal_with_kv_cache", "_generate_multimodal_full_forward"),
    },
}

METHOD_REPLACEMENTS = {
    "_generate_group_with_kv_cache": _dl.generate_group_with_kv_cache,
    "_generate_group_full_forward": _dl.generate_group_full_forward,
    "_generate_multimodal_with_kv_cache": _dl.generate_multimodal_with_kv_cache,
    "_generate_multimodal_full_forward": _dl.generate_multimodal_full_forward,
}

_saved: dict[tuple[str, str], object] = {}
_saved_methods: dict[tuple[str, str, str], object] = {}


def install(targets: dict[str, tuple[str, ...]] | None = None, *, strict: bool = False,
            methods: dict[str, dict[str, tuple[str, ...]]] | None = None):
    """Rebind the hot-path names in every importable target module, and the
    decode-loop methods on the adapter classes.

    Returns the list of ``(module, name)`` pairs (``(module, class.method)``
    for methods) that were replaced.  With ``strict`` a module that cannot be
    imported raises; otherwise it is skipped (a model family that is not
    installed)."""
    done = []
    for mod_name, classes in (METHOD_TARGETS if methods is None else methods).items():
        try:
            mod = importlib.import_module(mod_name)
        except ImportError:
            if strict:
                raise
            continue
        for cls_name, names in classes.items():
            cls = getattr(mod, cls_name, None)
            if cls is None:
                continue
            for name in names:
                if name not in cls.__dict__:
                    continue
                key = (mod_name, cls_name, name)
                if key not in _saved_methods:
                    _saved_methods[key] = cls.__dict__[name]
                setattr(cls, name, METHOD_REPLACEMENTS[name])
                done.append((mod_name, f"{cls_name}.{name}"))
    for mod_name, names in (TARGETS if targets is None else targets).items():
        try:
            mod = importlib.import_module(mod_name)
        except ImportError:
            if strict:
                raise
            continue
        for name in names:
            if not hasattr(mod, name):
                continue
            key = (mod_name, name)
            if key not in _saved:
                _saved[key] = getattr(mod, name)
            setattr(mod, name, REPLACEMENTS[name])
            done.append(key)
    return done


def uninstall() -> None:
    """Restore every name :func:`install` replaced."""
    for (mod_name, cls_name, name), orig in list(_saved_methods.items()):
        cls = getattr(importlib.import_module(mod_name), cls_name)
        setattr(cls, name, orig)
        del _saved_methods[(mod_name, cls_name, name)]
    for (mod_name, name), orig in list(_saved.items()):
        mod = importlib.import_module(mod_name)
        setattr(mod, name, orig)
        del _saved[(mod_name, name)]
