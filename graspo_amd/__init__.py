"""graspo_amd -- MI355X-native vocabulary-wide token path for GRASPO.

The rollout sampler and the selective log-softmax / entropy of the GRASPO
loss, as hand-written gfx950 HIP kernels behind a C ABI
(``include/graspo_tokpath.h``, ``libgraspo_tokpath.so``) and a thin PyTorch
extension (``torch.ops.graspo_tokpath``).

* :mod:`graspo_amd.ops` -- tensor-level entry points.
* :mod:`graspo_amd.tensor_utils` / :mod:`graspo_amd.graspo_loss` -- drop-ins
  with the reference's names and signatures.
* :mod:`graspo_amd.integration` -- installs the drop-ins into an imported
  ``graspo`` package without editing its call sites.

There is no CPU fallback: every op raises if the native libraries are not
built (``python -m graspo_amd.build``) or the tensors are not on a GPU.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgraspo_tokpath.so")
EXT_PATH = os.path.join(HERE, "_graspo_tokpath_ops.so")

_state: dict = {"lib": None, "ops": None}


def load():
    """Load libgraspo_tokpath.so and register torch.ops.graspo_tokpath.

    Raises RuntimeError when the libraries have not been built."""
    if _state["ops"] is not None:
        return _state["ops"]
    import torch  # torch first: the HIP runtime it loads is the one we bind to

    missing = [p for p in (LIB_PATH, EXT_PATH) if not os.path.exists(p)]
    if missing:
        raise RuntimeError(
            "graspo_amd: native libraries not built (missing "
            + ", ".join(os.path.basename(p) for p in missing)
            + "); run `python -m graspo_amd.build`"
        )
    _state["lib"] = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    torch.ops.load_library(EXT_PATH)
    _state["ops"] = torch.ops.graspo_tokpath
    return _state["ops"]


def native_library() -> ctypes.CDLL:
    """The ctypes handle of libgraspo_tokpath.so (loads it if needed)."""
    load()
    return _state["lib"]


__all__ = ["load", "native_library", "LIB_PATH", "EXT_PATH"]
