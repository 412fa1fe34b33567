"""CPU oracle for the vocabulary-wide token path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only to check or time the HIP path.
The product package (``graspo_amd``) never imports it and has no CPU fallback.

Two oracles live here:

* the *exact* oracle: ``tokpath_oracle.c`` through ctypes.  It restates the
  sampler contract of ``include/graspo_tokpath.h`` (fixed-point weights,
  exact integer top-p / draw comparisons) by sorting whole rows.  GPU ids,
  kept-set sizes and thresholds must equal it bit for bit.
* the *semantic* oracle: a literal fp64 torch restatement of the reference's
  sampler (src/graspo/backends/graspoflow/tensor_utils.py:649-683: temperature,
  softmax, descending sort, cumsum, shifted ``cum > top_p`` cut, renormalise,
  draw) and of its logprob (src/graspo/core/graspo_loss.py:19-21), extended
  with the repetition penalty / mask / top-k / supplied-uniform steps of the
  contract.  The exact oracle must agree with it everywhere except at measured
  near-ties, which the tests report.  ``torch.multinomial`` is replaced by the
  inverse CDF of the supplied uniform (the global-RNG draw cannot be pinned).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtokpath_oracle.so")

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
ROW_OK, ROW_NONFINITE, ROW_EMPTY, ROW_BAD_HISTORY, ROW_BAD_UNIFORM, ROW_BAD_TARGET = range(6)


class SamplerParams(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_int32),
        ("top_p", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
    ]


_lib = None


def build(force: bool = False) -> str:
    """Compile the C oracle with its Makefile; returns the library path."""
    src = os.path.join(HERE, "tokpath_oracle.c")
    if force or not os.path.exists(LIB_PATH) or os.path.getmtime(LIB_PATH) < os.path.getmtime(src):
        subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32, c_int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int
        L.gtp_oracle_detexp_fix.argtypes = [ctypes.c_float]
        L.gtp_oracle_detexp_fix.restype = ctypes.c_uint64
        L.gtp_oracle_floor_mul.argtypes = [ctypes.c_float, ctypes.c_uint64]
        L.gtp_oracle_floor_mul.restype = ctypes.c_uint64
        L.gtp_oracle_sample_rows.argtypes = [
            vp, c_int, i64, i64, i64, vp, i64, i64, vp, i64, vp,
            ctypes.POINTER(SamplerParams), vp, i64, vp, vp, vp, vp, vp, vp, vp,
        ]
        L.gtp_oracle_sample_rows.restype = c_int
        L.gtp_oracle_logprob_entropy_rows.argtypes = [vp, c_int, i64, i64, i64, vp, c_int, vp, vp, vp]
        L.gtp_oracle_logprob_entropy_rows.restype = c_int
        L.gtp_oracle_version.restype = ctypes.c_char_p
        del i32
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data


def logits_dtype_code(a: np.ndarray, is_bf16: bool = False) -> int:
    if a.dtype == np.float32:
        return DTYPE_F32
    if a.dtype == np.uint16:
        return DTYPE_BF16 if is_bf16 else DTYPE_F16
    if a.dtype == np.float16:
        return DTYPE_F16
    raise TypeError(f"unsupported logits dtype {a.dtype}")


def detexp_fix(d: float) -> int:
    return int(lib().gtp_oracle_detexp_fix(ctypes.c_float(d)))


def floor_mul(f: float, W: int) -> int:
    return int(lib().gtp_oracle_floor_mul(ctypes.c_float(f), ctypes.c_uint64(W)))


@dataclass
class SampleResult:
    ids: np.ndarray
    logprob: np.ndarray
    sampled_logprob: np.ndarray
    kept: np.ndarray
    thresh_value: np.ndarray
    thresh_id: np.ndarray
    status: np.ndarray


def sample_rows(
    logits: np.ndarray,
    dtype: int,
    *,
    temperature: float,
    top_k: int = 0,
    top_p: float = 1.0,
    repetition_penalty: float = 1.0,
    history: np.ndarray | None = None,
    allow_mask: np.ndarray | None = None,
    uniforms: np.ndarray | None = None,
    finished: np.ndarray | None = None,
    pad_token_id: int = 0,
    V: int | None = None,
) -> SampleResult:
    """Exact oracle.  ``logits`` is [B, row_stride] float32, or uint16 bit
    patterns of bf16/fp16 (``dtype`` says which)."""
    B, row_stride = logits.shape
    V = row_stride if V is None else V
    hist_len = 0 if history is None else history.shape[1]
    hist_stride = hist_len
    mask_stride = 0 if allow_mask is None else allow_mask.shape[1]
    if history is not None:
        history = np.ascontiguousarray(history, dtype=np.int32)
    if allow_mask is not None:
        allow_mask = np.ascontiguousarray(allow_mask, dtype=np.uint32)
    if uniforms is not None:
        uniforms = np.ascontiguousarray(uniforms, dtype=np.float32)
    if finished is not None:
        finished = np.ascontiguousarray(finished, dtype=np.uint8)
    logits = np.ascontiguousarray(logits)
    out = SampleResult(
        ids=np.empty(B, np.int64),
        logprob=np.empty(B, np.float32),
        sampled_logprob=np.empty(B, np.float32),
        kept=np.empty(B, np.int32),
        thresh_value=np.empty(B, np.float32),
        thresh_id=np.empty(B, np.int32),
        status=np.empty(B, np.int32),
    )
    p = SamplerParams(float(temperature), int(top_k), float(top_p), float(repetition_penalty))
    rc = lib().gtp_oracle_sample_rows(
        _ptr(logits), dtype, B, V, row_stride, _ptr(history), hist_len, hist_stride,
        _ptr(allow_mask), mask_stride, _ptr(uniforms), ctypes.byref(p), _ptr(finished),
        int(pad_token_id), _ptr(out.ids), _ptr(out.logprob), _ptr(out.sampled_logprob),
        _ptr(out.kept), _ptr(out.thresh_value), _ptr(out.thresh_id), _ptr(out.status),
    )
    if rc != 0:
        raise ValueError(f"gtp_oracle_sample_rows returned {rc}")
    return out


def logprob_entropy_rows(logits: np.ndarray, dtype: int, targets: np.ndarray, V: int | None = None):
    """Exact-arithmetic (fp64) logprob / entropy oracle; returns (lp, H, status)."""
    N, row_stride = logits.shape
    V = row_stride if V is None else V
    logits = np.ascontiguousarray(logits)
    t64 = targets.dtype == np.int64
    targets = np.ascontiguousarray(targets, dtype=np.int64 if t64 else np.int32)
    lp = np.empty(N, np.float32)
    H = np.empty(N, np.float32)
    st = np.empty(N, np.int32)
    rc = lib().gtp_oracle_logprob_entropy_rows(
        _ptr(logits), dtype, N, V, row_stride, _ptr(targets), int(t64), _ptr(lp), _ptr(H), _ptr(st)
    )
    if rc != 0:
        raise ValueError(f"gtp_oracle_logprob_entropy_rows returned {rc}")
    return lp, H, st


# ------------------------------------------------------------------ bits io

def bits_to_f32(a: np.ndarray, dtype: int) -> np.ndarray:
    """Exact fp32 values of a bf16/fp16 bit-pattern array (or pass fp32)."""
    if dtype == DTYPE_F32:
        return a.astype(np.float32)
    if dtype == DTYPE_BF16:
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.view(np.float16).astype(np.float32)


def mask_bits(allow_mask: np.ndarray, V: int) -> np.ndarray:
    """[B, ceil(V/32)] uint32 LSB-first words -> [B, V] bool."""
    bits = np.unpackbits(allow_mask.astype("<u4").view(np.uint8), axis=1, bitorder="little")
    return bits[:, :V].astype(bool)


# -------------------------------------------------------- semantic (fp64)

def penalize_f32(x: np.ndarray, history: np.ndarray | None, rho: float) -> np.ndarray:
    """HF-style repetition penalty on fp32 rows: one IEEE op per penalised id."""
    x = x.astype(np.float32, copy=True)
    if history is None or rho == 1.0:
        return x
    rho32 = np.float32(rho)
    V = x.shape[1]
    for b in range(x.shape[0]):
        h = history[b]
        ids = np.unique(h[(h >= 0) & (h < V)])
        v = x[b, ids]
        x[b, ids] = np.where(v < 0, v * rho32, v / rho32)
    return x


def sample_semantic(
    x: np.ndarray,
    *,
    temperature: float,
    top_k: int = 0,
    top_p: float = 1.0,
    repetition_penalty: float = 1.0,
    history: np.ndarray | None = None,
    allow_mask: np.ndarray | None = None,
    uniforms: np.ndarray | None = None,
):
    """Literal fp64 restatement of tensor_utils.py:649-683 (+ contract extensions).

    Returns per row (id, kept, cut_margin, draw_margin, p_sampled): the
    margins are the distance of the top-p comparison and of the uniform from
    the nearest decision boundary, so callers can tell near-ties from
    disagreements; p_sampled is the drawn token's probability in the
    renormalised kept set (tensor_utils.py:679-683), 1 for greedy rows."""
    import torch

    x = np.asarray(x, dtype=np.float32)
    B, V = x.shape
    xp = penalize_f32(x, history, repetition_penalty)
    allowed = np.ones((B, V), bool) if allow_mask is None else mask_bits(allow_mask, V)
    out = []
    for b in range(B):
        row = torch.from_numpy(xp[b].copy())
        if temperature > 0:
            row = row / np.float32(max(float(temperature), 1e-6))  # tensor_utils.py:656
        else:
            allow = torch.from_numpy(allowed[b])
            if not bool(allow.any()):
                out.append((-1, 0, np.inf, np.inf, np.nan))
                continue
            masked = torch.where(allow, row, torch.tensor(-np.inf))
            gid = int(torch.argmax(masked))  # tensor_utils.py:658 (NaN, then +inf, win)
            if not bool(allow[gid]):  # every allowed token is -inf: the first of them
                gid = int(allow.nonzero()[0])
            out.append((gid, 1, np.inf, np.inf, 1.0))
            continue
        y = row.double()
        y = torch.where(torch.from_numpy(allowed[b]), y, torch.tensor(-np.inf, dtype=torch.float64))
        valid = int(torch.isfinite(y).sum())
        # stable descending sort == order (y desc, id asc)
        ys, idx = torch.sort(y, descending=True, stable=True)
        nk = top_k if 0 < top_k < valid else valid
        probs = torch.softmax(ys[:nk], dim=-1)  # tensor_utils.py:672 (over the top-k)
        R = nk
        cut_margin = np.inf
        if 0.0 < top_p < 1.0:  # tensor_utils.py:673-678
            cum = torch.cumsum(probs, dim=-1)
            remove = cum > top_p
            remove[1:] = remove[:-1].clone()
            remove[0] = False
            R = int((~remove).sum())
            excl = torch.cat([torch.zeros(1, dtype=torch.float64), cum[:-1]])
            cut_margin = float((excl - top_p).abs().min())
        kept = probs[:R] / probs[:R].sum().clamp_min(1e-12)  # tensor_utils.py:679-680
        cdf = torch.cumsum(kept, dim=-1)
        u = float(uniforms[b])
        r = int(torch.searchsorted(cdf, torch.tensor([u], dtype=torch.float64), right=True)[0])
        r = min(r, R - 1)
        draw_margin = float((cdf - u).abs().min())
        out.append((int(idx[r]), R, cut_margin, draw_margin, float(kept[r])))
    return out


def logprob_entropy_semantic(x: np.ndarray, targets: np.ndarray):
    """fp64 log_softmax + gather (graspo_loss.py:19-21) and entropy."""
    import torch

    t = torch.from_numpy(np.asarray(x, dtype=np.float64))
    ls = torch.log_softmax(t, dim=-1)
    lp = ls.gather(-1, torch.from_numpy(targets.astype(np.int64)).unsqueeze(-1)).squeeze(-1)
    p = ls.exp()
    H = -(torch.where(p > 0, p * ls, torch.zeros_like(p))).sum(-1)
    return lp.numpy(), H.numpy()
