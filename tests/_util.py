"""Helpers shared by the tests: tensor <-> oracle conversions."""

from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O


def logits_to_oracle(x: torch.Tensor):
    """CPU numpy view of logits for the C oracle: (array, dtype code)."""
    x = x.detach().cpu().contiguous()
    if x.dtype == torch.bfloat16:
        return x.view(torch.int16).numpy().view(np.uint16), O.DTYPE_BF16
    if x.dtype == torch.float16:
        return x.view(torch.int16).numpy().view(np.uint16), O.DTYPE_F16
    return x.float().numpy(), O.DTYPE_F32


def _np(t):
    return None if t is None else t.detach().cpu().numpy()


def oracle_sample(logits: torch.Tensor, *, temperature, top_k=0, top_p=1.0,
                  repetition_penalty=1.0, history=None, allow_mask=None, uniforms=None,
                  finished=None, pad_token_id=0):
    a, dt = logits_to_oracle(logits)
    return O.sample_rows(
        a, dt, temperature=temperature, top_k=top_k, top_p=top_p,
        repetition_penalty=repetition_penalty, history=_np(history),
        allow_mask=_np(allow_mask), uniforms=_np(uniforms),
        finished=None if finished is None else _np(finished).astype(np.uint8),
        pad_token_id=pad_token_id,
    )


def oracle_logprob(logits: torch.Tensor, targets: torch.Tensor):
    a, dt = logits_to_oracle(logits)
    return O.logprob_entropy_rows(a, dt, _np(targets))


def f32(x: torch.Tensor) -> np.ndarray:
    return x.detach().cpu().float().numpy()
