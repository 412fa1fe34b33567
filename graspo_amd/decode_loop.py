"""Generation decode loops on the gfx950 token path.

Drop-in replacements for the adapters' decode-loop methods (same keyword
arguments, same ``(sequences, timings)`` result, and the same tokens as the
reference loop from the same RNG state):

=====================================================  ===========================================
method                                                 reference
=====================================================  ===========================================
``Qwen3Adapter._generate_group_with_kv_cache``          ``models/qwen3/adapter.py:259-318``
``Qwen3Adapter._generate_group_full_forward``           ``models/qwen3/adapter.py:320-363``
``_Qwen35GenerationMethods._generate_group_with_kv_cache``      ``models/qwen35_36/generation.py:225-284``
``_Qwen35GenerationMethods._generate_group_full_forward``       ``models/qwen35_36/generation.py:286-329``
``_Qwen35GenerationMethods._generate_multimodal_with_kv_cache`` ``models/qwen35_36/generation.py:518-584``
``_Qwen35GenerationMethods._generate_multimodal_full_forward``  ``models/qwen35_36/generation.py:586-641``
=====================================================  ===========================================

What changes against the reference loop body:

* The sampler reads the model's last-position logits in the model's dtype,
  as a strided view.  The reference's ``logits.float()`` copies the whole
  ``[B, S, V]`` output (at prefill, every prompt position) to fp32 first;
  bf16 -> fp32 is exact, so the sampled tokens are the same.
* Padding of finished rows happens inside the sampler; the EOS update, the
  new sequence and attention-mask columns and the all-finished count are one
  kernel (``gtp_decode_update_rows``) writing into buffers sized for
  ``max_new_tokens`` up front, instead of ``torch.cat`` of the whole
  sequence and four small launches per token.
* The host reads step i's all-finished count (copied to pinned memory
  asynchronously) only after it has queued the model forward of step i + 1,
  so the GPU never idles while the host checks ``bool(finished.all())``.
  When every row finished at step i that forward's output is discarded; at
  the last step no forward is queued (the reference runs one there and
  discards it).
* A sampler row error (NaN logits and the like) raises ``RuntimeError`` as
  the reference's ``torch.multinomial`` does, when that step's count is read.

``finished`` is updated in place, as the reference's ``finished |= ...`` does.
With ``synchronize_cuda_timing`` set, ``self._sync_timing()`` synchronises at
the same points as in the reference and the timings mean the same things.
"""

from __future__ import annotations

import time
from typing import Any, Callable

import torch
import torch.distributed as dist

from . import ops


class DecodeState:
    """Device buffers and the lagged stop flag of one decode loop."""

    def __init__(self, sequences: torch.Tensor, finished: torch.Tensor, eos_token_id: int,
                 pad_token_id: int, max_new_tokens: int):
        if sequences.device.type != "cuda":
            raise RuntimeError("graspo_amd decode loop: sequences must be on a GPU; "
                               "there is no CPU path")
        B, S0 = sequences.shape
        total = S0 + max(int(max_new_tokens), 0)
        dev = sequences.device
        self.seq = torch.empty((B, total), dtype=torch.int64, device=dev)
        self.seq[:, :S0].copy_(sequences)
        self.attn = torch.empty((B, total), dtype=torch.bool, device=dev)
        torch.ne(sequences, pad_token_id, out=self.attn[:, :S0])
        self.col = S0
        self.finished = finished
        self.eos = int(eos_token_id)
        self.pad = int(pad_token_id)
        self.flags = torch.zeros(2, dtype=torch.int32, device=dev)
        self._host = torch.empty((2, 2), dtype=torch.int32, pin_memory=True)
        self._steps = 0
        self._pending = None

    def sequences(self) -> torch.Tensor:
        """The sequence so far, [B, col] int64, contiguous."""
        return self.seq[:, : self.col].contiguous()

    def attention_mask(self) -> torch.Tensor:
        """``sequences().ne(pad_token_id)``, [B, col] bool, contiguous."""
        return self.attn[:, : self.col].contiguous()

    def step(self, logits: torch.Tensor, temperature: float, top_p: float) -> torch.Tensor:
        """Sample one token per row of ``logits`` [B, V] and record it; returns
        the int64 [B] ids (pad_token_id for rows already finished)."""
        out = ops.sample(logits, temperature=float(temperature), top_p=float(top_p),
                         finished=self.finished, pad_token_id=self.pad)
        ids = out.ids
        if dist.is_available() and dist.is_initialized():
            # rank 0's tokens everywhere, as _broadcast_and_pad_finished does
            dist.broadcast(ids, src=0)
        ops.decode_update(ids, out.status, self.finished, self.eos, self.pad, self.seq, self.attn,
                          self.col, self.flags)
        host = self._host[self._steps % 2]
        host.copy_(self.flags, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._pending = (ev, host, out.status)
        self.col += 1
        self._steps += 1
        return ids

    def all_finished(self) -> bool:
        """Whether every row has finished after the last :meth:`step` (waits
        for that step's update only)."""
        ev, host, status = self._pending
        ev.synchronize()
        if int(host[1]) > 0:
            ops.raise_on_bad_status(status, "_next_token_from_logits")
        return int(host[0]) == 0


def _decode(self, st: DecodeState, first_logits: Callable[[], torch.Tensor],
            forward_next: Callable[[torch.Tensor], torch.Tensor], *, max_new_tokens: int,
            temperature: float, top_p: float, prefill_sec: float):
    decode_started_at = time.monotonic()
    decode_tokens = 0
    sampling_sec = 0.0
    stop_check_sec = 0.0
    step_logits = first_logits() if max_new_tokens > 0 else None
    for i in range(max_new_tokens):
        self._sync_timing()
        sampling_started_at = time.monotonic()
        next_token = st.step(step_logits, temperature, top_p)
        self._sync_timing()
        sampling_sec += time.monotonic() - sampling_started_at
        decode_tokens += 1
        if i + 1 < max_new_tokens:
            step_logits = forward_next(next_token)  # queued ahead of the stop check
        self._sync_timing()
        stop_check_started_at = time.monotonic()
        all_finished = st.all_finished()
        self._sync_timing()
        stop_check_sec += time.monotonic() - stop_check_started_at
        if all_finished:
            break
    self._sync_timing()
    return st.sequences(), {
        "prefill_sec": prefill_sec,
        "decode_sec": time.monotonic() - decode_started_at,
        "decode_tokens": decode_tokens,
        "sampling_sec": sampling_sec,
        "stop_check_sec": stop_check_sec,
    }


def _rows_at(logits: torch.Tensor, attention_mask: torch.Tensor) -> torch.Tensor:
    """Each row's logits at its last attended position (the multimodal loops'
    first step, generation.py:542-544)."""
    lens = attention_mask.sum(dim=1) - 1
    return logits[torch.arange(logits.shape[0], device=logits.device), lens]


def generate_group_with_kv_cache(self, *, sequences: torch.Tensor, finished: torch.Tensor,
                                 eos_token_id: int, pad_token_id: int, max_new_tokens: int,
                                 temperature: float, top_p: float):
    """KV-cache decode loop (adapter.py:259-318, generation.py:225-284)."""
    assert self.model is not None
    st = DecodeState(sequences, finished, eos_token_id, pad_token_id, max_new_tokens)
    self._sync_timing()
    prefill_started_at = time.monotonic()
    logits, past_key_values = self.model(sequences, attention_mask=st.attention_mask(),
                                         use_cache=True)
    self._sync_timing()
    prefill_sec = time.monotonic() - prefill_started_at
    cache = [past_key_values]

    def forward_next(next_token):
        out, cache[0] = self.model(next_token.unsqueeze(1), attention_mask=st.attention_mask(),
                                   past_key_values=cache[0], use_cache=True)
        return out[:, -1, :]

    return _decode(self, st, lambda: logits[:, -1, :], forward_next,
                   max_new_tokens=max_new_tokens, temperature=temperature, top_p=top_p,
                   prefill_sec=prefill_sec)


def generate_group_full_forward(self, *, sequences: torch.Tensor, finished: torch.Tensor,
                                eos_token_id: int, pad_token_id: int, max_new_tokens: int,
                                temperature: float, top_p: float):
    """Full-forward decode loop (adapter.py:320-363, generation.py:286-329)."""
    assert self.model is not None
    st = DecodeState(sequences, finished, eos_token_id, pad_token_id, max_new_tokens)

    def forward(_next_token=None):
        return self.model(st.sequences(), attention_mask=st.attention_mask())[:, -1, :]

    return _decode(self, st, forward, forward, max_new_tokens=max_new_tokens,
                   temperature=temperature, top_p=top_p, prefill_sec=0.0)


def generate_multimodal_with_kv_cache(self, *, sequences: torch.Tensor,
                                      attention_mask: torch.Tensor,
                                      multimodal_inputs: dict[str, Any], finished: torch.Tensor,
                                      eos_token_id: int, pad_token_id: int, max_new_tokens: int,
                                      temperature: float, top_p: float):
    """Multimodal KV-cache decode loop (generation.py:518-584): the prefill
    takes the caller's attention mask and samples each row at its last
    attended position; later steps use ``sequences.ne(pad_token_id)``."""
    assert self.model is not None
    st = DecodeState(sequences, finished, eos_token_id, pad_token_id, max_new_tokens)
    self._sync_timing()
    prefill_started_at = time.monotonic()
    logits, past_key_values = self.model(sequences, attention_mask=attention_mask,
                                         multimodal_inputs=multimodal_inputs, use_cache=True)
    self._sync_timing()
    prefill_sec = time.monotonic() - prefill_started_at
    cache = [past_key_values]

    def forward_next(next_token):
        out, cache[0] = self.model(next_token.unsqueeze(1), attention_mask=st.attention_mask(),
                                   past_key_values=cache[0], use_cache=True)
        return out[:, -1, :]

    return _decode(self, st, lambda: _rows_at(logits, attention_mask), forward_next,
                   max_new_tokens=max_new_tokens, temperature=temperature, top_p=top_p,
                   prefill_sec=prefill_sec)


def generate_multimodal_full_forward(self, *, sequences: torch.Tensor,
                                     multimodal_inputs: dict[str, Any], finished: torch.Tensor,
                                     eos_token_id: int, pad_token_id: int, max_new_tokens: int,
                                     temperature: float, top_p: float):
    """Multimodal full-forward decode loop (generation.py:586-641): the first
    step samples each row at its last attended position, later steps at the
    last position."""
    assert self.model is not None
    st = DecodeState(sequences, finished, eos_token_id, pad_token_id, max_new_tokens)

    def first():
        mask = st.attention_mask()
        raw = self.model(st.sequences(), attention_mask=mask, multimodal_inputs=multimodal_inputs)
        return _rows_at(raw, mask)

    def forward_next(_next_token):
        raw = self.model(st.sequences(), attention_mask=st.attention_mask(),
                         multimodal_inputs=multimodal_inputs)
        return raw[:, -1, :]

    return _decode(self, st, first, forward_next, max_new_tokens=max_new_tokens,
                   temperature=temperature, top_p=top_p, prefill_sec=0.0)
