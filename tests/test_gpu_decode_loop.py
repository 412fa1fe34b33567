"""GPU parity of the decode-loop drop-ins (graspo_amd.decode_loop) against the
reference's loop bodies (models/qwen3/adapter.py:259-363,
models/qwen35_36/generation.py:518-641), restated below statement by
statement with the same sampler call, so that what is compared is the loop:
the bf16 strided logits instead of ``logits.float()``, the fused
pad / EOS / column / all-finished kernel and the lagged stop check.

The model is a deterministic toy LM whose logits depend on (token,
position); the EOS logit can be raised or lowered per position to force
every row to finish early, none to finish, or a mix.  Both loops draw their
uniforms from torch's generator after the same seed, so the tokens must be
identical, as must ``finished``, ``decode_tokens`` and the attention masks
the model saw."""

import pytest
import torch

from graspo_amd import decode_loop as dl
from graspo_amd import ops
from graspo_amd import tensor_utils as tu

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
V = 1000


class ToyLM:
    def __init__(self, eos, eos_bias, seed=0, nan_at=None):
        g = torch.Generator().manual_seed(seed)
        self.table = (torch.randn(97, V, generator=g) * 2.0).to(torch.bfloat16).to(DEV)
        self.eos, self.eos_bias, self.nan_at = eos, eos_bias, nan_at
        self.masks = []

    def _logits(self, ids, start):
        # an embedding lookup faults on an id outside [0, V): refuse it here
        assert bool(((ids >= 0) & (ids < V)).all()), f"id outside [0, {V}) fed to the model"
        L = ids.shape[1]
        pos = torch.arange(start, start + L, device=DEV)
        out = self.table[(ids * 31 + pos[None, :] * 7) % 97].clone()  # [B, L, V] bf16
        out[:, :, self.eos] += self.eos_bias(pos)[None, :].to(out.dtype)
        if self.nan_at is not None:
            row, p = self.nan_at
            hit = (pos == p).nonzero().flatten()
            if len(hit):
                out[row, hit] = float("nan")
        return out

    def __call__(self, ids, attention_mask=None, past_key_values=None, use_cache=False,
                 multimodal_inputs=None):
        self.masks.append(attention_mask.clone())
        start = past_key_values or 0
        assert attention_mask.shape == (ids.shape[0], start + ids.shape[1])
        out = self._logits(ids, start)
        return (out, start + ids.shape[1]) if use_cache else out


class Adapter:
    def __init__(self, model):
        self.model = model

    def _sync_timing(self):
        pass


# ---- the reference loops, restated (adapter.py:259-363, generation.py:518-641)

def ref_kv(model, sequences, finished, eos, pad, max_new, T, top_p):
    attention_mask = sequences.ne(pad)
    logits, pkv = model(sequences, attention_mask=attention_mask, use_cache=True)
    n = 0
    for _ in range(max_new):
        nt = tu._next_token_from_logits(logits.float()[:, -1, :], temperature=T, top_p=top_p)
        nt = tu._broadcast_and_pad_finished(nt, finished, pad)
        sequences = torch.cat([sequences, nt.unsqueeze(1)], dim=1)
        n += 1
        finished |= nt.eq(eos)
        if bool(finished.all()):
            break
        attention_mask = sequences.ne(pad)
        logits, pkv = model(nt.unsqueeze(1), attention_mask=attention_mask, past_key_values=pkv,
                            use_cache=True)
    return sequences, n


def ref_full(model, sequences, finished, eos, pad, max_new, T, top_p):
    n = 0
    for _ in range(max_new):
        attention_mask = sequences.ne(pad)
        logits = model(sequences, attention_mask=attention_mask).float()[:, -1, :]
        nt = tu._next_token_from_logits(logits, temperature=T, top_p=top_p)
        nt = tu._broadcast_and_pad_finished(nt, finished, pad)
        sequences = torch.cat([sequences, nt.unsqueeze(1)], dim=1)
        n += 1
        finished |= nt.eq(eos)
        if bool(finished.all()):
            break
    return sequences, n


def ref_mm_kv(model, sequences, attention_mask, finished, eos, pad, max_new, T, top_p):
    logits, pkv = model(sequences, attention_mask=attention_mask, multimodal_inputs={},
                        use_cache=True)
    lens = attention_mask.sum(dim=1) - 1
    step_logits = logits[torch.arange(logits.shape[0], device=DEV), lens]
    n = 0
    for _ in range(max_new):
        nt = tu._next_token_from_logits(step_logits.float(), temperature=T, top_p=top_p)
        nt = tu._broadcast_and_pad_finished(nt, finished, pad)
        sequences = torch.cat([sequences, nt.unsqueeze(1)], dim=1)
        n += 1
        finished |= nt.eq(eos)
        if bool(finished.all()):
            break
        attention_mask = sequences.ne(pad)
        logits, pkv = model(nt.unsqueeze(1), attention_mask=attention_mask, past_key_values=pkv,
                            use_cache=True)
        step_logits = logits[:, -1, :]
    return sequences, n


def ref_mm_full(model, sequences, finished, eos, pad, max_new, T, top_p):
    n = 0
    first = True
    for _ in range(max_new):
        attention_mask = sequences.ne(pad)
        raw = model(sequences, attention_mask=attention_mask, multimodal_inputs={}).float()
        if first:
            lens = attention_mask.sum(dim=1) - 1
            logits = raw[torch.arange(raw.shape[0], device=DEV), lens]
            first = False
        else:
            logits = raw[:, -1, :]
        nt = tu._next_token_from_logits(logits, temperature=T, top_p=top_p)
        nt = tu._broadcast_and_pad_finished(nt, finished, pad)
        sequences = torch.cat([sequences, nt.unsqueeze(1)], dim=1)
        n += 1
        finished |= nt.eq(eos)
        if bool(finished.all()):
            break
    return sequences, n


EOS, PAD = 7, 0
BIASES = {
    "all_finish": lambda pos: torch.where(pos >= 14, 60.0, 0.0),  # every row ends by position 14
    "none_finish": lambda pos: torch.full_like(pos, -60.0, dtype=torch.float32),
    "mixed": lambda pos: torch.full_like(pos, 4.5, dtype=torch.float32),
}


def _prompt(B, S0, seed, right_pad=False):
    g = torch.Generator().manual_seed(seed)
    seq = torch.randint(1, V, (B, S0), generator=g)
    seq[seq == EOS] = EOS + 1
    if right_pad:  # ragged prompts, padded on the right
        for b in range(B):
            seq[b, S0 - (b % 3):] = PAD
    return seq.to(DEV)


def _run_pair(kind, bias, T, top_p, max_new, B=8, S0=10, pre_finished=(), seed=0):
    seq0 = _prompt(B, S0, seed, right_pad=kind.startswith("mm"))
    fin_ref = torch.zeros(B, dtype=torch.bool, device=DEV)
    for b in pre_finished:
        fin_ref[b] = True
    fin_new = fin_ref.clone()
    m_ref, m_new = ToyLM(EOS, BIASES[bias], seed), ToyLM(EOS, BIASES[bias], seed)
    kw = dict(eos_token_id=EOS, pad_token_id=PAD, max_new_tokens=max_new, temperature=T,
              top_p=top_p)
    torch.manual_seed(1234 + seed)
    if kind == "kv":
        want, n_want = ref_kv(m_ref, seq0.clone(), fin_ref, EOS, PAD, max_new, T, top_p)
        torch.manual_seed(1234 + seed)
        got, timing = dl.generate_group_with_kv_cache(Adapter(m_new), sequences=seq0.clone(),
                                                      finished=fin_new, **kw)
    elif kind == "full":
        want, n_want = ref_full(m_ref, seq0.clone(), fin_ref, EOS, PAD, max_new, T, top_p)
        torch.manual_seed(1234 + seed)
        got, timing = dl.generate_group_full_forward(Adapter(m_new), sequences=seq0.clone(),
                                                     finished=fin_new, **kw)
    elif kind == "mm_kv":
        am = seq0.ne(PAD)
        want, n_want = ref_mm_kv(m_ref, seq0.clone(), am, fin_ref, EOS, PAD, max_new, T, top_p)
        torch.manual_seed(1234 + seed)
        got, timing = dl.generate_multimodal_with_kv_cache(
            Adapter(m_new), sequences=seq0.clone(), attention_mask=am, multimodal_inputs={},
            finished=fin_new, **kw)
    else:
        want, n_want = ref_mm_full(m_ref, seq0.clone(), fin_ref, EOS, PAD, max_new, T, top_p)
        torch.manual_seed(1234 + seed)
        got, timing = dl.generate_multimodal_full_forward(
            Adapter(m_new), sequences=seq0.clone(), multimodal_inputs={}, finished=fin_new, **kw)
    torch.cuda.synchronize()
    what = (kind, bias, T, top_p, max_new)
    assert got.dtype == torch.int64 and got.is_contiguous()
    assert torch.equal(got, want), (what, got.cpu(), want.cpu())
    assert torch.equal(fin_new, fin_ref), what
    assert timing["decode_tokens"] == n_want, (what, timing, n_want)
    assert set(timing) == {"prefill_sec", "decode_sec", "decode_tokens", "sampling_sec",
                           "stop_check_sec"}
    # the masks the model saw: the same sequence, except that the drop-in
    # queues one forward past the step where every row finished, and skips the
    # forward the reference runs (and discards) after its last step
    assert len(m_new.masks) - len(m_ref.masks) in (-1, 0, 1), what
    for a, b in zip(m_ref.masks, m_new.masks):
        assert torch.equal(a, b), what
    return n_want


@pytest.mark.parametrize("kind", ["kv", "full", "mm_kv", "mm_full"])
@pytest.mark.parametrize("bias,T,top_p", [("all_finish", 1.0, 0.9), ("none_finish", 0.7, 1.0),
                                          ("mixed", 1.0, 0.95), ("mixed", 0.0, 1.0)])
def test_loop_matches_reference(kind, bias, T, top_p):
    print("decode loop", kind, bias, T, top_p, flush=True)
    n = _run_pair(kind, bias, T, top_p, max_new=12)
    if bias == "all_finish":
        assert n <= 6  # stopped early: every row samples EOS from position 14 on
    if bias == "none_finish":
        assert n == 12


def test_pre_finished_rows_and_zero_steps():
    print("decode loop pre-finished", flush=True)
    _run_pair("kv", "mixed", 1.0, 0.9, max_new=10, pre_finished=(1, 5))
    _run_pair("kv", "mixed", 1.0, 0.9, max_new=0)
    # every row finished before the call: one step of pads, then stop
    n = _run_pair("kv", "mixed", 1.0, 0.9, max_new=6, pre_finished=tuple(range(8)))
    assert n == 1


def test_bad_row_raises_like_the_reference():
    print("decode loop nan row", flush=True)
    seq0 = _prompt(4, 6, 3)
    m = ToyLM(EOS, BIASES["none_finish"], 3, nan_at=(2, 8))
    fin = torch.zeros(4, dtype=torch.bool, device=DEV)
    with pytest.raises(RuntimeError, match="non-finite"):
        dl.generate_group_with_kv_cache(Adapter(m), sequences=seq0, finished=fin,
                                        eos_token_id=EOS, pad_token_id=PAD, max_new_tokens=8,
                                        temperature=1.0, top_p=0.9)


@pytest.mark.parametrize("B", [0, 1, 5, 1024, 3000])
def test_update_kernel_against_torch(B):
    g = torch.Generator().manual_seed(B)
    ids = torch.randint(0, 12, (B,), generator=g).to(DEV)
    fin = (torch.rand(B, generator=g) < 0.3).to(DEV)
    status = torch.where(torch.rand(B, generator=g) < 0.05, 1, 0).to(torch.int32).to(DEV)
    seq = torch.full((B, 9), -5, dtype=torch.int64, device=DEV)
    attn = torch.zeros((B, 9), dtype=torch.bool, device=DEV)
    flags = torch.full((2,), -1, dtype=torch.int32, device=DEV)
    ids[status.ne(0)] = -1  # the sampler's id for a bad row
    want_ids = torch.where(status.ne(0), torch.full_like(ids, 3), ids)  # padded in place
    want_fin = fin | want_ids.eq(EOS)
    fin_in = fin.clone()
    ops.decode_update(ids, status, fin_in, EOS, 3, seq, attn, 4, flags)
    torch.cuda.synchronize()
    assert torch.equal(ids, want_ids)
    assert torch.equal(fin_in, want_fin)
    assert torch.equal(seq[:, 4], want_ids) and bool((seq[:, :4] == -5).all())
    assert bool((seq[:, 5:] == -5).all())
    assert torch.equal(attn[:, 4], want_ids.ne(3)) and not bool(attn[:, :4].any())
    assert flags.tolist() == [int((~want_fin).sum()), int(status.ne(0).sum())]
