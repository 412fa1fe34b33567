"""GPU parity of the top-p kernel (bf16 rows, top-p without top-k,
V >= 65536) against the exact CPU oracle: ids, kept sizes, thresholds and
statuses bit for bit, logprobs within 1e-3.

Covers the decode loop's rows (the reference's _next_token_from_logits(
logits, temperature, top_p), tensor_utils.py:649-683), penalties above and
below 1 with exact ties between penalised and unpenalised values, values
with thousands of tokens (the cut and the draw inside one value), zeros,
flat rows whose kept set outgrows the capture pool (the rescan), rows the
kernel hands over to the row-wise path (values outside its bins, a value
held by more than 65535 tokens), status rows, vocabulary tails and workspace
reuse between the top-p and the split kernels."""

import numpy as np
import pytest
import torch

from graspo_amd import ops
from graspo_amd import workloads as W
from tests import _capi
from tests._util import oracle_sample
from tests.test_gpu_sampler import assert_parity, gpu_sample

pytestmark = pytest.mark.gpu


def aligned_rows(x):
    """[B, V] on the GPU as a view whose rows start 16 bytes apart (a row
    stride rounded up to 8 tokens), so the top-p kernel takes any V."""
    B, V = x.shape
    full = torch.zeros((B, (V + 7) // 8 * 8), dtype=x.dtype, device="cuda:0")
    full[:, :V] = x.to("cuda:0")
    return full[:, :V]


def _u(B, g):
    return torch.randint(0, 1 << 24, (B,), generator=g).float() * 2.0 ** -24


def one_workgroup_sample(x, **kw):
    """The call through the C ABI with a workspace too small for the split
    kernel, so that rows of a small batch take the one-workgroup kernel."""
    dev = torch.device("cuda:0")
    kw = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    if kw.get("finished") is not None:
        kw["finished"] = kw["finished"].to(torch.uint8)
    xd = x.to(dev)
    if xd.stride(1) != 1 or xd.data_ptr() % 16 != 0:
        xd = aligned_rows(x)
    out = _capi.sample_small_workspace(xd, **kw)
    return ops.SampleOutput(*[out[f] for f in ops.SampleOutput._fields])


def _check(x, what, **kw):
    """Both kernels against the oracle: the torch op (rows of batches up to
    128 split over several workgroups) and the one-workgroup kernel."""
    print("topp:", what, tuple(x.shape), {k: v for k, v in kw.items()
                                          if not isinstance(v, torch.Tensor)}, flush=True)
    g = gpu_sample(x, **kw)
    ref = oracle_sample(x, **kw)
    assert_parity(g, ref, what)
    if x.shape[0] <= 128 and not kw.get("top_k"):
        assert_parity(one_workgroup_sample(x, **kw), ref, what + " (one workgroup)")
    return g, ref


def test_decode_rows_large_vocab():
    """[256, 248320] bf16 N(0, 3), 10% of rows with a +12 spike, T 0.7,
    P 0.9: the decode loop's rows."""
    wl = W.sampler_workload(5)
    g = torch.Generator().manual_seed(77)
    _check(wl.logits, "decode rows", temperature=0.7, top_p=0.9, uniforms=_u(256, g))


@pytest.mark.parametrize("cfg", [2, 3, 5])
def test_workload_rows_top_p_only(cfg):
    """The workloads' rows with top-k off (configurations 2 and 3 are top-p
    only already; 5 keeps its history and mask)."""
    wl = W.sampler_workload(cfg, rows=64)
    kw = wl.kwargs()
    kw["top_k"] = 0
    _check(wl.logits, f"cfg{cfg} top-p only", **kw)


@pytest.mark.parametrize("rho", [0.5, 0.8, 1.3, 2.0])
def test_penalties(rho):
    """Penalised values move among the unpenalised ones; rho = 2 and 0.5 map
    bf16 values onto bf16 values, so penalised and unpenalised tokens tie."""
    B, V = 32, 100000
    g = torch.Generator().manual_seed(int(rho * 10))
    x = (torch.randn(B, V, generator=g) * 2.0).to(torch.bfloat16)
    hist = torch.randint(-1, V, (B, 3000), generator=g, dtype=torch.int32)
    # make the top tokens penalised in half of the rows
    top = x.float().topk(64, dim=-1).indices.to(torch.int32)
    hist[: B // 2, :64] = top[: B // 2]
    hist[:, 100:200] = hist[:, :100]  # duplicates
    for T, P in ((0.7, 0.9), (1.0, 0.5), (1.5, 0.99)):
        _check(x, f"rho {rho} T {T} P {P}", temperature=T, top_p=P, repetition_penalty=rho,
               history=hist, uniforms=_u(B, g))


def test_values_with_many_tokens():
    """Values on a 1/4 grid (thousands of tokens per value) and five-valued
    rows: the cut and the draw fall inside one value, positions inside it
    are integer quotients, ids come in id order."""
    B, V = 24, 131072
    g = torch.Generator().manual_seed(5)
    x = torch.round(torch.randn(B, V, generator=g) * 8) / 4
    x[8:16] = torch.randint(0, 5, (8, V), generator=g).float() * 0.5
    x[16:] = torch.round(torch.randn(8, V, generator=g) * 64) / 64
    x = x.to(torch.bfloat16)
    for P in (0.3, 0.9, 0.999):
        _check(x, f"grid rows P {P}", temperature=1.0, top_p=P, uniforms=_u(B, g))
    hist = torch.randint(0, V, (B, 500), generator=g, dtype=torch.int32)
    _check(x, "grid rows, penalised", temperature=0.8, top_p=0.95, repetition_penalty=2.0,
           history=hist, uniforms=_u(B, g))


def test_zeros_and_signs():
    """Exact zeros (their own value between the negative and positive
    bins), penalised zeros, and all-negative rows."""
    B, V = 16, 70000
    g = torch.Generator().manual_seed(6)
    x = torch.randn(B, V, generator=g)
    x[:, ::7] = 0.0
    x[4:8] = -x[4:8].abs() - 0.5
    x[4:8, ::11] = 0.0
    x[8:12] = -x[8:12].abs() - 3.0  # all negative, no zero
    x[12:, :1000] = 0.0
    x[12:, 1000:] = -5.0 + torch.randn(4, V - 1000, generator=g) * 0.1
    x = x.to(torch.bfloat16)
    hist = torch.arange(0, 700, dtype=torch.int32).repeat(B, 1)  # ids 0, 7, ... are zeros
    for kw in (dict(), dict(repetition_penalty=1.2, history=hist)):
        for P in (0.5, 0.95):
            _check(x, f"zeros P {P} {list(kw)}", temperature=0.9, top_p=P, uniforms=_u(B, g), **kw)


@pytest.mark.parametrize("T", [2.0, 5.0, 50.0])
def test_flat_rows_outgrow_the_pool(T):
    """High temperatures flatten the row: the kept set runs to tens of
    thousands of tokens, beyond what the pilot captures, so the cut's ids
    come from a rescan of the row."""
    B, V = 16, 151936
    g = torch.Generator().manual_seed(int(T))
    x = (torch.randn(B, V, generator=g) * 2.5).to(torch.bfloat16)
    u = _u(B, g)
    u[0], u[1] = 0.0, 1.0 - 2.0 ** -24
    _, ref = _check(x, f"flat T {T}", temperature=T, top_p=0.95, uniforms=u)
    assert ref.kept.max() > 8192  # beyond the pool


def test_masked_rows():
    """Structured-output rows: ~8% allowed, single allowed tokens, an empty
    mask, and masked rows with a history."""
    wl = W.sampler_workload(3, rows=64)
    bits = torch.rand(64, wl.shape[1], generator=torch.Generator().manual_seed(9)) < 0.08
    bits[5] = False
    bits[5, 12345] = True
    bits[6] = False
    kw = wl.kwargs()
    kw["allow_mask"] = W.pack_mask(bits)
    g, ref = _check(wl.logits, "masked", **kw)
    assert int(g.ids[5]) == 12345 and int(g.status[6]) == ops.ROW_EMPTY
    hist = torch.randint(0, wl.shape[1], (64, 2048), generator=torch.Generator().manual_seed(3),
                         dtype=torch.int32)
    kw.update(history=hist, repetition_penalty=1.1)
    _check(wl.logits, "masked with history", **kw)


def test_rows_handed_over_to_the_row_wise_path():
    """Rows outside the kernel's bounds run the row-wise path inside the same
    launch: a value beyond 2^24, a tiny nonzero value, a constant row (one
    value held by every token, beyond a 16-bit count), and a row whose
    penalised values crowd one range; the other rows of the batch stay on
    the top-p path."""
    B, V = 8, 70000
    g = torch.Generator().manual_seed(12)
    x = torch.randn(B, V, generator=g) * 2
    x[1, 500] = 3.0e7
    x[2, 600] = 1e-20
    x[3] = 1.25
    x[4, :] = torch.randn(V, generator=g) * 0.01  # values crowd near zero
    x = x.to(torch.bfloat16)
    hist = torch.full((B, 4000), -1, dtype=torch.int32)
    hist[4] = torch.arange(4000, dtype=torch.int32)
    for kw in (dict(), dict(history=hist, repetition_penalty=1.5)):
        _check(x, f"hand-over {list(kw)}", temperature=0.8, top_p=0.9, uniforms=_u(B, g), **kw)


@pytest.mark.parametrize("mode", ["mask", "mask + penalty"])
def test_masked_rows_handed_over(mode):
    """The masked variants' rows outside the kernel's bounds (an allowed -inf
    logit, a value beyond 2^24, a constant row whose one value every allowed
    token holds) run the row-wise path inside the same launch, in the split
    and the one-workgroup kernels; the other rows stay on the top-p path."""
    B, V = 8, 70000
    g = torch.Generator().manual_seed(21)
    x = torch.randn(B, V, generator=g) * 2
    x[1, 500] = 3.0e7
    x[2, 77] = float("-inf")
    x[3] = 1.25
    x = x.to(torch.bfloat16)
    bits = torch.rand(B, V, generator=g) < 0.3
    bits[1, 500] = True
    bits[2, 77] = True
    bits[3] = True  # 70000 allowed tokens of one value: beyond a 16-bit count
    kw = dict(temperature=0.8, top_p=0.9, uniforms=_u(B, g), allow_mask=W.pack_mask(bits))
    if mode == "mask + penalty":
        hist = torch.randint(0, V, (B, 3000), generator=g, dtype=torch.int32)
        hist[1, 0] = 500
        kw.update(history=hist, repetition_penalty=1.3)
    _check(x, f"handed over, {mode}", **kw)


def test_status_rows_and_padding():
    B, V = 8, 65536 + 5  # a vocabulary tail of 5 tokens
    g = torch.Generator().manual_seed(13)
    x = torch.randn(B, V, generator=g)
    x[0, 77] = float("nan")
    x[1, 99] = float("inf")
    x[2, V - 1] = 9.0  # the answer in the tail
    x = aligned_rows(x.to(torch.bfloat16))
    u = _u(B, g)
    u[3] = 1.0  # bad uniform
    hist = torch.zeros((B, 4), dtype=torch.int32)
    hist[4, 2] = V  # bad history id
    fin = torch.zeros(B, dtype=torch.bool)
    fin[5] = True
    got, ref = _check(x, "status rows", temperature=1.0, top_p=0.8, uniforms=u, history=hist,
                      repetition_penalty=1.1, finished=fin, pad_token_id=-9)
    assert got.status.tolist()[:5] == [1, 1, 0, 4, 3]
    assert int(got.ids[5]) == -9


def test_workspace_shared_with_the_split_kernel():
    """The torch glue keeps one workspace per stream for the arrival counters
    of the split top-k and split top-p kernels: alternate the two kinds of
    call (with rows that go to the row-wise path) and check every call."""
    g = torch.Generator().manual_seed(14)
    B, V = 64, 151936
    x = (torch.randn(B, V, generator=g) * 2.5).to(torch.bfloat16)
    x[3, 10] = 3.0e7  # handed over
    x[9] = 0.5        # handed over (one value, every token)
    for i in range(3):
        _check(x, f"alternate {i} top-p", temperature=0.9, top_p=0.9, uniforms=_u(B, g))
        _check(x, f"alternate {i} top-k", temperature=0.9, top_k=40, top_p=0.9,
               uniforms=_u(B, g))


def test_fuzz_large_vocab():
    """Random rows through the top-p kernel: scales, temperatures, top-p,
    masks and penalties drawn per case."""
    rng = np.random.default_rng(2024)
    for case in range(24):
        B = int(rng.integers(1, 9))
        V = int(rng.choice([65536, 65537, 100003, 151936, 248320, 262144]))
        g = torch.Generator().manual_seed(case)
        kind = case % 4
        if kind == 0:
            x = torch.randn(B, V, generator=g) * float(rng.uniform(0.5, 6))
        elif kind == 1:
            x = torch.round(torch.randn(B, V, generator=g) * 16) / 16
        elif kind == 2:
            x = torch.randn(B, V, generator=g) * 3
            x[:, rng.integers(0, V, 5)] += 15.0
        else:
            x = -torch.rand(B, V, generator=g) * 40
        x = aligned_rows(x.to(torch.bfloat16))
        kw = dict(temperature=float(rng.choice([0.3, 0.7, 1.0, 1.7])),
                  top_p=float(rng.choice([0.1, 0.5, 0.9, 0.95, 0.999])), uniforms=_u(B, g))
        if rng.random() < 0.5:
            kw["allow_mask"] = W.pack_mask(torch.rand(B, V, generator=g) < rng.uniform(0.02, 0.9))
        if rng.random() < 0.5:
            kw["history"] = torch.randint(-1, V, (B, int(rng.integers(1, 5000))), generator=g,
                                          dtype=torch.int32)
            kw["repetition_penalty"] = float(rng.choice([0.7, 1.05, 1.3, 2.0]))
        _check(x, f"fuzz {case}", **kw)
