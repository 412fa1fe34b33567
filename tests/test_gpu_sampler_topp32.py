"""GPU parity of the fp32 top-p kernel (fp32 rows, top-p without top-k,
V >= 65536) against the exact CPU oracle: ids, kept sizes, thresholds and
statuses bit for bit, logprobs within 1e-3.

Covers the reference's decode call _next_token_from_logits(logits.float(),
temperature, top_p) (tensor_utils.py:649-683) on rows whose values are bf16
values (ties by the thousand) and on rows that are not, penalties above and
below 1, masks, rows dominated by a few spiked tokens (the top list), rows
whose kept set outgrows the candidate array or whose spikes overflow the top
list (handed over to the row-wise path), status rows, vocabulary tails,
strided rows and random cases."""

import numpy as np
import pytest
import torch

from graspo_amd import ops, workloads as W
from tests._util import oracle_sample
from tests.test_gpu_sampler import assert_parity, gpu_sample

pytestmark = pytest.mark.gpu


def aligned_rows(x):
    """[B, V] fp32 on the GPU as a view whose rows start 16 bytes apart."""
    B, V = x.shape
    full = torch.zeros((B, (V + 3) // 4 * 4), dtype=x.dtype, device="cuda:0")
    full[:, :V] = x.to("cuda:0")
    return full[:, :V]


def _u(B, g):
    return torch.randint(0, 1 << 24, (B,), generator=g).float() * 2.0 ** -24


def _check(x, what, **kw):
    print("topp32:", what, tuple(x.shape), {k: v for k, v in kw.items()
                                            if not isinstance(v, torch.Tensor)}, flush=True)
    g = gpu_sample(x, **kw)
    ref = oracle_sample(x, **kw)
    assert_parity(g, ref, what)
    return g, ref


def _inexact(x, seed):
    g = torch.Generator().manual_seed(seed)
    y = x.float() + torch.rand(x.shape, generator=g) * 1e-3
    assert bool((y.to(torch.bfloat16).float() != y).any())
    return y


def test_decode_rows_not_bf16_values():
    """[128, 248320] N(0, 3) with spikes plus U(0, 1e-3), T 0.7, P 0.9."""
    wl = W.sampler_workload(5, rows=128)
    g = torch.Generator().manual_seed(71)
    _check(_inexact(wl.logits, 1), "decode fp32", temperature=0.7, top_p=0.9, uniforms=_u(128, g))


def test_decode_rows_bf16_values():
    """logits.float() of bf16 rows: every value a bf16 value, a handful of
    tokens per value at the cut."""
    wl = W.sampler_workload(5, rows=128)
    g = torch.Generator().manual_seed(72)
    _check(wl.logits.float(), "decode bf16 values", temperature=0.7, top_p=0.9,
           uniforms=_u(128, g))


@pytest.mark.parametrize("cfg", [2, 3, 5])
def test_workload_rows_top_p_only(cfg):
    """The workloads' rows as fp32 with top-k off (history, mask and penalty
    as the workload has them)."""
    wl = W.sampler_workload(cfg, rows=48)
    kw = wl.kwargs()
    kw["top_k"] = 0
    _check(_inexact(wl.logits, cfg), f"cfg{cfg} fp32", **kw)
    _check(wl.logits.float(), f"cfg{cfg} bf16 values", **kw)


@pytest.mark.parametrize("rho", [0.5, 1.3, 2.0])
def test_penalties(rho):
    B, V = 16, 151936
    g = torch.Generator().manual_seed(int(rho * 10))
    x = torch.randn(B, V, generator=g) * 3
    x[:, :50] = torch.randn(50, generator=g) * 3 + 9.0  # penalised ids among the top
    hist = torch.randint(-1, 200, (B, 3000), generator=g, dtype=torch.int32)
    _check(x, f"penalty {rho}", temperature=0.8, top_p=0.9, uniforms=_u(B, g), history=hist,
           repetition_penalty=rho)


def test_masked_rows():
    B, V = 16, 151936
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, V, generator=g) * 2.5
    bits = torch.rand(B, V, generator=g) < 0.08
    bits[3] = False
    bits[3, [7, 70000, 151935]] = True  # three allowed tokens
    bits[4] = False
    bits[4, :5000] = True               # none in the pilot's places but the first
    _check(x, "mask", temperature=0.7, top_p=0.9, uniforms=_u(B, g), allow_mask=W.pack_mask(bits))
    hist = torch.randint(0, V, (B, 2000), generator=g, dtype=torch.int32)
    _check(x, "mask + penalty", temperature=0.7, top_p=0.9, uniforms=_u(B, g),
           allow_mask=W.pack_mask(bits), history=hist, repetition_penalty=1.2)


def test_spiked_rows():
    """A few tokens far above the rest carry the weight (the top list); 700
    spiked tokens overflow it (handed over)."""
    B, V = 8, 248320
    g = torch.Generator().manual_seed(6)
    x = torch.randn(B, V, generator=g) * 3
    x[0, 1000] += 20.0
    x[1, [5, 6, 7, 8]] += 14.0
    x[2, 200000] += 2.0
    x[3, torch.randperm(V, generator=g)[:700]] += 25.0
    x[4, torch.randperm(V, generator=g)[:40]] = 30.0  # 40 equal tokens at the top
    for P in (0.5, 0.9, 0.999):
        _check(x, f"spikes P {P}", temperature=0.7, top_p=P, uniforms=_u(B, g))


@pytest.mark.parametrize("mode", ["penalty", "mask", "mask + penalty"])
def test_rows_handed_over_in_every_variant(mode):
    """Each variant's rows outside the kernel's bounds run the row-wise path
    inside the same launch: |y| >= 2^15, a top list beyond its capacity, a
    NaN (the row-wise path writes the status); the other rows stay on the
    fp32 top-p path."""
    B, V = 6, 131072
    g = torch.Generator().manual_seed(31)
    x = torch.randn(B, V, generator=g) * 2.5
    x[1, 1000] = 3.0e4
    x[2, torch.randperm(V, generator=g)[:700]] += 25.0
    x[3, 5] = float("nan")
    kw = dict(temperature=0.7, top_p=0.9, uniforms=_u(B, g))
    if "mask" in mode:
        bits = torch.rand(B, V, generator=g) < 0.5
        bits[1, 1000] = True
        bits[3, 5] = True
        kw["allow_mask"] = W.pack_mask(bits)
    if "penalty" in mode:
        hist = torch.randint(0, V, (B, 2000), generator=g, dtype=torch.int32)
        hist[1, 0] = 1000
        kw.update(history=hist, repetition_penalty=1.2)
    got, _ = _check(x, f"handed over, {mode}", **kw)
    assert int(got.status[3]) == ops.ROW_NONFINITE


@pytest.mark.parametrize("T,P", [(1.0, 0.9), (1.0, 0.95), (1.7, 0.99)])
def test_large_kept_sets(T, P):
    """Kept sets of 10^4 tokens and more: beyond the candidate array the row
    is handed over; either way bit-exact."""
    B, V = 6, 248320
    g = torch.Generator().manual_seed(int(T * 100 + P * 1000))
    x = torch.randn(B, V, generator=g) * 2.5
    _check(x, f"large kept {T} {P}", temperature=T, top_p=P, uniforms=_u(B, g))
    _check(x.to(torch.bfloat16).float(), f"large kept bf16 values {T} {P}", temperature=T,
           top_p=P, uniforms=_u(B, g))


def test_ties_at_the_cut():
    """Values on a coarse grid: hundreds of tokens share the y at the cut
    and the draw (the block-wide ranking of one bin)."""
    B, V = 8, 131072
    g = torch.Generator().manual_seed(8)
    x = torch.round(torch.randn(B, V, generator=g) * 4) / 4
    for T, P in ((0.7, 0.9), (1.0, 0.5), (2.0, 0.9)):
        _check(x, f"grid {T} {P}", temperature=T, top_p=P, uniforms=_u(B, g))


def test_status_rows_tail_and_stride():
    B, V = 10, 65536 + 3  # a vocabulary tail of 3 tokens
    g = torch.Generator().manual_seed(13)
    x = torch.randn(B, V, generator=g)
    x[0, 77] = float("nan")
    x[1, 99] = float("inf")
    x[2, V - 1] = 9.0  # the answer in the tail
    x[6, :] = float("-inf")
    x[6, 4] = 0.5      # one finite token
    x[7, 1000:] = float("-inf")
    x = aligned_rows(x)
    u = _u(B, g)
    u[3] = 1.0  # bad uniform
    hist = torch.zeros((B, 4), dtype=torch.int32)
    hist[4, 2] = V  # bad history id
    fin = torch.zeros(B, dtype=torch.bool)
    fin[5] = True
    bits = torch.ones(B, V, dtype=torch.bool)
    bits[8] = False  # no allowed token
    got, ref = _check(x, "status rows", temperature=1.0, top_p=0.8, uniforms=u, history=hist,
                      repetition_penalty=1.1, finished=fin, pad_token_id=-9,
                      allow_mask=W.pack_mask(bits))
    assert got.status.tolist()[:5] == [1, 1, 0, 4, 3]
    assert int(got.status[8]) == 2
    assert int(got.ids[5]) == -9
    assert int(got.ids[2]) == V - 1 or int(got.kept[2]) > 1


def test_fuzz_large_vocab():
    """Random fp32 rows through the fp32 top-p kernel: scales, temperatures,
    top-p, masks and penalties drawn per case."""
    rng = np.random.default_rng(3202)
    for case in range(20):
        B = int(rng.integers(1, 7))
        V = int(rng.choice([65536, 65539, 100003, 151936, 248320, 262144]))
        g = torch.Generator().manual_seed(case)
        kind = case % 4
        if kind == 0:
            x = torch.randn(B, V, generator=g) * float(rng.uniform(0.5, 6))
        elif kind == 1:
            x = (torch.randn(B, V, generator=g) * 3).to(torch.bfloat16).float()
        elif kind == 2:
            x = torch.randn(B, V, generator=g) * 3
            x[:, rng.integers(0, V, 5)] += 15.0
        else:
            x = -torch.rand(B, V, generator=g) * 40
        x = aligned_rows(x)
        kw = dict(temperature=float(rng.choice([0.3, 0.7, 1.0, 1.7])),
                  top_p=float(rng.choice([0.1, 0.5, 0.9, 0.95, 0.999])), uniforms=_u(B, g))
        if rng.random() < 0.5:
            kw["allow_mask"] = W.pack_mask(torch.rand(B, V, generator=g) < rng.uniform(0.02, 0.9))
        if rng.random() < 0.5:
            kw["history"] = torch.randint(-1, V, (B, int(rng.integers(1, 5000))), generator=g,
                                          dtype=torch.int32)
            kw["repetition_penalty"] = float(rng.choice([0.7, 1.05, 1.3, 2.0]))
        _check(x, f"fuzz {case}", **kw)


@pytest.mark.parametrize("T", [0.7, 0.3, 1.7])
def test_quotients_near_rounding_midpoints(T):
    """Every logit is chosen so that x / T lies within a few ulp of the
    midpoint between two fp32 values (y0 + ulp / 2, then x nudged by -1, 0 or
    +1 ulp): the kernel's division by T, a corrected reciprocal product
    accepted only when provably the IEEE quotient, must give the oracle's y
    bit for bit, which the threshold value output shows."""
    B, V = 16, 65536 + 5
    rng = np.random.default_rng(int(T * 1000))
    y0 = (rng.standard_normal((B, V)) * 4.0).astype(np.float32)
    y0[y0 == 0] = np.float32(1.0)
    mid = y0.astype(np.float64) + np.sign(y0) * np.spacing(np.abs(y0)).astype(np.float64) / 2
    x = (mid * np.float64(np.float32(T))).astype(np.float32)
    step = rng.integers(-1, 2, size=x.shape)
    x = np.where(step > 0, np.nextafter(x, np.float32(np.inf)),
                 np.where(step < 0, np.nextafter(x, np.float32(-np.inf)), x)).astype(np.float32)
    g = torch.Generator().manual_seed(5)
    xg = aligned_rows(torch.from_numpy(x))
    assert ops.sample_route(xg, temperature=T, top_p=0.9)[0] == ops.ROUTE_TOPP32
    _check(xg, f"midpoints T {T}", temperature=T, top_p=0.9, uniforms=_u(B, g))
