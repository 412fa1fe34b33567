"""GPU parity of the vocabulary-split sampler path (greedy and 1 <= top_k <=
128 on 16-byte aligned rows) against the exact CPU oracle.

Covers the row statuses in that path, vocabulary tails that do not fill a
16-byte vector, rho < 1, masks of every density, many rows (several
workgroups per CU), exact ties that overflow the candidate list, and repeated
calls on the same workspace with changing shapes."""

import numpy as np
import pytest
import torch

from graspo_amd import ops
from graspo_amd import workloads as W
from tests._util import oracle_sample
from tests.test_gpu_sampler import assert_parity, gpu_sample

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("top_k,temperature", [(5, 1.0), (1, 0.7), (128, 0.9), (0, 0.0)])
def test_status_rows_split_path(top_k, temperature):
    V = 4096
    x = torch.zeros(9, V)
    x[0, 3] = float("nan")
    x[1, 4] = float("inf")
    bits = torch.ones(9, V, dtype=torch.bool)
    bits[2] = False
    bits[3] = False
    bits[3, 39] = True
    hist = torch.full((9, 3), -1, dtype=torch.int32)
    hist[4, 1] = V
    hist[8, 0] = 7
    u = torch.full((9,), 0.5)
    u[5] = 1.0
    x[6] = float("-inf")
    x[7] = torch.arange(V, dtype=torch.float32) % 7
    x[8] = torch.randn(V, generator=torch.Generator().manual_seed(8))
    fin = torch.zeros(9, dtype=torch.bool)
    fin[7] = True
    kw = dict(temperature=temperature, top_k=top_k, top_p=0.8, repetition_penalty=1.2,
              history=hist, allow_mask=W.pack_mask(bits), uniforms=u, finished=fin,
              pad_token_id=-5)
    print("status rows", top_k, temperature, flush=True)
    assert_parity(gpu_sample(x, **kw), oracle_sample(x, **kw))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("V", [4099, 32773, 151936])
def test_vocab_tail_in_aligned_rows(dtype, V):
    """Rows 16-byte aligned (padded stride) but V not a multiple of the
    vector width: the last slice folds the tail tokens one by one."""
    g = torch.Generator().manual_seed(V)
    pad = (-V) % 8 + 8  # row stride a multiple of 8 elements: 16-byte aligned rows
    full = (torch.randn(5, V + pad, generator=g) * 3).to(dtype)
    full[:, V - 2] = 30.0  # a tail token must win sometimes
    u = W.uniforms_24(5, g, "cpu")
    dev = torch.device("cuda:0")
    view = full.to(dev)[:, :V]
    for kw in (dict(temperature=0.8, top_k=40, top_p=0.9), dict(temperature=0.0)):
        out = ops.sample(view, uniforms=u.to(dev), **kw)
        ref = oracle_sample(full[:, :V].contiguous(), uniforms=u, **kw)
        torch.cuda.synchronize()
        print(dtype, V, kw, flush=True)
        assert_parity(ops.SampleOutput(*[t.cpu() for t in out]), ref)


@pytest.mark.parametrize("seed", range(6))
def test_random_parameter_sweep(seed):
    rng = np.random.default_rng(seed)
    V = int(rng.choice([2048, 9000 * 8, 151936, 248320]))
    B = int(rng.choice([1, 3, 17]))
    dtype = [torch.bfloat16, torch.float16, torch.float32][seed % 3]
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, V, generator=g) * float(rng.uniform(0.5, 6))).to(dtype)
    density = float(rng.choice([0.002, 0.08, 0.5]))
    bits = torch.rand(B, V, generator=g) < density
    hist = torch.randint(-3, V, (B, int(rng.integers(1, 300))), generator=g, dtype=torch.int32)
    kw = dict(temperature=float(rng.choice([0.3, 0.7, 1.0, 2.5])),
              top_k=int(rng.choice([1, 2, 17, 64, 100, 128])),
              top_p=float(rng.choice([1.0, 0.5, 0.9, 0.99])),
              repetition_penalty=float(rng.choice([1.0, 1.3, 0.7])),
              history=hist, allow_mask=W.pack_mask(bits) if seed % 2 else None,
              uniforms=W.uniforms_24(B, g, "cpu"))
    print("sweep", seed, B, V, dtype, {k: v for k, v in kw.items() if not torch.is_tensor(v)},
          flush=True)
    assert_parity(gpu_sample(x, **kw), oracle_sample(x, **kw), f"seed {seed}")


def test_many_rows_one_launch():
    """B = 300 rows of the large-vocabulary workload: several rows per CU."""
    wl = W.sampler_workload(5, rows=300)
    print("many rows", wl.shape, flush=True)
    assert_parity(gpu_sample(wl.logits, **wl.kwargs()), oracle_sample(wl.logits, **wl.kwargs()))


@pytest.mark.parametrize("top_k", [1, 3, 128])
def test_exact_ties_overflow_candidates(top_k):
    """Thousands of tokens tied at the top of a slice: more than 1024 pass the
    key threshold, so the slice resolves its top-k by re-reading per digit."""
    V = 65536
    x = torch.zeros(4, V, dtype=torch.bfloat16)
    x[1, ::2] = 1.0
    x[2] = (torch.arange(V) % 3).to(torch.bfloat16)
    x[3, 5000:60000] = 2.0
    u = torch.tensor([0.0, 0.37, 0.999, 1 - 2**-24])
    for p in (1.0, 0.6):
        kw = dict(temperature=0.5, top_k=top_k, top_p=p, uniforms=u)
        print("ties", top_k, p, flush=True)
        assert_parity(gpu_sample(x, **kw), oracle_sample(x, **kw), f"k{top_k} p{p}")


def test_repeated_calls_reuse_workspace():
    """Consecutive calls with different row counts and k on one stream share
    the cached workspace; every call must match the oracle."""
    dev = torch.device("cuda:0")
    for i, (B, k) in enumerate([(8, 64), (40, 5), (8, 64), (3, 128), (40, 5)]):
        wl = W.sampler_workload(5, rows=B)
        kw = wl.kwargs()
        kw["top_k"] = k
        outs = [ops.sample(wl.logits.to(dev), **{n: (v.to(dev) if torch.is_tensor(v) else v)
                                                for n, v in kw.items()}) for _ in range(3)]
        torch.cuda.synchronize()
        ref = oracle_sample(wl.logits, **kw)
        print("repeat", i, B, k, flush=True)
        for o in outs:
            assert_parity(ops.SampleOutput(*[t.cpu() for t in o]), ref, f"call {i}")
