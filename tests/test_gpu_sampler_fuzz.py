"""Randomised GPU parity of the sampler against the exact CPU oracle.

Each case draws a batch shape, a logit distribution built to stress the
selection paths (few distinct values so that bins hold many tokens, exact
penalty ties with rho = 2, zeros and huge values kept one by one, spikes),
a repetition penalty with duplicated history ids, an allow mask, and the
temperature / top-k / top-p / uniform parameters; the GPU result (whichever
kernel the call routes to) must equal the oracle bit for bit."""

import numpy as np
import pytest
import torch

from graspo_amd import workloads as W
from tests._util import oracle_sample
from tests.test_gpu_sampler import assert_parity, gpu_sample

pytestmark = pytest.mark.gpu


def _logits(rng, B, V, kind):
    if kind == "normal":
        x = rng.normal(0.0, rng.uniform(0.5, 4.0), (B, V))
    elif kind == "few":
        vals = rng.normal(0.0, 2.0, int(rng.integers(1, 12)))
        x = vals[rng.integers(0, len(vals), (B, V))]
    elif kind == "grid":
        x = np.round(rng.normal(0.0, 3.0, (B, V)) * 4) / 4
    elif kind == "pow2":  # rho = 2 maps these onto each other exactly
        x = 2.0 ** rng.integers(-3, 4, (B, V)) * rng.choice([-1.0, 1.0], (B, V))
    else:  # "wild": zeros, huge and tiny magnitudes, spikes
        x = rng.normal(0.0, 2.0, (B, V))
        sel = rng.random((B, V))
        x[sel < 0.05] = 0.0
        x[(sel >= 0.05) & (sel < 0.06)] = 3.0e7
        x[(sel >= 0.06) & (sel < 0.07)] = 1.0e-13
        x[:, rng.integers(0, V)] += 20.0
    return torch.from_numpy(x.astype(np.float32))


@pytest.mark.parametrize("seed", range(12))
def test_random_cases(seed):
    rng = np.random.default_rng(1000 + seed)
    for case in range(12):
        B = int(rng.integers(1, 9))
        V = int(rng.choice([8, 37, 1000, 4096, 4099, 20000, 65536]))
        kind = str(rng.choice(["normal", "few", "grid", "pow2", "wild"]))
        dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.bfloat16, torch.float32,
                            torch.float16])
        x = _logits(rng, B, V, kind).to(dtype)
        T = float(rng.choice([0.0, 0.3, 1.0, 1.0, 5.0]))
        top_k = int(rng.choice([0, 0, 1, 5, 64, 200, 1000]))
        top_p = float(rng.choice([1.0, 0.5, 0.9, 0.99, 0.999]))
        rho = float(rng.choice([1.0, 1.0, 0.5, 1.3, 2.0]))
        kw = dict(temperature=T, top_k=top_k, top_p=top_p, repetition_penalty=rho)
        if rho != 1.0:
            L = int(rng.integers(1, 3 * V))
            kw["history"] = torch.from_numpy(
                rng.integers(-1, V, (B, L)).astype(np.int32))
        if rng.random() < 0.4:
            bits = torch.from_numpy(rng.random((B, V)) < rng.uniform(0.01, 0.9))
            bits[:, int(rng.integers(0, V))] = True
            kw["allow_mask"] = W.pack_mask(bits)
        u = (rng.integers(0, 1 << 24, B) * 2.0 ** -24).astype(np.float32)
        u[rng.random(B) < 0.1] = 0.0
        u[rng.random(B) < 0.1] = np.float32(1.0 - 2.0 ** -24)
        kw["uniforms"] = torch.from_numpy(u)
        what = f"seed {seed} case {case}: B{B} V{V} {kind} {dtype} {kw.keys()} T{T} k{top_k} " \
               f"p{top_p} rho{rho}"
        print(what, flush=True)
        assert_parity(gpu_sample(x, **kw), oracle_sample(x, **kw), what)
