"""GPU parity of the logprob-gradient kernel (gtp_logprob_backward_rows)
against an fp64 torch reference of g * (onehot - softmax), and of the
autograd drop-ins that use it: sequence_log_probs_from_logits, the hidden
path and sft_cross_entropy_loss (against torch.log_softmax / F.cross_entropy
autograd in fp32).

Tolerances: the kernel computes in fp32 and rounds once to the output
dtype, so an element may differ from the fp64 value by one rounding of the
output type plus a few fp32 ulps: 2^-8 relative for bf16, 2^-11 for fp16,
2e-6 for fp32 (plus 1e-7 absolute)."""

import pytest
import torch
import torch.nn.functional as F

from graspo_amd import ops
from graspo_amd.graspo_loss import sequence_log_probs_from_logits
from graspo_amd.sft_loss import sft_cross_entropy_loss

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
REL = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2e-6}


def _ref_grad(x, t, g, col_offset=0, lse=None):
    xd = x.double()
    if lse is None:
        lse = torch.logsumexp(xd, dim=1)
    p = torch.exp(xd - lse.double().unsqueeze(1))
    grad = -g.double().unsqueeze(1) * p
    V = x.shape[1]
    tl = t.long() - col_offset
    ok = (tl >= 0) & (tl < V)
    rows = torch.nonzero(ok).squeeze(1)
    grad[rows, tl[rows]] += g.double()[rows]
    return grad


def _check(got, ref, dtype, what):
    got = got.double().cpu()
    tol = REL[dtype] * ref.abs() + 1e-7
    err = (got - ref).abs() - tol
    assert float(err.max()) <= 0.0, (what, float((got - ref).abs().max()))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("V", [248320, 4099, 1000])
def test_kernel_matches_fp64(dtype, V):
    g0 = torch.Generator().manual_seed(V)
    N = 16
    x = (torch.randn(N, V, generator=g0) * 3.0).to(dtype)
    t = torch.randint(0, V, (N,), generator=g0)
    g = torch.randn(N, generator=g0)
    g[3] = 0.0  # an ignored row: zeros, not read
    x[5, 7] = 40.0
    t[5] = 7  # one-hot spike: gradient ~ 0 everywhere
    lse = torch.logsumexp(x.double(), dim=1).float()
    print("backward", dtype, V, flush=True)
    out = ops.logprob_backward(x.to(DEV), t.to(DEV), g.to(DEV), lse.to(DEV))
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == (N, V)
    _check(out, _ref_grad(x.float(), t, g, lse=lse), dtype, f"{dtype} V{V}")
    assert bool((out[3] == 0).all())


def test_strided_unaligned_and_chunk_offset():
    g0 = torch.Generator().manual_seed(5)
    N, V = 8, 5003
    full = (torch.randn(N, V + 13, generator=g0) * 2.0).to(torch.bfloat16).to(DEV)
    x = full[:, 1 : V + 1]  # row stride V + 13, rows not 16-byte aligned: scalar path
    t = torch.randint(0, V, (N,), generator=g0).to(DEV)
    g = torch.randn(N, generator=g0).to(DEV)
    lse = torch.logsumexp(x.double(), dim=1).float()
    out = ops.logprob_backward(x, t, g, lse)
    torch.cuda.synchronize()
    _check(out, _ref_grad(x.float().cpu(), t.cpu(), g.cpu(), lse=lse.cpu()), torch.bfloat16,
           "strided")
    # a vocabulary chunk: columns [2000, 3000) with the whole row's lse; targets
    # outside the chunk add no one-hot term
    chunk = x[:, 2000:3000].contiguous()
    t2 = t.clone()
    t2[0] = 2500
    out_c = ops.logprob_backward(chunk, t2, g, lse, col_offset=2000)
    torch.cuda.synchronize()
    _check(out_c, _ref_grad(chunk.float().cpu(), t2.cpu(), g.cpu(), 2000, lse.cpu()),
           torch.bfloat16, "chunk")


def test_out_argument_writes_in_place():
    g0 = torch.Generator().manual_seed(6)
    N, V = 4, 3000
    x = torch.randn(N, V, generator=g0).to(DEV)
    t = torch.randint(0, V, (N,), generator=g0).to(DEV)
    g = torch.ones(N, device=DEV)
    lse = torch.logsumexp(x, dim=1)
    buf = torch.full((N, V + 8), 7.0, device=DEV)
    ops.logprob_backward(x, t, g, lse, out=buf[:, :V])
    torch.cuda.synchronize()
    _check(buf[:, :V], _ref_grad(x.cpu(), t.cpu(), g.cpu(), lse=lse.cpu()), torch.float32, "out")
    assert bool((buf[:, V:] == 7.0).all())


def test_sequence_logprob_gradient_matches_autograd():
    g0 = torch.Generator().manual_seed(7)
    x = (torch.randn(2, 5, 32003, generator=g0) * 2.5).to(DEV).requires_grad_(True)
    ids = torch.randint(0, 32003, (2, 5), generator=g0).to(DEV)
    w = torch.randn(2, 5, generator=g0).to(DEV)
    (sequence_log_probs_from_logits(x, ids) * w).sum().backward()
    ref_x = x.detach().clone().requires_grad_(True)
    (torch.log_softmax(ref_x, -1).gather(-1, ids.unsqueeze(-1)).squeeze(-1) * w).sum().backward()
    torch.cuda.synchronize()
    assert float((x.grad - ref_x.grad).abs().max()) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sft_cross_entropy_matches_torch(dtype):
    g0 = torch.Generator().manual_seed(8)
    B, S, V = 3, 17, 30011
    x = (torch.randn(B, S, V, generator=g0) * 2.0).to(dtype).to(DEV).requires_grad_(True)
    labels = torch.randint(0, V, (B, S), generator=g0).to(DEV)
    labels[:, :5] = -100  # prompt positions
    labels[2, 9] = -100
    loss = sft_cross_entropy_loss(x, labels)
    loss.backward()
    xr = x.detach().float().clone().requires_grad_(True)
    ref = F.cross_entropy(xr[:, :-1].reshape(-1, V), labels[:, 1:].reshape(-1), ignore_index=-100)
    ref.backward()
    torch.cuda.synchronize()
    assert abs(float(loss) - float(ref)) <= 1e-5 * max(1.0, abs(float(ref)))
    assert x.grad.dtype == dtype
    gd = (x.grad.float() - xr.grad).abs()
    assert float(gd.max()) <= REL[dtype] * float(xr.grad.abs().max()) + 1e-7
    assert bool((x.grad[:, -1] == 0).all())


def test_sft_rejects_label_out_of_range():
    x = torch.randn(1, 4, 100, device=DEV)
    labels = torch.tensor([[0, 5, 100, 3]], device=DEV)
    with pytest.raises(RuntimeError):
        sft_cross_entropy_loss(x, labels)
