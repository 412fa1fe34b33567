"""The hidden-state logprob path's matrix-core route.

``gtp_f32_to_bf16_exact`` must return the upper 16 bits of every fp32 value
and flag exactly the inputs that are not bf16 values (nonzero lower bits,
NaN payloads there included), for aligned, unaligned and ragged lengths.

``_selected_token_log_probs_from_hidden`` must take the bf16 route when its
fp32 operands are bf16 values (as the reference's ``.float()`` copies are) --
the fused GEMM + lse kernel when H is a multiple of 128, the chunked GEMMs
otherwise -- stay in fp32 otherwise, and in every case agree with an fp64 evaluation of
the reference expression (tensor_utils.py:167-186) within 1e-4 -- well inside
the 1e-3 contract, since the bf16 x bf16 products are exact in fp32 and the
logits are kept in fp32."""

import pytest
import torch

from graspo_amd import ops
from graspo_amd import tensor_utils as TU

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("n", [1, 3, 4, 1000, 4099, 1 << 20])
@pytest.mark.parametrize("offset", [0, 1])
def test_narrowing_matches_truncation_and_flags(n, offset):
    g = torch.Generator().manual_seed(n + offset)
    exact = torch.randn(n + offset, generator=g).to(torch.bfloat16).float()
    src = exact.to(DEV)[offset:]  # offset 1: a 4-byte aligned, not 16-byte aligned start
    bf, flag = ops.to_bf16_exact(src)
    torch.cuda.synchronize()
    assert int(flag) == 0
    assert torch.equal(bf.cpu().view(torch.int16), exact[offset:].to(torch.bfloat16).view(torch.int16))
    for pos in {0, n // 2, n - 1}:
        bad = exact.clone()
        bits = bad.view(torch.int32)
        bits[offset + pos] |= 1  # one low bit: not a bf16 value
        _, flag = ops.to_bf16_exact(bad.to(DEV)[offset:])
        torch.cuda.synchronize()
        assert int(flag) == 1, (n, offset, pos)


def test_narrowing_specials():
    vals = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), float("nan"), 1e-40, -3.5])
    bf, flag = ops.to_bf16_exact(vals.to(DEV))
    torch.cuda.synchronize()
    assert int(flag) == 1  # 1e-40 (a subnormal) has low bits
    head = vals[:6].clone()
    head[5] = 2.0 ** -126
    bf, flag = ops.to_bf16_exact(head.to(DEV))
    torch.cuda.synchronize()
    assert int(flag) == 0
    upper = (head.view(torch.int32) >> 16).to(torch.int16)  # the contract: the upper 16 bits
    assert torch.equal(bf.cpu().view(torch.int16), upper)
    payload = torch.tensor([0x7F800001], dtype=torch.int32).view(torch.float32)  # NaN, low payload
    _, flag = ops.to_bf16_exact(payload.to(DEV))
    torch.cuda.synchronize()
    assert int(flag) == 1


def _reference_fp64(h, w, ids):
    logits = h.double() @ w.double().t()
    return logits.gather(-1, ids.unsqueeze(-1)).squeeze(-1) - torch.logsumexp(logits, -1)


@pytest.mark.parametrize("kind", ["fp32_of_bf16", "fp32_inexact", "bf16"])
def test_hidden_path_routes_and_accuracy(kind):
    g = torch.Generator().manual_seed(7)
    B, S, H, V = 2, 33, 256, 20000
    h = torch.randn(B, S, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(V, H, generator=g) * 0.15).to(torch.bfloat16)
    ids = torch.randint(0, V, (B, S), generator=g)
    if kind == "fp32_of_bf16":
        h_in, w_in = h.float(), w.float()
    elif kind == "fp32_inexact":
        h_in, w_in = h.float(), w.float() + 1e-6 * torch.randn(V, H, generator=g)
    else:
        h_in, w_in = h, w
    h_in, w_in, ids_d = h_in.to(DEV), w_in.to(DEV), ids.to(DEV)
    mc = TU._matrix_core_operands(h_in.reshape(-1, H), w_in)
    assert (mc is not None) == (kind != "fp32_inexact")
    # bf16 operands with H a multiple of 128 take the fused GEMM + lse kernel
    assert (mc is not None and ops.lm_head_supported(*mc)) == (kind != "fp32_inexact")
    print("hidden route", kind, flush=True)
    out = TU._selected_token_log_probs_from_hidden(h_in, w_in, ids_d, vocab_chunk_size=4096)
    ref = _reference_fp64(h_in.cpu(), w_in.cpu(), ids)
    err = float((out.double().cpu() - ref).abs().max())
    assert err <= 1e-4, (kind, err)


def test_hidden_path_gradients_on_the_bf16_route():
    g = torch.Generator().manual_seed(8)
    B, S, H, V = 2, 9, 64, 5000
    h = torch.randn(B, S, H, generator=g).to(torch.bfloat16).float().to(DEV).requires_grad_(True)
    w = (torch.randn(V, H, generator=g) * 0.2).to(torch.bfloat16).float().to(DEV)
    w.requires_grad_(True)
    ids = torch.randint(0, V, (B, S), generator=g).to(DEV)
    out = TU._selected_token_log_probs_from_hidden(h, w, ids, vocab_chunk_size=1024)
    gout = torch.randn(B, S, generator=g).to(DEV)
    (out * gout).sum().backward()
    h2 = h.detach().double().requires_grad_(True)
    w2 = w.detach().double().requires_grad_(True)
    logits = h2 @ w2.t()
    ref = logits.gather(-1, ids.unsqueeze(-1)).squeeze(-1) - torch.logsumexp(logits, -1)
    (ref * gout.double()).sum().backward()
    assert float((out.double() - ref).abs().max()) <= 1e-4
    assert float((h.grad.double() - h2.grad).abs().max()) <= 1e-4
    assert float((w.grad.double() - w2.grad).abs().max()) <= 1e-4


@pytest.mark.parametrize("V", [4099, 32768])
def test_split_gradient_is_the_fp32_gradient(V):
    """gtp_logprob_backward_split_rows: hi and lo are bf16 with hi the fp32
    gradient rounded to bf16 and |grad - hi - lo| <= 2^-16 |grad| (each bf16
    rounding is within 2^-8; + a tiny absolute floor), against the fp32 gradient kernel and fp64; rows with
    g == 0 are zeros; a column offset moves the one-hot term."""
    g0 = torch.Generator().manual_seed(V)
    N = 12
    x = (torch.randn(N, V, generator=g0) * 3.0).to(DEV)
    t = torch.randint(0, V, (N,), generator=g0).to(DEV)
    g = torch.randn(N, generator=g0).to(DEV)
    g[2] = 0.0
    x[4, 9] = 50.0
    t[4] = 9  # one-hot spike: the gradient is ~0 everywhere, computed without cancellation
    lse = torch.logsumexp(x.double(), dim=1).float()
    for off in (0, 17):
        hi, lo = ops.logprob_backward_split(x, t + off, g, lse, col_offset=off)
        full = ops.logprob_backward(x, t + off, g, lse, col_offset=off)
        torch.cuda.synchronize()
        assert torch.equal(hi, full.to(torch.bfloat16))
        s = hi.float() + lo.float()
        assert float(((s - full).abs() - full.abs() * 2.0 ** -16 - 1e-30).max()) <= 0.0
        xd = x.double()
        p = torch.exp(xd - lse.double().unsqueeze(1))
        ref = -g.double().unsqueeze(1) * p
        ref[torch.arange(N), t] += g.double()
        # the fp32 gradient's own bound (tests/test_gpu_logprob_backward.py)
        # plus the split's 2^-16
        assert float(((s.double() - ref).abs() - (2e-6 + 2.0 ** -16) * ref.abs() - 1e-7).max()) <= 0.0
        assert not bool(hi[2].float().any()) and not bool(lo[2].float().any())


@pytest.mark.parametrize("exact", [True, False])
def test_fp32_top_p_rows_take_the_bf16_kernel_when_exact(exact):
    """_next_token_from_logits on fp32 rows holding bf16 values (as the
    reference's logits.float() are) samples them through the bf16 kernels and
    returns exactly the ids of the bf16 rows and of the oracle on the fp32
    values; rows that are not bf16 values keep the fp32 path and still match
    the oracle."""
    from tests._util import oracle_sample

    g = torch.Generator().manual_seed(21)
    B, V = 16, 151936
    xb = (torch.randn(B, V, generator=g) * 2.5).to(torch.bfloat16)
    x32 = xb.float()
    if not exact:
        x32 = x32 + 1e-4 * torch.randn(B, V, generator=g)
    u = (torch.randint(0, 1 << 24, (B,), generator=g).float() * 2.0 ** -24)
    kw = dict(temperature=0.8, top_p=0.9, uniforms=u.to(DEV))
    print("fp32 top-p route", exact, flush=True)
    ids32 = TU._next_token_from_logits(x32.to(DEV), **kw)
    want = oracle_sample(x32, temperature=0.8, top_p=0.9, uniforms=u)
    assert torch.equal(ids32.cpu(), torch.from_numpy(want.ids)), exact
    if exact:
        idsb = TU._next_token_from_logits(xb.to(DEV), **kw)
        assert torch.equal(ids32, idsb)


def test_hidden_path_gradients_on_the_fused_route(monkeypatch):
    """K a multiple of 128: the forward keeps the fused kernel's fp32 logits
    and the backward runs bf16(-g p) through two matrix-core GEMMs, adding
    the one-hot term g [i == t] in fp32.  Each gradient element is within
    2^-8 * sum_i |g p_i w_i| (the bf16 rounding of -g p; doubled here for
    the fp32 sums) of the fp64 gradient; a missing or misplaced one-hot term
    is off by |g w_t| ~ the whole sum."""
    calls = []
    real = ops.lm_head_logprob_save
    monkeypatch.setattr(ops, "lm_head_logprob_save", lambda *a: calls.append(1) or real(*a))
    g = torch.Generator().manual_seed(9)
    B, S, H, V = 2, 150, 256, 5077
    h = torch.randn(B, S, H, generator=g).to(torch.bfloat16).float().to(DEV).requires_grad_(True)
    w = (torch.randn(V, H, generator=g) * 0.1).to(torch.bfloat16).float().to(DEV)
    w.requires_grad_(True)
    ids = torch.randint(0, V, (B, S), generator=g).to(DEV)
    ids[0, :4] = ids[1, 7]  # a target shared by several tokens (index_add of the one-hot term)
    gout = torch.randn(B, S, generator=g).to(DEV)
    gout[1, 3] = 0.0
    print("fused-route gradients", flush=True)
    out = TU._selected_token_log_probs_from_hidden(h, w, ids)
    (out * gout).sum().backward()
    assert calls, "the fused route with saved logits was not taken"
    h2 = h.detach().double().requires_grad_(True)
    w2 = w.detach().double().requires_grad_(True)
    logits = h2 @ w2.t()
    ref = logits.gather(-1, ids.unsqueeze(-1)).squeeze(-1) - torch.logsumexp(logits, -1)
    (ref * gout.double()).sum().backward()
    assert float((out.double() - ref).abs().max()) <= 1e-4
    p = torch.softmax(logits.detach(), -1).view(-1, V)
    gp = (gout.double().view(-1, 1).abs() * p)                       # |g| p  [N, V]
    bound_h = 2.0 ** -7 * (gp @ w2.detach().abs()) + 1e-6            # [N, H]
    bound_w = 2.0 ** -7 * (gp.t() @ h2.detach().abs().view(-1, H)) + 1e-6  # [V, H]
    err_h = (h.grad.double().view(-1, H) - h2.grad.view(-1, H)).abs()
    err_w = (w.grad.double() - w2.grad).abs()
    assert bool((err_h <= bound_h).all()), float((err_h - bound_h).max())
    assert bool((err_w <= bound_w).all()), float((err_w - bound_w).max())
    # the one-hot term alone is far outside the bound
    onehot = gout.double().view(-1, 1).abs() * w2.detach()[ids.view(-1)].abs()
    assert float((onehot - bound_h).max()) > 0
