"""GPU parity of the fused lm_head kernel (bf16 GEMM on the matrix cores
with the log-sum-exp in its epilogue, gtp_lm_head_logprob_rows) against an
fp64 evaluation of the reference's expression
(_selected_token_log_probs_from_hidden, tensor_utils.py:167-186):
logprob, entropy and logsumexp within 1e-4 absolute.

Shapes cover vocabulary and token tails (V and N not multiples of the
256 x 256 tile), a vocabulary smaller than one tile, one token, strided
hidden rows, int32 and int64 targets, bad targets, large logits, and the
full [8192, 4096] x [248320, 4096] case on sampled rows."""

import pytest
import torch

from graspo_amd import ops

pytestmark = pytest.mark.gpu

TOL = 1e-4


def fp64_reference(h, w, t):
    x = h.double() @ w.double().t()
    lse = torch.logsumexp(x, dim=-1)
    lp = x.gather(1, t.long().clamp(0, w.shape[0] - 1)[:, None])[:, 0] - lse
    logp = x - lse[:, None]
    ent = -(logp.exp() * logp).sum(-1)
    return lp, ent, lse


def _case(N, V, K, seed, scale=1.0, t64=False, hidden=None):
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    if hidden is None:
        hidden = torch.randn(N, K, generator=g, device="cuda:0").to(torch.bfloat16)
    w = (torch.randn(V, K, generator=g, device="cuda:0") * (scale / K ** 0.5)).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), generator=g, device="cuda:0",
                      dtype=torch.int64 if t64 else torch.int32)
    return hidden, w, t


def _check(h, w, t, what):
    print("lm_head:", what, tuple(h.shape), tuple(w.shape), flush=True)
    assert ops.lm_head_supported(h, w)
    lp, ent, lse = ops.lm_head_logprob(h, w, t)
    torch.cuda.synchronize()
    rlp, rent, rlse = fp64_reference(h, w, t)
    for name, a, b in (("logprob", lp, rlp), ("entropy", ent, rent), ("lse", lse, rlse)):
        err = (a.double() - b).abs().max().item()
        assert err <= TOL, f"{what}: {name} differs by {err}"
    return lp


@pytest.mark.parametrize("N,V,K", [(300, 1037, 256), (1, 256, 128), (257, 300, 128),
                                   (512, 100, 384), (1000, 40000, 1024), (256, 65536 + 255, 512)])
def test_shapes_and_tails(N, V, K):
    h, w, t = _case(N, V, K, seed=N + V + K)
    _check(h, w, t, f"N {N} V {V} K {K}")


def test_strided_hidden_and_int64_targets():
    g = torch.Generator(device="cuda:0").manual_seed(3)
    big = torch.randn(640, 1024 + 64, generator=g, device="cuda:0").to(torch.bfloat16)
    h = big[:, 32:32 + 1024]  # rows 1088 elements apart, 64-byte offset
    _, w, t = _case(640, 5000, 1024, seed=4, t64=True, hidden=h)
    _check(h, w, t, "strided hidden, int64 targets")


def test_large_logits():
    """Logits of several hundred: the online max and the merge of partial
    states across vocabulary groups must not overflow."""
    h, w, t = _case(384, 20000, 512, seed=5, scale=60.0)
    lp = _check(h, w, t, "large logits")
    assert torch.isfinite(lp).all()


def test_bad_targets_give_nan():
    h, w, t = _case(64, 3000, 256, seed=6)
    t[3] = -1
    t[9] = 3000
    lp, ent, lse = ops.lm_head_logprob(h, w, t)
    torch.cuda.synchronize()
    assert torch.isnan(lp[3]) and torch.isnan(lp[9])
    assert torch.isfinite(lp[torch.arange(64, device=lp.device) % 3 == 1]).all()
    assert torch.isfinite(ent).all() and torch.isfinite(lse).all()


def test_full_size_sampled_rows():
    """[8192, 4096] x [248320, 4096]: every row against the chunked
    hipBLASLt + lse path within 1e-4, and 64 sampled rows against fp64."""
    N, V, K = 8192, 248320, 4096
    h, w, t = _case(N, V, K, seed=7, scale=4.0)
    print("lm_head: full size", flush=True)
    lp, ent, lse = ops.lm_head_logprob(h, w, t)
    torch.cuda.synchronize()
    rows = torch.randperm(N, generator=torch.Generator().manual_seed(8))[:64].to("cuda:0")
    rlp, rent, rlse = fp64_reference(h[rows], w, t[rows])
    for name, a, b in (("logprob", lp[rows], rlp), ("entropy", ent[rows], rent),
                       ("lse", lse[rows], rlse)):
        err = (a.double() - b).abs().max().item()
        assert err <= TOL, f"full size: {name} differs by {err}"
    # every row against the chunked path (fp32 logits from hipBLASLt, lse kernel)
    state = ops.new_lse_state(N, h.device)
    for c, start in enumerate(range(0, V, 32768)):
        logits = torch.mm(h, w[start:start + 32768].t(), out_dtype=torch.float32)
        ops.lse_partial(logits, t, start, state, accumulate=c > 0)
        del logits
    clp, cent = ops.lse_finalize(state)
    assert (lp - clp).abs().max().item() <= 2 * TOL
    assert (ent - cent).abs().max().item() <= 2 * TOL


def test_strided_weight_rows():
    """lm_head weight rows farther apart than K (a column slice of a wider
    matrix): the buffer ranges and offsets follow the row stride."""
    g = torch.Generator(device="cuda:0").manual_seed(9)
    K = 512
    big = (torch.randn(3000, K + 136, generator=g, device="cuda:0") / K ** 0.5).to(torch.bfloat16)
    w = big[:, 64:64 + K]  # rows 648 elements apart, 128-byte offset
    h, _, t = _case(300, 3000, K, seed=10)
    assert w.stride(0) == K + 136
    _check(h, w, t, "strided weight")


@pytest.mark.parametrize("N,V,K", [(300, 1037, 256), (257, 300, 128), (1, 256, 128),
                                   (512, 100, 384), (1000, 40001, 1024)])
def test_save_keeps_the_logits(N, V, K):
    """gtp_lm_head_logprob_save_rows: the same logprob and lse as the kernel
    that writes no logits, and every logit of the product, vocabulary-major
    (token and vocabulary tails, a vocabulary below one tile), within 1e-4
    of fp64; a bad target is NaN with its status."""
    h, w, t = _case(N, V, K, seed=N + 2 * V + K)
    if N > 3:
        t[3] = V
    print("lm_head save:", (N, V, K), flush=True)
    lp, lse, logits_t, status = ops.lm_head_logprob_save(h, w, t)
    lp0, _, lse0 = ops.lm_head_logprob(h, w, t)
    torch.cuda.synchronize()
    assert tuple(logits_t.shape) == (V, N) and logits_t.dtype == torch.float32
    x = h.double() @ w.double().t()
    assert (logits_t.t().double() - x).abs().max().item() <= TOL
    ok = torch.ones(N, dtype=torch.bool, device=lp.device)
    if N > 3:
        ok[3] = False
        assert torch.isnan(lp[3]) and int(status[3]) == ops.ROW_BAD_TARGET
    assert bool((status[ok] == ops.ROW_OK).all())
    assert (lp[ok] - lp0[ok]).abs().max().item() <= 1e-6
    assert (lse - lse0).abs().max().item() <= 1e-6
    rlp, _, rlse = fp64_reference(h, w, t)
    assert (lp[ok].double() - rlp[ok]).abs().max().item() <= TOL
    assert (lse.double() - rlse).abs().max().item() <= TOL


@pytest.mark.parametrize("N,V,stride,off", [(4099, 300, 4099, 0), (8192, 2000, 8192, 0),
                                            (1000, 77, 1004, 0), (3, 5000, 3, 0),
                                            (777, 130, 781, 1)])
def test_softmax_grad_bf16(N, V, stride, off):
    """bf16(-g_n softmax(x_n)) of vocabulary-major logits: within 2^-8 of the
    fp64 value (plus the fp32 evaluation's ~3e-6 relative), zeros for a
    token with g == 0, any row stride, token and vocabulary tails, and
    logits that do not start on a 16-byte boundary (off = 1)."""
    g0 = torch.Generator(device="cuda:0").manual_seed(N + V)
    big = torch.randn(V, stride, generator=g0, device="cuda:0") * 3.0
    xt = big[:, off:off + N]            # [V, N], token n's logits are column n
    xt[9, min(4, N - 1)] = 50.0         # p ~ 1 at one token
    g = torch.randn(N, generator=g0, device="cuda:0")
    g[min(2, N - 1)] = 0.0
    lse = torch.logsumexp(xt.double(), dim=0).float()
    print("softmax grad:", N, V, stride, flush=True)
    gs, none = ops.softmax_grad_bf16(xt, g, lse)
    torch.cuda.synchronize()
    assert none is None
    assert gs.dtype == torch.bfloat16 and tuple(gs.shape) == (V, N)
    ref = -g.double().unsqueeze(0) * torch.exp(xt.double() - lse.double().unsqueeze(0))
    err = (gs.double() - ref).abs() - (2.0 ** -8 + 1e-5) * ref.abs() - 1e-38
    assert err.max().item() <= 0.0
    assert not bool(gs[:, min(2, N - 1)].float().any())
    # both layouts from one pass, and the token-major one alone: the same
    # values bit for bit
    print("softmax grad, both layouts:", N, V, stride, flush=True)
    gt2, gn2 = ops.softmax_grad_bf16(xt, g, lse, token_major=True)
    none, gn3 = ops.softmax_grad_bf16(xt, g, lse, vocab_major=False, token_major=True)
    torch.cuda.synchronize()
    assert none is None and tuple(gn2.shape) == (N, V) and tuple(gn3.shape) == (N, V)
    assert torch.equal(gt2, gs)
    assert torch.equal(gn2, gs.t()) and torch.equal(gn3, gs.t())
