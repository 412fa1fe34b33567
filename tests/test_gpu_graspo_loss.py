"""GPU parity of the fused GRASPO loss (gtp_graspo_loss_forward / _backward)
against the reference's torch expression (graspo_loss.py:10-16, 45-63) and
its autograd, in fp32 on the same device.  The loss may differ by summation
order only (1e-6 relative); per-token gradients by a few fp32 ulps."""

import pytest
import torch

from graspo_amd.graspo_loss import GRASPOLoss

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def reference_loss(lp, old, adv, mask, eps):
    ratio = (lp - old).exp()
    surr1 = ratio * adv
    surr2 = ratio.clamp(1 - eps, 1 + eps) * adv
    loss = -torch.min(surr1, surr2)
    if mask is None:
        return loss.mean(dim=-1).mean()
    denom = mask.sum(dim=-1).clamp_min(1)
    return ((loss * mask).sum(dim=-1) / denom).mean()


def _compare(lp, old, adv, mask, eps, what):
    a = lp.clone().requires_grad_(True)
    got = GRASPOLoss(eps)(a, old, adv, mask)
    got.backward()
    b = lp.clone().requires_grad_(True)
    want = reference_loss(b, old, adv, mask, eps)
    want.backward()
    torch.cuda.synchronize()
    assert abs(float(got) - float(want)) <= 1e-6 * max(1.0, abs(float(want))), (what, got, want)
    gd = (a.grad - b.grad).abs().max()
    assert float(gd) <= 1e-6 * max(1e-3, float(b.grad.abs().max())) + 1e-9, (what, float(gd))


@pytest.mark.parametrize("eps", [0.2, 0.1, 0.28])
def test_random_batches(eps):
    g = torch.Generator().manual_seed(int(eps * 100))
    B, T = 16, 2047
    lp = (-torch.rand(B, T, generator=g) * 3).to(DEV)
    old = (lp.cpu() + torch.randn(B, T, generator=g) * 0.3).to(DEV)
    adv = torch.randn(B, 1, generator=g).expand(B, T).contiguous().to(DEV)
    mask = (torch.rand(B, T, generator=g) < 0.7).to(DEV)
    mask[3] = False  # a sequence without actions: denominator 1, zero loss and gradient
    print("graspo loss", eps, flush=True)
    _compare(lp, old, adv, mask, eps, "bool mask")
    _compare(lp, old, adv, mask.float() * 0.5, eps, "weighted mask")
    _compare(lp, old, adv, None, eps, "no mask")


def test_ties_and_boundaries():
    """r = 1 with A = 0 (both surrogates equal), r exactly 1 with A != 0, and
    per-token advantages of both signs around the clip edges."""
    B, T = 4, 64
    lp = torch.zeros(B, T, device=DEV)
    old = torch.zeros(B, T, device=DEV)
    adv = torch.zeros(B, T, device=DEV)
    adv[1] = 1.0
    adv[2] = -1.0
    lp[2:] = torch.linspace(-0.5, 0.5, T, device=DEV)
    adv[3] = torch.linspace(-1, 1, T, device=DEV)
    mask = torch.ones(B, T, dtype=torch.bool, device=DEV)
    _compare(lp, old, adv, mask, 0.2, "ties")


def test_three_dim_input_and_broadcast_advantages():
    g = torch.Generator().manual_seed(3)
    lp = (-torch.rand(2, 3, 100, generator=g)).to(DEV)
    old = (lp.cpu() + 0.1 * torch.randn(2, 3, 100, generator=g)).to(DEV)
    adv = torch.randn(2, 3, 1, generator=g).to(DEV)
    mask = (torch.rand(2, 3, 100, generator=g) < 0.5).to(DEV)
    _compare(lp, old, adv.expand(2, 3, 100), mask, 0.2, "3-D")
    a = lp.clone().requires_grad_(True)
    got = GRASPOLoss(0.2)(a, old, adv, mask)  # advantages broadcast inside
    want = reference_loss(lp, old, adv, mask, 0.2)
    assert abs(float(got) - float(want)) <= 1e-6


def _compare_elementwise(lp, old, adv, mask, eps):
    """Loss and per-token gradient equal to torch's, NaN where torch has NaN."""
    a = lp.clone().requires_grad_(True)
    got = GRASPOLoss(eps)(a, old, adv, mask)
    got.backward()
    b = lp.clone().requires_grad_(True)
    want = reference_loss(b, old, adv, mask, eps)
    want.backward()
    torch.cuda.synchronize()
    torch.testing.assert_close(got.detach(), want.detach(), rtol=1e-6, atol=1e-7, equal_nan=True)
    assert torch.equal(a.grad.isnan(), b.grad.isnan()), (a.grad, b.grad)
    torch.testing.assert_close(a.grad, b.grad, rtol=1e-6, atol=1e-9, equal_nan=True)


def test_non_finite_logprobs_propagate_like_torch():
    """NaN and +-inf log-probs, at masked and unmasked positions: torch's min
    and clamp pass NaN through, NaN * 0 under the mask still poisons the
    sum, and autograd puts NaN on the same gradient positions."""
    B, T = 4, 16
    g = torch.Generator().manual_seed(11)
    lp = (-torch.rand(B, T, generator=g)).to(DEV)
    old = (lp.cpu() + 0.2 * torch.randn(B, T, generator=g)).to(DEV)
    adv = torch.randn(B, T, generator=g).to(DEV)
    mask = torch.ones(B, T, dtype=torch.bool, device=DEV)
    nan, inf = float("nan"), float("inf")
    lp[0, 3] = nan                      # unmasked NaN
    lp[1, 5] = nan                      # masked NaN
    mask[1, 5] = False
    lp[2, 7] = inf                      # r = inf with A > 0: s1 = inf
    adv[2, 7] = 1.5
    lp[2, 8] = -inf                     # r = 0
    lp[3, 2] = inf                      # r = inf with A = 0: s1 = NaN, masked
    adv[3, 2] = 0.0
    mask[3, 2] = False
    lp[3, 9] = inf                      # r = inf with A < 0: s1 = -inf
    adv[3, 9] = -0.5
    print("graspo loss non-finite: whole batch", flush=True)
    _compare_elementwise(lp, old, adv, mask, 0.2)
    # one sequence at a time, so a finite loss is compared where torch has one
    for b in range(B):
        print("graspo loss non-finite: sequence", b, flush=True)
        _compare_elementwise(lp[b:b + 1].contiguous(), old[b:b + 1].contiguous(),
                             adv[b:b + 1].contiguous(), mask[b:b + 1].contiguous(), 0.2)
    # NaN in the advantages, and a float mask of zero weight on a NaN
    adv2 = adv.clone()
    adv2[0, 0] = nan
    print("graspo loss non-finite: NaN advantage, float mask", flush=True)
    _compare_elementwise(lp, old, adv2, mask.float(), 0.2)
