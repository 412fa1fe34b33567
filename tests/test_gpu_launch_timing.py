"""The launch-timing hook (gtp_time_next_launch): the next sampler, logprob
or logprob-gradient kernel records the two events at its own dispatch start
and end, once, without changing any result."""

import pytest
import torch

from graspo_amd import ops

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _events():
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    b.record()
    return a, b


def test_hook_brackets_the_kernel_and_is_used_once():
    g = torch.Generator(device=DEV).manual_seed(3)
    x = (torch.randn(64, 151936, device=DEV, generator=g) * 2.0).to(torch.bfloat16)
    u = ops.draw_uniforms(64, DEV, g)
    kw = dict(temperature=0.7, top_k=64, top_p=0.9, uniforms=u)
    k0, k1 = _events()
    o0, o1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ops.time_next_launch(k0, k1)
    o0.record()
    a = ops.sample(x, **kw)
    o1.record()
    torch.cuda.synchronize()
    t_kernel, t_outer = k0.elapsed_time(k1), o0.elapsed_time(o1)
    print("sampler kernel", t_kernel, "around", t_outer, flush=True)
    assert 0.0 < t_kernel <= t_outer
    b = ops.sample(x, **kw)  # no hook: the events stay where they were
    torch.cuda.synchronize()
    assert k0.elapsed_time(k1) == t_kernel
    assert torch.equal(a.ids, b.ids) and torch.equal(a.sampled_logprob, b.sampled_logprob)


def test_hook_on_logprob_and_gradient():
    g = torch.Generator(device=DEV).manual_seed(4)
    x = (torch.randn(256, 32768, device=DEV, generator=g) * 2.0).to(torch.bfloat16)
    t = torch.randint(0, 32768, (256,), device=DEV, generator=g)
    k0, k1 = _events()
    ops.time_next_launch(k0, k1)
    lp, H, st = ops.logprob_entropy(x, t)
    torch.cuda.synchronize()
    assert k0.elapsed_time(k1) > 0.0
    lp2, H2, _ = ops.logprob_entropy(x, t)
    assert torch.equal(lp, lp2) and torch.equal(H, H2)
    lse = x.gather(1, t.unsqueeze(1)).squeeze(1).float() - lp
    gl = torch.randn(256, device=DEV, generator=g)
    k2, k3 = _events()
    ops.time_next_launch(k2, k3)
    d1 = ops.logprob_backward(x, t, gl, lse)
    torch.cuda.synchronize()
    assert k2.elapsed_time(k3) > 0.0
    assert torch.equal(d1, ops.logprob_backward(x, t, gl, lse))


def test_hook_needs_existing_events():
    with pytest.raises(RuntimeError):
        ops.time_next_launch(torch.cuda.Event(enable_timing=True),
                             torch.cuda.Event(enable_timing=True))


def test_hook_spans_a_row_that_takes_the_row_wise_path():
    """A top-p call is one launch: a row outside the top-p kernel's bounds (a
    -inf logit is outside its bins) runs the row-wise path in the same
    kernel, so its time shows in the hooked interval."""
    g = torch.Generator(device=DEV).manual_seed(5)
    x = (torch.randn(128, 151936, device=DEV, generator=g) * 2.0).to(torch.bfloat16)
    u = ops.draw_uniforms(128, DEV, g)
    kw = dict(temperature=0.7, top_p=0.9, uniforms=u)
    xh = x.clone()
    xh[5, 77] = float("-inf")
    times = {}
    for name, xx in (("plain", x), ("handed_over", xh)):
        ops.sample(xx, **kw)  # warm
        k0, k1 = _events()
        o0, o1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ops.time_next_launch(k0, k1)
        o0.record()
        out = ops.sample(xx, **kw)
        o1.record()
        torch.cuda.synchronize()
        times[name] = (k0.elapsed_time(k1), o0.elapsed_time(o1))
        assert bool((out.status == 0).all())
    print("top-p call (hooked, around):", times, flush=True)
    (t0, a0), (t1, a1) = times["plain"], times["handed_over"]
    assert 0.0 < t0 <= a0 and 0.0 < t1 <= a1
    assert t1 - t0 > 0.5 * (a1 - a0) > 0.0
