"""Benchmark of the vocabulary-wide token path on one MI355X.

A step is one pass of the hot path over the large-vocabulary workload:
the sampler over a bf16 [256, 248320] batch (repetition penalty over a
4096-token history, 8%-density allow mask, T 0.7, top-k 64, top-p 0.9) and
one logprob/entropy pass over bf16 [8192, 248320] with int32 targets.
Inputs are generated on the GPU and resident in HBM before timing; two
sampler batches alternate and the 4 GB logprob pass between them evicts the
256 MB MALL, so every sampler launch reads its logits from HBM.  In a timed
step each kernel runs alone: the host waits for the GPU to drain before
each launch, so that no kernel shares the GPU with the last workgroups of
the one before it.

Prints ONE JSON line.  ``value`` is sampled rows/s of the sampler kernel;
``logprob_tokens_per_s`` is the logprob kernel's throughput.  Kernel times
come from HIP events on the stream the kernels are launched on (torch's
current stream, which the ops use), recorded at each kernel's own dispatch
start and end through the library's launch hook (gtp_time_next_launch,
hipExtLaunchKernelGGL), as rocprofv3 times a kernel.  Events recorded around
a launch also count the event packets' idle microseconds and, the GPU being
drained before each timed launch, the host's launch latency; those figures
are reported beside as ``avg_us_events_around_launch``.  The side
measurements below run before the timed steps, and the step itself runs
untimed for PREWARM_S seconds before the W warm-up steps (reported as
``prewarm``), so that the timed steps run at the GPU's steady state.

``rooflines.logprob_backward`` times the logprob gradient kernel over the
same [8192, 248320] logits (read once, bf16 gradient written once).

``graspo_loss`` times forward + backward of the fused GRASPO loss against
the reference's torch expression over [16, 2048] token logprobs.

``decode_loop`` times the generation loop's own per-token work at the
[256, 248320] bf16 shape: the decode-loop drop-in against the reference's
loop body, both on this library's sampler, with a stand-in model.

``hidden_logprobs`` times the hidden-state logprob path (8192 tokens, hidden
4096, vocabulary 248320) as the callers use it, against the reference's fp32
expression, with the bf16 GEMM's TFLOP/s against the matrix-core peak.

``per_config`` adds the other sampler workloads (fp32 [8,151936]; bf16
[64,151936] top-p only; bf16 [64,151936] masked; the [256,248320] rows with
top-p only -- the decode loop's T 0.7 / P 0.9 rows, and the same with the
history and mask -- on the top-p kernel), each call timed alone (a
read-only pass over a 512 MB buffer evicts the MALL and the GPU drains
before every launch; every call is one kernel launch), and the loss-side
logprob workload: bf16 [32768,151936] x 2 passes (policy and reference
logits) in 4 chunks of 8192 rows each.

``stream_floor_us`` is the kernel time of gtp_stream_read_rows over the
same logits (a read-only pass with the samplers' access pattern: one
1024-thread workgroup per row, 16-byte non-temporal loads), MALL evicted:
the streaming floor the sampler kernels are compared with.

``cpu_baseline`` times the reference's CPU path (oracle/cpu_reference.py)
on bounded samples of every configuration, with all host threads, and names
the host CPU.

``--calibrate-copy`` runs only a 1 GiB device-to-device copy (the reference
kernel whose rocprof FETCH_SIZE / WRITE_SIZE scale the HBM traffic counters).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0
PREWARM_S = 0.3  # seconds of untimed steps before the warm-up steps
REPO = os.path.dirname(os.path.abspath(__file__))
SAMPLER_KERNEL = "sampler_split_kernel<bf16>"
LOGPROB_KERNEL = "logprob_entropy_kernel<bf16>"
BACKWARD_KERNEL = "logprob_backward_kernel<bf16>"
TRAFFIC_FILE = os.path.join(REPO, "profiles", "hbm_traffic_large_vocab.md")
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_rate(fn, units: int, min_seconds: float) -> float:
    fn()  # warmup
    reps, t0 = 0, time.perf_counter()
    while reps < 2 or time.perf_counter() - t0 < min_seconds:
        fn()
        reps += 1
    return units * reps / (time.perf_counter() - t0)


def cpu_baseline_configs(min_seconds: float = 3.0):
    """The reference's CPU path on bounded samples of configurations 1-4
    (config 5 is the headline cpu_baseline): rows/s for the samplers,
    tokens/s for the logprob workload."""
    from graspo_amd import workloads as W
    from oracle import cpu_reference as CR

    out = {}
    for cfg, rows in ((1, 8), (2, 16), (3, 16)):
        w = W.sampler_workload(cfg, device="cpu", rows=rows)
        bits = None if w.allow_mask is None else W.unpack_mask(w.allow_mask, w.logits.shape[1])
        kw = dict(temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                  repetition_penalty=w.repetition_penalty, history=w.history,
                  allow_mask_bits=bits, uniforms=w.uniforms)
        r = _cpu_rate(lambda: CR.sample_rows(w.logits, **kw), rows, min_seconds)
        out[f"config{cfg}"] = {"value": round(r, 2), "unit": "rows/s",
                               "sample": f"{rows} rows of {list(w.logits.shape[1:])} "
                                         f"{str(w.logits.dtype).replace('torch.', '')}"}
    x, t = W.logprob_workload(4, device="cpu", rows=256)
    r = _cpu_rate(lambda: CR.logprob_entropy_rows(x, t), 256, min_seconds)
    out["config4"] = {"value": round(r, 2), "unit": "tokens/s",
                      "sample": "256 rows of bf16 [32768, 151936] (pass 0)"}
    return out


def cpu_baseline(wl_cpu, lx_cpu, lt_cpu, min_seconds: float = 10.0):
    """The reference's CPU path (oracle/cpu_reference.py), timed on a bounded
    sample of the same workload with all host threads."""
    import torch

    from graspo_amd import workloads as W
    from oracle import cpu_reference as CR

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count() or 1
    torch.set_num_threads(threads)
    rows = wl_cpu.logits.shape[0]
    x = wl_cpu.logits
    bits = W.unpack_mask(wl_cpu.allow_mask, x.shape[1])
    kw = dict(temperature=wl_cpu.temperature, top_k=wl_cpu.top_k, top_p=wl_cpu.top_p,
              repetition_penalty=wl_cpu.repetition_penalty, history=wl_cpu.history,
              allow_mask_bits=bits, uniforms=wl_cpu.uniforms)
    CR.sample_rows(x, **kw)  # warmup
    reps, t0 = 0, time.perf_counter()
    while reps < 3 or time.perf_counter() - t0 < min_seconds:
        CR.sample_rows(x, **kw)
        reps += 1
    s_rows = rows * reps / (time.perf_counter() - t0)
    lrows = lx_cpu.shape[0]
    CR.logprob_entropy_rows(lx_cpu, lt_cpu)
    reps, t0 = 0, time.perf_counter()
    while reps < 3 or time.perf_counter() - t0 < min_seconds:
        CR.logprob_entropy_rows(lx_cpu, lt_cpu)
        reps += 1
    l_tok = lrows * reps / (time.perf_counter() - t0)
    return {
        "value": round(s_rows, 2),
        "unit": "rows/s",
        "cores": threads,
        "kind": "port",
        "sample": f"sampler: {rows} rows of the bf16 [256, 248320] batch (same penalty, mask, "
                  f"T, top-k, top-p), full V, >= {min_seconds:.0f} s; logprob: {lrows} rows of "
                  f"bf16 [8192, 248320] -> {l_tok:.1f} tokens/s",
        "logprob_tokens_per_s": round(l_tok, 2),
        "cpu_model": cpu_model(),
        "configs": cpu_baseline_configs(),
    }


def profiled_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` (a name, optionally with its
    workload shape) as measured by rocprofv3 FETCH_SIZE and WRITE_SIZE
    counters (scaled by the copy-kernel calibration), read from the committed
    profile summary's ``traffic_bytes <key> <bytes>`` lines, whose key is the
    name with spaces removed.  None when no such line exists."""
    key = kernel.replace(" ", "")
    try:
        with open(TRAFFIC_FILE) as f:
            for ln in f:
                parts = ln.strip().strip("`").split()
                if len(parts) == 3 and parts[0] == "traffic_bytes" and parts[1] == key:
                    return int(parts[2])
    except OSError:
        pass
    return None


def calibrate_copy(iters: int = 5) -> None:
    """1 GiB device-to-device copies: FETCH_SIZE and WRITE_SIZE of this kernel
    should each read 1 GiB = 1048576 KiB per dispatch."""
    import torch

    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": n, "iters": iters}), flush=True)


def kernel_events(n: int):
    """n pairs of timing events for ops.time_next_launch, each recorded once
    so that it exists; the hook then re-records them at a kernel's own
    dispatch start and end."""
    import torch

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n)]
    for e0, e1 in evs:
        e0.record()
        e1.record()
    return evs


def evict(flush) -> None:
    """Evicts the 256 MB last-level cache (MALL) with a read-only pass over a
    512 MB buffer, then waits for the GPU to drain: the next kernel starts
    cold, alone on the GPU, with no dirty lines to write back (an in-place
    write pass instead leaves 512 MB dirty, and the next kernel pays for
    their write-back: the configuration-5 sampler measured 41 against
    37.6 us)."""
    import torch

    flush.amax()
    torch.cuda.synchronize()


def stream_floor_us(x, flush, iters: int = 10) -> float:
    """Average kernel time of gtp_stream_read_rows over the rows of ``x``
    (a read-only pass with the samplers' access pattern), MALL evicted
    before each launch: the streaming floor."""
    import ctypes

    import torch

    import graspo_amd
    from graspo_amd import ops

    lib = ctypes.CDLL(graspo_amd.LIB_PATH)
    fn = lib.gtp_stream_read_rows
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                   ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    rows, cols = x.shape
    out = torch.zeros(rows, dtype=torch.int32, device=x.device)
    args = (x.data_ptr(), rows, cols * x.element_size(), x.stride(0) * x.element_size(),
            out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    for _ in range(2):
        assert fn(*args) == 0
    evs = kernel_events(iters)
    for e0, e1 in evs:
        evict(flush)
        ops.time_next_launch(e0, e1)
        assert fn(*args) == 0
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in evs) / iters * 1e3


def time_sampler_config(cfg: int, dev, iters: int, flush, kernel: str = SAMPLER_KERNEL,
                        override: dict | None = None, drop: tuple = (), what: str | None = None,
                        transform=None):
    """Average kernel time of one sampler launch on workload ``cfg`` (its
    parameters changed by ``override``, inputs in ``drop`` removed, its
    logits replaced by ``transform(logits)`` when given) with the MALL
    evicted before every launch."""
    import torch

    from graspo_amd import ops
    from graspo_amd import workloads as W

    wl = W.sampler_workload(cfg, device=dev)
    if transform is not None:
        wl.logits = transform(wl.logits)
    kw = wl.kwargs()
    for k in drop:
        kw.pop(k, None)
    kw.update(override or {})
    for _ in range(2):
        ops.sample(wl.logits, **kw)
    evs = kernel_events(iters)
    for e0, e1 in evs:
        evict(flush)
        ops.time_next_launch(e0, e1)
        ops.sample(wl.logits, **kw)
    torch.cuda.synchronize()
    us = sum(a.elapsed_time(b) for a, b in evs) / iters * 1e3
    B, V = wl.logits.shape
    nbytes = wl.logits.numel() * wl.logits.element_size() + B * 16
    if kw.get("allow_mask") is not None:
        nbytes += B * ((V + 31) // 32) * 4
    if kw.get("history") is not None:
        nbytes += kw["history"].numel() * 4
    floor = stream_floor_us(wl.logits, flush)
    out = {
        "shape": [B, V], "dtype": str(wl.logits.dtype).replace("torch.", ""), "kernel": kernel,
        "avg_us": round(us, 2), "rows_per_s": round(B / (us * 1e-6), 1),
        "algorithmic_bytes": nbytes, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
        "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "stream_floor_us": round(floor, 2),
        "traffic": profiled_traffic(kernel + f" [{B}, {V}]"),
    }
    if what:
        out["what"] = what
    return out


def time_logprob_config4(dev, chunk: int = 8192):
    """The loss-side workload: bf16 [32768, 151936] logits with int32
    targets, for the policy and the reference pass (different seeds), each
    processed as 4 chunks of 8192 rows; every chunk launch timed through the
    launch hook."""
    import torch

    from graspo_amd import ops
    from graspo_amd import workloads as W

    passes = [W.logprob_workload(4, device=dev, pass_index=p) for p in (0, 1)]
    N, V = passes[0][0].shape
    ops.logprob_entropy(passes[0][0][:chunk], passes[0][1][:chunk])
    evs = kernel_events(2 * (N // chunk))
    torch.cuda.synchronize()
    i = 0
    for x, t in passes:
        for s0 in range(0, N, chunk):
            ops.time_next_launch(*evs[i])
            ops.logprob_entropy(x[s0:s0 + chunk], t[s0:s0 + chunk])
            i += 1
    torch.cuda.synchronize()
    us = [a.elapsed_time(b) * 1e3 for a, b in evs]
    avg = sum(us) / len(us)
    nbytes = W.logprob_algorithmic_bytes(chunk, V, 2)
    del passes
    return {
        "shape": [N, V], "passes": 2, "chunk_rows": chunk, "chunks": len(us),
        "kernel": LOGPROB_KERNEL, "avg_us_per_chunk": round(avg, 2),
        "total_ms_both_passes": round(sum(us) / 1e3, 3),
        "tokens_per_s": round(2 * N / (sum(us) * 1e-6), 1),
        "algorithmic_bytes_per_chunk": nbytes,
        "gbs": round(nbytes / (avg * 1e-6) / 1e9, 1),
        "frac": round(nbytes / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "traffic": profiled_traffic(LOGPROB_KERNEL + f" [{chunk}, {V}]"),
    }


def time_graspo_loss(dev, B: int = 16, T: int = 2048, iters: int = 50):
    """Forward + backward of the GRASPO PPO-clip loss over [B, T] token
    logprobs: the fused kernels against the reference's torch expression
    (graspo_loss.py:10-16, 45-63) on the same device."""
    import torch

    from graspo_amd.graspo_loss import GRASPOLoss

    g = torch.Generator(device=dev).manual_seed(0)
    lp = -torch.rand(B, T, device=dev, generator=g) * 3
    old = lp + 0.3 * torch.randn(B, T, device=dev, generator=g)
    adv = torch.randn(B, 1, device=dev, generator=g).expand(B, T).contiguous()
    mask = torch.rand(B, T, device=dev, generator=g) < 0.7

    def ref(x):
        ratio = (x - old).exp()
        loss = -torch.min(ratio * adv, ratio.clamp(0.8, 1.2) * adv)
        return ((loss * mask).sum(dim=-1) / mask.sum(dim=-1).clamp_min(1)).mean()

    fused = GRASPOLoss(0.2)
    out = {}
    for name, fn in (("fused_us", lambda x: fused(x, old, adv, mask)), ("torch_us", ref)):
        for _ in range(3):
            x = lp.clone().requires_grad_(True)
            fn(x).backward()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        xs = [lp.clone().requires_grad_(True) for _ in range(iters)]
        torch.cuda.synchronize()
        e0.record()
        for x in xs:
            fn(x).backward()
        e1.record()
        torch.cuda.synchronize()
        out[name] = round(e0.elapsed_time(e1) / iters * 1e3, 2)
    out["shape"] = [B, T]
    out["what"] = "forward + backward per call, HIP events around 50 back-to-back calls"
    return out


def time_hidden_logprobs(dev, N: int = 8192, H: int = 4096, V: int = 248320):
    """The hidden-state logprob path at N tokens x H x V (tensor_utils.py:
    167-186 with the callers' fp32 copies of bf16 hidden states and lm_head,
    qwen3/model.py:361-365): the drop-in (exact bf16 narrowing, then the
    fused bf16 GEMM + log-sum-exp kernel) against the reference's expression
    in fp32 on the same device, the fused kernel's call on bf16 operands,
    and hipBLASLt's bf16 GEMM alone over the reference's chunks (fp32
    output); TFLOP/s are reported against the 2.5 PFLOP/s dense bf16 peak."""
    import torch
    import torch.nn.functional as F

    from graspo_amd import ops
    from graspo_amd import tensor_utils as TU

    g = torch.Generator(device=dev).manual_seed(11)
    h = torch.randn(N, H, device=dev, generator=g).to(torch.bfloat16).float()
    w = (torch.randn(V, H, device=dev, generator=g) * 0.02).to(torch.bfloat16).float()
    ids = torch.randint(0, V, (N,), device=dev, generator=g)
    chunk = 32768

    def reference():
        sel = (h * w.index_select(0, ids)).sum(dim=-1)
        lse = None
        for start in range(0, V, chunk):
            c = torch.logsumexp(F.linear(h, w[start:start + chunk]), dim=-1)
            lse = c if lse is None else torch.logaddexp(lse, c)
        return sel - lse

    def dropin():
        return TU._selected_token_log_probs_from_hidden(h, w, ids)

    hb, wb = h.to(torch.bfloat16), w.to(torch.bfloat16)

    def gemm_only():
        for start in range(0, V, chunk):
            torch.mm(hb, wb[start:start + chunk].t(), out_dtype=torch.float32)

    def fused():
        return ops.lm_head_logprob(hb, wb, ids)

    def clock(fn, reps):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            out = fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps, out

    ours_ms, lp = clock(dropin, 5)
    gemm_ms, _ = clock(gemm_only, 5)
    fused_ms, _ = clock(fused, 5)
    # the GEMM-with-lse kernel alone, HIP events from the dispatch itself
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    e1.record()
    kern = []
    for _ in range(5):
        ops.time_next_launch(e0, e1)
        fused()
        torch.cuda.synchronize()
        kern.append(e0.elapsed_time(e1))
    kern_ms = sorted(kern)[len(kern) // 2]
    ref_ms, lp_ref = clock(reference, 2)
    # forward + backward (gradients of hidden and lm_head), as training uses it
    gout = torch.randn(N, device=dev, generator=g)

    def train(fn):
        def step():
            h.grad = None
            w.grad = None
            (fn() * gout).sum().backward()
        return step

    h.requires_grad_(True)
    w.requires_grad_(True)
    ours_fb_ms, _ = clock(train(dropin), 2)
    gh_ours, gw_ours = h.grad.clone(), w.grad.clone()
    ref_fb_ms, _ = clock(train(reference), 1)
    grad_diff = max(float((gh_ours - h.grad).abs().max()), float((gw_ours - w.grad).abs().max()))
    h.requires_grad_(False)
    w.requires_grad_(False)
    del gh_ours, gw_ours
    h.grad = None
    w.grad = None
    flops = 2.0 * N * H * V
    return {
        "shape": {"tokens": N, "hidden": H, "vocab": V, "chunk": chunk},
        "dropin_ms": round(ours_ms, 3), "reference_fp32_ms": round(ref_ms, 3),
        "gemm_bf16_ms": round(gemm_ms, 3),
        "gemm_tflops": round(flops / (gemm_ms * 1e-3) / 1e12, 1),
        "gemm_frac_bf16_peak": round(flops / (gemm_ms * 1e-3) / 2.5e15, 4),
        "fused_ms": round(fused_ms, 3), "fused_kernel_ms": round(kern_ms, 3),
        "fused_tflops": round(flops / (fused_ms * 1e-3) / 1e12, 1),
        "fused_frac_bf16_peak": round(flops / (fused_ms * 1e-3) / 2.5e15, 4),
        "dropin_tflops": round(flops / (ours_ms * 1e-3) / 1e12, 1),
        "max_abs_diff_vs_reference": round(float((lp - lp_ref).abs().max()), 7),
        "dropin_fwd_bwd_ms": round(ours_fb_ms, 3), "reference_fwd_bwd_ms": round(ref_fb_ms, 3),
        "max_abs_grad_diff_vs_reference": round(grad_diff, 9),
        "what": "fp32 inputs holding bf16 values, as the callers pass them (the drop-in "
                "narrows them, then runs the fused GEMM+lse kernel); fused = the kernel's "
                "call on bf16 operands (GEMM+lse, target dots, merge), fused_kernel = the "
                "GEMM+lse kernel alone; gemm_bf16 = hipBLASLt over the same chunks with fp32 "
                "output; HIP events, 5 (drop-in, GEMM, fused) and 2 (reference) forward calls, "
                "2 and 1 forward+backward calls, each after one warm-up",
    }


def time_decode_loop(dev, B: int = 256, V: int = 248320, steps: int = 24):
    """Per-token cost of the generation loop's own work at [B, V] bf16 logits:
    the decode-loop drop-in (graspo_amd.decode_loop) against the reference's
    loop body (models/qwen3/adapter.py:283-311: logits.float(), sampler,
    pad, cat, EOS update, bool(finished.all())) on the same sampler.  The
    model is a stand-in that returns resident logits, so only the loop is
    timed; no row reaches EOS, so both loops run every step."""
    import torch

    from graspo_amd import decode_loop as dl
    from graspo_amd import tensor_utils as tu

    g = torch.Generator(device=dev).manual_seed(5)
    logits = (torch.randn(B, 1, V, device=dev, generator=g) * 3.0).to(torch.bfloat16)
    seq0 = torch.randint(0, V, (B, 64), device=dev, generator=g)
    eos, pad = V + 7, 0  # never sampled

    class _Model:
        def __call__(self, ids, attention_mask=None, past_key_values=None, use_cache=False):
            return (logits, 0) if use_cache else logits

    class _Adapter:
        model = _Model()

        def _sync_timing(self):
            pass

    def reference_loop(n):
        sequences = seq0.clone()
        finished = torch.zeros(B, dtype=torch.bool, device=dev)
        out, pkv = _Adapter.model(sequences, attention_mask=sequences.ne(pad), use_cache=True)
        for _ in range(n):
            nt = tu._next_token_from_logits(out.float()[:, -1, :], temperature=0.7, top_p=0.9)
            nt = tu._broadcast_and_pad_finished(nt, finished, pad)
            sequences = torch.cat([sequences, nt.unsqueeze(1)], dim=1)
            finished |= nt.eq(eos)
            if bool(finished.all()):
                break
            out, pkv = _Adapter.model(nt.unsqueeze(1), attention_mask=sequences.ne(pad),
                                      past_key_values=pkv, use_cache=True)
        return sequences

    def fused_loop(n):
        finished = torch.zeros(B, dtype=torch.bool, device=dev)
        return dl.generate_group_with_kv_cache(
            _Adapter(), sequences=seq0, finished=finished, eos_token_id=eos, pad_token_id=pad,
            max_new_tokens=n, temperature=0.7, top_p=0.9)[0]

    res = {}
    for name, fn in (("fused_us_per_step", fused_loop), ("reference_loop_us_per_step",
                                                         reference_loop)):
        fn(3)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        s = fn(steps)
        torch.cuda.synchronize()
        res[name] = round((time.perf_counter() - t0) / steps * 1e6, 1)
        assert s.shape == (B, 64 + steps)
    res["shape"] = [B, V]
    res["what"] = (f"wall time per token over a {steps}-token loop, KV-cache form, T 0.7, "
                   "top-p 0.9, bf16 logits resident (the reference body samples their fp32 "
                   "copy)")
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-per-config", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "rows are independent, so N GPUs would each run B/N rows of the same kernels",
              file=sys.stderr)
        return 2

    import torch

    if args.calibrate_copy:
        calibrate_copy()
        return 0

    import graspo_amd
    from graspo_amd import ops
    from graspo_amd import workloads as W

    graspo_amd.load()
    dev = torch.device("cuda:0")
    wl = W.sampler_workload(5, device=dev)
    wl_b = W.SamplerWorkload(**{**wl.__dict__, "logits": wl.logits.clone()})
    batches = [wl, wl_b]
    lx, lt = W.logprob_workload(5, device=dev)
    B, V = wl.logits.shape
    N = lx.shape[0]
    torch.cuda.synchronize()

    def step(i, evs=None):
        # evs: events around the two launches (0-2) and, through the launch
        # hook, at each kernel's own start and end (3-4 sampler, 5-6 logprob).
        # Timed steps wait for the GPU to drain before each launch, so that a
        # kernel never shares the GPU with the last workgroups of the one
        # before it (the sampler right behind the logprob pass measured 43.2
        # us that way, 37.6 us alone); the logprob pass of the previous step
        # has evicted the sampler's rows from the MALL with reads only.
        w = batches[i % 2]
        if evs:
            torch.cuda.synchronize()
            evs[0].record()
            ops.time_next_launch(evs[3], evs[4])
        ops.sample(w.logits, **w.kwargs())
        if evs:
            evs[1].record()
            torch.cuda.synchronize()
            evs[7].record()
            ops.time_next_launch(evs[5], evs[6])
        ops.logprob_entropy(lx, lt)
        if evs:
            evs[2].record()

    # The side measurements run first: about a second of GPU work, after
    # which the GPU runs at its steady-state clocks (a cold GPU ran the
    # sampler's first timed steps at 56 us, settling to ~37 us over 20 steps).
    side = {}
    # the gradient of the logprob pass (one read of the logits, one write of
    # the bf16 gradient), the kernel behind the autograd backward
    g_lp = torch.randn(N, device=dev)
    lp_f, _, _ = ops.logprob_entropy(lx, lt)
    lse = lx.gather(1, lt.long().unsqueeze(1)).squeeze(1).float() - lp_f
    grad = torch.empty_like(lx)
    for _ in range(2):
        ops.logprob_backward(lx, lt, g_lp, lse, out=grad)
    bevs = kernel_events(10)
    for e0, e1 in bevs:
        ops.time_next_launch(e0, e1)
        ops.logprob_backward(lx, lt, g_lp, lse, out=grad)
    torch.cuda.synchronize()
    b_ms = sum(a.elapsed_time(b) for a, b in bevs) / len(bevs)
    b_bytes = 2 * N * V * lx.element_size() + N * (lt.element_size() + 4 + 4)
    b_gbs = b_bytes / (b_ms * 1e-3) / 1e9
    side["logprob_backward"] = {
        "bound": "hbm", "achieved": round(b_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(b_gbs / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(BACKWARD_KERNEL),
        "kernel": BACKWARD_KERNEL, "algorithmic_bytes": b_bytes, "avg_us": round(b_ms * 1e3, 2)}
    del grad, g_lp, lse, lp_f
    side["graspo_loss"] = time_graspo_loss(dev)
    side["decode_loop"] = time_decode_loop(dev)
    side["hidden_logprobs"] = time_hidden_logprobs(dev)
    # the step itself, untimed, for PREWARM_S before the W warm-up steps: a
    # GPU coming from other work or from idle ran the sampler's first steps
    # at 48-58 us, settling at ~37 us only after some tens of steps of this
    # same loop
    prewarm_steps, t_pw = 0, time.perf_counter()
    while time.perf_counter() - t_pw < PREWARM_S:
        step(prewarm_steps)
        prewarm_steps += 1
        if prewarm_steps % 32 == 0:
            torch.cuda.synchronize()
    for i in range(args.warmup):
        step(i)
    # per step: events around the sampler launch (0, 1) and after the logprob
    # launch (2), the hook's pairs (3-4, 5-6), and before the logprob launch (7)
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)]
              + [e for pair in kernel_events(2) for e in pair]
              + [torch.cuda.Event(enable_timing=True)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i, events[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # kernel time: the events the launch hook records at each kernel's own
    # dispatch; events recorded around a launch on the drained GPU also count
    # the host's launch latency
    s_ms = sum(e[3].elapsed_time(e[4]) for e in events) / args.steps
    l_ms = sum(e[5].elapsed_time(e[6]) for e in events) / args.steps
    s_ev_us = sum(e[0].elapsed_time(e[1]) for e in events) / args.steps * 1e3
    l_ev_us = sum(e[7].elapsed_time(e[2]) for e in events) / args.steps * 1e3

    s_bytes = wl.algorithmic_bytes()
    l_bytes = W.logprob_algorithmic_bytes(N, V, lx.element_size())
    s_gbs = s_bytes / (s_ms * 1e-3) / 1e9
    l_gbs = l_bytes / (l_ms * 1e-3) / 1e9
    roof_s = {"bound": "hbm", "achieved": round(s_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
              "frac": round(s_gbs / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(SAMPLER_KERNEL),
              "kernel": SAMPLER_KERNEL, "algorithmic_bytes": s_bytes,
              "avg_us": round(s_ms * 1e3, 2), "avg_us_events_around_launch": round(s_ev_us, 2)}
    roof_l = {"bound": "hbm", "achieved": round(l_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
              "frac": round(l_gbs / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(LOGPROB_KERNEL),
              "kernel": LOGPROB_KERNEL, "algorithmic_bytes": l_bytes,
              "avg_us": round(l_ms * 1e3, 2), "avg_us_events_around_launch": round(l_ev_us, 2)}
    dominant = roof_l if l_ms >= s_ms else roof_s
    line = {
        "metric": "sampled rows/sec and logprob tokens/sec; achieved HBM GB/s vs MI355X peak",
        "value": round(B / (s_ms * 1e-3), 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "large-vocab sampler bf16 [256,248320] (hist 4096, rho 1.05, mask 8%, "
                        "T 0.7, top-k 64, top-p 0.9) + logprob/entropy bf16 [8192,248320]",
            "sampler_batch": B, "vocab": V, "logprob_rows": N, "input_dtype": "bf16",
            "parallelism": "single-gpu",
        },
        "prewarm": {"seconds": PREWARM_S, "steps": prewarm_steps,
                    "what": "the step run untimed before the warm-up steps, so that the "
                            "timed steps run at the GPU's steady state"},
        "logprob_tokens_per_s": round(N / (l_ms * 1e-3), 1),
        "roofline": dominant,
        "rooflines": {"sampler": roof_s, "logprob": roof_l},
        "per_config": None,
        "cpu_baseline": None,
    }
    line["rooflines"]["logprob_backward"] = side["logprob_backward"]
    for k in ("graspo_loss", "decode_loop", "hidden_logprobs"):
        line[k] = side[k]
    del lx, lt, batches, wl_b
    flush = torch.zeros(128 << 20, dtype=torch.float32, device=dev)  # 512 MB
    roof_s["stream_floor_us"] = round(stream_floor_us(wl.logits, flush), 2)
    if not args.no_per_config:
        topp = "sampler_topp_kernel<bf16>"
        pc = {
            f"sampler_{name}": time_sampler_config(cfg, dev, 20, flush, kernel)
            for cfg, name, kernel in ((1, "fp32_8x151936", "sampler_split_kernel<fp32>"),
                                      (2, "bf16_64x151936_top_p", "sampler_topps_kernel<bf16> penalty"),
                                      (3, "bf16_64x151936_masked", topp + " mask"))
        }
        pc["sampler_bf16_256x248320_decode_top_p"] = time_sampler_config(
            5, dev, 20, flush, topp, override={"temperature": 0.7, "top_p": 0.9, "top_k": 0},
            drop=("history", "allow_mask"),
            what="the decode loop's rows: the [256,248320] logits, T 0.7, top-p 0.9, "
                 "no top-k, history or mask")
        pc["sampler_bf16_256x248320_masked_history_top_p"] = time_sampler_config(
            5, dev, 20, flush, topp + " mask penalty", override={"top_k": 0},
            what="configuration 5's inputs with top-k off (mask, history, penalty, "
                 "T 0.7, top-p 0.9)")
        def fp32_inexact(x):
            g = torch.Generator(device=x.device).manual_seed(5)
            return x.float() + torch.rand(x.shape, generator=g, device=x.device) * 1e-3

        pc["sampler_fp32_256x248320_decode_top_p"] = time_sampler_config(
            5, dev, 10, flush, "sampler_topp32_kernel<fp32>",
            override={"temperature": 0.7, "top_p": 0.9, "top_k": 0},
            drop=("history", "allow_mask"), transform=fp32_inexact,
            what="fp32 rows that are not bf16 values (configuration 5's logits + U(0, 1e-3)), "
                 "T 0.7, top-p 0.9: the fp32 top-p kernel (two reads of the rows)")
        pc["logprob_bf16_32768x151936"] = time_logprob_config4(dev)
        line["per_config"] = pc
    del flush
    if not args.no_cpu_baseline:
        cw = W.sampler_workload(5, device="cpu", rows=32)
        clx, clt = W.logprob_workload(5, device="cpu", rows=64)
        line["cpu_baseline"] = cpu_baseline(cw, clx, clt)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
