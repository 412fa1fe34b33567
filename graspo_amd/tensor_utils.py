"""Drop-ins for the hot-path helpers of
``src/graspo/backends/graspoflow/tensor_utils.py``.

Same names, same keyword-only signatures and the same return types as the
reference; the extra keywords default to "off", so existing call sites need
no edit.  All arithmetic runs in the gfx950 kernels of
``libgraspo_tokpath.so``; torch is used for allocation, the vocabulary-chunk
GEMMs of the hidden-state path, and the backward passes.
"""

from __future__ import annotations

import torch
import torch.distributed as dist
from torch.nn import functional as F  # noqa: N812

from . import ops


def _fp32_top_p_kernel_takes(logits: torch.Tensor, temperature: float, top_k: int,
                             top_p: float) -> bool:
    """Whether an fp32 call without history or mask goes to the fp32 top-p
    kernel, as the library's own routing decides (gtp_sample_route)."""
    route, _ = ops.sample_route(logits, temperature=temperature, top_k=top_k, top_p=top_p)
    return route == ops.ROUTE_TOPP32


def _bf16_when_exact(logits: torch.Tensor, temperature: float, top_k: int,
                     top_p: float = 1.0) -> torch.Tensor:
    """fp32 rows as their bf16 copy when every value is a bf16 value -- the
    reference's callers pass ``logits.float()`` of a bf16 model -- and the
    call would otherwise take the row-wise kernel (sampling without a top-k
    of at most 128, other than the top-p rows the fp32 top-p kernel reads
    directly, which is faster than the narrowing and its host
    synchronisation): the value-histogram kernel takes bf16 rows only, and
    the samples are the same because the float inputs are.  Costs one pass
    over the rows and one host synchronisation."""
    if (logits.dtype != torch.float32 or logits.dim() != 2 or not logits.is_cuda
            or not temperature > 0 or 1 <= top_k <= 128
            or _fp32_top_p_kernel_takes(logits, temperature, top_k, top_p)):
        return logits
    bf, inexact = ops.to_bf16_exact(logits)
    return bf if int(inexact) == 0 else logits


def _next_token_from_logits(
    logits: torch.Tensor,
    *,
    temperature: float,
    top_p: float,
    top_k: int = 0,
    repetition_penalty: float = 1.0,
    history: torch.Tensor | None = None,
    allow_mask: torch.Tensor | None = None,
    uniforms: torch.Tensor | None = None,
    generator: torch.Generator | None = None,
    check_status: bool = True,
) -> torch.Tensor:
    """Next token per row (reference: tensor_utils.py:649-658).

    ``temperature <= 0`` is greedy (argmax, lowest id on ties); otherwise the
    row is divided by ``max(temperature, 1e-6)`` and sampled under top-k /
    top-p from ``uniforms`` (drawn from torch's generator when omitted, as the
    reference's ``torch.multinomial`` does).  Returns int64 [B].  fp32 rows
    holding bf16 values take the bf16 kernels when the status is checked
    (that check synchronises anyway)."""
    if check_status:
        logits = _bf16_when_exact(logits, float(temperature), int(top_k), float(top_p))
    out = ops.sample(
        logits,
        temperature=float(temperature),
        top_k=top_k,
        top_p=float(top_p),
        repetition_penalty=repetition_penalty,
        history=history,
        allow_mask=allow_mask,
        uniforms=uniforms,
        generator=generator,
    )
    if check_status:
        ops.raise_on_bad_status(out.status, "_next_token_from_logits")
    return out.ids


def _sample_next_token(
    logits: torch.Tensor,
    *,
    top_p: float,
    top_k: int = 0,
    uniforms: torch.Tensor | None = None,
    generator: torch.Generator | None = None,
    check_status: bool = True,
) -> torch.Tensor:
    """Sample from already temperature-scaled logits (reference:
    tensor_utils.py:671-683): softmax, top-p cut with the first token always
    kept, renormalise, draw.  Division by 1.0 is exact, so this is the
    sampler at temperature 1."""
    return _next_token_from_logits(
        logits, temperature=1.0, top_p=top_p, top_k=top_k, uniforms=uniforms,
        generator=generator, check_status=check_status,
    )


def _broadcast_and_pad_finished(
    next_token: torch.Tensor,
    finished: torch.Tensor,
    pad_token_id: int,
) -> torch.Tensor:
    """Rank 0's ids to every rank, then ``pad_token_id`` for finished rows
    (reference: tensor_utils.py:661-668).  On one GPU there is no broadcast;
    the sampler can also fold the padding itself (``finished=`` of
    :func:`graspo_amd.ops.sample`)."""
    if dist.is_available() and dist.is_initialized():
        dist.broadcast(next_token, src=0)
    return next_token.masked_fill(finished, pad_token_id)


# ------------------------------------------------------------- logprobs

def _matrix_core_operands(h2: torch.Tensor, weight: torch.Tensor,
                          targets: torch.Tensor | None = None):
    """bf16 operands for the chunk GEMMs, or None to multiply in the inputs'
    own dtype.

    bf16 / fp16 inputs are used as they are.  fp32 inputs -- the reference's
    callers pass ``hidden.float()`` and ``lm_head.weight.float()``, fp32
    copies of bf16 tensors -- are narrowed to bf16 in one pass that also
    reports whether every value is a bf16 value.  When it is, a bf16 x bf16
    product is exact in fp32, so a matrix-core GEMM with fp32 output computes
    the same products as the reference's fp32 GEMM (only the summation order
    differs); otherwise the fp32 GEMM is kept.

    With ``targets`` an id outside [0, V) raises, as the reference's
    ``index_select`` does; that flag and the exactness flag are read in one
    host synchronisation."""
    V = weight.shape[0]
    bad = None
    if targets is not None and targets.numel():
        bad = ((targets < 0) | (targets >= V)).any().to(torch.int32).view(1).to(h2.device)
    mc, inexact = None, None
    if h2.dtype in (torch.bfloat16, torch.float16) and weight.dtype == h2.dtype:
        mc = (h2, weight)
    elif h2.dtype == torch.float32 and weight.dtype == torch.float32 and h2.is_cuda:
        hb, fh = ops.to_bf16_exact(h2)
        wb, fw = ops.to_bf16_exact(weight)
        mc, inexact = (hb, wb), fh | fw
    flags = [f for f in (inexact, bad) if f is not None]
    if flags:
        vals = torch.cat(flags).tolist()
        if bad is not None and vals[-1]:
            raise RuntimeError(
                "_selected_token_log_probs_from_hidden: an output id is outside [0, vocab_size)")
        if inexact is not None and vals[0]:
            mc = None
    return mc


def _chunk_logits(h2, weight, mc, start, chunk):
    """fp32 logits of vocabulary columns [start, start + chunk)."""
    if mc is not None:
        hb, wb = mc
        return torch.mm(hb, wb[start : start + chunk].t(), out_dtype=torch.float32)
    return F.linear(h2, weight[start : start + chunk]).float()


class _SelectedLogProbsFromHidden(torch.autograd.Function):
    """log_softmax(h W^T)[target] without materialising [N, V] logits for a
    forward-only call.  When the operands are bf16 values (K a multiple of
    128) the forward is one fused kernel: the bf16 GEMM on the matrix cores
    with the log-sum-exp in its epilogue; when a gradient is wanted the same
    kernel also keeps the fp32 logits, as the reference's autograd keeps
    every chunk's logits for ``logsumexp``'s backward, and the backward is
    one pass over them (bf16 of -g * softmax) and two bf16 GEMMs with fp32
    output, the one-hot term g * [i == t] added in fp32.  Other operands
    fold vocabulary chunks of the GEMM into a running (m, s) state with the
    lse kernel and recompute each chunk's softmax in the backward."""

    @staticmethod
    def forward(ctx, hidden, weight, output_ids, chunk):
        H = hidden.shape[-1]
        h2 = hidden.reshape(-1, H)
        t = output_ids.reshape(-1)
        N, V = h2.shape[0], weight.shape[0]
        # raises for an id outside [0, V), as the reference's index_select does
        mc = _matrix_core_operands(h2, weight, t)
        logits = None
        if N and mc is not None and ops.lm_head_supported(*mc):
            if ctx.needs_input_grad[0] or ctx.needs_input_grad[1]:
                lp, lse, logits, _ = ops.lm_head_logprob_save(mc[0], mc[1], t)
            else:
                # one kernel: the bf16 GEMM with the log-sum-exp in its
                # epilogue, no [N, V] logits (the vocabulary chunking is the
                # kernel's tiling)
                lp, _, lse = ops.lm_head_logprob(mc[0], mc[1], t)
        else:
            state = ops.new_lse_state(N, hidden.device)
            # (running each chunk's lse on a second stream beside the next
            # GEMM was slower: 21.4 against 16.5 ms at 8192 x 4096 x 248320)
            for c, start in enumerate(range(0, V, chunk)):
                chunk_logits = _chunk_logits(h2, weight, mc, start, chunk)
                ops.lse_partial(chunk_logits, t, start, state, accumulate=c > 0)
            lp, _ = ops.lse_finalize(state)
            lse = state[:, 0] + torch.log(state[:, 1])
        saved = (h2, weight, t, lse) + (mc if mc is not None else ())
        if logits is not None:
            saved = saved + (logits,)
        ctx.save_for_backward(*saved)
        ctx.has_mc = mc is not None
        ctx.has_logits = logits is not None
        ctx.chunk = chunk
        ctx.out_shape = output_ids.shape
        return lp.view(output_ids.shape)

    @staticmethod
    def backward(ctx, grad_out):
        saved = ctx.saved_tensors
        h2, weight, t, lse = saved[:4]
        mc = saved[4:6] if ctx.has_mc else None
        g = grad_out.reshape(-1).to(torch.float32)
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if ctx.has_logits:
            # d lp_n / d x_ni = [i == t_n] - p_ni: the softmax part in bf16
            # (each element within 2^-8 of -g p) through the matrix cores,
            # the one-hot part in fp32.  grad_W takes it vocabulary-major
            # (gs_t [V, N]) and grad_h token-major (gs [N, V]), the layout on
            # which each GEMM runs fastest (12.4 against 14.4 ms for grad_h
            # at 8192 x 4096 x 248320), both written by one pass
            hb, wb = mc
            gs_t, gs = ops.softmax_grad_bf16(saved[6], g, lse, vocab_major=need_w,
                                             token_major=need_h)
            tl = t.long()
            gt = g.unsqueeze(1)
            grad_h = grad_w = None
            if need_h:
                grad_h = torch.mm(gs, wb, out_dtype=torch.float32)
                del gs
                grad_h += gt * wb.index_select(0, tl).float()
                grad_h = grad_h.to(h2.dtype).view(*ctx.out_shape, h2.shape[-1])
            if need_w:
                grad_w = torch.mm(gs_t, hb, out_dtype=torch.float32)
                grad_w.index_add_(0, tl, gt * hb.float())
                grad_w = grad_w.to(weight.dtype)
            return grad_h, grad_w, None, None
        # the bf16 route accumulates grad_h over the chunks in fp32
        acc_dtype = torch.float32 if mc is not None else h2.dtype
        grad_h = torch.zeros(h2.shape, dtype=acc_dtype, device=h2.device) if need_h else None
        grad_w = torch.empty_like(weight) if need_w else None
        for start in range(0, weight.shape[0], ctx.chunk):
            w_c = weight[start : start + ctx.chunk]
            # g * (onehot - softmax) of this chunk's logits, one kernel pass
            logits = _chunk_logits(h2, weight, mc, start, ctx.chunk)
            if mc is not None:
                # bf16 matrix cores with fp32 output: the gradient kernel
                # writes gc = hi + lo in bf16 (|gc - hi - lo| <= 2^-16 |gc|),
                # multiplied against the exact bf16 operands: the products
                # carry about 16 significant bits
                hb, wb = mc
                hi, lo = ops.logprob_backward_split(logits, t, g, lse, col_offset=start)
                del logits
                w_b = wb[start : start + ctx.chunk]
                if need_h:
                    grad_h += torch.mm(hi, w_b, out_dtype=torch.float32)
                    grad_h += torch.mm(lo, w_b, out_dtype=torch.float32)
                if need_w:
                    gw = (torch.mm(hi.t(), hb, out_dtype=torch.float32)
                          + torch.mm(lo.t(), hb, out_dtype=torch.float32))
                    grad_w[start : start + ctx.chunk] = gw.to(weight.dtype)
                continue
            gc = ops.logprob_backward(logits, t, g, lse, col_offset=start)
            if need_h:
                grad_h += gc.to(h2.dtype) @ w_c.to(h2.dtype)
            if need_w:
                grad_w[start : start + ctx.chunk] = (gc.t() @ h2.to(gc.dtype)).to(weight.dtype)
        if grad_h is not None:
            grad_h = grad_h.to(h2.dtype).view(*ctx.out_shape, h2.shape[-1])
        return grad_h, grad_w, None, None


def _selected_token_log_probs_from_hidden(
    hidden_states: torch.Tensor,
    lm_head_weight: torch.Tensor,
    output_ids: torch.Tensor,
    *,
    vocab_chunk_size: int = 32768,
) -> torch.Tensor:
    """logit[target] - logsumexp over the vocabulary, fp32 [*output_ids.shape]
    (reference: tensor_utils.py:167-186).  When the operands are bf16 values,
    as the reference's ``.float()`` copies of bf16 tensors are, the forward
    is one kernel: the bf16 GEMM on the matrix cores (fp32 accumulation) with
    the logsumexp in its epilogue, and the target logit as an fp32 dot
    product like the reference's ``selected_logits``.  Other operands keep
    the reference's ``vocab_chunk_size`` GEMMs with the lse kernel as the
    logsumexp / logaddexp fold.
    Differentiable in ``hidden_states`` and ``lm_head_weight``; on the bf16
    route the gradient GEMMs also run on matrix cores.  With the fused
    forward (K a multiple of 128) the softmax part of the logit gradient,
    -g * p, is rounded once to bf16 (each element within 2^-8 of it) and the
    one-hot part g * [i == t] is added in fp32, so a gradient element is
    within 2^-8 * sum_i |g p_i w_i| of the fp32 one; the chunked route
    splits the fp32 logit gradient into two bf16 parts (hi + lo, within
    2^-16 of it)."""
    return _SelectedLogProbsFromHidden.apply(
        hidden_states, lm_head_weight, output_ids, int(vocab_chunk_size)
    )
