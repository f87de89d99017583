"""LM head + GRPO step over token chunks, in the manner of Liger-Kernel's
fused linear cross-entropy.

The reference names "a Liger-style fused-LM-head extension" as its follow-up
(docs/FINAL_REPORT.md:439-450): the LM-head projection and the loss run
together so that the ``[B, S, V]`` logits are never materialised.  With the
GRPO loss at token level the gradient of the loss with respect to the logits
is known inside the forward (``klp_grpo_step`` writes it in the same pass
over the logits that computes the log-probabilities), so each chunk of tokens
goes through

    logits_c  = hidden_c @ weight^T                  (library GEMM, [c, V])
    klp_grpo_step(logits_c)                          (logp, entropy, loss, d_logits_c)
    d_hidden_c = d_logits_c @ weight                 (library GEMM)
    d_weight  += d_logits_c^T @ hidden_c             (library GEMM, float32 accumulator)

and is dropped before the next chunk: peak memory is two ``[c, V]`` buffers
instead of the full logits and their gradient, and the backward has nothing
left to recompute (it hands over d_hidden and d_weight, scaled by the loss's
upstream gradient when that is not 1).

Same loss, results and restrictions as :func:`kernel_opt.fused_grpo_step`
(token-level importance weights; ``logp`` / ``entropy`` returned as
constants).  Inputs ``fused_grpo_step`` cannot take in one pass (sequence-level
weights, rows above ``klp_grpo_step_max_vocab``, rows not 16-byte aligned) run
the unfused composition on the whole logits instead.
"""
from __future__ import annotations

import torch

from ._library import DTYPE_CODES, lib
from .grpo import fused_grpo_loss
from .grpo_step import _check_grad_scale, grpo_step_launch, grpo_token_weights, scale_by_upstream
from .ops import fused_logprob_entropy

__all__ = ["fused_linear_grpo_step"]

# Default chunking: each [chunk, V] buffer (a chunk's logits, then its
# d_logits) is held to about this many bytes, and the tokens are split into
# the fewest chunks that respect it, of equal size.  Fewer, larger chunks keep
# the library GEMMs efficient and skip the float32 d_weight accumulator
# entirely when one chunk suffices; 4 GiB per buffer is small beside 288 GB of
# HBM.
DEFAULT_CHUNK_BYTES = 4 << 30


def default_chunk_tokens(n_tokens: int, vocab: int, elem_bytes: int) -> int:
    """Tokens per chunk for the default: the fewest equal chunks whose
    [chunk, vocab] buffers stay within DEFAULT_CHUNK_BYTES."""
    max_tok = max(1, DEFAULT_CHUNK_BYTES // max(1, vocab * elem_bytes))
    n_chunks = max(1, -(-n_tokens // max_tok))
    return max(1, -(-n_tokens // n_chunks))


def _accumulate_f32(acc, a, b):
    """acc + a @ b in float32 (acc None: a @ b), for bf16 / fp16 / fp32
    operands: the GEMM accumulates in float32 and, where torch offers it
    (aten::mm.dtype / addmm.dtype), writes float32 directly into `acc`;
    otherwise the product is rounded to the operands' dtype first."""
    if a.dtype == torch.float32:
        return torch.mm(a, b) if acc is None else acc.addmm_(a, b)
    if _HAS_OUT_DTYPE:
        if acc is None:
            return torch.mm(a, b, out_dtype=torch.float32)
        return torch.addmm(acc, a, b, out_dtype=torch.float32, out=acc)
    part = torch.mm(a, b).float()
    return part if acc is None else acc.add_(part)


_HAS_OUT_DTYPE = hasattr(torch.ops.aten.mm, "dtype") and hasattr(torch.ops.aten.addmm, "dtype")


class _FusedLinearGrpoStep(torch.autograd.Function):

    @staticmethod
    def forward(ctx, hidden, weight, targets, old, ref, adv, wts, params, chunk):
        temperature, eps_low, eps_high, beta, grad_scale = params
        D = hidden.size(-1)
        V = weight.size(0)
        h2 = hidden.reshape(-1, D)
        N = h2.size(0)
        t = targets.reshape(-1)
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dev = hidden.device
        f32 = lambda: torch.empty(N, dtype=torch.float32, device=dev)  # noqa: E731
        logp, ent, loss_tok = f32(), f32(), f32()
        d_hidden = torch.empty_like(h2) if need_h else None
        d_weight = None
        single = chunk >= N
        step_params = (temperature, eps_low, eps_high, beta, 1, grad_scale)  # per-token adv.
        for n0 in range(0, N, chunk):
            n1 = min(N, n0 + chunk)
            c = n1 - n0
            hc = h2[n0:n1]
            logits = torch.mm(hc, weight.t())
            lp, en, _lse, lt, d = grpo_step_launch(
                logits.view(1, c, V), t[n0:n1].view(1, c), old[n0:n1], ref[n0:n1]
                if ref is not None else None, adv[n0:n1], wts[n0:n1], step_params)
            del logits
            logp[n0:n1] = lp.view(-1)
            ent[n0:n1] = en.view(-1)
            loss_tok[n0:n1] = lt.view(-1)
            d2 = d.view(c, V)
            if need_h:
                torch.mm(d2, weight, out=d_hidden[n0:n1])
            if need_w:
                if single:
                    d_weight = torch.mm(d2.t(), hc)
                else:
                    d_weight = _accumulate_f32(d_weight, d2.t(), hc)
            del d, d2
        if need_w and not single and d_weight.dtype != weight.dtype:
            d_weight = d_weight.to(weight.dtype)
        ctx.grads = (d_hidden, d_weight)
        ctx.grad_scale = grad_scale
        ctx.hidden_shape = hidden.shape
        logp, ent = logp.view(targets.shape), ent.view(targets.shape)
        ctx.mark_non_differentiable(logp, ent)
        return loss_tok.sum(), logp, ent

    @staticmethod
    def backward(ctx, g_loss, _g_logp, _g_ent):
        grads = ctx.grads
        if grads is None:
            raise RuntimeError("fused_linear_grpo_step: the backward can run only once per "
                               "forward (retain_graph replays are not supported)")
        ctx.grads = None
        d_hidden, d_weight = grads
        if g_loss is None:
            return (None,) * 9
        # The upstream gradient stays on the device (no host synchronisation):
        # multiplied in float32 by its ratio to the declared grad_scale, one
        # rounding to the dtype; equal to it (1 by default) writes nothing.
        if d_hidden is not None:
            d_hidden = scale_by_upstream(d_hidden, g_loss, ctx.grad_scale).view(ctx.hidden_shape)
        if d_weight is not None:
            scale_by_upstream(d_weight, g_loss, ctx.grad_scale)
        return d_hidden, d_weight, None, None, None, None, None, None, None


def _step_supported(V, dtype) -> bool:
    if dtype not in DTYPE_CODES:
        return False
    esz = torch.empty((), dtype=dtype).element_size()
    return V <= lib.klp_grpo_step_max_vocab(DTYPE_CODES[dtype]) and (V * esz) % 16 == 0


def fused_linear_grpo_step(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                           old_logp: torch.Tensor, advantages: torch.Tensor,
                           mask: torch.Tensor | None = None,
                           ref_logp: torch.Tensor | None = None, *, eps_low: float = 0.2,
                           eps_high: float | None = None, beta: float = 0.0,
                           loss_type: str = "bnpo", importance_level: str = "token",
                           max_completion_length: int | None = None,
                           normalizer: float | None = None, temperature: float | None = None,
                           chunk_tokens: int | None = None, return_stats: bool = False,
                           grad_scale: float = 1.0):
    """GRPO loss of the LM head ``hidden @ weight^T`` over token chunks;
    differentiable in ``hidden`` and ``weight``.

    Args:
        hidden: ``[B, S, D]`` (bf16 / fp16 / fp32) on the GPU.
        weight: ``[V, D]``, same dtype (``nn.Linear`` layout).
        targets: ``[B, S]`` int64.
        old_logp, advantages, mask, ref_logp and the loss keywords: as
            :func:`kernel_opt.fused_grpo_loss`; ``temperature`` divides the
            logits.
        chunk_tokens: tokens per chunk.  Peak extra memory is about
            ``2 * chunk_tokens * V`` elements, plus a float32 ``[V, D]``
            accumulator for ``d_weight`` when there is more than one chunk.
            Smaller chunks cost GEMM efficiency.  Default: the fewest equal
            chunks whose ``[chunk, V]`` buffers stay within 4 GiB
            (:data:`DEFAULT_CHUNK_BYTES`).
        grad_scale: the upstream gradient the caller's backward will send
            into the loss (``1 / k`` under ``k`` gradient-accumulation steps),
            as :func:`kernel_opt.fused_grpo_step` takes it: the gradients are
            computed already multiplied by it, and the backward writes
            nothing when the upstream gradient equals it.

    Returns ``(loss, logp, entropy)`` (``+ stats`` with ``return_stats``);
    ``logp`` and ``entropy`` are float32 ``[B, S]`` constants.
    """
    if hidden.dim() != 3:
        raise RuntimeError(f"hidden must be [B, S, D], got shape {tuple(hidden.shape)}")
    if not (hidden.is_cuda and weight.is_cuda and targets.is_cuda):
        raise RuntimeError("hidden, weight and targets must be GPU tensors")
    B, S, D = hidden.shape
    if weight.dim() != 2 or weight.size(1) != D:
        raise RuntimeError(f"weight must be [V, {D}], got {tuple(weight.shape)}")
    if weight.dtype != hidden.dtype:
        raise RuntimeError("hidden and weight must have the same dtype")
    if tuple(targets.shape) != (B, S) or targets.dtype != torch.int64:
        raise RuntimeError(f"targets must be int64 [{B}, {S}]")
    if importance_level not in ("token", "sequence"):
        raise ValueError(f"importance_level must be 'token' or 'sequence', got {importance_level!r}")
    T = 1.0 if temperature is None else float(temperature)
    if not (T > 0.0 and T != float("inf")):
        raise RuntimeError(f"temperature must be finite and > 0, got {T}")
    gs = _check_grad_scale(grad_scale)
    V = weight.size(0)
    chunk = (default_chunk_tokens(B * S, V, hidden.element_size()) if chunk_tokens is None
             else int(chunk_tokens))
    if chunk < 1:
        raise ValueError("chunk_tokens must be >= 1")
    loss_kw = dict(eps_low=eps_low, eps_high=eps_high, beta=beta, loss_type=loss_type,
                   importance_level=importance_level,
                   max_completion_length=max_completion_length, normalizer=normalizer)
    if importance_level != "token" or B * S == 0 or not _step_supported(V, hidden.dtype):
        # The unfused composition over the whole logits.
        logits = torch.matmul(hidden, weight.t())
        logp, ent, _ = fused_logprob_entropy(logits, targets, temperature)
        loss, stats = fused_grpo_loss(logp, old_logp, advantages, mask, ref_logp, **loss_kw)
        return (loss, logp, ent, stats) if return_stats else (loss, logp, ent)

    dev = hidden.device

    def f32(x, name, shape):
        if x.device != dev:
            raise RuntimeError(f"{name} must be on {dev}")
        x = x.detach().to(torch.float32)
        if tuple(x.shape) != shape:
            raise RuntimeError(f"{name} has shape {tuple(x.shape)}, expected {shape}")
        return x.contiguous()

    old = f32(old_logp, "old_logp", (B, S))
    adv = (f32(advantages, "advantages", (B,)).unsqueeze(1).expand(B, S)
           if advantages.dim() == 1 else f32(advantages, "advantages", (B, S)))
    m = (f32(mask, "mask", (B, S)) if mask is not None
         else torch.ones((B, S), dtype=torch.float32, device=dev))
    ref = f32(ref_logp, "ref_logp", (B, S)) if (beta != 0.0 and ref_logp is not None) else None
    wts = grpo_token_weights(m, loss_type, max_completion_length, normalizer)
    eh = eps_low if eps_high is None else eps_high
    params = (T, float(eps_low), float(eh), float(beta), gs)
    flat = lambda x: None if x is None else x.reshape(-1).contiguous()  # noqa: E731
    loss, logp, ent = _FusedLinearGrpoStep.apply(
        hidden, weight, targets.contiguous(), flat(old), flat(ref), flat(adv), flat(wts),
        params, chunk)
    if not return_stats:
        return loss, logp, ent
    with torch.no_grad():
        _, stats = fused_grpo_loss(logp, old, advantages, m, ref, **loss_kw)
    return loss, logp, ent, stats
