"""Fused GRPO step: per-token logprob / entropy, GRPO loss and d_logits in one
pass over the logits.

The reference's GRPO step runs, one after another, the logprob kernel
(python/kernel_opt/trainer.py:38-130), the eager loss
(examples/compare_one_step.py:232-236) and, in the backward, the logprob
backward: the logits are read twice (forward, backward) and d_logits written
once.  With token-level importance weights the gradient of the batch loss
with respect to a token's log-probability is known as soon as that token's
log-probability is, so ``klp_grpo_step`` keeps each row of logits in
registers, computes logprob / entropy, the token's loss and its gradient,
and writes the row's d_logits at once: one read of the logits instead of two.

``fused_grpo_step`` returns the loss and the per-token log-probabilities and
entropies; ``loss.backward()`` hands the precomputed d_logits to autograd.
The same numbers come out of

    logp, ent, _ = fused_logprob_entropy(logits, targets, temperature)
    loss, _ = fused_grpo_loss(logp, old_logp, advantages, mask, ref_logp, ...)

up to float32 rounding; that composition is also what runs when the fused
step does not apply (sequence-level importance weights, rows longer than
``klp_grpo_step_max_vocab``, rows not 16-byte aligned).

Restrictions of the fused path, by construction:
  * only the loss is differentiable: ``logp`` and ``entropy`` are returned
    as constants (an extra loss term on them would get no gradient; use the
    composition above for that);
  * the backward can run once per forward (no ``retain_graph`` replays);
  * an upstream gradient other than exactly 1 on the loss (e.g. a loss
    scaled before ``backward()``) costs one extra pass over d_logits, and
    telling the two apart reads the scalar back to the host.
"""
from __future__ import annotations

import collections
import math
import threading

import numpy as np
import torch

from . import _C
from ._library import (DTYPE_CODES, KLP_GRPO_LOSS_BNPO, KLP_GRPO_STEP_SCHED_BYTES,
                       KLP_GRPO_TOKEN_WEIGHTS_WORKSPACE_BYTES, binding, capturing, check_status,
                       device_guard, keep_for_capture, lib, ptr, stream_handle)
from .grpo import fused_grpo_loss
from .ops import fused_logprob_entropy

__all__ = ["fused_grpo_step", "grpo_token_weights", "grpo_step_launch"]


_ptr = ptr


def _f32_reciprocal(v) -> float:
    """fp32(1) / fp32(v), rounded once in float32 (what dividing a float32
    tensor gives), as a Python float: multiplying a float32 tensor by it needs
    no device copy of a host scalar (no synchronisation, capturable)."""
    return float(np.float32(1.0) / np.float32(v))


def grpo_token_weights(mask: torch.Tensor, loss_type: str = "bnpo",
                       max_completion_length: int | None = None,
                       normalizer: float | None = None) -> torch.Tensor:
    """Weight of each token's loss in the batch loss (float32 ``[B, S]``):
    the mask divided by the loss type's normaliser, as ``fused_grpo_loss``
    applies it ("grpo": B * max(row mask sum, 1); "bnpo": max(mask sum, 1);
    "dr_grpo": B * max_completion_length (default S); "dapo": normalizer)."""
    m = mask.to(torch.float32)
    B, S = m.shape
    if loss_type == "grpo":
        den = m.sum(dim=1, keepdim=True).clamp(min=1.0) * float(B)
        return m * (1.0 / den)
    if loss_type == "bnpo":
        return m * (1.0 / m.sum().clamp(min=1.0))
    if loss_type == "dr_grpo":
        L = S if max_completion_length is None else max_completion_length
        return m * _f32_reciprocal(B * L)
    if loss_type == "dapo":
        if normalizer is None:
            raise ValueError("loss_type='dapo' needs `normalizer`")
        return m * _f32_reciprocal(normalizer)
    raise ValueError(f"unknown loss_type {loss_type!r}")


def _fused_supported(logits: torch.Tensor, rows) -> bool:
    """True when klp_grpo_step accepts these logits (row capacity and
    16-byte aligned rows of whole 16-byte vectors)."""
    if rows is None or logits.dtype not in DTYPE_CODES:
        return False
    V = logits.size(-1)
    esz = logits.element_size()
    if V > lib.klp_grpo_step_max_vocab(DTYPE_CODES[logits.dtype]):
        return False
    _, s_outer, s_inner = rows
    return ((V * esz) % 16 == 0 and logits.data_ptr() % 16 == 0
            and (s_inner * esz) % 16 == 0 and (s_outer * esz) % 16 == 0)


# klp_grpo_step's row counters, one per (device, raw stream handle): each is
# zeroed once, when allocated on its stream, and every launch leaves it zero,
# so launches on one stream can share it.  At most _SCHED_KEEP are kept,
# least recently used dropped first (the caching allocator reuses a dropped
# one only in its stream's order).  A call under graph capture gets a counter
# of its own instead (kept for the life of the process): graphs captured on
# one stream and replayed concurrently would otherwise race on a shared one.
_sched_lock = threading.Lock()
_scheds: collections.OrderedDict = collections.OrderedDict()
_SCHED_KEEP = 16


def _sched(device_index: int, stream: int) -> torch.Tensor:
    """The row counter of (device, stream); the device must be current and
    ``stream`` its current stream."""
    if capturing():
        # torch.zeros fills with a kernel, which a graph replays correctly.
        return keep_for_capture(torch.zeros(KLP_GRPO_STEP_SCHED_BYTES // 8, dtype=torch.int64,
                                            device=torch.device("cuda", device_index)))
    key = (device_index, stream)
    with _sched_lock:
        buf = _scheds.get(key)
        if buf is None:
            buf = torch.zeros(KLP_GRPO_STEP_SCHED_BYTES // 8, dtype=torch.int64,
                              device=torch.device("cuda", device_index))
            _scheds[key] = buf
        _scheds.move_to_end(key)
        while len(_scheds) > _SCHED_KEEP:
            _scheds.popitem(last=False)
        return buf


def grpo_step_launch(logits, targets, old, ref, adv, weight, params):
    """One klp_grpo_step call, no autograd: returns float32 ``logp``,
    ``entropy``, ``lse``, ``loss_tok`` ``[B, S]`` and ``d_logits`` (dense,
    logits dtype).  ``old`` / ``ref`` / ``adv`` / ``weight`` are float32,
    contiguous, on the logits' device; ``params`` = (temperature, eps_low,
    eps_high, beta, adv_per_token, grad_scale): ``d_logits`` is the loss's
    gradient times ``grad_scale``."""
    temperature, eps_low, eps_high, beta, per_token, grad_scale = params
    B, S, V = logits.shape
    dev = logits.device
    rows = _C.row_layout(logits)
    if rows is None:
        raise RuntimeError("logits must be contiguous")
    logp, ent, lse, loss_tok = (torch.empty((B, S), dtype=torch.float32, device=dev)
                                for _ in range(4))
    d_logits = torch.empty((B, S, V), dtype=logits.dtype, device=dev)
    with device_guard(dev.index):
        stream = stream_handle(dev.index)
        rc = lib.klp_grpo_step(_ptr(logits), DTYPE_CODES[logits.dtype], B * S, V, *rows,
                               _ptr(targets), float(temperature), _ptr(old), _ptr(ref),
                               _ptr(adv), _ptr(weight), S, eps_low, eps_high, beta, per_token,
                               float(grad_scale), _ptr(logp), _ptr(ent), _ptr(lse), _ptr(loss_tok), _ptr(d_logits),
                               _ptr(_sched(dev.index, stream)), stream)
    check_status(rc)
    return logp, ent, lse, loss_tok, d_logits


def scale_by_upstream(t: torch.Tensor, g: torch.Tensor, applied: float = 1.0) -> torch.Tensor:
    """``t *= g / applied`` in place (``t`` contiguous, already scaled by the
    declared upstream gradient ``applied``; ``g`` a one-element tensor on
    ``t``'s device) without reading ``g`` on the host: klp_rescale_inplace
    reads it on the device, multiplies in float32 by ``g / applied`` (``g``
    itself when ``applied`` is 1) and rounds once to ``t``'s dtype (as
    ``t * float(g)`` would), and writes nothing when ``g == applied``."""
    if not t.is_contiguous():
        raise RuntimeError("scale_by_upstream needs a contiguous tensor")
    g32 = g.detach().to(device=t.device, dtype=torch.float32).reshape(1).contiguous()
    with device_guard(t.device.index):
        stream = stream_handle(t.device.index)
        rc = lib.klp_rescale_inplace(_ptr(t), DTYPE_CODES[t.dtype], t.numel(), _ptr(g32),
                                     float(applied), stream)
    check_status(rc)
    return t


class _FusedGrpoStep(torch.autograd.Function):

    @staticmethod
    def forward(ctx, logits, targets, old, ref, adv, weight, params):
        logp, ent, _lse, loss_tok, d_logits = grpo_step_launch(logits, targets, old, ref, adv,
                                                               weight, params)
        ctx.d_logits = d_logits
        ctx.grad_scale = params[5]
        ctx.mark_non_differentiable(logp, ent)
        return loss_tok.sum(), logp, ent

    @staticmethod
    def backward(ctx, g_loss, _g_logp, _g_ent):
        d = ctx.d_logits
        if d is None:
            raise RuntimeError("fused_grpo_step: the backward can run only once per forward "
                               "(retain_graph replays are not supported)")
        ctx.d_logits = None
        if g_loss is None or not ctx.needs_input_grad[0]:
            return None, None, None, None, None, None, None
        # The upstream gradient stays on the device (no host synchronisation);
        # exactly the declared grad_scale (1 by default) leaves d as it is.
        return (scale_by_upstream(d, g_loss, ctx.grad_scale), None, None, None, None, None,
                None)


def fused_grpo_step(logits: torch.Tensor, targets: torch.Tensor, old_logp: torch.Tensor,
                    advantages: torch.Tensor, mask: torch.Tensor | None = None,
                    ref_logp: torch.Tensor | None = None, *, eps_low: float = 0.2,
                    eps_high: float | None = None, beta: float = 0.0, loss_type: str = "bnpo",
                    importance_level: str = "token", max_completion_length: int | None = None,
                    normalizer: float | None = None, temperature: float | None = None,
                    return_stats: bool = False, grad_scale: float = 1.0):
    """GRPO loss of ``logits`` ``[B, S, V]`` (the completion window, rows as
    :func:`kernel_opt.fused_logprob_entropy` accepts them) for ``targets``
    ``[B, S]`` (int64), differentiable in ``logits``.

    The loss arguments are those of :func:`kernel_opt.fused_grpo_loss`;
    ``temperature`` divides the logits as in ``fused_logprob_entropy``.

    ``grad_scale`` declares the upstream gradient the caller's backward will
    send into the loss: 1 for ``loss.backward()``, ``1 / k`` when a trainer
    divides the loss by ``k`` gradient-accumulation steps.  The fused kernel
    writes d_logits already multiplied by it, so the backward writes nothing
    when the upstream gradient equals it; any other upstream gradient is
    still applied (one more pass over d_logits, multiplied by the ratio).
    It changes no value beyond rounding, and the unfused composition ignores
    it.

    Returns ``(loss, logp, entropy)``, or ``(loss, logp, entropy, stats)``
    with ``return_stats`` (stats as ``fused_grpo_loss`` returns them).
    ``logp`` and ``entropy`` are float32 ``[B, S]`` constants when the fused
    path runs.
    """
    if logits.dim() != 3:
        raise RuntimeError(f"logits must be [B, S, V], got shape {tuple(logits.shape)}")
    if not logits.is_cuda:
        raise RuntimeError("logits must be a GPU tensor")
    B, S, V = logits.shape
    if tuple(targets.shape) != (B, S):
        raise RuntimeError(f"targets has shape {tuple(targets.shape)}, expected {(B, S)}")
    if targets.device != logits.device:
        # Checked before either path is chosen: the fused kernel would
        # otherwise read a host pointer as device memory.
        raise RuntimeError(f"targets must be on {logits.device}, got {targets.device}")
    if importance_level not in ("token", "sequence"):
        raise ValueError(f"importance_level must be 'token' or 'sequence', got {importance_level!r}")
    t = 1.0 if temperature is None else float(temperature)
    if not (t > 0.0 and t != float("inf")):
        raise RuntimeError(f"temperature must be finite and > 0, got {t}")
    gs = _check_grad_scale(grad_scale)
    loss_kw = dict(eps_low=eps_low, eps_high=eps_high, beta=beta, loss_type=loss_type,
                   importance_level=importance_level,
                   max_completion_length=max_completion_length, normalizer=normalizer)

    wants_grad = torch.is_grad_enabled() and logits.requires_grad
    if (wants_grad and importance_level == "token" and B * S > 0 and targets.is_contiguous()
            and targets.dtype == torch.int64):
        eh = eps_low if eps_high is None else eps_high
        kind, scale = _weight_kind(B, S, loss_type, max_completion_length, normalizer)
        # The compiled binding (binding/klp_torch.cpp) runs the conversions,
        # the token weights and the autograd op below in C++; under graph
        # capture it declines and this module's statement of them runs.
        try:
            out = binding.fused_grpo_step(logits, targets, old_logp, advantages, mask,
                                          ref_logp, t, float(eps_low), float(eh), float(beta),
                                          kind, scale, gs)
        except binding.CaptureDeclined:
            out = _fused_python(logits, targets, old_logp, advantages, mask, ref_logp, t,
                                float(eps_low), float(eh), float(beta), loss_type,
                                max_completion_length, normalizer, gs)
        if out is not None:
            loss, logp, ent = out
            if not return_stats:
                return loss, logp, ent
            with torch.no_grad():
                _, stats = fused_grpo_loss(logp, old_logp, advantages, mask, ref_logp, **loss_kw)
            return loss, logp, ent, stats
    # The unfused composition: same loss, logp / entropy differentiable.  It
    # also serves calls that need no gradient (evaluation, logging,
    # torch.no_grad()): the fused kernel would allocate and write a full
    # [B, S, V] d_logits that nothing reads.
    logp, ent, _ = fused_logprob_entropy(logits, targets, temperature)
    loss, stats = fused_grpo_loss(logp, old_logp, advantages, mask, ref_logp, **loss_kw)
    return (loss, logp, ent, stats) if return_stats else (loss, logp, ent)


# Mask dtypes klp_grpo_token_weights reads (KLP_MASK_U8 / _I32 / _I64).
_MASK_CODES = {torch.bool: 0, torch.uint8: 0, torch.int32: 1, torch.int64: 2}


def _device_token_weights(mask, B, S, dev, kind, scale):
    """grpo_token_weights' bits by klp_grpo_token_weights (a bool / integer
    mask, or none), or None where the eager statement has to run: a floating
    mask, or a fixed normaliser whose float32 reciprocal is not finite and
    > 0.  Under graph capture the workspace is the captured call's own."""
    if mask is not None and (mask.dtype not in _MASK_CODES or mask.device != dev
                             or tuple(mask.shape) != (B, S)):
        return None
    if kind == 2 and not (0.0 < float(np.float32(scale)) < float("inf")):
        return None
    m = None if mask is None else mask.detach().contiguous()
    weight = torch.empty((B, S), dtype=torch.float32, device=dev)
    ws = None
    if kind == KLP_GRPO_LOSS_BNPO:
        ws = torch.empty(KLP_GRPO_TOKEN_WEIGHTS_WORKSPACE_BYTES, dtype=torch.uint8, device=dev)
        if capturing():
            ws = keep_for_capture(ws)
    with device_guard(dev.index):
        check_status(lib.klp_grpo_token_weights(
            ptr(m), 0 if m is None else _MASK_CODES[m.dtype], B, S, kind, float(scale),
            ptr(weight), ptr(ws), stream_handle(dev.index)))
    return weight


def _check_grad_scale(grad_scale) -> float:
    """``grad_scale`` as a float, finite and non-zero in float32 (the
    kernels take it as float32)."""
    gs = float(grad_scale)
    if not (math.isfinite(gs) and abs(gs) <= float(np.finfo(np.float32).max)
            and np.float32(gs) != 0):
        raise ValueError(f"grad_scale must be finite and non-zero in float32, got {grad_scale}")
    return gs


def _weight_kind(B, S, loss_type, max_completion_length, normalizer):
    """(kind, scale) of grpo_token_weights for the compiled binding: 0 "grpo",
    1 "bnpo", 2 a fixed normaliser with its float32 reciprocal."""
    if loss_type == "grpo":
        return 0, 1.0
    if loss_type == "bnpo":
        return 1, 1.0
    if loss_type == "dr_grpo":
        L = S if max_completion_length is None else max_completion_length
        return 2, _f32_reciprocal(B * L)
    if loss_type == "dapo":
        if normalizer is None:
            raise ValueError("loss_type='dapo' needs `normalizer`")
        return 2, _f32_reciprocal(normalizer)
    raise ValueError(f"unknown loss_type {loss_type!r}")


def _fused_python(logits, targets, old_logp, advantages, mask, ref_logp, t, eps_low, eps_high,
                  beta, loss_type, max_completion_length, normalizer, grad_scale=1.0):
    """The fused path in Python (graph capture): (loss, logp, entropy), or
    None when klp_grpo_step does not take these logits."""
    if not _fused_supported(logits, _C.row_layout(logits)):
        return None
    B, S, _ = logits.shape
    dev = logits.device

    def f32(x, name, shape):
        if x.device != dev:
            raise RuntimeError(f"{name} must be on {dev}")
        x = x.detach().to(torch.float32)
        if tuple(x.shape) != shape:
            raise RuntimeError(f"{name} has shape {tuple(x.shape)}, expected {shape}")
        return x.contiguous()

    old = f32(old_logp, "old_logp", (B, S))
    per_token = advantages.dim() != 1
    adv = f32(advantages, "advantages", (B, S) if per_token else (B,))
    ref = f32(ref_logp, "ref_logp", (B, S)) if (beta != 0.0 and ref_logp is not None) else None
    kind, scale = _weight_kind(B, S, loss_type, max_completion_length, normalizer)
    weight = _device_token_weights(mask, B, S, dev, kind, scale)
    if weight is None:
        m = (f32(mask, "mask", (B, S)) if mask is not None
             else torch.ones((B, S), dtype=torch.float32, device=dev))
        weight = grpo_token_weights(m, loss_type, max_completion_length, normalizer).contiguous()
    params = (t, eps_low, eps_high, beta, int(per_token), grad_scale)
    return _FusedGrpoStep.apply(logits, targets, old, ref, adv, weight, params)
