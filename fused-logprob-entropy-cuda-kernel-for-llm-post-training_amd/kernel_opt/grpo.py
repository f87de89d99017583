"""Fused GRPO policy loss over per-token log-probabilities.

The reference plans this as kernel "K2 fused_grpo_loss" (notes/PLAN.md:59)
and writes the loss out in eager PyTorch in examples/compare_one_step.py:232-236:

    ratio = (new_logp - old).exp()
    surr = -torch.minimum(ratio * A, ratio.clamp(1 - eps, 1 + eps) * A)
    loss = (surr * mask).sum() / mask.sum()

``fused_grpo_loss`` computes that loss, and the variants TRL's GRPOTrainer
offers around it, in two small HIP launches (row sums, then the batch sums)
instead of a chain of elementwise kernels; its backward is one more launch.

Per token, with w = new_logp - old_logp (``importance_level="token"``) or the
row's masked mean of it (``"sequence"``):
    c1 = exp(w),  c2 = clamp(c1, 1 - eps_low, 1 + eps_high),
    loss_tok = -min(c1 * A, c2 * A) + beta * (exp(ref - new) - (ref - new) - 1)
and the loss divides the masked sum of ``loss_tok`` by
    "grpo":     n_seqs * max(row mask sum, 1), row by row (mean of row means);
    "bnpo":     max(batch mask sum, 1)  (the reference's formula, with mask.sum() >= 1);
    "dr_grpo":  n_seqs * max_completion_length;
    "dapo":     ``normalizer``.
Gradients flow to ``logp`` only; the other inputs are constants, as the
detached old / reference log-probabilities and advantages are in GRPO.
With no tokens (B = 0 or S = 0) the loss is 0.
"""
from __future__ import annotations

import torch

from ._library import (KLP_GRPO_LOSS_BNPO, KLP_GRPO_LOSS_FIXED, KLP_GRPO_LOSS_GRPO,
                       KLP_GRPO_SEQUENCE, KLP_GRPO_TOKEN, binding, check_status, device_guard,
                       lib, ptr, stream_handle)

__all__ = ["fused_grpo_loss"]

_LEVELS = {"token": KLP_GRPO_TOKEN, "sequence": KLP_GRPO_SEQUENCE}


_ptr = ptr


def _f32(t, name, shape, device):
    if t is None:
        return None
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device != device:
        raise RuntimeError(f"{name} must be on {device}")
    t = t.detach().to(torch.float32)
    if tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    return t.contiguous()


def _config(B, S, loss_type, importance_level, max_completion_length, normalizer):
    if importance_level not in _LEVELS:
        raise ValueError(f"importance_level must be 'token' or 'sequence', got {importance_level!r}")
    norm = 1.0
    if loss_type == "grpo":
        kind = KLP_GRPO_LOSS_GRPO
    elif loss_type == "bnpo":
        kind = KLP_GRPO_LOSS_BNPO
    elif loss_type == "dr_grpo":
        kind = KLP_GRPO_LOSS_FIXED
        norm = float(B * (S if max_completion_length is None else max_completion_length))
    elif loss_type == "dapo":
        if normalizer is None:
            raise ValueError("loss_type='dapo' needs `normalizer`")
        kind = KLP_GRPO_LOSS_FIXED
        norm = float(normalizer)
    else:
        raise ValueError(f"unknown loss_type {loss_type!r}")
    return kind, _LEVELS[importance_level], norm


class _FusedGrpoLoss(torch.autograd.Function):

    @staticmethod
    def forward(ctx, logp, old_logp, ref_logp, advantages, mask, params):
        B, S = logp.shape
        dev = logp.device
        lp = logp.detach().contiguous()
        ws = torch.empty(lib.klp_grpo_workspace_bytes(B), dtype=torch.uint8, device=dev)
        loss = torch.empty(1, dtype=torch.float32, device=dev)
        stats = torch.empty(4, dtype=torch.float32, device=dev)
        with device_guard(dev.index):
            stream = stream_handle(dev.index)
            rc = lib.klp_grpo_fwd(_ptr(lp), _ptr(old_logp), _ptr(ref_logp), _ptr(advantages),
                                  _ptr(mask), B, S, *params, _ptr(loss), _ptr(stats), _ptr(ws),
                                  ws.numel(), stream)
        check_status(rc)
        ctx.save_for_backward(lp, old_logp, ref_logp, advantages, mask, ws)
        ctx.params = params
        ctx.mark_non_differentiable(stats)
        return loss.view(()), stats

    @staticmethod
    def backward(ctx, g_loss, _g_stats):
        lp, old_logp, ref_logp, advantages, mask, ws = ctx.saved_tensors
        if g_loss is None or not ctx.needs_input_grad[0]:
            return None, None, None, None, None, None
        B, S = lp.shape
        g = g_loss.detach().to(torch.float32).reshape(1).contiguous()
        d = torch.empty_like(lp)
        dev = lp.device
        with device_guard(dev.index):
            stream = stream_handle(dev.index)
            rc = lib.klp_grpo_bwd(_ptr(lp), _ptr(old_logp), _ptr(ref_logp), _ptr(advantages),
                                  _ptr(mask), B, S, *ctx.params, _ptr(g), _ptr(d), _ptr(ws),
                                  ws.numel(), stream)
        check_status(rc)
        return d, None, None, None, None, None


def fused_grpo_loss(logp: torch.Tensor, old_logp: torch.Tensor, advantages: torch.Tensor,
                    mask: torch.Tensor | None = None, ref_logp: torch.Tensor | None = None, *,
                    eps_low: float = 0.2, eps_high: float | None = None, beta: float = 0.0,
                    loss_type: str = "bnpo", importance_level: str = "token",
                    max_completion_length: int | None = None,
                    normalizer: float | None = None):
    """GRPO loss of per-token log-probabilities ``logp`` ``[B, S]`` (the
    output of :func:`kernel_opt.fused_logprob_entropy`), differentiable in
    ``logp``.

    Args:
        old_logp: ``[B, S]`` log-probabilities of the sampling policy.
        advantages: ``[B]`` (one per completion) or ``[B, S]``.
        mask: ``[B, S]`` completion mask (bool / int / float), ``None`` = all ones.
        ref_logp: ``[B, S]`` reference-model log-probabilities for the KL
            term (used when ``beta != 0``).
        eps_low, eps_high: clip range ``[1 - eps_low, 1 + eps_high]``;
            ``eps_high`` defaults to ``eps_low``.
        loss_type: "grpo", "bnpo", "dr_grpo" or "dapo" (see the module docstring).

    Returns:
        ``(loss, stats)``: the scalar loss (float32) and a float32 ``[4]``
        tensor of masked means over all tokens: KL estimate, "clipped low"
        (c1 < 1 - eps_low with A < 0), "clipped high" (c1 > 1 + eps_high
        with A > 0), and clipped either way.
    """
    if logp.dim() != 2:
        raise RuntimeError(f"logp must be [B, S], got shape {tuple(logp.shape)}")
    kind, level, norm = _config(logp.size(0), logp.size(1), loss_type, importance_level,
                                max_completion_length, normalizer)
    eh = eps_low if eps_high is None else eps_high
    for name, t in (("old_logp", old_logp), ("advantages", advantages), ("mask", mask),
                    ("ref_logp", ref_logp)):
        if t is not None and not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a tensor")
    # The compiled binding runs the checks, conversions and launches below in
    # C++ (binding/klp_torch.cpp); under graph capture it declines and this
    # Python statement of them runs.
    try:
        return tuple(binding.fused_grpo_loss(logp, old_logp, advantages, mask, ref_logp,
                                             float(eps_low), float(eh), float(beta), norm, kind,
                                             level))
    except binding.CaptureDeclined:
        pass
    if not logp.is_cuda:
        raise RuntimeError("logp must be a GPU tensor")
    if logp.dtype != torch.float32:
        raise RuntimeError("logp must be float32")
    B, S = logp.shape
    dev = logp.device
    old = _f32(old_logp, "old_logp", (B, S), dev)
    if advantages.dim() == 1:
        adv, per_token = _f32(advantages, "advantages", (B,), dev), 0
    else:
        adv, per_token = _f32(advantages, "advantages", (B, S), dev), 1
    m = _f32(mask, "mask", (B, S), dev)
    ref = _f32(ref_logp, "ref_logp", (B, S), dev) if beta != 0.0 else None
    if B == 0 or S == 0:
        # No tokens: every normaliser sees an empty (zero) masked sum.
        return logp.sum() * 0.0, torch.zeros(4, dtype=torch.float32, device=dev)
    params = (float(eps_low), float(eh), float(beta), norm, kind, level, per_token)
    return _FusedGrpoLoss.apply(logp, old, ref, adv, m, params)
