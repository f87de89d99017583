"""Python entry points over the HIP kernels (reference python/kernel_opt/ops.py).

Public entry points, with the reference's names and semantics:
  - ``fused_logprob_entropy(logits, targets)`` — autograd-aware; use from
    training code (reference ops.py:92-111).
  - ``fused_logprob_entropy_forward(logits, targets)`` — forward only, no
    autograd graph; benchmarks and no-grad paths (ops.py:41-46).
  - ``fused_logprob_entropy_naive(logits, targets)`` — one thread per row,
    never fast; correctness anchor (ops.py:33-38).

Each returns ``(logprob, entropy, lse)``, fp32 tensors shaped like
``targets``:
    logprob[i] = logits[i, targets[i]] - logsumexp(logits[i])
    entropy[i] = -sum_v softmax(logits[i])[v] * log_softmax(logits[i])[v]
    lse[i]     = logsumexp(logits[i])
A target outside ``[0, V)`` gives ``logprob = -lse`` (as the reference).

Input rule: the reference asserts ``logits.is_contiguous()``.  Here the
assertion is relaxed to "the last dim has unit stride and the rows are
reachable through at most two leading strides", which admits the shifted
slice ``logits[:, :-1, :]`` of a ``[B, L, V]`` tensor without a copy.
"""
from __future__ import annotations

import torch

from . import _C


def _check_inputs(logits: torch.Tensor, targets: torch.Tensor):
    """reference ops.py:16-21 (AssertionError on violation)."""
    assert logits.is_cuda and targets.is_cuda
    assert _C.row_layout(logits) is not None and targets.is_contiguous()
    assert targets.dtype == torch.int64
    assert logits.shape[:-1] == targets.shape, \
        f"logits[...,V]={logits.shape} vs targets[...]={targets.shape}"


def _alloc_outputs(targets: torch.Tensor):
    """reference ops.py:24-30."""
    out_shape = targets.shape
    return (
        torch.empty(out_shape, device=targets.device, dtype=torch.float32),
        torch.empty(out_shape, device=targets.device, dtype=torch.float32),
        torch.empty(out_shape, device=targets.device, dtype=torch.float32),
    )


def fused_logprob_entropy_naive(logits: torch.Tensor, targets: torch.Tensor):
    """Naive forward (one thread per row, scalar V loop)."""
    _check_inputs(logits, targets)
    logprob, entropy, lse = _alloc_outputs(targets)
    _C.fused_logprob_entropy_naive(logits, targets, logprob, entropy, lse)
    return logprob, entropy, lse


def fused_logprob_entropy_forward(logits: torch.Tensor, targets: torch.Tensor):
    """Forward only (no autograd).  Use in benches / no-grad paths."""
    _check_inputs(logits, targets)
    logprob, entropy, lse = _alloc_outputs(targets)
    _C.fused_logprob_entropy_v1(logits, targets, logprob, entropy, lse)
    return logprob, entropy, lse


class _FusedLogprobEntropy(torch.autograd.Function):
    """Forward + backward as one autograd op (reference ops.py:49-89).

    Forward saves (logits, targets, lse, entropy).  Backward recomputes
    p = exp(x - lse) in a single streaming pass and allocates only the
    gradient itself.  Outputs that are not used downstream reach backward as
    ``None`` (grad materialisation is off) and are passed to the kernel as
    null pointers, where the reference allocates and fills zero tensors.
    """

    @staticmethod
    def forward(ctx, logits, targets):
        _check_inputs(logits, targets)
        logprob, entropy, lse = _alloc_outputs(targets)
        _C.fused_logprob_entropy_v1(logits, targets, logprob, entropy, lse)
        ctx.save_for_backward(logits, targets, lse, entropy)
        ctx.set_materialize_grads(False)
        return logprob, entropy, lse

    @staticmethod
    def backward(ctx, g_logp, g_ent, g_lse):
        logits, targets, lse, entropy = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None

        def prep(g):
            return None if g is None else g.to(torch.float32, copy=False).contiguous()

        d_logits = torch.empty(logits.shape, dtype=logits.dtype, device=logits.device)
        _C.fused_logprob_entropy_v1_backward(
            logits, targets, lse, entropy, prep(g_logp), prep(g_ent), prep(g_lse), d_logits)
        return d_logits, None


def fused_logprob_entropy(logits: torch.Tensor, targets: torch.Tensor):
    """Fused logprob + entropy + logsumexp, autograd-aware.

    Replaces TRL's ``selective_log_softmax(logits, targets)`` +
    ``entropy_from_logits(logits)`` with a single streaming pass per row,
    plus a streaming backward that recomputes softmax from the saved lse.

    Args:
        logits:  [..., V] bf16 / fp16 / fp32 on the GPU (rows with unit
                 stride; see the module docstring for the layout rule).
        targets: [...]    int64, contiguous, on the GPU.

    Returns:
        (logprob, entropy, lse), each [...] fp32.  ``targets`` has no gradient.
    """
    return _FusedLogprobEntropy.apply(logits, targets)
