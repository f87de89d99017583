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

The eager entry points run in the compiled binding (``binding/klp_torch.cpp``):
the assertions, allocations and launches, and for ``fused_logprob_entropy``
the autograd function itself (a C++ ``torch::autograd::Function`` with the
forward and backward of ``_FusedLogprobEntropy`` below), so a call costs a
few us of host time instead of the ~36 us (forward) and ~100 us (forward +
backward) the same steps took in Python.  ``_FusedLogprobEntropy`` remains
the Python statement of that op (reference ops.py:49-89), over the same
launchers; calls made while the current stream is being captured into a graph
run it (the binding declines them).
"""
from __future__ import annotations

import torch

from . import _C
from ._library import binding


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
    try:
        return tuple(binding.fused_logprob_entropy_naive_op(logits, targets))
    except binding.CaptureDeclined:
        pass
    _check_inputs(logits, targets)
    logprob, entropy, lse = _alloc_outputs(targets)
    _C.fused_logprob_entropy_naive(logits, targets, logprob, entropy, lse)
    return logprob, entropy, lse


def fused_logprob_entropy_forward(logits: torch.Tensor, targets: torch.Tensor,
                                  temperature: float | None = None):
    """Forward only (no autograd).  Use in benches / no-grad paths."""
    try:
        return tuple(binding.fused_logprob_entropy_forward(logits, targets, temperature))
    except binding.CaptureDeclined:
        pass
    _check_inputs(logits, targets)
    logprob, entropy, lse = _alloc_outputs(targets)
    _C.fwd_launch(logits, targets, logprob, entropy, lse, temperature=temperature)
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
    def forward(ctx, logits, targets, temperature=None):
        _check_inputs(logits, targets)
        logprob, entropy, lse = _alloc_outputs(targets)
        _C.fwd_launch(logits, targets, logprob, entropy, lse, temperature=temperature)
        ctx.save_for_backward(logits, targets, lse, entropy)
        ctx.temperature = temperature
        ctx.set_materialize_grads(False)
        return logprob, entropy, lse

    @staticmethod
    def backward(ctx, g_logp, g_ent, g_lse):
        logits, targets, lse, entropy = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None

        def prep(g):
            return None if g is None else g.to(torch.float32, copy=False).contiguous()

        d_logits = torch.empty(logits.shape, dtype=logits.dtype, device=logits.device)
        _C.bwd_launch(logits, targets, lse, entropy, prep(g_logp), prep(g_ent), prep(g_lse),
                      d_logits, temperature=ctx.temperature)
        return d_logits, None, None


# ---------------------------------------------------------------------------
# torch.library registration: lets torch.compile trace through the op without
# a graph break (the reference's autograd.Function breaks the graph,
# notes/stage3_findings.md:75-94).  Eager calls take the compiled autograd function.
# ---------------------------------------------------------------------------
@torch.library.custom_op("kernel_opt::fused_logprob_entropy", mutates_args=(),
                         device_types="cuda")
def _op_forward(logits: torch.Tensor, targets: torch.Tensor,
                temperature: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    _check_inputs(logits, targets)
    logprob, entropy, lse = _alloc_outputs(targets)
    _C.fwd_launch(logits, targets, logprob, entropy, lse, temperature=temperature)
    return logprob, entropy, lse


@_op_forward.register_fake
def _(logits, targets, temperature):
    return tuple(targets.new_empty(targets.shape, dtype=torch.float32) for _ in range(3))


@torch.library.custom_op("kernel_opt::fused_logprob_entropy_backward", mutates_args=(),
                         device_types="cuda")
def _op_backward(logits: torch.Tensor, targets: torch.Tensor, lse: torch.Tensor,
                 entropy: torch.Tensor, g_logp: torch.Tensor | None, g_ent: torch.Tensor | None,
                 g_lse: torch.Tensor | None, temperature: float) -> torch.Tensor:
    def prep(g):
        return None if g is None else g.to(torch.float32, copy=False).contiguous()

    d_logits = torch.empty(logits.shape, dtype=logits.dtype, device=logits.device)
    _C.bwd_launch(logits, targets, lse, entropy, prep(g_logp), prep(g_ent), prep(g_lse),
                  d_logits, temperature=temperature)
    return d_logits


@_op_backward.register_fake
def _(logits, targets, lse, entropy, g_logp, g_ent, g_lse, temperature):
    return torch.empty(logits.shape, dtype=logits.dtype, device=logits.device)


def _op_setup_context(ctx, inputs, output):
    logits, targets, temperature = inputs
    _logprob, entropy, lse = output
    ctx.save_for_backward(logits, targets, lse, entropy)
    ctx.temperature = temperature


def _op_backward_rule(ctx, g_logp, g_ent, g_lse):
    logits, targets, lse, entropy = ctx.saved_tensors
    d = _op_backward(logits, targets, lse, entropy, g_logp, g_ent, g_lse, ctx.temperature)
    return d, None, None


_op_forward.register_autograd(_op_backward_rule, setup_context=_op_setup_context)


def fused_logprob_entropy(logits: torch.Tensor, targets: torch.Tensor,
                          temperature: float | None = None):
    """Fused logprob + entropy + logsumexp, autograd-aware.

    Replaces TRL's ``selective_log_softmax(logits, targets)`` +
    ``entropy_from_logits(logits)`` with a single streaming pass per row,
    plus a streaming backward that recomputes softmax from the saved lse.

    Args:
        logits:  [..., V] bf16 / fp16 / fp32 on the GPU (rows with unit
                 stride; see the module docstring for the layout rule).
        targets: [...]    int64, contiguous, on the GPU.

        temperature: optional sampling temperature T > 0.  The kernels then
                 work on ``logits / T`` (each logit multiplied by fp32(1/T) as
                 it is loaded) and the gradient is taken with respect to the
                 unscaled ``logits``.  This replaces a separate
                 ``logits.div_(T)`` pass; ``None`` or 1 is the plain op.

    Returns:
        (logprob, entropy, lse), each [...] fp32.  ``targets`` has no gradient.

    Under ``torch.compile`` the call goes through the registered op
    ``torch.ops.kernel_opt.fused_logprob_entropy`` (traced without a graph
    break); eagerly it runs the compiled autograd function, which skips the
    dispatcher.
    """
    if torch.compiler.is_compiling():
        return torch.ops.kernel_opt.fused_logprob_entropy(
            logits, targets, 1.0 if temperature is None else float(temperature))
    try:
        return tuple(binding.fused_logprob_entropy(logits, targets, temperature))
    except binding.CaptureDeclined:
        return _FusedLogprobEntropy.apply(logits, targets, temperature)
