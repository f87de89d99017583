"""Fused LM head + per-token logprob / entropy.

``fused_linear_logprob_entropy(hidden, weight, targets)`` returns what
``fused_logprob_entropy(hidden @ weight.T, targets)`` returns, without
materialising the ``[N, V]`` logits in the forward: one MFMA GEMM kernel folds
each block of logits into the online softmax state as it is produced
(klp_lmh_fwd, csrc/klp_lmhead.hip).  The reference names this as its
follow-up (docs/FINAL_REPORT.md:439-450) and does not build it.

The logits are the fp32 sums of the bf16 products, not rounded to bf16 as a
bf16 matmul output would be; the results are therefore closer to the exact
values than the unfused bf16 path.

Backward: klp_lmh_bwd_logits recomputes every logits block with the same
MFMA order as the forward (so the softmax is rebuilt from the very values
behind the saved lse) and writes d_logits in bf16; d_hidden = d_logits @ W
and d_weight = d_logits^T @ hidden are plain library GEMMs.  Nothing of size
[N, V] is kept between forward and backward.
``fused_linear_logprob_entropy_forward`` is the no-grad entry point (GRPO's
old-policy and reference log-probabilities).
"""
from __future__ import annotations

import collections
import threading

import torch

from ._library import check_status, device_guard, lib, ptr, stream_handle

__all__ = ["fused_linear_logprob_entropy", "fused_linear_logprob_entropy_forward"]


_ptr = ptr


# Forward workspaces, one per (device, stream), the 16 most recently used
# kept (as kernel_opt._C keeps its split-row workspaces).
_ws_lock = threading.Lock()
_ws: collections.OrderedDict = collections.OrderedDict()
_WS_KEEP = 16


def _workspace(dev, stream, nbytes):
    """The workspace of (device, raw handle of its current stream), allocated
    on that stream."""
    key = (dev.index, stream)
    with _ws_lock:
        buf = _ws.get(key)
        if buf is None or buf.numel() < nbytes:
            with torch.cuda.stream(torch.cuda.current_stream(dev)):
                buf = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
            _ws[key] = buf
        _ws.move_to_end(key)
        while len(_ws) > _WS_KEEP:
            _ws.popitem(last=False)
        return buf


def _check(hidden, weight, targets):
    if not (hidden.is_cuda and weight.is_cuda and targets.is_cuda):
        raise RuntimeError("hidden, weight and targets must be GPU tensors")
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise RuntimeError("hidden and weight must be bfloat16")
    if targets.dtype != torch.int64:
        raise RuntimeError("targets must be int64")
    D = hidden.size(-1)
    if weight.dim() != 2 or weight.size(1) != D:
        raise RuntimeError(f"weight must be [V, {D}], got {tuple(weight.shape)}")
    if tuple(hidden.shape[:-1]) != tuple(targets.shape):
        raise RuntimeError("hidden[..., D] and targets[...] must have the same leading shape")
    if weight.stride(-1) != 1:
        raise RuntimeError("weight rows must have unit stride")
    h2 = hidden.reshape(-1, D)
    if h2.size(0) > 0 and h2.stride(-1) != 1:
        raise RuntimeError("hidden rows must have unit stride")
    return h2, targets.reshape(-1).contiguous()


def _ld(t: torch.Tensor) -> int:
    return t.stride(0) if t.size(0) > 1 else t.size(1)


class _FusedLinearLogprobEntropy(torch.autograd.Function):

    @staticmethod
    def forward(ctx, hidden, weight, targets, temperature):
        outs = fused_linear_logprob_entropy_forward(hidden, weight, targets, temperature)
        ctx.save_for_backward(hidden, weight, targets, outs[2], outs[1])
        ctx.temperature = temperature
        ctx.set_materialize_grads(False)
        return outs

    @staticmethod
    def backward(ctx, g_logp, g_ent, g_lse):
        hidden, weight, targets, lse, ent = ctx.saved_tensors
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (need_h or need_w):
            return None, None, None, None
        h2, t = _check(hidden, weight, targets)
        N, D, V = h2.size(0), h2.size(1), weight.size(0)
        if N == 0:
            return (torch.zeros_like(hidden) if need_h else None,
                    torch.zeros_like(weight) if need_w else None, None, None)

        def prep(g):
            return None if g is None else g.to(torch.float32, copy=False).reshape(-1).contiguous()

        gl, ge, gs = prep(g_logp), prep(g_ent), prep(g_lse)
        ld_d = (V + 3) // 4 * 4
        d = torch.empty(N, ld_d, dtype=torch.bfloat16, device=hidden.device)
        T = 1.0 if ctx.temperature is None else float(ctx.temperature)
        with device_guard(hidden.device.index):
            stream = stream_handle(hidden.device.index)
            rc = lib.klp_lmh_bwd_logits(
                _ptr(h2), _ld(h2), _ptr(weight), _ld(weight), N, V, D, _ptr(t), T,
                _ptr(lse), _ptr(ent), None if gl is None else _ptr(gl),
                None if ge is None else _ptr(ge), None if gs is None else _ptr(gs),
                _ptr(d), ld_d, stream)
        check_status(rc)
        dl = d[:, :V]
        dh = torch.mm(dl, weight).reshape(hidden.shape) if need_h else None
        dw = torch.mm(dl.t(), h2) if need_w else None
        return dh, dw, None, None


def fused_linear_logprob_entropy(hidden: torch.Tensor, weight: torch.Tensor,
                                 targets: torch.Tensor, temperature: float | None = None):
    """Autograd-aware fused LM head + logprob / entropy: gradients flow to
    ``hidden`` and ``weight`` (see :func:`fused_linear_logprob_entropy_forward`
    for the arguments and the module docstring for the backward)."""
    return _FusedLinearLogprobEntropy.apply(hidden, weight, targets, temperature)


def fused_linear_logprob_entropy_forward(hidden: torch.Tensor, weight: torch.Tensor,
                                         targets: torch.Tensor,
                                         temperature: float | None = None):
    """Args:
        hidden: ``[..., D]`` bf16 on the GPU, rows with unit stride (the
            leading dims must flatten to one stride).
        weight: ``[V, D]`` bf16 (an ``nn.Linear`` weight), rows with unit stride.
        targets: ``[...]`` int64, same leading shape as ``hidden``.
        temperature: optional T > 0; logits are multiplied by fp32(1/T).
    D must be a multiple of 64 and both row strides multiples of 8.

    Returns ``(logprob, entropy, lse)``, float32, shaped like ``targets``.
    """
    h2, t = _check(hidden, weight, targets)
    D = h2.size(1)
    N, V = h2.size(0), weight.size(0)
    out = [torch.empty(targets.shape, dtype=torch.float32, device=hidden.device)
           for _ in range(3)]
    if N == 0:
        return tuple(out)
    T = 1.0 if temperature is None else float(temperature)
    dev = hidden.device
    with device_guard(dev.index):
        stream = stream_handle(dev.index)
        ws = _workspace(dev, stream, lib.klp_lmh_workspace_bytes(N, V, D))
        rc = lib.klp_lmh_fwd(_ptr(h2), _ld(h2), _ptr(weight), _ld(weight),
                             N, V, D, _ptr(t), T, _ptr(out[0]), _ptr(out[1]), _ptr(out[2]),
                             _ptr(ws), ws.numel(), stream)
    check_status(rc)
    return tuple(out)
