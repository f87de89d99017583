"""Fused LM head + per-token logprob / entropy (forward).

``fused_linear_logprob_entropy_forward(hidden, weight, targets)`` returns
what ``fused_logprob_entropy_forward(hidden @ weight.T, targets)`` returns,
without materialising the ``[N, V]`` logits: one MFMA GEMM kernel folds each
block of logits into the online softmax state as it is produced (klp_lmh_fwd,
csrc/klp_lmhead.hip).  The reference names this as its follow-up
(docs/FINAL_REPORT.md:439-450) and does not build it.

The logits are the fp32 sums of the bf16 products, not rounded to bf16 as a
bf16 matmul output would be; the results are therefore closer to the exact
values than the unfused bf16 path.  No autograd: for the no-grad
log-probabilities of GRPO (old policy and reference model).
"""
from __future__ import annotations

import ctypes

import torch

from ._library import check_status, lib

__all__ = ["fused_linear_logprob_entropy_forward"]


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


_ws = {}


def _workspace(dev, stream, nbytes):
    key = (dev.index, stream.cuda_stream)
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        with torch.cuda.stream(stream):
            buf = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
        _ws[key] = buf
    return buf


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
    h2 = hidden.reshape(-1, D)
    if h2.stride(-1) != 1 and h2.size(0) > 0:
        raise RuntimeError("hidden rows must have unit stride")
    if weight.stride(-1) != 1:
        raise RuntimeError("weight rows must have unit stride")
    t = targets.reshape(-1).contiguous()
    N, V = h2.size(0), weight.size(0)
    out = [torch.empty(targets.shape, dtype=torch.float32, device=hidden.device)
           for _ in range(3)]
    if N == 0:
        return tuple(out)
    T = 1.0 if temperature is None else float(temperature)
    dev = hidden.device
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev)
        ws = _workspace(dev, stream, lib.klp_lmh_workspace_bytes(N, V, D))
        ld_h = h2.stride(0) if N > 1 else D
        rc = lib.klp_lmh_fwd(_ptr(h2), ld_h, _ptr(weight), weight.stride(0) if V > 1 else D,
                             N, V, D, _ptr(t), T, _ptr(out[0]), _ptr(out[1]), _ptr(out[2]),
                             _ptr(ws), ws.numel(), ctypes.c_void_p(stream.cuda_stream))
    check_status(rc)
    return tuple(out)
