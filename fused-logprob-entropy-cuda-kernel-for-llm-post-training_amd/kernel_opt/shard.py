"""Per-shard pieces of a vocab-parallel logprob / entropy (the LM head's
logits split along the vocabulary over ranks).

Each rank holds columns ``[vocab_offset, vocab_offset + V_shard)`` of the
logits.  The sharded forward is

    state = shard_state(logits_shard, targets, vocab_offset)     # [..., 4] fp32
    states = all_gather(state)                                    # [P, ..., 4]
    logp, entropy, lse = merge_shard_states(states, targets, shard_vocab, vocab)

and the backward is local: :func:`shard_backward` with the merged lse /
entropy.  The exchange is 16 bytes per row; every rank merges in shard order
and holds the same outputs.  This module provides the per-rank parts (C ABI
klp_fwd_shard / klp_fwd_shard_merge / klp_bwd_temp); the exchange is the
caller's collective.  The reference has no multi-GPU path.
"""
from __future__ import annotations

import torch

from . import _C
from ._library import DTYPE_CODES, check_status, device_guard, lib, ptr, stream_handle

__all__ = ["shard_state", "merge_shard_states", "shard_backward"]


_ptr = ptr


def shard_state(logits_shard: torch.Tensor, targets: torch.Tensor, vocab_offset: int,
                temperature: float | None = None) -> torch.Tensor:
    """Online state of each row over this shard: float32 ``[..., 4]``
    (max, sum-exp, sum-x-exp in the kernels' units, target logit or 0).
    ``targets`` index the full vocabulary."""
    rows = _C.row_layout(logits_shard)
    if rows is None:
        raise RuntimeError("logits must be contiguous")
    if logits_shard.dtype not in DTYPE_CODES:
        raise RuntimeError("logits dtype must be bf16, fp16, or fp32")
    if targets.dtype != torch.int64 or tuple(targets.shape) != tuple(logits_shard.shape[:-1]):
        raise RuntimeError("targets must be int64 shaped like the leading dims of logits")
    V = logits_shard.size(-1)
    N = logits_shard.numel() // V if V else 0
    t = targets.contiguous()
    state = torch.empty(*targets.shape, 4, dtype=torch.float32, device=logits_shard.device)
    T = 1.0 if temperature is None else float(temperature)
    with device_guard(logits_shard.device.index):
        stream = stream_handle(logits_shard.device.index)
        rc = lib.klp_fwd_shard(_ptr(logits_shard), DTYPE_CODES[logits_shard.dtype], N, V, *rows,
                               _ptr(t), int(vocab_offset), T, _ptr(state),
                               stream)
    check_status(rc)
    return state


def merge_shard_states(states: torch.Tensor, targets: torch.Tensor, shard_vocab: int,
                       vocab: int):
    """Merge ``states`` ``[P, ..., 4]`` (shard k = columns ``[k * shard_vocab,
    ...)``) in shard order; returns float32 ``(logp, entropy, lse)`` shaped
    like ``targets``."""
    P = states.size(0)
    if tuple(states.shape[1:]) != tuple(targets.shape) + (4,):
        raise RuntimeError("states must be [P, *targets.shape, 4]")
    s = states.to(torch.float32).contiguous()
    t = targets.contiguous()
    outs = [torch.empty(targets.shape, dtype=torch.float32, device=states.device)
            for _ in range(3)]
    with device_guard(states.device.index):
        stream = stream_handle(states.device.index)
        rc = lib.klp_fwd_shard_merge(_ptr(s), P, t.numel(), _ptr(t), int(shard_vocab),
                                     int(vocab), *[_ptr(o) for o in outs],
                                     stream)
    check_status(rc)
    return tuple(outs)


def shard_backward(logits_shard: torch.Tensor, targets: torch.Tensor, vocab_offset: int,
                   lse: torch.Tensor, entropy: torch.Tensor, g_logp=None, g_ent=None,
                   g_lse=None, temperature: float | None = None) -> torch.Tensor:
    """d_logits of this shard (dense, logits dtype) from the merged ``lse`` /
    ``entropy``: the backward kernel with targets relative to the shard."""
    def prep(g):
        return None if g is None else g.to(torch.float32).contiguous()

    d = torch.empty(logits_shard.shape, dtype=logits_shard.dtype, device=logits_shard.device)
    _C.bwd_launch(logits_shard, (targets - int(vocab_offset)).contiguous(), prep(lse),
                  prep(entropy), prep(g_logp), prep(g_ent), prep(g_lse), d,
                  temperature=temperature)
    return d
