"""LM head + per-token logprob / entropy without the ``[N, V]`` logits.

``fused_linear_logprob_entropy(hidden, weight, targets)`` returns what
``fused_logprob_entropy(hidden @ weight.T, targets)`` returns, and so does its
backward, while neither pass holds the ``[N, V]`` logits (or their gradient):
the Liger-style head the reference names as its follow-up
(docs/FINAL_REPORT.md:439-450, 490-493) and does not build.

Two implementations:

``impl="chunked"`` (default) walks the vocabulary in chunks
(:func:`vocab_chunks`: 32768 columns for small batches, ~16K for larger
ones).  Per chunk a library GEMM writes the chunk's logits (``[N, chunk]``
in the input dtype, at most 128 MiB) and ``klp_fwd_chunk`` folds them into
each token's online state; the last chunk's launch merges the chunk states
in chunk order and writes the outputs.  The weight is read once and the
logits never exist as one ``[N, V]`` tensor.  The backward recomputes each
chunk with the same GEMM call (bit-identical logits), applies ``klp_bwd``
with chunk-relative targets, and accumulates ``d_hidden += d_chunk @
W_chunk`` (fp32) and ``d_weight[chunk] = d_chunk^T @ hidden``.  Numerics are
the unfused path's: logits rounded once to the input dtype by the GEMM.

``impl="mfma"`` is the hand-written gfx950 kernel (klp_lmh_fwd,
csrc/klp_lmhead.hip): the GEMM with the logprob / entropy reduction as its
epilogue, logits kept as fp32 MFMA sums (never rounded), bf16 inputs, hidden
size a multiple of 64.  Its backward recomputes chunks of logits with the
same MFMA order (klp_lmh_bwd_logits on a slice of the weight) and runs the
same two library GEMMs per chunk.  It is slower than the library GEMM at
these shapes (1024 tokens of Qwen2.5-7B's head, bench.py's lm_head leg:
forward 1.30-1.32 ms, 34% of the bf16 MFMA peak, against 0.93 ms for the
library GEMM) and is kept as a correct alternative, not tuned further.

At 1024 tokens the chunked forward runs within ~2% of the unfused one, on
either side from box to box (bench.py's lm_head leg: 0.9356 against 0.9279 ms
on one box, 0.901-0.954 against 0.911-0.948 ms on three others), while it holds 64 MiB of
extra memory where the unfused path holds 297 MiB of logits; at 8192 tokens
6.33 against 6.42 ms, 131 against 2376 MiB.

The backward of either head recomputes the logits, one GEMM more than the
unfused path's backward: that is the price of not holding them (measured
forward + backward at 1024 tokens: 4.64-4.72 ms chunked, 3.83-3.87 ms
unfused, with 135 MiB against 297 MiB beyond the inputs and gradients).  When the loss is
known in the forward, :func:`kernel_opt.fused_linear_grpo_step` computes the
gradients there and needs no recompute.

``fused_linear_logprob_entropy_forward`` is the no-grad entry point (GRPO's
old-policy and reference log-probabilities).
"""
from __future__ import annotations

import collections
import threading

import torch

from . import _C
from ._library import DTYPE_CODES, check_status, device_guard, lib, ptr, stream_handle
from .linear_grpo import _accumulate_f32

__all__ = ["fused_linear_logprob_entropy", "fused_linear_logprob_entropy_forward", "vocab_chunk",
           "vocab_chunks"]


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


def _check(hidden, weight, targets, impl):
    if impl not in ("chunked", "mfma"):
        raise ValueError(f"impl must be 'chunked' or 'mfma', got {impl!r}")
    if not (hidden.is_cuda and weight.is_cuda and targets.is_cuda):
        raise RuntimeError("hidden, weight and targets must be GPU tensors")
    if impl == "mfma" and (hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16):
        raise RuntimeError("hidden and weight must be bfloat16")
    if hidden.dtype not in DTYPE_CODES or weight.dtype != hidden.dtype:
        raise RuntimeError("hidden and weight must share one dtype: bf16, fp16 or fp32")
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


# Vocabulary chunk of the chunked head.  Small batches (a chunk of
# CHUNK_COLS_WIDE columns within CHUNK_WIDE_MAX_BYTES: up to 1024 bf16 tokens)
# take chunks of CHUNK_COLS_WIDE columns, the last one holding the rest.
# Larger batches take about CHUNK_COLS columns, balanced over the vocabulary
# in whole multiples of 1024 (so that no small tail GEMM runs), and fewer
# while one chunk of logits would exceed CHUNK_MAX_BYTES, half of the 256 MB
# Infinity Cache, so that the logprob pass over a chunk reads it from the
# cache.  The library GEMM's speed at the chunk shape dominates, and it does
# not follow the width monotonically.  Measured at Qwen2.5-7B's head
# (V = 152064, D = 3584; forward, forward + backward, ms; two runs):
#   1024 tokens: 32768 columns 0.934-0.940, 4.75-4.76; balanced 15360
#                0.975-0.979, 4.79; unfused 0.927-0.932, 3.84
#   2048 tokens: balanced 15360 1.75-1.76, 8.40-8.44; 16384 1.70-1.71,
#                9.80-9.82 (its backward GEMMs are slow); unfused 1.70, 7.04
#   4096 tokens: balanced 15360 3.34, 15.22-15.24; 8192 3.30-3.31,
#                15.30-15.31; unfused 3.25-3.27, 12.94
#   8192 tokens: balanced 8192 6.39-6.40, 30.40-30.46; unfused 6.41-6.43, 24.65
# The forward and the backward use the same chunks: the backward recomputes
# each chunk's logits with the same GEMM call, hence the same values.
# In the small-batch regime a last chunk wider than CHUNK_COLS_WIDE / 2 is
# cut into CHUNK_COLS_WIDE / 2 columns plus the rest: the library GEMM runs
# widths of 16384 and 32768 columns at 5.0-5.1 us per 1024 columns (1024
# tokens, D = 3584), but 18432-22528 at 6.2-6.8 us (V = 152064's remainder of
# 20992: 138.8 us, against 83.4 + ~36 us as 16384 + 4608).  Qwen2.5-7B's head
# at 1024 tokens, forward, one box, launches queued (host-issued): chunks
# 4 x 32768 + 20992 950.3 (927.2) us, 4 x 32768 + 16384 + 4608 942.4
# (908.4) us, unfused 957.7 (923.2) us.
CHUNK_COLS_WIDE = 32768
CHUNK_WIDE_MAX_BYTES = 64 << 20
CHUNK_COLS = 16384
CHUNK_MAX_BYTES = 128 << 20


def vocab_chunk(n_tokens: int, vocab: int, elem_bytes: int = 2,
                chunk_vocab: int | None = None) -> int:
    """Columns per chunk of the chunked head (the last chunk may hold
    fewer)."""
    if chunk_vocab is not None:
        if chunk_vocab < 1:
            raise ValueError(f"chunk_vocab must be >= 1, got {chunk_vocab}")
        return min(int(chunk_vocab), max(vocab, 1))
    if n_tokens * CHUNK_COLS_WIDE * elem_bytes <= CHUNK_WIDE_MAX_BYTES:
        return min(vocab, CHUNK_COLS_WIDE)
    cols = CHUNK_COLS
    while cols > 1024 and n_tokens * cols * elem_bytes > CHUNK_MAX_BYTES:
        cols //= 2
    n_chunks = max(1, -(-vocab // cols))
    per = -(-vocab // n_chunks)
    return min(vocab, -(-per // 1024) * 1024)


def vocab_chunks(n_tokens: int, vocab: int, elem_bytes: int = 2,
                 chunk_vocab: int | None = None) -> list:
    """``(first column, width)`` of every vocabulary chunk of the chunked
    head, in order: chunks of :func:`vocab_chunk` columns, the last one the
    rest; in the small-batch regime a rest of at least half a chunk plus 1024
    columns is cut in two (``CHUNK_COLS_WIDE // 2`` columns, then the
    remainder).  The forward and the backward use the same chunks."""
    vc = vocab_chunk(n_tokens, vocab, elem_bytes, chunk_vocab)
    plan = [(c0, min(vc, vocab - c0)) for c0 in range(0, vocab, vc)]
    wide = n_tokens * CHUNK_COLS_WIDE * elem_bytes <= CHUNK_WIDE_MAX_BYTES
    half = CHUNK_COLS_WIDE // 2
    if chunk_vocab is None and wide and plan and half + 1024 <= plan[-1][1] < CHUNK_COLS_WIDE:
        c0, n = plan[-1]
        plan[-1:] = [(c0, half), (c0 + half, n - half)]
    return plan


def _chunk_logits(buf, h2, weight, c0, n):
    """logits[:, c0:c0+n] = h2 @ weight[c0:c0+n]^T into a contiguous view of
    ``buf`` (the same call, hence the same values, in forward and backward)."""
    out = buf[: h2.size(0) * n].view(h2.size(0), n)
    torch.mm(h2, weight[c0:c0 + n].t(), out=out)
    return out


def _forward_chunked(h2, weight, t, T, plan, out):
    N = h2.size(0)
    n_chunks = len(plan)
    dev = h2.device
    states = torch.empty(n_chunks, N, 4, dtype=torch.float32, device=dev)
    buf = torch.empty(N * max(n for _, n in plan), dtype=h2.dtype, device=dev)
    code = DTYPE_CODES[h2.dtype]
    with device_guard(dev.index):
        stream = stream_handle(dev.index)
        for c, (c0, n) in enumerate(plan):
            lg = _chunk_logits(buf, h2, weight, c0, n)
            check_status(lib.klp_fwd_chunk(_ptr(lg), code, N, n, *_C.row_layout(lg), _ptr(t),
                                           c0, T, _ptr(states), c, n_chunks, _ptr(out[0]),
                                           _ptr(out[1]), _ptr(out[2]), stream))


def _backward_chunked(h2, weight, t, T, plan, lse, ent, gl, ge, gs, need_h, need_w, impl):
    """d_hidden (fp32, or None) and d_weight (weight dtype, or None), one
    vocabulary chunk of ``plan`` at a time: d_logits exist for one chunk
    only."""
    N, D, V = h2.size(0), h2.size(1), weight.size(0)
    dev = h2.device
    dh = torch.zeros(N, D, dtype=torch.float32, device=dev) if need_h else None
    dw = torch.empty(V, D, dtype=weight.dtype, device=dev) if need_w else None
    cols = max(n for _, n in plan)
    d_buf = torch.empty(N * (-(-cols // 4) * 4), dtype=weight.dtype, device=dev)
    lg_buf = torch.empty(N * cols, dtype=h2.dtype, device=dev) if impl == "chunked" else None
    with device_guard(dev.index):
        stream = stream_handle(dev.index)
        for c0, n in plan:
            tc = t - c0  # chunk-relative: a target outside the chunk adds no one-hot term
            if impl == "chunked":
                lg = _chunk_logits(lg_buf, h2, weight, c0, n)
                d = d_buf[: N * n].view(N, n)
                check_status(lib.klp_bwd_temp(_ptr(lg), DTYPE_CODES[lg.dtype], N, n,
                                              *_C.row_layout(lg),
                                              _ptr(tc), T, _ptr(lse), _ptr(ent), _ptr(gl),
                                              _ptr(ge), _ptr(gs), _ptr(d), stream))
            else:
                ld_d = -(-n // 4) * 4
                dpad = d_buf[: N * ld_d].view(N, ld_d)
                w_c = weight[c0:c0 + n]
                check_status(lib.klp_lmh_bwd_logits(
                    _ptr(h2), _ld(h2), _ptr(w_c), _ld(weight), N, n, D, _ptr(tc), T, _ptr(lse),
                    _ptr(ent), _ptr(gl), _ptr(ge), _ptr(gs), _ptr(dpad), ld_d, stream))
                d = dpad[:, :n]
            w_c = weight[c0:c0 + n]
            if need_h:
                _accumulate_f32(dh, d, w_c)
            if need_w:
                torch.mm(d.t(), h2, out=dw[c0:c0 + n])
    return dh, dw


class _FusedLinearLogprobEntropy(torch.autograd.Function):

    @staticmethod
    def forward(ctx, hidden, weight, targets, temperature, impl, chunk_vocab):
        outs = fused_linear_logprob_entropy_forward(hidden, weight, targets, temperature,
                                                    impl=impl, chunk_vocab=chunk_vocab)
        ctx.save_for_backward(hidden, weight, targets, outs[2], outs[1])
        ctx.temperature = temperature
        ctx.impl = impl
        ctx.chunk_vocab = chunk_vocab
        ctx.set_materialize_grads(False)
        return outs

    @staticmethod
    def backward(ctx, g_logp, g_ent, g_lse):
        hidden, weight, targets, lse, ent = ctx.saved_tensors
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        none = (None,) * 4
        if not (need_h or need_w):
            return (None, None) + none
        h2, t = _check(hidden, weight, targets, ctx.impl)
        N, V = h2.size(0), weight.size(0)
        if N == 0:
            return (torch.zeros_like(hidden) if need_h else None,
                    torch.zeros_like(weight) if need_w else None) + none

        def prep(g):
            return None if g is None else g.to(torch.float32, copy=False).reshape(-1).contiguous()

        T = 1.0 if ctx.temperature is None else float(ctx.temperature)
        plan = vocab_chunks(N, V, h2.element_size(), ctx.chunk_vocab)
        dh, dw = _backward_chunked(h2, weight, t, T, plan, lse.reshape(-1), ent.reshape(-1),
                                   prep(g_logp), prep(g_ent), prep(g_lse), need_h, need_w,
                                   ctx.impl)
        if dh is not None:
            dh = dh.to(hidden.dtype).reshape(hidden.shape)
        return (dh, dw) + none


def fused_linear_logprob_entropy(hidden: torch.Tensor, weight: torch.Tensor,
                                 targets: torch.Tensor, temperature: float | None = None, *,
                                 impl: str = "chunked", chunk_vocab: int | None = None):
    """Autograd-aware LM head + logprob / entropy: gradients flow to
    ``hidden`` and ``weight`` (see :func:`fused_linear_logprob_entropy_forward`
    for the arguments and the module docstring for the backward)."""
    return _FusedLinearLogprobEntropy.apply(hidden, weight, targets, temperature, impl,
                                            chunk_vocab)


def fused_linear_logprob_entropy_forward(hidden: torch.Tensor, weight: torch.Tensor,
                                         targets: torch.Tensor,
                                         temperature: float | None = None, *,
                                         impl: str = "chunked",
                                         chunk_vocab: int | None = None):
    """Args:
        hidden: ``[..., D]`` on the GPU, rows with unit stride (the leading
            dims must flatten to one stride).
        weight: ``[V, D]`` (an ``nn.Linear`` weight) of hidden's dtype, rows
            with unit stride.
        targets: ``[...]`` int64, same leading shape as ``hidden``.
        temperature: optional T > 0; logits are multiplied by fp32(1/T).
        impl: ``"chunked"`` (bf16 / fp16 / fp32) or ``"mfma"`` (bf16, D a
            multiple of 64, both row strides multiples of 8).
        chunk_vocab: columns per vocabulary chunk (chunked head, and the
            backward of both); default :func:`vocab_chunks`.

    Returns ``(logprob, entropy, lse)``, float32, shaped like ``targets``.
    """
    h2, t = _check(hidden, weight, targets, impl)
    D = h2.size(1)
    N, V = h2.size(0), weight.size(0)
    out = [torch.empty(targets.shape, dtype=torch.float32, device=hidden.device)
           for _ in range(3)]
    if N == 0:
        return tuple(out)
    T = 1.0 if temperature is None else float(temperature)
    if not (T > 0.0 and T != float("inf")):
        raise RuntimeError(f"temperature must be finite and > 0, got {T}")
    if impl == "chunked":
        _forward_chunked(h2, weight, t, T, vocab_chunks(N, V, h2.element_size(), chunk_vocab),
                         out)
        return tuple(out)
    dev = hidden.device
    with device_guard(dev.index):
        stream = stream_handle(dev.index)
        ws = _workspace(dev, stream, lib.klp_lmh_workspace_bytes(N, V, D))
        rc = lib.klp_lmh_fwd(_ptr(h2), _ld(h2), _ptr(weight), _ld(weight),
                             N, V, D, _ptr(t), T, _ptr(out[0]), _ptr(out[1]), _ptr(out[2]),
                             _ptr(ws), ws.numel(), stream)
    check_status(rc)
    return tuple(out)
