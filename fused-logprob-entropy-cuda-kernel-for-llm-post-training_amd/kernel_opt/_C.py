"""``kernel_opt._C`` — the reference's pybind11 module, restated over the C ABI.

Same three functions, same argument order and out-parameter convention as
the reference's ``csrc/bindings.cpp:17-27``:

* ``fused_logprob_entropy_naive(logits, targets, logprob, entropy, lse_out)``
* ``fused_logprob_entropy_v1(logits, targets, logprob, entropy, lse_out)``
* ``fused_logprob_entropy_v1_backward(logits, targets, lse, entropy,
  g_logp, g_ent, g_lse, d_logits)``

Tensor checks raise ``RuntimeError`` with the reference's ``TORCH_CHECK``
messages (``csrc/fused_logprob.cu:294-311,362-374,412-424``).  Differences:

* ``logits`` need not be contiguous: any tensor whose last dim has unit
  stride and whose rows are reachable through at most two leading strides is
  accepted (e.g. the shifted slice ``logits[:, :-1, :]``); anything else
  still raises "logits must be contiguous".
* In the backward, ``g_logp``/``g_ent``/``g_lse`` may be ``None`` (an all-zero
  upstream gradient), so callers need not materialise zero tensors.
* Work runs on the current stream of ``logits``' device, with that device
  made current for the call.

The three functions, and ``fwd_launch`` / ``bwd_launch`` without a pinned
launch shape, are the compiled binding's (``binding/klp_torch.cpp``, loaded
as ``_library.binding``): the checks, workspace and launch in C++, a few us
of host time per call.  A pinned launch shape (the tuning ABI, for sweeps and
tests) goes through ctypes, and so does every call while the current stream
is being captured into a graph (the binding declines those with
``binding.CaptureDeclined`` before it allocates or launches anything).
"""
from __future__ import annotations

import collections
import ctypes
import threading

import torch

from ._library import (DTYPE_CODES, binding, capturing, check_status, device_guard,
                       keep_for_capture, lib, ptr, stream_handle)

__all__ = [
    "fused_logprob_entropy_naive",
    "fused_logprob_entropy_v1",
    "fused_logprob_entropy_v1_backward",
    "row_layout",
    "fwd_launch",
    "bwd_launch",
    "default_config",
]


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def row_layout(t: torch.Tensor):
    """Return ``(rows_inner, stride_outer, stride_inner)`` addressing the rows
    of ``t`` (see include/kernel_opt_hip.h), or ``None`` when the rows cannot
    be reached with unit-stride rows and at most two leading strides."""
    if t.dim() == 0:
        return None
    if t.is_contiguous():
        # Fast path, same result as _row_layout_walk for two or more rows:
        # one run of rows V elements apart.
        V = t.size(-1)
        n = t.numel() // V if V else 0
        if n >= 2:
            return (n, 0, V)
    return _row_layout_walk(t)


def _row_layout_walk(t: torch.Tensor):
    """row_layout by merging the leading dims' strides (any tensor of rank
    >= 1)."""
    if t.size(-1) > 1 and t.stride(-1) != 1:
        return None
    dims = [(s, st) for s, st in zip(t.shape[:-1], t.stride()[:-1]) if s != 1]
    merged: list[list[int]] = []
    for size, stride in dims:
        if merged and merged[-1][1] == stride * size:
            merged[-1] = [merged[-1][0] * size, stride]
        else:
            merged.append([size, stride])
    n_rows = 1
    for s in t.shape[:-1]:
        n_rows *= s
    if not merged:
        return (max(n_rows, 1), 0, 0)
    if len(merged) == 1:
        return (merged[0][0], 0, merged[0][1])
    if len(merged) == 2:
        return (merged[1][0], merged[0][1], merged[1][1])
    return None


# Split-row workspaces (partial states), one per (device, stream) so that
# launches sharing one are ordered by their stream.  No initialisation needed.
# At most _WS_KEEP are kept, least recently used dropped first: each was
# allocated on its own stream, so the caching allocator hands a dropped one
# out again only in that stream's order, after the launches that used it.
_ws_lock = threading.Lock()
_workspaces: collections.OrderedDict = collections.OrderedDict()
_WS_KEEP = 16


def _workspace(device_index: int, stream: int, nbytes: int):
    """The workspace of (device, raw stream handle) holding at least
    ``nbytes``; the device must be current and ``stream`` its current
    stream.  Workspaces start zero-filled (by a fill kernel, not a memset),
    as the split-row forward needs; it leaves them zero.  Under graph
    capture every call gets a workspace of its own, kept for the life of the
    process: graphs captured on one stream would otherwise share one and race
    when replayed concurrently."""
    if nbytes == 0:
        return None
    if capturing():
        return keep_for_capture(
            torch.empty(nbytes, dtype=torch.uint8, device=device_index).zero_())
    key = (device_index, stream)
    with _ws_lock:
        buf = _workspaces.get(key)
        if buf is None or buf.numel() < nbytes:
            # Allocated on the stream that uses it (the caching allocator then
            # reuses it only in that stream's order).
            with torch.cuda.stream(torch.cuda.current_stream(device_index)):
                buf = torch.empty(nbytes, dtype=torch.uint8, device=device_index).zero_()
            _workspaces[key] = buf
        _workspaces.move_to_end(key)
        while len(_workspaces) > _WS_KEEP:
            _workspaces.popitem(last=False)
        return buf


_ptr = ptr


def _common_forward_checks(logits, targets, logprob, entropy, lse_out, per_output: bool):
    _require(logits.is_cuda, "logits must be CUDA")
    _require(targets.is_cuda, "targets must be CUDA")
    rows = row_layout(logits)
    _require(rows is not None, "logits must be contiguous")
    _require(targets.dtype == torch.int64, "targets must be int64")
    if per_output:
        _require(logprob.dtype == torch.float32, "logprob must be float32")
        _require(entropy.dtype == torch.float32, "entropy must be float32")
        _require(lse_out.dtype == torch.float32, "lse must be float32")
    else:
        _require(logprob.dtype == torch.float32 and entropy.dtype == torch.float32
                 and lse_out.dtype == torch.float32, "outputs must be float32")
    _require(logits.dtype in DTYPE_CODES, "logits dtype must be bf16, fp16, or fp32")
    V = logits.size(-1)
    _require(V > 0, "logits last dim (vocab) must be >= 1")
    N = logits.numel() // V
    _require(targets.numel() == N, "targets numel must match leading dims of logits")
    _require(logprob.numel() == N and entropy.numel() == N and lse_out.numel() == N,
             "output tensor numels must equal leading-dim count")
    _require(targets.is_contiguous(), "targets must be contiguous")
    _require(logprob.is_contiguous() and entropy.is_contiguous() and lse_out.is_contiguous(),
             "outputs must be contiguous")
    d = logits.get_device()
    _require(targets.get_device() == d and logprob.get_device() == d
             and entropy.get_device() == d and lse_out.get_device() == d,
             "all tensors must be on the device of logits")
    return rows, N, V


def _temperature(temperature, config):
    if temperature is None or float(temperature) == 1.0:
        return None
    _require(config is None, "a launch shape cannot be pinned together with a temperature")
    t = float(temperature)
    _require(t > 0.0 and t != float("inf"), f"temperature must be finite and > 0, got {t}")
    return t


def fwd_launch(logits, targets, logprob, entropy, lse_out, config=None, temperature=None) -> None:
    """Forward into caller-allocated outputs.  ``config`` = ``(waves, unroll,
    splits, flags)`` pins a launch shape (tuning ABI); ``None`` lets the
    native dispatcher choose.  ``temperature`` T divides the logits (as
    x * fp32(1/T)) inside the kernel."""
    if config is None:
        try:
            binding.fwd_launch(logits, targets, logprob, entropy, lse_out, temperature)
            return
        except binding.CaptureDeclined:
            pass
    rows, N, V = _common_forward_checks(logits, targets, logprob, entropy, lse_out, False)
    temp = _temperature(temperature, config)
    if N == 0:
        return
    code = DTYPE_CODES[logits.dtype]
    dev = logits.get_device()
    with device_guard(dev):
        stream = stream_handle(dev)
        if config is None:
            nbytes = lib.klp_fwd_workspace_bytes(code, N, V)
        else:
            nbytes = lib.klp_fwd_workspace_bytes_ex(N, int(config[2]))
        ws = _workspace(dev, stream, nbytes)
        args = [_ptr(logits), code, N, V, rows[0], rows[1], rows[2], _ptr(targets),
                _ptr(logprob), _ptr(entropy), _ptr(lse_out), _ptr(ws),
                0 if ws is None else ws.numel()]
        if temp is not None:
            rc = lib.klp_fwd_temp(*args[:8], temp, *args[8:], stream)
        elif config is None:
            rc = lib.klp_fwd(*args, stream)
        else:
            w, u, sp, fl = (int(c) for c in config)
            rc = lib.klp_fwd_ex(*args, w, u, sp, fl, stream)
    check_status(rc)


def fused_logprob_entropy_v1(logits, targets, logprob, entropy, lse_out) -> None:
    """Production forward (reference csrc/fused_logprob.cu:355-403)."""
    fwd_launch(logits, targets, logprob, entropy, lse_out)


def fused_logprob_entropy_naive(logits, targets, logprob, entropy, lse_out) -> None:
    """Naive forward, one thread per row (reference csrc/fused_logprob.cu:405-458)."""
    try:
        binding.fused_logprob_entropy_naive(logits, targets, logprob, entropy, lse_out)
        return
    except binding.CaptureDeclined:
        pass
    rows, N, V = _common_forward_checks(logits, targets, logprob, entropy, lse_out, True)
    if N == 0:
        return
    dev = logits.get_device()
    with device_guard(dev):
        rc = lib.klp_fwd_naive(_ptr(logits), DTYPE_CODES[logits.dtype], N, V, rows[0], rows[1],
                               rows[2], _ptr(targets), _ptr(logprob), _ptr(entropy),
                               _ptr(lse_out), stream_handle(dev))
    check_status(rc)


def _backward_checks(logits, targets, lse, entropy, g_logp, g_ent, g_lse, d_logits):
    _require(logits.is_cuda, "logits must be contiguous CUDA")
    rows = row_layout(logits)
    _require(rows is not None, "logits must be contiguous CUDA")
    _require(targets.dtype == torch.int64, "targets must be int64")
    _require(lse.dtype == torch.float32 and entropy.dtype == torch.float32,
             "saved lse / entropy must be fp32")
    grads = [g for g in (g_logp, g_ent, g_lse) if g is not None]
    _require(all(g.dtype == torch.float32 for g in grads), "upstream gradients must be fp32")
    _require(all(g.is_contiguous() for g in grads), "upstream gradients must be contiguous")
    _require(d_logits.dtype == logits.dtype and d_logits.is_contiguous()
             and d_logits.shape == logits.shape,
             "d_logits must match logits dtype/shape and be contiguous")
    _require(logits.dtype in DTYPE_CODES, "logits dtype must be bf16, fp16, or fp32")
    V = logits.size(-1)
    _require(V > 0, "logits last dim (vocab) must be >= 1")
    N = logits.numel() // V
    _require(targets.numel() == N and lse.numel() == N and entropy.numel() == N
             and all(g.numel() == N for g in grads), "leading-dim count mismatch")
    _require(targets.is_contiguous() and lse.is_contiguous() and entropy.is_contiguous(),
             "targets / saved lse / entropy must be contiguous")
    d = logits.get_device()
    _require(all(t.get_device() == d for t in [targets, lse, entropy, d_logits] + grads),
             "all tensors must be on the device of logits")
    return rows, N, V


def bwd_launch(logits, targets, lse, entropy, g_logp, g_ent, g_lse, d_logits,
               config=None, temperature=None) -> None:
    """Backward into caller-allocated ``d_logits``; ``config`` and
    ``temperature`` as in fwd_launch (the gradient is with respect to the
    unscaled logits)."""
    if config is None:
        try:
            binding.bwd_launch(logits, targets, lse, entropy, g_logp, g_ent, g_lse, d_logits,
                               temperature)
            return
        except binding.CaptureDeclined:
            pass
    rows, N, V = _backward_checks(logits, targets, lse, entropy, g_logp, g_ent, g_lse, d_logits)
    temp = _temperature(temperature, config)
    if N == 0:
        return
    dev = logits.get_device()
    with device_guard(dev):
        stream = stream_handle(dev)
        args = [_ptr(logits), DTYPE_CODES[logits.dtype], N, V, rows[0], rows[1], rows[2],
                _ptr(targets), _ptr(lse), _ptr(entropy), _ptr(g_logp), _ptr(g_ent),
                _ptr(g_lse), _ptr(d_logits)]
        if temp is not None:
            rc = lib.klp_bwd_temp(*args[:8], temp, *args[8:], stream)
        elif config is None:
            rc = lib.klp_bwd(*args, stream)
        else:
            w, u, sp, fl = (int(c) for c in config)
            rc = lib.klp_bwd_ex(*args, w, u, sp, fl, stream)
    check_status(rc)


def fused_logprob_entropy_v1_backward(logits, targets, lse, entropy, g_logp, g_ent, g_lse,
                                      d_logits) -> None:
    """Backward (reference csrc/fused_logprob.cu:284-346)."""
    bwd_launch(logits, targets, lse, entropy, g_logp, g_ent, g_lse, d_logits)


def default_config(which: str, dtype: torch.dtype, n_rows: int, vocab: int):
    """Launch shape ``(waves, unroll, splits, flags)`` the native
    dispatcher picks for the forward (``which="fwd"``) or backward."""
    out = [ctypes.c_int(0) for _ in range(4)]
    lib.klp_default_config(0 if which == "fwd" else 1, DTYPE_CODES[dtype], n_rows, vocab,
                           *[ctypes.byref(o) for o in out])
    return tuple(o.value for o in out)
