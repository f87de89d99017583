"""The compiled binding (binding/klp_torch.cpp) on the CPU: it loads, exports
the reference's _C names and the ops entry points, computes the same row
addressing as the Python shim, and raises the reference's exception types
(AssertionError from the ops asserts, RuntimeError from the _C checks)
before touching the GPU."""
from __future__ import annotations

import pytest
import torch


def _binding():
    from kernel_opt._library import binding
    return binding


def test_exports():
    b = _binding()
    for name in ("fused_logprob_entropy_v1", "fused_logprob_entropy_naive",
                 "fused_logprob_entropy_v1_backward", "fwd_launch", "bwd_launch",
                 "fused_logprob_entropy", "fused_logprob_entropy_forward",
                 "fused_logprob_entropy_naive_op", "row_layout", "workspaces_cached",
                 "fused_grpo_loss", "fused_grpo_step"):
        assert callable(getattr(b, name)), name
    assert issubclass(b.InputAssertionError, AssertionError)


def _views():
    x = torch.zeros(4, 6, 10)
    y = torch.zeros(3, 5, 7, 9)
    return [x, x[:, :-1, :], x[:, 1:, :], x[1], x[:2, :3], x[:, :, :5], x[:, ::2, :],
            x[::2], x[:, 2], x[0, 0], x[:1], x[:, :1], x.transpose(0, 1), x[..., ::2],
            y, y[:, :, :-1, :], y[:, 1:, 1:, :], y[1:2, :, ::3, :], torch.zeros(0, 5),
            torch.zeros(1, 7), torch.zeros(7), torch.zeros(2, 1, 3)]


def test_row_layout_matches_python_shim():
    from kernel_opt import _C
    b = _binding()
    for i, v in enumerate(_views()):
        assert b.row_layout(v) == _C.row_layout(v), (i, tuple(v.shape), v.stride())
    assert b.row_layout(torch.tensor(1.0)) is None


def test_ops_entry_points_assert_on_cpu_tensors():
    b = _binding()
    x = torch.zeros(2, 8)
    t = torch.zeros(2, dtype=torch.int64)
    for f in (b.fused_logprob_entropy, b.fused_logprob_entropy_forward,
              b.fused_logprob_entropy_naive_op):
        with pytest.raises(AssertionError):
            f(x, t)


def test_c_entry_points_raise_reference_messages():
    b = _binding()
    x = torch.zeros(2, 8)
    t = torch.zeros(2, dtype=torch.int64)
    o = [torch.zeros(2) for _ in range(3)]
    with pytest.raises(RuntimeError, match="logits must be CUDA"):
        b.fused_logprob_entropy_v1(x, t, *o)
    with pytest.raises(RuntimeError, match="logits must be CUDA"):
        b.fwd_launch(x, t, *o, 0.7)
    with pytest.raises(RuntimeError, match="logits must be contiguous CUDA"):
        b.fused_logprob_entropy_v1_backward(x, t, o[0], o[1], None, None, None, x)
    with pytest.raises(RuntimeError, match="logits must be contiguous CUDA"):
        b.bwd_launch(x, t, o[0], o[1], None, None, None, x, None)


def test_grpo_loss_errors_before_the_gpu():
    """The GRPO loss through the binding raises what grpo.py's Python
    statement raises, for the checks that need no GPU."""
    from kernel_opt import fused_grpo_loss
    b = _binding()
    lp = torch.zeros(2, 3)
    adv = torch.zeros(2)
    args = (1.0, 0.2, 0.2, 0.0, 1.0, 0, 0)
    with pytest.raises(RuntimeError, match=r"logp must be \[B, S\], got shape \(6,\)"):
        b.fused_grpo_loss(lp.reshape(-1), lp, adv, None, None, *args[1:5], 0, 0)
    with pytest.raises(RuntimeError, match="logp must be a GPU tensor"):
        b.fused_grpo_loss(lp, lp, adv, None, None, *args[1:5], 0, 0)
    with pytest.raises(RuntimeError, match="logp must be a GPU tensor"):
        fused_grpo_loss(lp, lp, adv)
    with pytest.raises(RuntimeError, match=r"logp must be \[B, S\]"):
        fused_grpo_loss(lp.reshape(-1), lp, adv)
    with pytest.raises(TypeError, match="mask must be a tensor"):
        fused_grpo_loss(lp, lp, adv, mask=[1, 0])
    with pytest.raises(ValueError, match="loss_type"):
        fused_grpo_loss(lp, lp, adv, loss_type="nope")
