"""The gradient checker used by the GPU tests, exercised on the CPU with
known answers: the oracle's own rounded gradient passes, a 2-ulp error on an
element fails, and a cancellation-dominated element is judged against fp32
evaluation noise rather than its own (tiny) ulp."""
import numpy as np
import torch

from klp_testutil import grad_check, seeded_logits, seeded_targets


def _setup(dtype, V=300, N=4):
    x = seeded_logits((N, V), dtype, seed=5)
    t = seeded_targets((N,), V, seed=5)
    return x, t


def _fwd(oracle, x, t):
    lp, h, l = oracle.forward(x, t.numpy())
    return torch.tensor(l, dtype=torch.float32), torch.tensor(h, dtype=torch.float32)


def test_exact_rounding_passes_and_two_ulps_fail(oracle):
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        x, t = _setup(dtype)
        lse, ent = _fwd(oracle, x, t)
        gl = torch.full((4,), 0.7)
        d_ref = oracle.backward(x, t.numpy(), lse.numpy(), ent.numpy(), g_logp=gl.numpy())
        d = torch.from_numpy(d_ref).to(dtype)  # torch's RNE rounding of the float64 values
        worst, _ = grad_check(oracle, x, t, lse, ent, d, g_logp=gl)
        assert worst <= 1.0, (dtype, worst)
        # push the largest non-target element 2 ulps away (16-bit dtypes), or
        # by 1e-5 relative (fp32, whose bar allows exp-argument rounding)
        j = int(np.argsort(-np.abs(d_ref[0]))[1])
        bad = d.clone()
        if dtype == torch.float32:
            bad[0, j] = bad[0, j] * (1 + 1e-5)
        else:
            bits = bad.view(torch.int16)
            bits[0, j] += 2
        worst_bad, _ = grad_check(oracle, x, t, lse, ent, bad, g_logp=gl)
        assert worst_bad > 1.0, (dtype, worst_bad)


def test_cancellation_uses_fp32_noise(oracle):
    """V = 1: d = p*(g_lse - g_logp) + g_logp with p = 1, exactly 0; an fp32
    evaluation leaves ~1e-8 of noise, which must pass, while 1e-3 must not."""
    x = torch.tensor([[3.0]])
    t = torch.tensor([0])
    lse, ent = torch.tensor([3.0]), torch.tensor([0.0])
    gl = torch.tensor([0.3])
    ok = torch.tensor([[1.5e-8]])
    assert grad_check(oracle, x, t, lse, ent, ok, g_logp=gl)[0] <= 1.0
    bad = torch.tensor([[1e-3]])
    assert grad_check(oracle, x, t, lse, ent, bad, g_logp=gl)[0] > 1.0
