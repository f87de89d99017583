"""Randomised GPU parity of the logprob op (forward and backward) against the
float64 oracle, through the public entry point.

Each case draws, from a fixed seed (reproducible; the case is printed on
failure): the dtype; the batch shape (1-3 leading dims); the vocabulary
(1 to 70 000, odd sizes included); the row layout on the GPU (contiguous, the
shifted slice [..., :-1, :] of a longer tensor, rows narrowed from wider ones,
rows starting one element past a 16-byte boundary); the logit scale; a
temperature or none; which upstream gradients the loss uses.  Targets include
both ends of the row and one out of range; a few logits are -inf (never a
row's target) and one row has all logits equal.  Bars: the north-star forward
tolerance (1e-5 fp32, 2e-5 bf16 / fp16 inputs) and the gradient bar of
oracle/checks.py (1 ulp of the output dtype, or the fp32 evaluation noise
where the exact value is a cancellation).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from klp_testutil import FWD_TOL, grad_check

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = (torch.bfloat16, torch.float16, torch.float32)
VOCABS = (1, 2, 7, 8, 9, 31, 64, 100, 257, 1000, 4097, 8192, 12289, 32000, 50257, 70000)


def draw_case(seed):
    r = np.random.default_rng(seed)
    nd = int(r.integers(1, 4))
    layout = str(r.choice(["contiguous", "shifted", "narrowed", "offset"]))
    return dict(seed=seed,
                dtype=DTYPES[int(r.integers(3))],
                V=int(r.choice(VOCABS)),
                lead=[int(r.integers(1, 6)) for _ in range(nd)],
                layout="contiguous" if layout == "shifted" and nd < 2 else layout,
                scale=float(r.choice([0.5, 2.0, 4.0])),
                temperature=None if r.random() < 0.5 else float(r.choice([0.6, 1.0, 1.7])),
                grads=str(r.choice(["all", "logp", "ent", "lse", "logp+ent"])))


def build_rows(case):
    """The case's logits as contiguous CPU rows [n, V], and targets [n]."""
    g = torch.Generator().manual_seed(case["seed"])
    V, n = case["V"], int(np.prod(case["lead"]))
    x = (torch.randn(n, V, generator=g) * case["scale"]).to(case["dtype"])
    t = torch.randint(0, V, (n,), generator=g)
    t[0] = V - 1
    if n > 1:
        t[1] = 0
    if n > 2:
        t[2] = -1 if case["seed"] % 2 else V
    if V > 1:
        # -inf logits, never at a row's (clamped) target, so no row is all -inf
        for k in torch.randint(0, n * V, (max(1, n * V // 997),), generator=g).tolist():
            i, j = divmod(k, V)
            if j != int(t[i].clamp(0, V - 1)):
                x[i, j] = float("-inf")
    if n > 3:
        x[3] = 1.25
    return x, t


def to_device_layout(case, rows):
    """(leaf, view): a device tensor in the case's layout holding `rows`, and
    the [*lead, V] view of it that the op is given."""
    lead, V, n = case["lead"], case["V"], rows.size(0)
    rv = rows.view(*lead, V)
    if case["layout"] == "shifted":
        full = torch.zeros(*lead[:-1], lead[-1] + 1, V, dtype=rows.dtype)
        full[..., :-1, :] = rv
        leaf = full.to(DEV).requires_grad_(True)
        return leaf, leaf[..., :-1, :]
    if case["layout"] == "narrowed":
        full = torch.zeros(*lead, V + 5, dtype=rows.dtype)
        full[..., 3:3 + V] = rv
        leaf = full.to(DEV).requires_grad_(True)
        return leaf, leaf[..., 3:3 + V]
    if case["layout"] == "offset":
        flat = torch.zeros(n * V + 1, dtype=rows.dtype)
        flat[1:] = rows.reshape(-1)
        leaf = flat.to(DEV).requires_grad_(True)
        return leaf, leaf[1:].view(*lead, V)
    leaf = rv.to(DEV).requires_grad_(True)
    return leaf, leaf


def grad_rows(case, leaf):
    """The gradient of the op's input, as [n, V] rows, from the leaf's."""
    V, d = case["V"], leaf.grad
    if case["layout"] == "shifted":
        d = d[..., :-1, :]
    elif case["layout"] == "narrowed":
        d = d[..., 3:3 + V]
    elif case["layout"] == "offset":
        d = d[1:]
    return d.reshape(-1, V)


def _f64(z):
    return z.detach().double().cpu().numpy().reshape(-1)


@pytest.mark.parametrize("seed", range(60))
def test_random_case(seed, oracle):
    from kernel_opt import fused_logprob_entropy
    case = draw_case(1000 + seed)
    rows, t = build_rows(case)
    n, V, T = rows.size(0), case["V"], case["temperature"]
    leaf, xd = to_device_layout(case, rows)
    td = t.view(*case["lead"]).to(DEV)
    gen = torch.Generator().manual_seed(case["seed"] + 1)
    gl, ge, gs = (torch.randn(n, generator=gen) for _ in range(3))
    use = case["grads"]
    with_l = "logp" in use or use == "all"
    with_e = "ent" in use or use == "all"
    with_s = use in ("lse", "all")

    lp, ent, lse = fused_logprob_entropy(xd, td, T)
    loss = torch.zeros((), device=DEV)
    if with_l:
        loss = loss + (lp.reshape(-1) * gl.to(DEV)).sum()
    if with_e:
        loss = loss + (ent.reshape(-1) * ge.to(DEV)).sum()
    if with_s:
        loss = loss + (lse.reshape(-1) * gs.to(DEV)).sum()
    loss.backward()
    torch.cuda.synchronize()

    label = f"case {case}"
    ref = oracle.forward(rows, t.numpy(), temperature=T)
    tol = FWD_TOL[case["dtype"]]
    for name, o, rv in zip(("logp", "entropy", "lse"), (lp, ent, lse), ref):
        got = _f64(o)
        same_inf = np.isinf(got) & np.isinf(rv) & (np.sign(got) == np.sign(rv))
        err = np.where(same_inf, 0.0, np.abs(got - rv))
        assert np.all(err <= tol), f"{label}: {name} max err {np.nanmax(err):.3g}"

    worst, detail = grad_check(oracle, rows, t, lse.reshape(-1), ent.reshape(-1),
                               grad_rows(case, leaf), g_logp=gl if with_l else None,
                               g_ent=ge if with_e else None, g_lse=gs if with_s else None,
                               temperature=T)
    assert worst <= 1.0, f"{label}: gradient {detail}"
