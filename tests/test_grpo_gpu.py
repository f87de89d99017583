"""GPU parity of the fused GRPO loss (klp_grpo.hip) against the float64
oracle (oracle/grpo_oracle.py, pinned in tests/test_grpo_cpu.py).

Bar: the fp32 kernels against the float64 oracle on the same float32
inputs: loss within 1e-5 of the scale of the summed terms, statistics within
1e-6, every gradient element within 1e-5 of the largest gradient magnitude
plus 1e-5 relative.  Repeated calls are bitwise identical.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from oracle.grpo_oracle import grpo_loss

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(B, S, seed, adv_per_token=False, zero_row=False, spread=0.4):
    g = np.random.default_rng(seed)
    new = g.normal(-2.0, 1.0, (B, S)).astype(np.float32)
    old = (new + g.normal(0.0, spread, (B, S))).astype(np.float32)
    ref = (new + g.normal(0.0, spread, (B, S))).astype(np.float32)
    adv = g.normal(0.0, 1.0, (B, S) if adv_per_token else (B,)).astype(np.float32)
    mask = (g.random((B, S)) < 0.7).astype(np.float32)
    if zero_row:
        mask[0] = 0.0
    return new, old, ref, adv, mask


def run(new, old, ref, adv, mask, **kw):
    from kernel_opt import fused_grpo_loss
    lp = torch.tensor(new, device=DEV, requires_grad=True)
    t = lambda a: None if a is None else torch.tensor(a, device=DEV)
    loss, stats = fused_grpo_loss(lp, t(old), t(adv), t(mask), t(ref), **kw)
    loss.backward()
    return loss.item(), stats.cpu().numpy(), lp.grad.cpu().numpy()


def check(new, old, ref, adv, mask, kw, okw):
    loss, stats, grad = run(new, old, ref, adv, mask, **kw)
    e_loss, e_stats, e_grad = grpo_loss(new, old, adv, mask, ref, **okw)
    assert abs(loss - e_loss) <= 1e-5 * max(1.0, abs(e_loss)), (loss, e_loss)
    np.testing.assert_allclose(stats, e_stats, rtol=0, atol=1e-6)
    gmax = np.abs(e_grad).max() if e_grad.size else 0.0
    err = np.abs(grad - e_grad)
    bound = 1e-5 * gmax + 1e-5 * np.abs(e_grad)
    assert np.all(err <= bound), f"grad err {err.max():.3g} (max |g| {gmax:.3g})"


VARIANTS = list(itertools.product(("grpo", "bnpo", "dr_grpo", "dapo"), ("token", "sequence"),
                                  (0.0, 0.04), (False, True)))


@pytest.mark.parametrize("loss_type,level,beta,adv_tok", VARIANTS)
def test_matches_oracle(loss_type, level, beta, adv_tok):
    B, S = 7, 333
    new, old, ref, adv, mask = case(B, S, seed=11, adv_per_token=adv_tok, zero_row=True)
    kw = dict(eps_low=0.2, eps_high=0.28, beta=beta, loss_type=loss_type,
              importance_level=level, max_completion_length=400, normalizer=1234.0)
    norm = {"dr_grpo": B * 400.0, "dapo": 1234.0}.get(loss_type, 1.0)
    okw = dict(eps_low=0.2, eps_high=0.28, beta=beta,
               loss_type=loss_type if loss_type in ("grpo", "bnpo") else "fixed",
               level=level, norm_const=norm)
    check(new, old, ref, adv, mask, kw, okw)


def test_reference_formula_defaults():
    """Defaults (bnpo, token level, eps 0.2 both ways, no KL) are the
    reference's loss (examples/compare_one_step.py:232-236)."""
    from oracle import eager_ref
    new, old, _, adv, mask = case(4, 300, seed=12, adv_per_token=True)
    loss, _, grad = run(new, old, None, adv, mask)
    lp = torch.tensor(new, dtype=torch.float64, requires_grad=True)
    e = eager_ref.reference_grpo_loss(lp, torch.tensor(old, dtype=torch.float64),
                                      torch.tensor(adv, dtype=torch.float64),
                                      torch.tensor(mask, dtype=torch.float64), 0.2)
    e.backward()
    assert abs(loss - e.item()) <= 1e-5 * max(1.0, abs(e.item()))
    g = lp.grad.numpy()
    assert np.all(np.abs(grad - g) <= 1e-5 * np.abs(g).max() + 1e-5 * np.abs(g))


@pytest.mark.parametrize("B,S", [(1, 1), (1, 5000), (64, 1), (16, 2048), (300, 17)])
def test_shapes(B, S):
    new, old, ref, adv, mask = case(B, S, seed=13 + B + S)
    check(new, old, ref, adv, mask, dict(beta=0.04, loss_type="grpo"),
          dict(beta=0.04, loss_type="grpo"))


def test_no_mask_and_all_masked():
    new, old, ref, adv, _ = case(3, 100, seed=14)
    check(new, old, ref, adv, None, dict(loss_type="bnpo"), dict(loss_type="bnpo"))
    zero = np.zeros((3, 100), np.float32)
    loss, stats, grad = run(new, old, ref, adv, zero, loss_type="grpo")
    assert loss == 0.0 and np.all(grad == 0.0) and np.all(stats == 0.0)


def test_bool_mask_and_upstream_gradient_scale():
    from kernel_opt import fused_grpo_loss
    new, old, ref, adv, mask = case(5, 64, seed=15)
    lp = torch.tensor(new, device=DEV, requires_grad=True)
    loss, _ = fused_grpo_loss(lp, torch.tensor(old, device=DEV), torch.tensor(adv, device=DEV),
                              torch.tensor(mask > 0, device=DEV))
    (3.0 * loss).backward()
    _, _, e_grad = grpo_loss(new, old, adv, mask)
    g = lp.grad.cpu().numpy()
    assert np.all(np.abs(g - 3.0 * e_grad) <= 1e-5 * np.abs(3.0 * e_grad).max()
                  + 1e-5 * np.abs(3.0 * e_grad))


def test_deterministic():
    new, old, ref, adv, mask = case(40, 1000, seed=16)
    outs = [run(new, old, ref, adv, mask, beta=0.04, loss_type="grpo") for _ in range(3)]
    for o in outs[1:]:
        assert o[0] == outs[0][0]
        assert np.array_equal(o[1], outs[0][1]) and np.array_equal(o[2], outs[0][2])


def test_empty_batch():
    from kernel_opt import fused_grpo_loss
    lp = torch.zeros(3, 0, device=DEV, requires_grad=True)
    loss, stats = fused_grpo_loss(lp, lp.detach(), torch.zeros(3, device=DEV))
    loss.backward()
    assert loss.item() == 0.0 and stats.shape == (4,) and lp.grad.shape == (3, 0)


def test_invalid_arguments_raise():
    from kernel_opt import fused_grpo_loss
    lp = torch.zeros(2, 3, device=DEV)
    adv = torch.zeros(2, device=DEV)
    with pytest.raises(RuntimeError, match="eps_low"):
        fused_grpo_loss(lp, lp, adv, eps_low=-0.1)
    with pytest.raises(ValueError, match="loss_type"):
        fused_grpo_loss(lp, lp, adv, loss_type="nope")
    with pytest.raises(ValueError, match="normalizer"):
        fused_grpo_loss(lp, lp, adv, loss_type="dapo")
    with pytest.raises(RuntimeError, match="shape"):
        fused_grpo_loss(lp, lp[:1], adv)
