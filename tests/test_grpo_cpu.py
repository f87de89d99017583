"""CPU pins of the float64 GRPO-loss oracle (oracle/grpo_oracle.py).

The oracle's loss, statistics and hand-derived gradient are checked against
  * float64 torch autograd of the reference's own loss
    (examples/compare_one_step.py:232-236, restated verbatim in
    oracle/eager_ref.reference_grpo_loss);
  * float64 torch autograd of the eager restatement of every variant
    (oracle/eager_ref.eager_grpo_loss);
  * central finite differences;
  * closed forms (old == new gives ratio 1: loss = -sum(A m) / den).
Each planted mistake (`mutant`) must fail at least one of these.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from oracle import eager_ref
from oracle.grpo_oracle import grpo_loss


def make_case(B, S, seed, adv_per_token=False, zero_row=False, spread=0.4):
    g = np.random.default_rng(seed)
    new = g.normal(-2.0, 1.0, (B, S))
    old = new + g.normal(0.0, spread, (B, S))
    ref = new + g.normal(0.0, spread, (B, S))
    adv = g.normal(0.0, 1.0, (B, S) if adv_per_token else (B,))
    mask = (g.random((B, S)) < 0.7).astype(np.float64)
    if zero_row:
        mask[0] = 0.0
    return new, old, ref, adv, mask


def torch_eager(new, old, ref, adv, mask, **kw):
    t = lambda a: torch.tensor(a, dtype=torch.float64)
    lp = t(new).requires_grad_(True)
    loss, stats = eager_ref.eager_grpo_loss(lp, t(old), t(adv), t(mask),
                                            None if ref is None else t(ref), **kw)
    loss.backward()
    return loss.item(), stats.numpy(), lp.grad.numpy()


VARIANTS = list(itertools.product(("grpo", "bnpo", "fixed"), ("token", "sequence"),
                                  (0.0, 0.04), (False, True)))


def test_matches_reference_formula_and_autograd():
    """bnpo / token / symmetric eps / no KL is the reference's loss exactly."""
    new, old, _, adv, mask = make_case(6, 50, seed=1, adv_per_token=True)
    lp = torch.tensor(new, requires_grad=True)
    ref_loss = eager_ref.reference_grpo_loss(lp, torch.tensor(old), torch.tensor(adv),
                                             torch.tensor(mask), 0.2)
    ref_loss.backward()
    loss, _, grad = grpo_loss(new, old, adv, mask, eps_low=0.2, loss_type="bnpo")
    assert abs(loss - ref_loss.item()) <= 1e-12 * max(1.0, abs(loss))
    np.testing.assert_allclose(grad, lp.grad.numpy(), rtol=1e-12, atol=1e-15)


@pytest.mark.parametrize("loss_type,level,beta,adv_tok", VARIANTS)
def test_matches_eager_autograd(loss_type, level, beta, adv_tok):
    new, old, ref, adv, mask = make_case(5, 40, seed=2, adv_per_token=adv_tok, zero_row=True)
    kw = dict(eps_low=0.2, eps_high=0.28, beta=beta, loss_type=loss_type, level=level,
              norm_const=123.0)
    e_loss, e_stats, e_grad = torch_eager(new, old, ref, adv, mask, **kw)
    loss, stats, grad = grpo_loss(new, old, adv, mask, ref, **kw)
    assert abs(loss - e_loss) <= 1e-12 * max(1.0, abs(loss))
    np.testing.assert_allclose(stats, e_stats, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(grad, e_grad, rtol=1e-11, atol=1e-15)


@pytest.mark.parametrize("loss_type,level", [("grpo", "token"), ("bnpo", "sequence"),
                                             ("fixed", "token")])
def test_gradient_matches_finite_differences(loss_type, level):
    new, old, ref, adv, mask = make_case(3, 7, seed=3)
    kw = dict(eps_low=0.2, eps_high=0.3, beta=0.05, loss_type=loss_type, level=level,
              norm_const=10.0)
    _, _, grad = grpo_loss(new, old, adv, mask, ref, **kw)
    h = 1e-6
    fd = np.zeros_like(new)
    for idx in np.ndindex(new.shape):
        up, dn = new.copy(), new.copy()
        up[idx] += h
        dn[idx] -= h
        fd[idx] = (grpo_loss(up, old, adv, mask, ref, **kw)[0]
                   - grpo_loss(dn, old, adv, mask, ref, **kw)[0]) / (2 * h)
    np.testing.assert_allclose(grad, fd, rtol=1e-6, atol=1e-9)


def test_closed_form_ratio_one():
    """old == new: every ratio is 1 (inside the clip range), no KL."""
    g = np.random.default_rng(4)
    new = g.normal(-1.0, 1.0, (4, 9))
    adv = g.normal(0.0, 1.0, (4,))
    mask = (g.random((4, 9)) < 0.6).astype(np.float64)
    loss, stats, grad = grpo_loss(new, new, adv, mask, loss_type="bnpo")
    den = max(mask.sum(), 1.0)
    assert loss == pytest.approx(-(adv[:, None] * mask).sum() / den, rel=1e-14)
    np.testing.assert_allclose(grad, -adv[:, None] * mask / den, rtol=1e-14)
    assert stats[1] == stats[2] == stats[3] == 0.0


def test_clipped_tokens_have_no_ratio_gradient():
    # A > 0 and ratio far above 1 + eps: the clamped term is the min, no gradient
    new = np.full((1, 3), -1.0)
    old = new - 1.0          # ratio = e
    loss, stats, grad = grpo_loss(new, old, np.array([2.0]), loss_type="bnpo")
    assert np.all(grad == 0.0)
    assert loss == pytest.approx(-1.2 * 2.0)
    assert stats[2] == 1.0 and stats[1] == 0.0


@pytest.mark.parametrize("mutant", [1, 2, 3, 4, 5])
def test_planted_mistakes_are_caught(mutant):
    caught = []
    for loss_type, level, beta, adv_tok in VARIANTS:
        new, old, ref, adv, mask = make_case(5, 40, seed=2, adv_per_token=adv_tok,
                                             zero_row=True, spread=0.6)
        kw = dict(eps_low=0.2, eps_high=0.28, beta=beta, loss_type=loss_type, level=level,
                  norm_const=123.0)
        e_loss, e_stats, e_grad = torch_eager(new, old, ref, adv, mask, **kw)
        with np.errstate(all="ignore"):
            loss, stats, grad = grpo_loss(new, old, adv, mask, ref, mutant=mutant, **kw)
        ok = (abs(loss - e_loss) <= 1e-12 * max(1.0, abs(e_loss))
              and np.allclose(stats, e_stats, rtol=1e-12, atol=1e-15)
              and np.allclose(grad, e_grad, rtol=1e-11, atol=1e-15))
        caught.append(not ok)
    assert any(caught), f"mutant {mutant} passes every pin"
