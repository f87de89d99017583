"""float64 numpy restatement of the GRPO policy loss and its gradient.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the HIP
kernels in klp_grpo.hip.  The product never imports it.

Follows the reference's loss, examples/compare_one_step.py:232-236:
    ratio = (new_logp - old).exp()
    surr = -min(ratio * A, ratio.clamp(1 - eps, 1 + eps) * A)
    loss = (surr * mask).sum() / mask.sum()
generalised as documented in include/kernel_opt_hip.h (klp_grpo_fwd):
separate eps_low / eps_high, the KL term beta * (exp(r - lp) - (r - lp) - 1),
sequence-level importance weights, and the "grpo" / "bnpo" / fixed
normalisers.  The gradient is derived by hand, with PyTorch's conventions
for the eager expression (a tie of min() sends half the gradient to each
side; clamp() passes the gradient on its closed interval).

Pinned (tests/test_grpo_cpu.py): loss and gradient against float64 torch
autograd of the reference's own formula and of an eager restatement of every
variant (oracle/eager_ref.py), against finite differences, and against
closed forms (old == new gives ratio 1; the clip region has zero ratio
gradient).  `mutant` plants one mistake each, for the tests that show those
pins catch it.
"""
from __future__ import annotations

import numpy as np

LOSS_TYPES = ("grpo", "bnpo", "fixed")


def grpo_loss(logp, old_logp, advantages, mask=None, ref_logp=None, *, eps_low=0.2,
              eps_high=None, beta=0.0, loss_type="bnpo", level="token", norm_const=1.0,
              mutant=0):
    """Returns (loss, stats[4], d loss / d logp) in float64.

    mutant: 0 none; 1 the upper clip bound uses eps_low; 2 the KL gradient
    loses its sign; 3 the "grpo" normaliser forgets the max(., 1) clamp;
    4 the clipped branch keeps the ratio gradient; 5 the sequence-level
    weight is the unmasked mean.
    """
    lp = np.asarray(logp, np.float64)
    lo = np.asarray(old_logp, np.float64)
    B, S = lp.shape
    m = np.ones((B, S)) if mask is None else np.asarray(mask, np.float64)
    A = np.asarray(advantages, np.float64)
    A = np.broadcast_to(A[:, None], (B, S)) if A.ndim == 1 else A
    eh = eps_low if eps_high is None else eps_high
    lo_b, hi_b = 1.0 - eps_low, 1.0 + (eps_low if mutant == 1 else eh)

    row_m = m.sum(1)
    if level == "sequence":
        if mutant == 5:
            w = np.broadcast_to(((lp - lo).sum(1) / S)[:, None], (B, S))
        else:
            w = np.broadcast_to((((lp - lo) * m).sum(1) / np.maximum(row_m, 1.0))[:, None],
                                (B, S))
    else:
        w = lp - lo
    c1 = np.exp(w)
    c2 = np.clip(c1, lo_b, hi_b)
    a, b = c1 * A, c2 * A
    da = c1 * A
    inside = (c1 >= lo_b) & (c1 <= hi_b)
    db = da if mutant == 4 else np.where(inside, da, 0.0)
    dmin = np.where(a < b, da, np.where(b < a, db, 0.5 * da + 0.5 * db))
    tok = -np.minimum(a, b)
    dw = -dmin
    kl = np.zeros((B, S))
    dkl = np.zeros((B, S))
    if ref_logp is not None and beta != 0.0:
        r = np.asarray(ref_logp, np.float64)
        d = r - lp
        kl = np.exp(d) - d - 1.0
        tok = tok + beta * kl
        dkl = beta * (np.exp(d) - 1.0) if mutant == 2 else beta * (1.0 - np.exp(d))

    total_m = m.sum()
    if loss_type == "grpo":
        den_row = row_m if mutant == 3 else np.maximum(row_m, 1.0)
        loss = ((tok * m).sum(1) / den_row).mean()
        scale = np.broadcast_to((1.0 / (B * den_row))[:, None], (B, S))
    elif loss_type == "bnpo":
        loss = (tok * m).sum() / max(total_m, 1.0)
        scale = np.full((B, S), 1.0 / max(total_m, 1.0))
    elif loss_type == "fixed":
        loss = (tok * m).sum() / norm_const
        scale = np.full((B, S), 1.0 / norm_const)
    else:
        raise ValueError(loss_type)

    if level == "sequence":
        # w is shared by the row: d loss / d lp_s = (sum_s' scale m dw) * m_s / max(row_m, 1)
        row_term = (scale * m * dw).sum(1) / np.maximum(row_m, 1.0)
        grad = row_term[:, None] * (np.ones((B, S)) if mutant == 5 else m) + dkl * m * scale
    else:
        grad = (dw + dkl) * m * scale

    den = max(total_m, 1.0)
    low = ((c1 < lo_b) & (A < 0)).astype(np.float64)
    high = ((c1 > hi_b) & (A > 0)).astype(np.float64)
    stats = np.array([(kl * m).sum() / den, (low * m).sum() / den, (high * m).sum() / den,
                      ((low + high) * m).sum() / den])
    return float(loss), stats, grad
