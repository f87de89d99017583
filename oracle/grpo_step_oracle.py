"""float64 oracle of the fused GRPO step (klp_grpo_step.hip).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the fused
step.  The product never imports it.

The fused step is the chain rule through two pinned oracles:
  1. per-token logprob / entropy / lse of the logits: the C oracle
     (klp_oracle.c), which restates the reference kernel
     csrc/fused_logprob.cu:114-241;
  2. the GRPO loss of those log-probabilities and its gradient g = d loss /
     d logp: grpo_oracle.grpo_loss (examples/compare_one_step.py:232-236,
     generalised as in include/kernel_opt_hip.h);
  3. d loss / d logits = the logprob backward with upstream g_logp = g and
     g_ent = g_lse = 0: the C oracle's backward (csrc/fused_logprob.cu:
     243-282).
Pinned (tests/test_grpo_step_cpu.py): the composed gradient against float64
torch autograd of the eager pipeline (log_softmax, gather, the eager loss)
and against central finite differences of the composed loss; `mutant`
plants a mistake in the composition for the tests that show those pins
catch it.
"""
from __future__ import annotations

import numpy as np

from . import grpo_oracle, klp_oracle


def grpo_step(logits, targets, old_logp, advantages, mask=None, ref_logp=None, *,
              eps_low=0.2, eps_high=None, beta=0.0, loss_type="bnpo", norm_const=1.0,
              dtype=None, temperature=None, mutant=0):
    """Returns (loss, logp, entropy, d_logits, stats), float64.

    logits: [B, S, V] storage (as klp_oracle accepts); targets int64 [B, S].
    mutant: 0 none; 1 the entropy gradient is fed into the logprob backward
    (g_ent = g instead of 0); 2 the upstream gradient is taken as g_lse
    instead of g_logp.
    """
    o = klp_oracle.get()
    logp, ent, lse = o.forward(logits, targets, dtype, temperature=temperature)
    loss, stats, g = grpo_oracle.grpo_loss(logp, old_logp, advantages, mask, ref_logp,
                                           eps_low=eps_low, eps_high=eps_high, beta=beta,
                                           loss_type=loss_type, level="token",
                                           norm_const=norm_const)
    if mutant == 1:
        d = o.backward(logits, targets, lse, ent, g_logp=g, g_ent=g, dtype=dtype,
                       temperature=temperature)
    elif mutant == 2:
        d = o.backward(logits, targets, lse, ent, g_lse=g, dtype=dtype, temperature=temperature)
    else:
        d = o.backward(logits, targets, lse, ent, g_logp=g, dtype=dtype, temperature=temperature)
    return loss, logp, ent, d, stats


def token_weights(mask, B, S, loss_type="bnpo", norm_const=1.0):
    """float64 weight of each token's loss in the batch loss (mask over the
    loss type's normaliser)."""
    m = np.ones((B, S)) if mask is None else np.asarray(mask, np.float64)
    if loss_type == "grpo":
        return m / (B * np.maximum(m.sum(1, keepdims=True), 1.0))
    if loss_type == "bnpo":
        return m / max(m.sum(), 1.0)
    if loss_type == "fixed":
        return m / norm_const
    raise ValueError(loss_type)
