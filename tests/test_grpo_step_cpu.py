"""CPU pins of the fused GRPO step's oracle (oracle/grpo_step_oracle.py) and
of the product's token weights.

The oracle composes the logprob oracle, the GRPO-loss oracle and the logprob
backward.  The composition is checked against
  * float64 torch autograd of the eager pipeline the fused step replaces
    (log_softmax, gather, oracle/eager_ref.eager_grpo_loss), with and
    without a temperature, for every loss type, with the KL term and with
    per-token advantages, ignore-index targets and masked tokens;
  * central finite differences of the composed loss;
and each planted mistake (`mutant`) must fail the autograd pin.
``grpo_token_weights`` (the product's float32 weights) is checked against
the float64 weights of the oracle.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from oracle import eager_ref
from oracle.grpo_step_oracle import grpo_step, token_weights

IGNORE = -100


def make_case(B, S, V, seed, adv_per_token=False):
    g = np.random.default_rng(seed)
    x = (g.normal(0.0, 2.0, (B, S, V))).astype(np.float32)
    t = g.integers(0, V, (B, S)).astype(np.int64)
    t[0, 1] = IGNORE
    mask = (g.random((B, S)) < 0.75).astype(np.float64)
    mask[0, 0] = 1.0
    adv = g.normal(0.0, 1.0, (B, S) if adv_per_token else (B,))
    return g, x, t, mask, adv


def eager_pipeline(x, t, old, adv, mask, ref, temperature=None, **kw):
    """float64 torch autograd of logits -> logp -> GRPO loss; returns
    (loss, d loss / d logits)."""
    s = 1.0 if temperature is None else float(np.float32(1.0 / temperature))
    # The kernels' scaled logit fp32(x * fp32(1/T)), then float64.
    xs = torch.tensor((x * np.float32(s)).astype(np.float32), dtype=torch.float64,
                      requires_grad=True)
    tt = torch.tensor(t)
    valid = (tt >= 0) & (tt < x.shape[-1])
    lsm = torch.log_softmax(xs, dim=-1)
    picked = lsm.gather(-1, tt.clamp(0, x.shape[-1] - 1).unsqueeze(-1)).squeeze(-1)
    logp = torch.where(valid, picked, -torch.logsumexp(xs, dim=-1))
    f = lambda a: None if a is None else torch.tensor(a, dtype=torch.float64)
    loss, _ = eager_ref.eager_grpo_loss(logp, f(old), f(adv), f(mask), f(ref), **kw)
    loss.backward()
    return loss.item(), xs.grad.numpy() * s


def old_ref_from(oracle_logp, g):
    old = oracle_logp + g.normal(0.0, 0.3, oracle_logp.shape)
    ref = oracle_logp + g.normal(0.0, 0.3, oracle_logp.shape)
    return old, ref


CASES = list(itertools.product(("grpo", "bnpo", "fixed"), (0.0, 0.04), (False, True)))


@pytest.mark.parametrize("loss_type,beta,adv_tok", CASES)
@pytest.mark.parametrize("temperature", [None, 0.7])
def test_composition_matches_eager_autograd(loss_type, beta, adv_tok, temperature, oracle):
    g, x, t, mask, adv = make_case(3, 6, 41, seed=5, adv_per_token=adv_tok)
    lp0, _, _ = oracle.forward(x, t, "fp32", temperature=temperature)
    old, ref = old_ref_from(lp0, g)
    kw = dict(eps_low=0.2, eps_high=0.28, beta=beta, loss_type=loss_type, norm_const=37.0)
    loss, logp, _, d, _ = grpo_step(x, t, old, adv, mask, ref, temperature=temperature,
                                     dtype="fp32", **kw)
    e_loss, e_d = eager_pipeline(x, t, old, adv, mask, ref, temperature=temperature,
                                 eps_low=0.2, eps_high=0.28, beta=beta, loss_type=loss_type,
                                 norm_const=37.0)
    assert abs(loss - e_loss) <= 1e-12 * max(1.0, abs(e_loss))
    np.testing.assert_allclose(d, e_d, rtol=1e-9, atol=1e-13)


def test_composition_matches_finite_differences():
    from oracle import klp_oracle
    g, x, t, mask, adv = make_case(2, 4, 23, seed=6)
    lp0, _, _ = klp_oracle.get().forward(x, t, "fp32")
    old, ref = old_ref_from(lp0, g)
    kw = dict(eps_low=0.2, eps_high=0.28, beta=0.04, loss_type="grpo", dtype="fp32")
    _, _, _, d, _ = grpo_step(x, t, old, adv, mask, ref, **kw)
    rng = np.random.default_rng(7)
    idx = [tuple(rng.integers(0, n) for n in x.shape) for _ in range(24)]
    idx += [(b, s, int(t[b, s])) for b in range(2) for s in range(4) if t[b, s] >= 0]
    for i in idx:
        xp, xm = x.copy(), x.copy()
        xp[i] = np.float32(float(x[i]) + 1e-3)
        xm[i] = np.float32(float(x[i]) - 1e-3)
        h = float(xp[i]) - float(xm[i])
        lp_, _, _, _, _ = grpo_step(xp, t, old, adv, mask, ref, **kw)
        lm_, _, _, _, _ = grpo_step(xm, t, old, adv, mask, ref, **kw)
        fd = (lp_ - lm_) / h
        assert abs(fd - d[i]) <= 1e-6 * max(1e-3, abs(d[i])) + 1e-10, (i, fd, d[i])


@pytest.mark.parametrize("mutant", [1, 2])
def test_planted_mistakes_are_caught(mutant, oracle):
    g, x, t, mask, adv = make_case(3, 6, 41, seed=5)
    lp0, _, _ = oracle.forward(x, t, "fp32")
    old, ref = old_ref_from(lp0, g)
    kw = dict(eps_low=0.2, eps_high=0.28, beta=0.04, loss_type="bnpo")
    _, _, _, d, _ = grpo_step(x, t, old, adv, mask, ref, mutant=mutant, dtype="fp32", **kw)
    _, e_d = eager_pipeline(x, t, old, adv, mask, ref, **kw)
    assert not np.allclose(d, e_d, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("loss_type", ["grpo", "bnpo", "dr_grpo", "dapo"])
def test_token_weights_match_oracle(loss_type):
    from kernel_opt.grpo_step import grpo_token_weights
    B, S = 5, 37
    g = np.random.default_rng(8)
    mask = (g.random((B, S)) < 0.6).astype(np.float32)
    mask[1] = 0.0  # an empty row: its normaliser clamps to 1
    w = grpo_token_weights(torch.tensor(mask), loss_type, max_completion_length=50,
                           normalizer=123.0).numpy()
    kind = loss_type if loss_type in ("grpo", "bnpo") else "fixed"
    norm = {"dr_grpo": B * 50.0, "dapo": 123.0}.get(loss_type, 1.0)
    e = token_weights(mask, B, S, kind, norm)
    np.testing.assert_allclose(w, e, rtol=2 ** -23, atol=0)
    assert np.all(w[1] == 0.0)


def test_default_chunk_tokens():
    """fused_linear_grpo_step's default chunking: the fewest chunks whose
    [chunk, V] buffers fit DEFAULT_CHUNK_BYTES, of equal size (the last one
    at most n_chunks - 1 tokens shorter), covering every token."""
    from kernel_opt.linear_grpo import DEFAULT_CHUNK_BYTES, default_chunk_tokens
    assert default_chunk_tokens(8192, 152064, 2) == 8192           # one chunk
    assert default_chunk_tokens(32768, 152064, 2) == 10923         # 3 chunks (14122 max)
    assert default_chunk_tokens(1, 152064, 4) == 1
    rng = np.random.default_rng(0)
    for _ in range(2000):
        n = int(rng.integers(1, 1 << 20))
        v = int(rng.integers(1, 1 << 19))
        esz = int(rng.choice([2, 4]))
        c = default_chunk_tokens(n, v, esz)
        k = -(-n // c)  # chunks used
        max_tok = max(1, DEFAULT_CHUNK_BYTES // (v * esz))
        assert 1 <= c <= max(1, min(n, max_tok))
        assert k == -(-n // max_tok)                   # fewest chunks that fit
        assert n - (k - 1) * c >= c - (k - 1)          # balanced: short last chunk by < k
