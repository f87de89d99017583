"""float64 restatement of the fused LM head forward (klp_lmh_fwd).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker.  The product
never imports it.

logits = (hidden @ weight^T) in float64 from the exact bf16 values (every
product of two bf16 numbers is exact in float64; a K-term sum of them is
within K * 2^-53 relative), times fp32(1/T); then the reference's output
formulas (csrc/fused_logprob.cu:221-224: lse = m + log Z, logprob =
x_t - lse, entropy = log Z - T/Z, in the stable float64 form) with the
reference's target rule (a target outside [0, V) leaves x_t = 0).

Pinned in tests/test_lmh_cpu.py against the float64 C oracle of the
logprob forward (oracle/klp_oracle.c) on integer inputs whose logits are
exact in fp32, against a pure-Python loop on tiny shapes, and against the
uniform closed form (identical weight rows: entropy = lse - x = log V).
`backward` (the reference's closed form, csrc/fused_logprob.cu:233-238,
chained through the linear layer) is pinned against float64 torch autograd
of the eager formulas.
"""
from __future__ import annotations

import numpy as np


def bf16_to_f64(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 storage -> float64 (exact)."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def scale_of(temperature):
    """The float nearest 1/fp32(T): the temperature crosses the C ABI as a
    float (1.0 for None)."""
    if temperature is None:
        return 1.0
    return float(np.float32(1.0 / float(np.float32(temperature))))


def logits(hidden_bits, weight_bits, temperature=None):
    h = bf16_to_f64(hidden_bits)
    w = bf16_to_f64(weight_bits)
    return (h @ w.T) * scale_of(temperature)


def forward(hidden_bits, weight_bits, targets, temperature=None):
    """(logprob, entropy, lse) float64 [N]."""
    x = logits(hidden_bits, weight_bits, temperature)
    N, V = x.shape
    m = x.max(axis=1, keepdims=True)
    e = np.exp(x - m)
    z = e.sum(axis=1)
    lse = m[:, 0] + np.log(z)
    p = e / z[:, None]
    ent = lse - (p * x).sum(axis=1)
    t = np.asarray(targets, np.int64)
    valid = (t >= 0) & (t < V)
    xt = np.where(valid, x[np.arange(N), np.clip(t, 0, V - 1)], 0.0)
    return xt - lse, ent, lse


def magnitude(hidden_bits, weight_bits):
    """Per-token max over v of sum_k |h_k w_k|: the scale of the fp32
    accumulation error of each logit."""
    return (np.abs(bf16_to_f64(hidden_bits)) @ np.abs(bf16_to_f64(weight_bits)).T).max(axis=1)


def backward(hidden_bits, weight_bits, targets, g_logp=None, g_ent=None, g_lse=None,
             temperature=None):
    """(d_hidden, d_weight, d_logits) float64 for upstream gradients of
    (logprob, entropy, lse); None means zero.  d_logits is with respect to
    the unscaled logits hidden @ weight^T."""
    h = bf16_to_f64(hidden_bits)
    w = bf16_to_f64(weight_bits)
    s = scale_of(temperature)
    x = (h @ w.T) * s
    N, V = x.shape
    m = x.max(axis=1, keepdims=True)
    lse = m[:, 0] + np.log(np.exp(x - m).sum(axis=1))
    lp = x - lse[:, None]
    p = np.exp(lp)
    ent = -(p * lp).sum(axis=1)
    z = np.zeros(N)
    gl = z if g_logp is None else np.asarray(g_logp, np.float64).reshape(-1)
    ge = z if g_ent is None else np.asarray(g_ent, np.float64).reshape(-1)
    gs = z if g_lse is None else np.asarray(g_lse, np.float64).reshape(-1)
    c0 = gs - gl - ge * ent
    d = p * (c0[:, None] - ge[:, None] * lp)
    t = np.asarray(targets, np.int64).reshape(-1)
    ok = (t >= 0) & (t < V)
    d[np.arange(N)[ok], t[ok]] += gl[ok]
    d *= s
    return d @ w, d.T @ h, d
