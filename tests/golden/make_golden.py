"""Writes tests/golden/klp_golden.npz: known-answer fixtures for the fused
logprob/entropy forward and backward.

The reference ships no golden vectors (its tests draw inputs from the CUDA
RNG), so these are computed here, from seeded inputs, with textbook
two-pass float64 formulas in numpy only — independent of the C oracle and of
the kernels:
    lse = m + log(sum exp(x - m)),  p = exp(x - lse),
    logp = x_t - lse (0 - lse for an out-of-range target),
    H = -sum p log p  (entries equal to -inf have p = 0 and are left out),
    d = p * (g_lse - g_logp - g_ent * (log p + H)) + [v == t] g_logp.
The gradient is evaluated from lse/H rounded to float32 (`lse32`, `ent32`),
which is what a backward kernel receives from the forward, so a test can
feed exactly these saved values to the kernel.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "klp_golden.npz")


def f32_to_bf16_bits(x32: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits, round to nearest even (inputs finite or -inf)."""
    b = x32.astype(np.float32).view(np.uint32).astype(np.uint64)
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    out = np.where(np.isneginf(x32), 0xFF80, rounded)
    return out.astype(np.uint16)


def bits_to_f64(bits: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "fp32":
        return bits.astype(np.float64)
    if dtype == "fp16":
        return bits.view(np.float16).astype(np.float64)
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def forward64(x, t):
    n, V = x.shape
    lse = np.empty(n)
    ent = np.empty(n)
    logp = np.empty(n)
    for i in range(n):
        row = x[i]
        fin = row[~np.isneginf(row)]
        m = fin.max()
        z = np.exp(fin - m).sum()
        lse[i] = m + np.log(z)
        p = np.exp(fin - lse[i])
        ent[i] = -(p * (fin - lse[i])).sum()
        logp[i] = (row[t[i]] if 0 <= t[i] < V else 0.0) - lse[i]
    return logp, ent, lse


def backward64(x, t, lse, ent, gl, ge, gs):
    n, V = x.shape
    d = np.zeros((n, V))
    for i in range(n):
        lp = x[i] - lse[i]
        with np.errstate(invalid="ignore"):
            p = np.where(np.isneginf(x[i]), 0.0, np.exp(lp))
            lp = np.where(np.isneginf(x[i]), 0.0, lp)
        d[i] = p * (gs[i] - gl[i] - ge[i] * (lp + ent[i]))
        if 0 <= t[i] < V:
            d[i, t[i]] += gl[i]
    return d


def make_case(name, dtype, n, V, seed, scale=2.0, spike=None, neg_inf=0.0, bad_target=False):
    r = np.random.default_rng(seed)
    x32 = (r.standard_normal((n, V)) * scale).astype(np.float32)
    t = r.integers(0, V, n).astype(np.int64)
    if spike is not None:
        j = r.integers(0, V, n)
        x32[np.arange(n), j] += np.float32(spike)
        t = np.where(r.random(n) < 0.6, j, t)
    if neg_inf > 0:
        mask = r.random((n, V)) < neg_inf
        x32[mask] = -np.inf
    if bad_target:
        t[0] = -100
    if dtype == "fp32":
        bits = x32
    elif dtype == "fp16":
        bits = x32.astype(np.float16).view(np.uint16)
    else:
        bits = f32_to_bf16_bits(x32)
    x = bits_to_f64(bits, dtype)
    logp, ent, lse = forward64(x, t)
    gl = r.standard_normal(n) * 0.5
    ge = r.standard_normal(n) * 0.5
    gs = r.standard_normal(n) * 0.5
    lse32 = lse.astype(np.float32)
    ent32 = ent.astype(np.float32)
    d = backward64(x, t, lse32.astype(np.float64), ent32.astype(np.float64), gl, ge, gs)
    return {f"{name}/dtype": np.array(dtype), f"{name}/logits_bits": bits, f"{name}/targets": t,
            f"{name}/logp": logp, f"{name}/entropy": ent, f"{name}/lse": lse,
            f"{name}/lse32": lse32, f"{name}/ent32": ent32,
            f"{name}/g_logp": gl.astype(np.float32), f"{name}/g_ent": ge.astype(np.float32),
            f"{name}/g_lse": gs.astype(np.float32), f"{name}/d": d}


CASES = [
    dict(name="fp32_randn", dtype="fp32", n=3, V=1000, seed=1, bad_target=True),
    dict(name="bf16_randn", dtype="bf16", n=4, V=5003, seed=2),
    dict(name="fp16_spiked", dtype="fp16", n=4, V=4099, seed=3, scale=3.0, spike=18.0),
    dict(name="bf16_neg_inf", dtype="bf16", n=2, V=3001, seed=4, neg_inf=0.3),
    dict(name="fp32_tiny", dtype="fp32", n=3, V=7, seed=5),
    dict(name="bf16_wide", dtype="bf16", n=1, V=32768, seed=6, scale=2.5),
]


def main():
    data = {"cases": np.array([c["name"] for c in CASES])}
    for c in CASES:
        # the gradient of the fixture must use exactly the fp32 g_* it stores
        case = make_case(**c)
        data.update(case)
    # recompute d with the stored float32 upstream grads
    for c in CASES:
        k = c["name"]
        x = bits_to_f64(data[f"{k}/logits_bits"], c["dtype"])
        data[f"{k}/d"] = backward64(
            x, data[f"{k}/targets"], data[f"{k}/lse32"].astype(np.float64),
            data[f"{k}/ent32"].astype(np.float64), data[f"{k}/g_logp"].astype(np.float64),
            data[f"{k}/g_ent"].astype(np.float64), data[f"{k}/g_lse"].astype(np.float64))
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
