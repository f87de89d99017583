"""Independent checks ("pins") of the float64 oracle.

Each pin compares the oracle with something that does not restate its
formulas: a two-pass float64 brute force, a closed form, an invariant, a
finite difference, an explicit Jacobian, or numpy/torch conversions.  Every
pin returns None on success or a failure message.  tests/test_oracle.py
requires all of them to pass; tests/test_oracle_mutants.py requires every
deliberately broken oracle build to fail at least one.
"""
from __future__ import annotations

import math

import numpy as np
import torch

RNG_SEED = 20251201


def _rng(k=0):
    return np.random.default_rng(RNG_SEED + k)


def brute_forward(x64: np.ndarray, t: np.ndarray):
    """Two-pass float64 log-softmax: the textbook definition, row by row.
    -inf entries have probability 0 and are left out of every sum."""
    x64 = np.atleast_2d(x64)
    out = []
    for row, tg in zip(x64, np.atleast_1d(t)):
        fin = row[row != -np.inf]
        m = fin.max()
        e = np.exp(fin - m)
        z = e.sum()
        lse = m + math.log(z)
        p = e / z
        ent = -np.sum(p * np.log(p, where=p > 0, out=np.zeros_like(p)))
        lp = (row[tg] if 0 <= tg < row.size else 0.0) - lse
        out.append((lp, ent, lse))
    return [np.array(v) for v in zip(*out)]


def _case(kind, V, n=4, k=0, scale=2.0):
    r = _rng(k)
    x = (r.standard_normal((n, V)) * scale).astype(np.float32)
    t = r.integers(0, V, n).astype(np.int64)
    return x, t


def _close(a, b, tol, what):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    if a.shape != b.shape:
        return f"{what}: shape {a.shape} vs {b.shape}"
    same_nan = np.isnan(a) == np.isnan(b)
    if not same_nan.all():
        return f"{what}: NaN pattern differs"
    ok = ~np.isnan(a)
    both_inf = np.isinf(a) & np.isinf(b) & (np.sign(a) == np.sign(b))
    diff = np.where(both_inf, 0.0, np.abs(a - b))
    err = diff[ok].max() if ok.any() else 0.0
    return None if err <= tol else f"{what}: max err {err:.3g} > {tol:.3g}"


# ---------------------------------------------------------------------------
# forward pins
# ---------------------------------------------------------------------------
def pin_brute_force(o):
    for k, V in enumerate([1, 2, 3, 17, 64, 1000, 5003]):
        x, t = _case("randn", V, n=5, k=k)
        got = o.forward(x, t, dtype="fp32")
        ref = brute_forward(x.astype(np.float64), t)
        for g, r, nm in zip(got, ref, ("logp", "entropy", "lse")):
            msg = _close(g, r, 1e-11 * max(1.0, math.log(V)), f"brute V={V} {nm}")
            if msg:
                return msg
    return None


def pin_uniform(o):
    for V in (1, 2, 7, 4096, 152064):
        x = np.zeros((2, V), np.float32)
        lp, h, l = o.forward(x, np.array([0, V - 1]), dtype="fp32")
        lv = math.log(V)
        for val, exp, nm in ((h, lv, "entropy"), (l, lv, "lse"), (lp, -lv, "logp")):
            if np.abs(val - exp).max() > 1e-12 * max(1, lv):
                return f"uniform V={V} {nm}: {val} vs {exp}"
    return None


def pin_two_element(o):
    r = _rng(1)
    ab = (r.standard_normal((20, 2)) * 3).astype(np.float32)
    t = (r.integers(0, 2, 20)).astype(np.int64)
    lp, h, l = o.forward(ab, t, dtype="fp32")
    a, b = ab[:, 0].astype(np.float64), ab[:, 1].astype(np.float64)
    p = 1.0 / (1.0 + np.exp(b - a))           # P(first)
    ent = -(p * np.log(p) + (1 - p) * np.log1p(-p))
    lse = np.logaddexp(a, b)
    logp = np.where(t == 0, np.log(p), np.log1p(-p))
    for g, e, nm in ((h, ent, "entropy"), (l, lse, "lse"), (lp, logp, "logp")):
        msg = _close(g, e, 1e-12, f"two-element {nm}")
        if msg:
            return msg
    return None


def pin_spike(o):
    """Row of zeros with one spike K at j: closed forms of lse, logp and H."""
    for V, K, j in ((1000, 18.0, 5), (128256, 18.0, 70000), (50, -3.0, 49)):
        x = np.zeros((1, V), np.float32)
        x[0, j] = K
        z = (V - 1) + math.exp(K)
        pj = math.exp(K) / z
        q = 1.0 / z
        H = -(pj * math.log(pj) + (V - 1) * q * math.log(q))
        lp, h, l = o.forward(x, np.array([j]), dtype="fp32")
        lp0, _, _ = o.forward(x, np.array([(j + 1) % V]), dtype="fp32")
        checks = ((l[0], math.log(z), "lse"), (h[0], H, "entropy"),
                  (lp[0], math.log(pj), "logp@spike"), (lp0[0], math.log(q), "logp@other"))
        for g, e, nm in checks:
            if abs(g - e) > 1e-11 * max(1.0, abs(e)):
                return f"spike V={V} {nm}: {g} vs {e}"
    return None


def pin_shift_and_permutation(o):
    r = _rng(2)
    V = 777
    # values k/8 keep x + 64 exact in float32
    x = (r.integers(-64, 64, (3, V)) / 8.0).astype(np.float32)
    t = r.integers(0, V, 3).astype(np.int64)
    lp, h, l = o.forward(x, t, dtype="fp32")
    lp2, h2, l2 = o.forward(x + np.float32(64.0), t, dtype="fp32")
    for a, b, nm in ((lp, lp2, "logp"), (h, h2, "entropy"), (l + 64.0, l2, "lse")):
        msg = _close(a, b, 1e-10, f"shift {nm}")
        if msg:
            return msg
    perm = r.permutation(V)
    inv = np.argsort(perm)
    lp3, h3, l3 = o.forward(x[:, perm], inv[t], dtype="fp32")
    for a, b, nm in ((lp, lp3, "logp"), (h, h3, "entropy"), (l, l3, "lse")):
        msg = _close(a, b, 1e-10, f"permutation {nm}")
        if msg:
            return msg
    return None


def pin_targets_out_of_range(o):
    x, _ = _case("randn", 300, n=4, k=3)
    t = np.array([-100, -1, 300, 10**9], np.int64)
    lp, _, l = o.forward(x, t, dtype="fp32")
    return _close(lp, -l, 0.0, "out-of-range target logp = -lse")


def pin_target_value(o):
    """logp + lse must equal the target's logit exactly (float64)."""
    x, t = _case("randn", 4099, n=8, k=4)
    lp, _, l = o.forward(x, t, dtype="fp32")
    return _close(lp + l, x[np.arange(8), t].astype(np.float64), 1e-12, "logp + lse = x_t")


def pin_negative_infinity(o):
    """-inf entries are skipped: equal to the row with them removed."""
    r = _rng(5)
    V = 500
    x = (r.standard_normal((3, V)) * 2).astype(np.float32)
    mask = r.random((3, V)) < 0.4
    mask[:, 0] = True   # first element masked too
    x[mask] = -np.inf
    t = np.array([int(np.nonzero(~mask[0])[0][0]), int(np.nonzero(mask[1])[0][1]), V + 1])
    lp, h, l = o.forward(x, t, dtype="fp32")
    ref = brute_forward(x.astype(np.float64), t)
    for g, e, nm in zip((lp, h, l), ref, ("logp", "entropy", "lse")):
        msg = _close(g, e, 1e-11, f"-inf {nm}")
        if msg:
            return msg
    xa = np.full((1, 10), -np.inf, np.float32)
    lp, h, l = o.forward(xa, np.array([2]), dtype="fp32")
    if not (l[0] == -np.inf and math.isnan(h[0]) and math.isnan(lp[0])):
        return f"all -inf row: got lse={l[0]} H={h[0]} logp={lp[0]}"
    return None


def pin_nan_propagates(o):
    x, t = _case("randn", 64, n=2, k=6)
    x[0, 10] = np.nan
    lp, h, l = o.forward(x, t, dtype="fp32")
    if not (math.isnan(l[0]) and math.isnan(h[0])):
        return "NaN logit must make lse and entropy NaN"
    if math.isnan(l[1]):
        return "NaN leaked into another row"
    return None


def pin_combine_associative(o):
    r = _rng(7)
    V = 3000
    row = (r.standard_normal(V) * 2).astype(np.float32)
    whole = o.segment_state(row, 0, V, dtype="fp32")
    for trial in range(5):
        cuts = np.sort(r.choice(np.arange(1, V), size=6, replace=False))
        bounds = [0, *cuts.tolist(), V]
        states = [o.segment_state(row, a, b, dtype="fp32") for a, b in zip(bounds, bounds[1:])]
        if trial % 2:
            states = states[::-1]
        acc = np.array([-np.inf, 0.0, 0.0])
        for s in states:
            acc = o.combine(acc, s)
        lp1 = o.finalize(whole, 0.0)
        lp2 = o.finalize(acc, 0.0)
        if max(abs(a - b) for a, b in zip(lp1, lp2)) > 1e-12:
            return f"combine over {bounds}: {lp1} vs {lp2}"
    empty = np.array([-np.inf, 0.0, 0.0])
    if not np.array_equal(o.combine(whole, empty), whole) or \
            not np.array_equal(o.combine(empty, whole), whole):
        return "the empty state must be the identity of combine"
    return None


def pin_naive_matches(o):
    x, t = _case("randn", 2000, n=4, k=8)
    a = o.forward(x, t, dtype="fp32")
    b = o.forward(x, t, dtype="fp32", naive=True)
    for g, e, nm in zip(a, b, ("logp", "entropy", "lse")):
        msg = _close(g, e, 1e-11, f"naive vs v1 {nm}")
        if msg:
            return msg
    x[1, 5] = -np.inf
    _, h, l = o.forward(x, t, dtype="fp32", naive=True)
    if not math.isnan(h[1]) or not np.isfinite(l[1]):
        return "naive: a -inf logit after the first must give NaN entropy, finite lse"
    return None


# ---------------------------------------------------------------------------
# backward pins
# ---------------------------------------------------------------------------
def _grads(n, k):
    r = _rng(100 + k)
    return [r.standard_normal(n) * 0.5 for _ in range(3)]


def pin_backward_finite_difference(o):
    """Central differences of L = sum(gl*logp + ge*H + gs*lse) through the
    float64 forward, against the backward."""
    for k, V in enumerate((5, 37)):
        x, t = _case("randn", V, n=2, k=20 + k, scale=1.5)
        x64 = x.astype(np.float64)
        gl, ge, gs = _grads(2, k)
        lp, h, l = brute_forward(x64, t)
        d = o.backward(x, t, l, h, g_logp=gl, g_ent=ge, g_lse=gs, dtype="fp32")

        def loss(xx):
            a, b, c = brute_forward(xx, t)
            return float(np.sum(gl * a + ge * b + gs * c))
        eps = 1e-6
        fd = np.zeros_like(x64)
        for i in range(x64.shape[0]):
            for j in range(V):
                xp, xm = x64.copy(), x64.copy()
                xp[i, j] += eps
                xm[i, j] -= eps
                fd[i, j] = (loss(xp) - loss(xm)) / (2 * eps)
        msg = _close(d, fd, 2e-8, f"finite differences V={V}")
        if msg:
            return msg
    return None


def pin_backward_jacobian(o):
    """Explicit softmax Jacobian J = diag(p) - p p^T:
    dlogp_t/dx = e_t - p, dlse/dx = p, dH/dx = -J^T (log p + 1)."""
    V = 40
    x, t = _case("randn", V, n=3, k=30)
    gl, ge, gs = _grads(3, 3)
    lp, h, l = brute_forward(x.astype(np.float64), t)
    d = o.backward(x, t, l, h, g_logp=gl, g_ent=ge, g_lse=gs, dtype="fp32")
    for i in range(3):
        xi = x[i].astype(np.float64)
        p = np.exp(xi - l[i])
        J = np.diag(p) - np.outer(p, p)
        e_t = np.zeros(V)
        e_t[t[i]] = 1.0
        ref = gl[i] * (e_t - p) + gs[i] * p - ge[i] * (J.T @ (np.log(p) + 1.0))
        msg = _close(d[i], ref, 1e-13, f"jacobian row {i}")
        if msg:
            return msg
    return None


def pin_backward_sum_and_nones(o):
    x, t = _case("randn", 1001, n=4, k=31)
    gl, ge, gs = _grads(4, 4)
    lp, h, l = brute_forward(x.astype(np.float64), t)
    d = o.backward(x, t, l, h, g_logp=gl, g_ent=ge, g_lse=gs, dtype="fp32")
    msg = _close(d.sum(axis=1), gs, 1e-12, "sum_v d = g_lse")
    if msg:
        return msg
    d0 = o.backward(x, t, l, h, g_logp=gl, dtype="fp32")
    d1 = o.backward(x, t, l, h, g_logp=gl, g_ent=np.zeros(4), g_lse=np.zeros(4), dtype="fp32")
    if not np.array_equal(d0, d1):
        return "None upstream gradients must act as zeros"
    # out-of-range target: no one-hot term, so the row sums to g_lse - 0
    t2 = t.copy()
    t2[0] = -100
    lp2 = lp.copy()
    d2 = o.backward(x, t2, l, h, g_logp=gl, g_ent=ge, g_lse=gs, dtype="fp32")
    if abs(d2[0].sum() - (gs[0] - gl[0])) > 1e-12:
        return "out-of-range target must drop the one-hot term"
    del lp2
    return None


def pin_backward_negative_infinity(o):
    x, t = _case("randn", 300, n=2, k=32)
    x[0, :50] = -np.inf
    t[0] = 100
    gl, ge, gs = _grads(2, 5)
    lp, h, l = brute_forward(x.astype(np.float64), t)
    d = o.backward(x, t, l, h, g_logp=gl, g_ent=ge, g_lse=gs, dtype="fp32")
    if not (d[0, :50] == 0).all():
        return "-inf logits must get gradient 0"
    # the rest equals the gradient of the row without them
    xr = x[0:1, 50:]
    tr = t[0:1] - 50
    lpr, hr, lr = brute_forward(xr.astype(np.float64), tr)
    dr = o.backward(xr, tr, lr, hr, g_logp=gl[:1], g_ent=ge[:1], g_lse=gs[:1], dtype="fp32")
    return _close(d[0, 50:], dr[0], 1e-13, "-inf row remainder")


# ---------------------------------------------------------------------------
# conversion pins
# ---------------------------------------------------------------------------
def pin_up_conversions(o):
    bits = np.arange(65536, dtype=np.uint16)
    f16 = o.to_f32(bits, "fp16")
    ref16 = bits.view(np.float16).astype(np.float32)
    if not np.array_equal(np.isnan(f16), np.isnan(ref16)) or \
            not np.array_equal(f16[~np.isnan(f16)], ref16[~np.isnan(ref16)]):
        return "fp16 -> f32 differs from numpy"
    bf = o.to_f32(bits, "bf16")
    refb = torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).float().numpy()
    if not np.array_equal(np.isnan(bf), np.isnan(refb)) or \
            not np.array_equal(bf[~np.isnan(bf)], refb[~np.isnan(refb)]):
        return "bf16 -> f32 differs from torch"
    return None


def _special_values():
    r = _rng(40)
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 70000.0, 1e-8, 5.96e-8, 2.98e-8,
            2.9802322387695312e-08, 6.103515625e-05, 6.1e-05, 3.4e38, 3.3895313892515355e+38,
            1e-40, -1e-45, 1.00390625, 1.01171875, 1.0078125, float("inf"), -float("inf")]
    vals += list(r.standard_normal(4000) * 10.0 ** r.integers(-12, 8, 4000))
    # exact ties for bf16: 1 + (2k+1) * 2^-8
    vals += [1.0 + (2 * k + 1) * 2.0 ** -8 for k in range(64)]
    vals += [2.0 ** -24 * (k + 0.5) for k in range(64)]  # fp16 subnormal ties
    return np.array(vals, np.float64)


def pin_down_conversions(o):
    v = _special_values()
    got16 = o.round_to(v, "fp16")
    with np.errstate(over="ignore"):
        ref16 = v.astype(np.float16).view(np.uint16)  # numpy: correctly rounded, RNE
    if not np.array_equal(got16, ref16):
        i = int(np.nonzero(got16 != ref16)[0][0])
        return f"f64 -> fp16 of {v[i]!r}: {got16[i]:#06x} vs numpy {ref16[i]:#06x}"
    # bf16: compare on float32-representable inputs against torch's RNE
    v32 = v.astype(np.float32)
    gotb = o.round_to(v32.astype(np.float64), "bf16")
    refb = torch.from_numpy(v32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    if not np.array_equal(gotb, refb):
        i = int(np.nonzero(gotb != refb)[0][0])
        return f"f32 -> bf16 of {v32[i]!r}: {gotb[i]:#06x} vs torch {refb[i]:#06x}"
    return None


def _scaled(x32, T):
    """numpy's own fp32 product x * s, as float64, where s is the float
    nearest 1/fp32(T) (the temperature crosses the C ABI as a float)."""
    s = np.float32(1.0 / float(np.float32(T)))
    return (x32.astype(np.float32) * s).astype(np.float64), float(s)


def pin_temperature_forward(o):
    """Temperature T: brute force on the logits scaled by fp32(1/fp32(T)) in numpy;
    T = 1 is exactly the plain forward."""
    x, t = _case("randn", 2001, n=4, k=50)
    for T in (0.7, 1.3, 2.0):
        xs, _ = _scaled(x, T)
        got = o.forward(x, t, dtype="fp32", temperature=T)
        ref = brute_forward(xs, t)
        for g, r, nm in zip(got, ref, ("logp", "entropy", "lse")):
            msg = _close(g, r, 1e-11, f"temperature {T} {nm}")
            if msg:
                return msg
    a = o.forward(x, t, dtype="fp32", temperature=1.0)
    b = o.forward(x, t, dtype="fp32")
    if not all(np.array_equal(u, v) for u, v in zip(a, b)):
        return "temperature 1 must equal the plain forward"
    return None


def pin_temperature_backward(o):
    """d/dx of L(x / T) = (1/T) * (the softmax-Jacobian gradient at x / T)."""
    V = 60
    x, t = _case("randn", V, n=3, k=51)
    gl, ge, gs = _grads(3, 6)
    for T in (0.6, 1.7):
        xs, s = _scaled(x, T)
        lp, h, l = brute_forward(xs, t)
        d = o.backward(x, t, l, h, g_logp=gl, g_ent=ge, g_lse=gs, dtype="fp32", temperature=T)
        for i in range(3):
            p = np.exp(xs[i] - l[i])
            J = np.diag(p) - np.outer(p, p)
            e_t = np.zeros(V)
            e_t[t[i]] = 1.0
            ref = s * (gl[i] * (e_t - p) + gs[i] * p - ge[i] * (J.T @ (np.log(p) + 1.0)))
            msg = _close(d[i], ref, 1e-13, f"temperature {T} jacobian row {i}")
            if msg:
                return msg
    return None


ALL_PINS = [
    pin_brute_force, pin_uniform, pin_two_element, pin_spike, pin_shift_and_permutation,
    pin_targets_out_of_range, pin_target_value, pin_negative_infinity, pin_nan_propagates,
    pin_combine_associative, pin_naive_matches, pin_backward_finite_difference,
    pin_backward_jacobian, pin_backward_sum_and_nones, pin_backward_negative_infinity,
    pin_up_conversions, pin_down_conversions, pin_temperature_forward, pin_temperature_backward,
]
