"""The five BASELINE.json configurations at full size on the GPU.

At full size the oracle runs on a subset of rows (the first and last row
blocks); the whole batch is checked through size-independent properties:
  * finite outputs, 0 <= entropy <= log V, logp <= 0, max <= lse <= max + log V;
  * every row's gradient sums to g_lse (= 0 here) within the rounding bound
    sum|d| * 2^-p (p = significand bits of the output dtype) plus fp32 noise;
  * launch-shape invariance: the forward with another launch shape equals
    the default one to fp32 reduction-order noise;
  * determinism: a second run is bitwise identical;
  * on the oracle rows, the north star's literal gradient bar against the
    reference's fp32 eager path (autograd of the fp32 formulas, rounded to the
    output dtype): bf16 / fp16 gradients (C2-C4) within 1 ulp of it except
    where ours is the closer to the exact value; fp32 gradients (C1, C5) no
    farther from the exact value than the eager path at the worst element
    and in the median,
    1 fp32 ulp being below either's evaluation noise.  Each config prints
    its counts.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from klp_testutil import FWD_TOL, grad_check

pytestmark = pytest.mark.gpu

SIG_BITS = {torch.bfloat16: 8, torch.float16: 11, torch.float32: 24}


def _run(name):
    import bench
    from kernel_opt import _C

    inp = bench.make_inputs(name, "cuda")
    x, t = inp["logits"], inp["targets"]
    gl, ge = inp["g_logp"].contiguous(), inp["g_ent"].contiguous()
    lp, h, l = [torch.empty(t.shape, device="cuda") for _ in range(3)]
    _C.fused_logprob_entropy_v1(x, t, lp, h, l)
    d = torch.empty(x.shape, dtype=x.dtype, device="cuda")
    _C.fused_logprob_entropy_v1_backward(x, t, l, h, gl, ge, None, d)
    torch.cuda.synchronize()
    return inp, (lp, h, l), d


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5"])
def test_config_full_size(name, oracle):
    from kernel_opt import _C

    print(f"\n[config {name}] generating inputs", flush=True)
    inp, (lp, h, l), d = _run(name)
    x, t = inp["logits"], inp["targets"]
    V = x.size(-1)
    N = x.numel() // V
    dt = x.dtype
    print(f"[config {name}] N={N} V={V} {dt} ran fwd+bwd", flush=True)

    # --- whole-batch properties -------------------------------------------
    lp_f, h_f, l_f = lp.reshape(-1), h.reshape(-1), l.reshape(-1)
    assert torch.isfinite(lp_f).all() and torch.isfinite(h_f).all() and torch.isfinite(l_f).all()
    assert (h_f >= -1e-5).all() and (h_f <= math.log(V) + 1e-4).all()
    assert (lp_f <= 1e-5).all()
    x2 = x.reshape(-1, V) if x.is_contiguous() else None
    xmax = (x2.max(dim=1).values.float() if x2 is not None
            else torch.stack([x[b].float().max(dim=-1).values for b in range(x.size(0))]).reshape(-1))
    assert (l_f >= xmax - 1e-5).all() and (l_f <= xmax + math.log(V) + 1e-4).all()

    d2 = d.reshape(-1, V)
    row_sum = torch.zeros(N, dtype=torch.float64, device="cuda")
    row_abs = torch.zeros(N, dtype=torch.float64, device="cuda")
    for r0 in range(0, N, 1024):
        blk = d2[r0:r0 + 1024].double()
        row_sum[r0:r0 + 1024] = blk.sum(dim=1)
        row_abs[r0:r0 + 1024] = blk.abs().sum(dim=1)
    bound = row_abs * (2.0 ** -(SIG_BITS[dt] - 1) + 1e-6) + 1e-30
    if dt == torch.float16:
        bound = bound + V * 2.0 ** -25  # half of fp16's subnormal spacing, per element
    assert (row_sum.abs() <= bound).all(), \
        f"sum of gradients off by {float((row_sum.abs() / bound).max()):.3g}x the rounding bound"

    # --- launch-shape invariance + determinism ------------------------------
    lp1, h1, l1 = [torch.empty_like(lp) for _ in range(3)]
    _C.fwd_launch(x, t, lp1, h1, l1, config=(8, 4, 1, 0))
    assert (l1 - l).abs().max().item() <= 4e-6 * max(1.0, l.abs().max().item())
    assert (h1 - h).abs().max().item() <= 4e-6 * max(1.0, h.abs().max().item())
    lp2, h2, l2 = [torch.empty_like(lp) for _ in range(3)]
    _C.fused_logprob_entropy_v1(x, t, lp2, h2, l2)
    assert torch.equal(lp2, lp) and torch.equal(h2, h) and torch.equal(l2, l)

    # --- oracle on the first and last row blocks ----------------------------
    rows = list(range(0, min(64, N))) + list(range(max(64, N - 64), N))
    idx = torch.tensor(rows, device="cuda")
    xs = torch.stack([x.reshape(-1, V)[r] for r in rows]) if x.is_contiguous() else \
        torch.stack([x[r // x.size(1), r % x.size(1)] for r in rows])
    x_cpu = xs.cpu()
    t_cpu = t.reshape(-1)[idx].cpu()
    r_lp, r_h, r_l = oracle.forward(x_cpu, t_cpu.numpy())
    for nm, ours, ref in (("logp", lp_f, r_lp), ("entropy", h_f, r_h), ("lse", l_f, r_l)):
        err = np.abs(ours[idx].cpu().double().numpy() - ref).max()
        assert err <= FWD_TOL[dt], f"{name} {nm}: {err:.3g} > {FWD_TOL[dt]}"
    worst, detail = grad_check(oracle, x_cpu, t_cpu, l_f[idx], h_f[idx], d2[idx],
                               g_logp=inp["g_logp"].reshape(-1)[idx],
                               g_ent=inp["g_ent"].reshape(-1)[idx])
    assert worst <= 1.0, f"{name}: gradient {detail}"
    print(f"[config {name}] ok: grad {detail}", flush=True)

    # --- the north star's literal gradient bar on the same rows -------------
    # Against the reference's fp32 path itself (autograd of the fp32 formulas
    # on the upcast logits, tests/test_logprob.py:17-25 of the reference),
    # rounded to the output dtype: every element within 1 ulp of it, except
    # where the eager path is itself further from the exact (float64) value,
    # and there ours must be the closer one.
    from oracle import eager_ref
    from klp_testutil import DTYPE_NAME, WIDTH, bits_of, storage_bits, ulp_diff
    gl_r = inp["g_logp"].reshape(-1)[idx].contiguous()
    ge_r = inp["g_ent"].reshape(-1)[idx].contiguous()
    xf = xs.float().requires_grad_(True)
    e_lp, e_h, _ = eager_ref.ref_fp32(xf, t.reshape(-1)[idx])
    (e_lp * gl_r + e_h * ge_r).sum().backward()
    eager = xf.grad.to(dt)
    width = WIDTH[dt]
    d_vs_eager = ulp_diff(storage_bits(d2[idx]), storage_bits(eager), width)
    exact = oracle.backward(x_cpu, t_cpu.numpy(), r_l, r_h, gl_r.cpu().double().numpy(),
                            ge_r.cpu().double().numpy(), None)
    exact_bits = bits_of(oracle.round_to(exact, DTYPE_NAME[dt]))
    d_ours = ulp_diff(storage_bits(d2[idx]), exact_bits.reshape(d_vs_eager.shape), width)
    d_eager = ulp_diff(storage_bits(eager), exact_bits.reshape(d_vs_eager.shape), width)
    far = d_vs_eager > 1
    print(f"[config {name}] vs fp32 eager path ({len(rows)} rows, {d_vs_eager.size} elements): "
          f"{int(far.sum())} elements > 1 ulp apart (max {int(d_vs_eager.max())}); "
          f"ulps from exact: ours max {int(d_ours.max())} median {np.median(d_ours):.0f}, "
          f"eager max {int(d_eager.max())} median {np.median(d_eager):.0f}", flush=True)
    if width == 16:
        bad = far & (d_ours >= d_eager)
        assert not bad.any(), (f"{name}: {int(bad.sum())} elements > 1 ulp from the fp32 eager "
                               f"path without being closer to the exact value")
    else:
        # fp32 output: 1 fp32 ulp is below the evaluation noise of any fp32
        # computation of these gradients (the saved fp32 lse alone, rounded
        # at magnitude ~12, moves p by up to 4 ulps, in ours and in the
        # eager path alike); the eager path itself lands tens of ulps from
        # the exact value.  The bound: ours no farther from the exact value
        # than the eager path, at the worst element and in the median (C1:
        # 19 vs 42 ulps, medians 3 vs 4; C5: 29 vs 72, medians 5 vs 8,
        # printed above), on top of grad_check's noise bound.
        assert d_ours.max() <= d_eager.max(), \
            (f"{name}: ours up to {int(d_ours.max())} ulps from the exact gradient, the fp32 "
             f"eager path {int(d_eager.max())}")
        assert np.median(d_ours) <= np.median(d_eager), \
            (f"{name}: ours {np.median(d_ours):.0f} ulps from the exact gradient in the median, "
             f"the fp32 eager path {np.median(d_eager):.0f}")
