"""The five BASELINE.json configurations at full size on the GPU.

At full size the oracle runs on a subset of rows (the first and last row
blocks); the whole batch is checked through size-independent properties:
  * finite outputs, 0 <= entropy <= log V, logp <= 0, max <= lse <= max + log V;
  * every row's gradient sums to g_lse (= 0 here) within the rounding bound
    sum|d| * 2^-p (p = significand bits of the output dtype) plus fp32 noise;
  * launch-shape invariance: the forward with another launch shape equals
    the default one to fp32 reduction-order noise;
  * determinism: a second run is bitwise identical.
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
