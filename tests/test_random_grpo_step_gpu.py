"""Randomised GPU parity of the fused GRPO step (klp_grpo_step through the C
ABI, and kernel_opt.fused_grpo_step) against the float64 oracle and the
unfused kernels.

Each case draws, from a fixed seed (the case is printed before it runs):
the dtype; B and S; a vocabulary the step's row kernel takes (whole 16-byte
vectors, up to the row capacity); the row layout (contiguous, or the shifted
slice [:, :-1, :] of a longer tensor); the loss type (grpo, bnpo, dr_grpo,
dapo with a random normaliser); a KL term with reference log-probabilities
or none; per-sequence or per-token advantages; the mask (none, bool, int32,
int64, float32, bf16; some rows all masked); a temperature or none; and the
declared upstream gradient grad_scale (1, 0.25, 1/3, -2).  Bars:
  * logp / entropy / lse: the north-star forward tolerance against the
    oracle (1e-5 fp32, 2e-5 bf16 / fp16);
  * the loss: the sum of the kernel's per-token terms, within 1e-5 relative
    of the unfused GRPO loss at the kernel's logp;
  * d_logits: bit for bit klp_bwd's output for the same row statistics and
    the per-token gradient g_logp * grad_scale, where g_logp is the unfused
    GRPO loss's gradient (klp_grpo_bwd), and within the oracle's gradient
    bar (oracle/checks.py) of the float64 gradient;
  * the public entry point: loss * grad_scale backpropagated through
    fused_grpo_step leaves exactly that d_logits in logits.grad, and its
    logp / entropy are the C ABI's.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from klp_testutil import FWD_TOL, grad_check

pytestmark = pytest.mark.gpu
DEV = "cuda"
IGNORE = -100
DTYPES = (torch.bfloat16, torch.float16, torch.float32)
# Vocabularies of whole 16-byte vectors for every dtype (multiples of 8), up
# to the fp32 row capacity (77 824) and, for 16-bit dtypes, bf16's (155 648).
VOCABS_ANY = (8, 64, 1000, 4096, 8200, 32000, 50304, 77824)
VOCABS_16 = (128256, 152064, 155648)
MASKS = ("none", "bool", "int32", "int64", "float32", "bf16")
LOSSES = ("grpo", "bnpo", "dr_grpo", "dapo")
SEEDS = range(40)


def draw_case(seed):
    r = np.random.default_rng(1000 + seed)
    dtype = DTYPES[int(r.integers(3))]
    vocabs = VOCABS_ANY + (VOCABS_16 if dtype != torch.float32 else ())
    return dict(seed=seed, dtype=dtype,
                B=int(r.integers(1, 5)), S=int(r.integers(1, 24)),
                V=int(r.choice(vocabs)),
                shifted=bool(r.random() < 0.4),
                loss_type=str(r.choice(LOSSES)),
                normalizer=float(r.choice([1.0, 37.0, 1000.0])),
                beta=float(r.choice([0.0, 0.04])),
                per_token=bool(r.random() < 0.4),
                mask=str(r.choice(MASKS)),
                temperature=None if r.random() < 0.5 else float(r.choice([0.7, 1.3])),
                grad_scale=float(r.choice([1.0, 0.25, 1.0 / 3.0, -2.0])),
                scale=float(r.choice([1.0, 2.0, 4.0])))


def build(c):
    g = torch.Generator().manual_seed(c["seed"])
    B, S, V = c["B"], c["S"], c["V"]
    L = S + 1 if c["shifted"] else S
    full = (torch.randn(B, L, V, generator=g) * c["scale"]).to(c["dtype"])
    x_cpu = full[:, :S, :].contiguous()
    x = full.to(DEV)
    x = x[:, :-1, :] if c["shifted"] else x
    t = torch.randint(0, V, (B, S), generator=g)
    t[0, 0] = V - 1
    if S > 1:
        t[-1, -1] = 0
        t[0, 1] = IGNORE
    m01 = torch.rand(B, S, generator=g) < 0.75
    m01[0, 0] = True
    if B > 1 and c["seed"] % 3 == 0:
        m01[-1] = False
    adv = torch.randn((B, S) if c["per_token"] else (B,), generator=g)
    kinds = {"bool": torch.bool, "int32": torch.int32, "int64": torch.int64,
             "float32": torch.float32, "bf16": torch.bfloat16}
    if c["mask"] == "none":  # no mask: every token counts
        return x_cpu, x, t, None, torch.ones(B, S), adv
    return x_cpu, x, t, m01.to(kinds[c["mask"]]), m01.float(), adv


@pytest.mark.parametrize("seed", SEEDS)
def test_random_fused_grpo_step(seed, oracle):
    import kernel_opt as ko
    from kernel_opt import _C
    from kernel_opt.grpo_step import grpo_step_launch, grpo_token_weights
    c = draw_case(seed)
    print(f"random grpo step: {c}", flush=True)
    x_cpu, x, t, mask, mf, adv = build(c)
    B, S, V, T, cs = c["B"], c["S"], c["V"], c["temperature"], c["grad_scale"]
    e_lp, e_ent, e_lse = oracle.forward(x_cpu, t.numpy(), temperature=T)
    gen = torch.Generator().manual_seed(seed + 7)
    old = (torch.from_numpy(e_lp).float() + 0.3 * torch.randn(B, S, generator=gen)).to(DEV)
    ref = (torch.from_numpy(e_lp).float() + 0.3 * torch.randn(B, S, generator=gen)).to(DEV)
    ref = ref if c["beta"] != 0.0 else None
    extra = dict(normalizer=c["normalizer"]) if c["loss_type"] == "dapo" else {}
    td, advd, maskd = t.to(DEV), adv.to(DEV), None if mask is None else mask.to(DEV)

    # The C ABI.
    w = grpo_token_weights(mf.to(DEV), c["loss_type"], **extra).contiguous()
    params = (1.0 if T is None else T, 0.2, 0.28, c["beta"], int(c["per_token"]), cs)
    lp, ent, lse, lt, d = grpo_step_launch(x, td, old, ref, advd, w, params)
    tol = FWD_TOL[c["dtype"]]
    for name, ours, e in (("logp", lp, e_lp), ("entropy", ent, e_ent), ("lse", lse, e_lse)):
        err = np.abs(ours.cpu().double().numpy() - e).max()
        assert err <= tol, f"{name}: {err:.3g} > {tol}"

    # The unfused GRPO loss at the kernel's logp, and klp_bwd with its
    # gradient times grad_scale.
    lpu = lp.detach().clone().requires_grad_(True)
    loss_u, _ = ko.fused_grpo_loss(lpu, old, advd, mf.to(DEV), ref, eps_low=0.2, eps_high=0.28,
                                   beta=c["beta"], loss_type=c["loss_type"], **extra)
    loss_u.backward()
    g = lpu.grad
    loss = lt.sum()
    assert abs(loss.item() - loss_u.item()) <= 1e-5 * max(1.0, abs(loss_u.item())), \
        (loss.item(), loss_u.item())
    d_ref = torch.empty(x.shape, dtype=x.dtype, device=DEV)
    _C.bwd_launch(x, td, lse, ent, (g * cs).contiguous(), None, None, d_ref, temperature=T)
    assert torch.equal(d, d_ref), "d_logits differ from klp_bwd with g_logp * grad_scale"
    worst, detail = grad_check(oracle, x_cpu, t, lse, ent, d.cpu(), g_logp=g * cs,
                               temperature=T)
    assert worst <= 1.0, detail

    # The public entry point, the declared upstream gradient sent.
    leaf = x.detach().clone().requires_grad_(True)
    kw = dict(eps_low=0.2, eps_high=0.28, beta=c["beta"], loss_type=c["loss_type"],
              temperature=T, grad_scale=cs, **extra)
    lossp, lpp, entp = ko.fused_grpo_step(leaf, td, old, advd, maskd, ref, **kw)
    assert "FusedGrpoStep" in lossp.grad_fn.name(), lossp.grad_fn.name()
    (lossp * cs).backward()
    assert torch.equal(lpp, lp) and torch.equal(entp, ent)
    assert torch.equal(lossp, loss)
    assert torch.equal(leaf.grad, d)
