"""GPU parity of the chunked LM head + GRPO step (kernel_opt.fused_linear_grpo_step).

Bars:
  * one chunk against the autograd composition logits = hidden @ weight^T ->
    fused_grpo_step -> backward, on the same GEMM: loss, logp, entropy and
    d_hidden equal; d_weight within the fp32-accumulation noise of a bf16 GEMM
    (the composition's backward runs the weight GEMM in the other layout);
  * several chunks against the per-chunk composition run here by hand on the
    same chunk GEMMs (grpo_step_launch with the same per-token weights, then
    d_hidden = d_logits @ W and d_weight accumulated chunk by chunk in float32):
    equal, so the chunking itself adds nothing;
  * a small case against the float64 oracle (oracle/grpo_step_oracle.py on the
    GEMM's bf16 logits, then float64 products): logp / entropy within 2e-5,
    the loss within 1e-5 relative, d_hidden and d_weight within
    2^-7 (|d| @ |M|) + 2^-8 |ref| (one bf16 rounding of d_logits and of the
    product);
  * sequence-level weights run the unfused composition; a frozen weight; a
    scaled loss.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ko():
    import kernel_opt
    return kernel_opt


def make(B, S, D, V, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(B, S, D, generator=g).to(dtype)
    w = (torch.randn(V, D, generator=g) * 3.0 / math.sqrt(D)).to(dtype)
    t = torch.randint(0, V, (B, S), generator=g)
    t[0, 1] = -100
    mask = (torch.rand(B, S, generator=g) < 0.8).float()
    adv = torch.randn(B, generator=g)
    old = -torch.rand(B, S, generator=g) * 8 - 4
    ref = old + 0.2 * torch.randn(B, S, generator=g)
    return [x.to(DEV) for x in (h, w, t, mask, adv, old, ref)]


KW = dict(eps_low=0.2, eps_high=0.28, beta=0.04, loss_type="grpo")


def test_one_chunk_matches_autograd_composition():
    ko = _ko()
    h, w, t, mask, adv, old, ref = make(2, 96, 256, 4096, seed=1)
    B, S, D = h.shape
    ha = h.clone().requires_grad_(True)
    wa = w.clone().requires_grad_(True)
    la, lpa, enta = ko.fused_linear_grpo_step(ha, wa, t, old, adv, mask, ref, chunk_tokens=B * S,
                                              **KW)
    la.backward()
    hb = h.clone().requires_grad_(True)
    wb = w.clone().requires_grad_(True)
    logits = torch.mm(hb.view(-1, D), wb.t()).view(B, S, -1)
    lb, lpb, entb = ko.fused_grpo_step(logits, t, old, adv, mask, ref, **KW)
    lb.backward()
    assert torch.equal(la, lb) and torch.equal(lpa, lpb) and torch.equal(enta, entb)
    assert not lpa.requires_grad and not enta.requires_grad
    assert torch.equal(ha.grad, hb.grad)
    # d_weight: same products, GEMM in the other layout.
    ref_dw = wb.grad.float()
    bound = 2.0 ** -7 * ref_dw.abs() + 1e-6 * ref_dw.abs().max()
    assert torch.all((wa.grad.float() - ref_dw).abs() <= bound)


@pytest.mark.parametrize("chunk", [7, 64, 200])
def test_chunks_match_per_chunk_composition(chunk):
    from kernel_opt.grpo_step import grpo_step_launch, grpo_token_weights
    ko = _ko()
    h, w, t, mask, adv, old, ref = make(3, 70, 128, 2048, seed=2 + chunk)
    B, S, D = h.shape
    V = w.size(0)
    N = B * S
    ha = h.clone().requires_grad_(True)
    wa = w.clone().requires_grad_(True)
    loss, lp, ent = ko.fused_linear_grpo_step(ha, wa, t, old, adv, mask, ref, chunk_tokens=chunk,
                                              **KW)
    loss.backward()
    # The composition by hand, chunk by chunk.
    h2 = h.view(N, D)
    wts = grpo_token_weights(mask, "grpo").reshape(-1).contiguous()
    adv_t = adv.unsqueeze(1).expand(B, S).reshape(-1).contiguous()
    params = (1.0, 0.2, 0.28, 0.04, 1, 1.0)
    lps, ents, lts, dhs = [], [], [], []
    dw = None  # float32, accumulated inside the GEMM
    for n0 in range(0, N, chunk):
        n1 = min(N, n0 + chunk)
        c = n1 - n0
        logits = torch.mm(h2[n0:n1], w.t())
        a, b_, _, lt, d = grpo_step_launch(logits.view(1, c, V), t.view(-1)[n0:n1].view(1, c),
                                           old.reshape(-1)[n0:n1], ref.reshape(-1)[n0:n1],
                                           adv_t[n0:n1], wts[n0:n1], params)
        lps.append(a.view(-1)); ents.append(b_.view(-1)); lts.append(lt.view(-1))
        dhs.append(torch.mm(d.view(c, V), w))
        if dw is None:
            dw = torch.mm(d.view(c, V).t(), h2[n0:n1], out_dtype=torch.float32)
        else:
            torch.addmm(dw, d.view(c, V).t(), h2[n0:n1], out_dtype=torch.float32, out=dw)
    assert torch.equal(lp.view(-1), torch.cat(lps)) and torch.equal(ent.view(-1), torch.cat(ents))
    assert torch.equal(loss, torch.cat(lts).sum())
    assert torch.equal(ha.grad.view(N, D), torch.cat(dhs))
    assert torch.equal(wa.grad, dw.to(w.dtype))


def test_matches_oracle():
    from oracle.grpo_oracle import grpo_loss
    from oracle.grpo_step_oracle import grpo_step
    ko = _ko()
    h, w, t, mask, adv, old, ref = make(2, 6, 64, 1024, seed=3)
    B, S, D = h.shape
    ha = h.clone().requires_grad_(True)
    wa = w.clone().requires_grad_(True)
    loss, lp, ent = ko.fused_linear_grpo_step(ha, wa, t, old, adv, mask, ref, chunk_tokens=5,
                                              **KW)
    loss.backward()
    # Oracle on the GEMM's own bf16 logits (rows computed one chunk at a time
    # as the op does; compared to the full GEMM they agree here, checked below).
    logits = torch.mm(h.view(-1, D), w.t())
    chunked = torch.cat([torch.mm(h.view(-1, D)[n0:n0 + 5], w.t()) for n0 in range(0, B * S, 5)])
    assert torch.equal(logits, chunked)
    x = logits.view(B, S, -1).cpu().view(torch.int16).numpy().view(np.uint16)
    okw = dict(eps_low=0.2, eps_high=0.28, beta=0.04, loss_type="grpo")
    e_loss, e_lp, e_ent, e_d, _ = grpo_step(x, t.cpu().numpy(), old.cpu().numpy(),
                                            adv.cpu().numpy(), mask.cpu().numpy(),
                                            ref.cpu().numpy(), dtype="bf16", **okw)
    assert np.abs(lp.cpu().double().numpy() - e_lp).max() <= 2e-5
    assert np.abs(ent.cpu().double().numpy() - e_ent).max() <= 2e-5
    # The loss at the kernel's logp (its own 2e-5 logp error aside).
    k_loss, _, _ = grpo_loss(lp.cpu().double().numpy(), old.cpu().numpy(), adv.cpu().numpy(),
                             mask.cpu().numpy(), ref.cpu().numpy(), **okw)
    assert abs(loss.item() - k_loss) <= 1e-5 * max(1.0, abs(k_loss))
    d64 = e_d.reshape(B * S, -1)
    h64 = h.view(-1, D).cpu().double().numpy()
    w64 = w.cpu().double().numpy()
    for ours, ref_, bound in (
            (ha.grad.view(-1, D), d64 @ w64, np.abs(d64) @ np.abs(w64)),
            (wa.grad, d64.T @ h64, np.abs(d64).T @ np.abs(h64))):
        o = ours.cpu().double().numpy()
        assert np.all(np.abs(o - ref_) <= 2.0 ** -7 * bound + 2.0 ** -8 * np.abs(ref_) + 1e-12)


def test_sequence_level_runs_the_composition():
    ko = _ko()
    h, w, t, mask, adv, old, ref = make(2, 16, 64, 512, seed=4)
    B, S, D = h.shape
    ha = h.clone().requires_grad_(True)
    la, lpa, _ = ko.fused_linear_grpo_step(ha, w, t, old, adv, mask, ref,
                                           importance_level="sequence", **KW)
    la.backward()
    hb = h.clone().requires_grad_(True)
    lpb, _, _ = ko.fused_logprob_entropy(torch.matmul(hb, w.t()), t)
    lb, _ = ko.fused_grpo_loss(lpb, old, adv, mask, ref, importance_level="sequence", **KW)
    lb.backward()
    assert torch.equal(la, lb) and torch.equal(lpa, lpb)
    assert torch.equal(ha.grad, hb.grad)


def test_frozen_weight_and_scaled_loss():
    ko = _ko()
    h, w, t, mask, adv, old, ref = make(2, 40, 128, 1024, seed=5)
    ha = h.clone().requires_grad_(True)
    la, _, _ = ko.fused_linear_grpo_step(ha, w, t, old, adv, mask, ref, chunk_tokens=33, **KW)
    la.backward()
    hb = h.clone().requires_grad_(True)
    wb = w.clone().requires_grad_(True)
    lb, _, _ = ko.fused_linear_grpo_step(hb, wb, t, old, adv, mask, ref, chunk_tokens=33, **KW)
    (lb * 0.5).backward()
    assert torch.equal(la, lb)
    assert torch.equal(hb.grad, (ha.grad.float() * 0.5).to(h.dtype))
    with pytest.raises(RuntimeError, match="only once"):
        la.backward()
    # The same upstream gradient declared as grad_scale: applied in the
    # forward (a power of two, so the same bits), nothing left for the
    # backward to write.
    hc = h.clone().requires_grad_(True)
    wc = w.clone().requires_grad_(True)
    lc, _, _ = ko.fused_linear_grpo_step(hc, wc, t, old, adv, mask, ref, chunk_tokens=33,
                                         grad_scale=0.5, **KW)
    (lc * 0.5).backward()
    assert torch.equal(lc, lb)
    assert torch.equal(hc.grad, hb.grad) and torch.equal(wc.grad, wb.grad)


def test_qwen_head_shape_chunks():
    """Qwen2.5-7B's head (D = 3584, V = 152064) with 1024 tokens in chunks of
    384 against one chunk: the loss within 1e-5 relative; logp / entropy equal
    where the chunk GEMMs reproduce the full GEMM's logits, else within twice
    the row's largest logit difference (logp and H move by at most that)."""
    ko = _ko()
    h, w, t, mask, adv, old, ref = make(4, 256, 3584, 152064, seed=6)
    B, S, D = h.shape
    out_a = ko.fused_linear_grpo_step(h, w, t, old, adv, mask, ref, chunk_tokens=384, **KW)
    out_b = ko.fused_linear_grpo_step(h, w, t, old, adv, mask, ref, chunk_tokens=1024, **KW)
    assert abs(out_a[0].item() - out_b[0].item()) <= 1e-5 * max(1.0, abs(out_b[0].item()))
    h2 = h.view(-1, D)
    full = torch.mm(h2, w.t())
    chunked = torch.cat([torch.mm(h2[n0:n0 + 384], w.t()) for n0 in range(0, B * S, 384)])
    dx = (full.float() - chunked.float()).abs().amax(dim=-1).view(B, S)
    del full, chunked
    for a, b in zip(out_a[1:], out_b[1:]):
        assert torch.all((a - b).abs() <= 2 * dx + 2e-5)


def test_default_chunking_is_one_chunk_when_it_fits():
    """Without chunk_tokens, tokens that fit the default budget run as one
    chunk: the same results as chunk_tokens = all tokens."""
    ko = _ko()
    h, w, t, mask, adv, old, ref = make(2, 48, 128, 2048, seed=7)
    B, S, D = h.shape
    outs = []
    for chunk in (None, B * S):
        hh = h.clone().requires_grad_(True)
        ww = w.clone().requires_grad_(True)
        loss, lp, ent = ko.fused_linear_grpo_step(hh, ww, t, old, adv, mask, ref,
                                                  chunk_tokens=chunk, **KW)
        loss.backward()
        outs.append((loss, lp, ent, hh.grad, ww.grad))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_vocab_chunked_head_then_grpo_loss():
    """The memory-bounded alternative: the vocabulary-chunked LM head
    (fused_linear_logprob_entropy) then fused_grpo_loss, through autograd.
    Same loss and gradients as the token-chunked fused step up to the bf16
    rounding of each logit (the two compute the logits with different GEMM
    calls): loss within 1e-3 relative, gradients within 5% of their largest
    element, as the chunked head's own composition test."""
    ko = _ko()
    h, w, t, mask, adv, old, ref = make(2, 64, 256, 5000, seed=31)
    ha = h.clone().requires_grad_(True)
    wa = w.clone().requires_grad_(True)
    lp, _, _ = ko.fused_linear_logprob_entropy(ha, wa, t, chunk_vocab=1536)
    la, _ = ko.fused_grpo_loss(lp, old, adv, mask, ref, **KW)
    la.backward()
    hb = h.clone().requires_grad_(True)
    wb = w.clone().requires_grad_(True)
    lb, _, _ = ko.fused_linear_grpo_step(hb, wb, t, old, adv, mask, ref, **KW)
    lb.backward()
    assert torch.isfinite(la) and abs(la.item() - lb.item()) <= 1e-3 * max(1.0, abs(lb.item()))
    for a, b in ((ha.grad, hb.grad), (wa.grad, wb.grad)):
        a, b = a.float(), b.float()
        assert (a - b).abs().max() <= 0.05 * b.abs().max()
