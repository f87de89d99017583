"""GPU parity of the fused LM head forward (klp_lmh_fwd) against the float64
oracle (oracle/lmh_oracle.py, pinned in tests/test_lmh_cpu.py).

Bar: the kernel accumulates each logit in fp32 (MFMA, 16-term blocks), so a
logit can be off by about sqrt(D / 16) roundings of the running sum of
|h_k w_k|; logprob, entropy and lse inherit at most the largest logit error
of their row plus the fp32 softmax noise.  Per token:
    |ours - oracle| <= 2e-5 + 8 * 2^-24 * sqrt(D / 16) * max_v sum_k |h_k w_k|.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import lmh_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make(N, V, D, seed, w_std=None, spike=False):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(N, D, generator=g).to(torch.bfloat16)
    w = (torch.randn(V, D, generator=g) * (w_std or 3.0 / math.sqrt(D))).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), generator=g)
    if spike:
        w[t[: min(N, V)] % V] *= 4
    return h, w, t


def bits(x):
    return x.contiguous().view(torch.int16).numpy().view(np.uint16)


def check(h, w, t, temperature=None, hidden_dev=None, targets_dev=None, label=""):
    from kernel_opt import fused_linear_logprob_entropy_forward
    hd = hidden_dev if hidden_dev is not None else h.to(DEV)
    td = targets_dev if targets_dev is not None else t.to(DEV)
    outs = fused_linear_logprob_entropy_forward(hd, w.to(DEV), td, temperature)
    ref = lmh_oracle.forward(bits(h), bits(w), t.numpy(), temperature)
    D = h.size(-1)
    mag = lmh_oracle.magnitude(bits(h), bits(w))
    scale = lmh_oracle.scale_of(temperature)
    tol = 2e-5 + 8 * 2.0 ** -24 * math.sqrt(D / 16) * mag * scale
    for name, o, r in zip(("logp", "entropy", "lse"), outs, ref):
        err = np.abs(o.cpu().double().numpy().reshape(-1) - r)
        assert np.all(err <= tol), f"{label} {name}: max err {err.max():.3g}, tol {tol.min():.3g}"
    return outs


@pytest.mark.parametrize("N,V,D", [(1, 1, 64), (5, 300, 64), (128, 256, 128), (130, 1000, 256),
                                   (257, 4099, 192), (64, 151936 // 8, 896)])
def test_matches_oracle(N, V, D):
    h, w, t = make(N, V, D, seed=N + V + D)
    check(h, w, t, label=f"{N}x{V}x{D}")


def test_headline_vocab_and_hidden():
    """Qwen2.5-7B's head: V = 152064, D = 3584, with 300 tokens."""
    h, w, t = make(300, 152064, 3584, seed=7, spike=True)
    check(h, w, t, label="qwen7b head")


def test_temperature_and_out_of_range_targets():
    h, w, t = make(200, 3000, 320, seed=8)
    t[::7] = -100
    t[3::11] = 3000
    outs = check(h, w, t, temperature=0.7)
    lp, _, lse = (o.cpu() for o in outs)
    bad = (t < 0) | (t >= 3000)
    assert torch.equal(lp[bad], -lse[bad])


def test_strided_hidden_and_leading_dims():
    g = torch.Generator().manual_seed(9)
    full = torch.randn(3, 41, 128, generator=g).to(torch.bfloat16)
    w = (torch.randn(999, 128, generator=g) * 0.25).to(torch.bfloat16)
    t = torch.randint(0, 999, (3, 40), generator=g)
    view = full.to(DEV)[:, :-1, :]
    outs = check(full[:, :-1, :].reshape(-1, 128), w, t.reshape(-1), hidden_dev=view,
                 targets_dev=t.to(DEV))
    assert outs[0].shape == (3, 40)


def test_matches_unfused_path_up_to_bf16_logit_rounding():
    """The unfused path (bf16 matmul, then the logprob kernel) rounds every
    logit to bf16; the fused one does not.  Both stay within the bf16
    rounding of the logits of each other."""
    from kernel_opt import fused_linear_logprob_entropy_forward, fused_logprob_entropy_forward
    h, w, t = make(256, 20000, 512, seed=10)
    hd, wd, td = h.to(DEV), w.to(DEV), t.to(DEV)
    fused = fused_linear_logprob_entropy_forward(hd, wd, td)
    logits = (hd @ wd.T)
    unfused = fused_logprob_entropy_forward(logits, td)
    half_ulp = logits.float().abs().amax(dim=1) * 2.0 ** -8
    for f, u in zip(fused, unfused):
        assert torch.all((f - u).abs() <= 2 * half_ulp + 1e-5)


def test_deterministic():
    from kernel_opt import fused_linear_logprob_entropy_forward
    h, w, t = make(333, 7777, 256, seed=11)
    hd, wd, td = h.to(DEV), w.to(DEV), t.to(DEV)
    a = fused_linear_logprob_entropy_forward(hd, wd, td)
    b = fused_linear_logprob_entropy_forward(hd, wd, td)
    assert all(torch.equal(x, y) for x, y in zip(a, b))


def test_invalid_arguments_raise():
    from kernel_opt import fused_linear_logprob_entropy_forward
    h = torch.zeros(4, 100, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(10, 100, dtype=torch.bfloat16, device=DEV)
    t = torch.zeros(4, dtype=torch.int64, device=DEV)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        fused_linear_logprob_entropy_forward(h, w, t)
    with pytest.raises(RuntimeError, match="bfloat16"):
        fused_linear_logprob_entropy_forward(h.float(), w, t)


# ---------------------------------------------------------------------------
# Backward (klp_lmh_bwd_logits + library GEMMs)
# ---------------------------------------------------------------------------
def _grads(N, V, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(N, generator=g) for _ in range(3))


def _bwd_check(h, w, t, gl, ge, gs, temperature=None, need_w=True):
    from kernel_opt import fused_linear_logprob_entropy
    hd = h.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(need_w)
    lp, ent, lse = fused_linear_logprob_entropy(hd, wd, t.to(DEV), temperature)
    loss = 0
    for out, gg in ((lp, gl), (ent, ge), (lse, gs)):
        if gg is not None:
            loss = loss + (out * gg.to(DEV)).sum()
    loss.backward()
    ref_dh, ref_dw, ref_dl = lmh_oracle.backward(
        bits(h), bits(w), t.numpy(), *(None if gg is None else gg.numpy() for gg in (gl, ge, gs)),
        temperature=temperature)
    hf, wf = lmh_oracle.bf16_to_f64(bits(h)), lmh_oracle.bf16_to_f64(bits(w))
    # bf16 rounding of d_logits and of the GEMM outputs (fp32 accumulation)
    bound_h = 2.0 ** -7 * (np.abs(ref_dl) @ np.abs(wf)) + 2.0 ** -8 * np.abs(ref_dh) + 1e-7
    err_h = np.abs(hd.grad.float().cpu().numpy() - ref_dh)
    assert np.all(err_h <= bound_h), f"d_hidden err {err_h.max():.3g}"
    if need_w:
        bound_w = 2.0 ** -7 * (np.abs(ref_dl).T @ np.abs(hf)) + 2.0 ** -8 * np.abs(ref_dw) + 1e-7
        err_w = np.abs(wd.grad.float().cpu().numpy() - ref_dw)
        assert np.all(err_w <= bound_w), f"d_weight err {err_w.max():.3g}"
    else:
        assert wd.grad is None


@pytest.mark.parametrize("N,V,D", [(130, 1000, 256), (64, 4099, 192), (300, 2001, 128)])
def test_backward_matches_oracle(N, V, D):
    h, w, t = make(N, V, D, seed=20 + N)
    t[::9] = -100
    _bwd_check(h, w, t, *_grads(N, V, 21))


def test_backward_temperature_and_partial_grads():
    h, w, t = make(100, 3000, 256, seed=22)
    gl, ge, _ = _grads(100, 3000, 23)
    _bwd_check(h, w, t, gl, None, None, temperature=0.7)
    _bwd_check(h, w, t, None, ge, None, need_w=False)


def test_backward_d_logits_against_oracle():
    """The recomputed d_logits, rounded once to bf16, against the float64
    closed form: within one bf16 rounding of each value plus the fp32
    evaluation noise of its row."""
    import ctypes
    from kernel_opt import fused_linear_logprob_entropy_forward
    from kernel_opt._library import lib
    N, V, D = 96, 3001, 192
    h, w, t = make(N, V, D, seed=24)
    gl, ge, gs = _grads(N, V, 25)
    hd, wd, td = h.to(DEV), w.to(DEV), t.to(DEV)
    lp, ent, lse = fused_linear_logprob_entropy_forward(hd, wd, td)
    ld = (V + 3) // 4 * 4 + 8
    d = torch.full((N, ld), 7.0, dtype=torch.bfloat16, device=DEV)
    G = [x.to(DEV) for x in (gl, ge, gs)]
    P = lambda x: ctypes.c_void_p(x.data_ptr())
    rc = lib.klp_lmh_bwd_logits(P(hd), D, P(wd), D, N, V, D, P(td), 1.0, P(lse), P(ent),
                                P(G[0]), P(G[1]), P(G[2]), P(d), ld,
                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    got = d[:, :V].float().cpu().numpy()
    v4 = (V + 3) // 4 * 4
    assert torch.all(d[:, V:v4].cpu() == 0.0)  # the last group of four, zero-filled
    assert torch.all(d[:, v4:].cpu() == 7.0)   # columns past it untouched
    _, _, ref = lmh_oracle.backward(bits(h), bits(w), t.numpy(), gl.numpy(), ge.numpy(),
                                    gs.numpy())
    row_noise = 2.0 ** -20 * np.abs(ref).max(axis=1, keepdims=True)
    assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + row_noise)


def test_backward_matches_unfused_path():
    """Same gradients as logits = hidden @ weight^T followed by the
    autograd logprob kernel, up to the bf16 rounding of the logits."""
    from kernel_opt import fused_linear_logprob_entropy, fused_logprob_entropy
    h, w, t = make(200, 5000, 256, seed=26)
    gl, ge, _ = _grads(200, 5000, 27)
    res = []
    for fused in (True, False):
        hd = h.to(DEV).requires_grad_(True)
        wd = w.to(DEV).requires_grad_(True)
        td = t.to(DEV)
        if fused:
            lp, ent, _ = fused_linear_logprob_entropy(hd, wd, td)
        else:
            lp, ent, _ = fused_logprob_entropy(hd @ wd.T, td)
        ((lp * gl.to(DEV)).sum() + (ent * ge.to(DEV)).sum()).backward()
        res.append((hd.grad.float(), wd.grad.float()))
    for a, b in zip(res[0], res[1]):
        scale = b.abs().max()
        assert (a - b).abs().max() <= 0.05 * scale
