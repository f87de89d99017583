"""GPU parity of the fused LM head (kernel_opt.lmhead), both implementations.

MFMA head (impl="mfma", klp_lmh_fwd) against the float64 oracle
(oracle/lmh_oracle.py, pinned in tests/test_lmh_cpu.py).  The kernel
accumulates each logit in fp32 (MFMA, 16-term blocks), so a logit can be off
by about sqrt(D / 16) roundings of the running sum of |h_k w_k|; logprob,
entropy and lse inherit at most the largest logit error of their row plus the
fp32 softmax noise.  Per token:
    |ours - oracle| <= 2e-5 + 8 * 2^-24 * sqrt(D / 16) * max_v sum_k |h_k w_k|.

Chunked head (impl="chunked", the default): the library GEMM rounds each
logit once to the input dtype, so the bar is the logprob kernels' own bar on
those logits (the float64 logits oracle, oracle/klp_oracle.py, on the chunk
GEMMs' output), plus a float64 check of the head itself whose bound follows
from the logit rounding: with every logit within eps of exact, lse moves by
at most eps, logp by 2 eps and the entropy by eps * sqrt(Var_p(x)) to first
order (the derivative of H is -p_v (x_v - mean_p x)).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import lmh_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make(N, V, D, seed, w_std=None, spike=False, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(N, D, generator=g).to(dtype)
    w = (torch.randn(V, D, generator=g) * (w_std or 3.0 / math.sqrt(D))).to(dtype)
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
    outs = fused_linear_logprob_entropy_forward(hd, w.to(DEV), td, temperature, impl="mfma")
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
    fused = fused_linear_logprob_entropy_forward(hd, wd, td, impl="mfma")
    logits = (hd @ wd.T)
    unfused = fused_logprob_entropy_forward(logits, td)
    half_ulp = logits.float().abs().amax(dim=1) * 2.0 ** -8
    for f, u in zip(fused, unfused):
        assert torch.all((f - u).abs() <= 2 * half_ulp + 1e-5)


def test_deterministic():
    from kernel_opt import fused_linear_logprob_entropy_forward
    h, w, t = make(333, 7777, 256, seed=11)
    hd, wd, td = h.to(DEV), w.to(DEV), t.to(DEV)
    for impl in ("mfma", "chunked"):
        a = fused_linear_logprob_entropy_forward(hd, wd, td, impl=impl)
        b = fused_linear_logprob_entropy_forward(hd, wd, td, impl=impl)
        assert all(torch.equal(x, y) for x, y in zip(a, b)), impl


def test_invalid_arguments_raise():
    from kernel_opt import fused_linear_logprob_entropy_forward
    h = torch.zeros(4, 100, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(10, 100, dtype=torch.bfloat16, device=DEV)
    t = torch.zeros(4, dtype=torch.int64, device=DEV)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        fused_linear_logprob_entropy_forward(h, w, t, impl="mfma")
    with pytest.raises(RuntimeError, match="bfloat16"):
        fused_linear_logprob_entropy_forward(h.float(), w.float(), t, impl="mfma")
    with pytest.raises(RuntimeError, match="share one dtype"):
        fused_linear_logprob_entropy_forward(h.float(), w, t)
    with pytest.raises(ValueError, match="impl"):
        fused_linear_logprob_entropy_forward(h, w, t, impl="dense")
    with pytest.raises(ValueError, match="chunk_vocab"):
        fused_linear_logprob_entropy_forward(h, w, t, chunk_vocab=0)
    with pytest.raises(RuntimeError, match="temperature"):
        fused_linear_logprob_entropy_forward(h, w, t, 0.0)


# ---------------------------------------------------------------------------
# Backward (klp_lmh_bwd_logits + library GEMMs)
# ---------------------------------------------------------------------------
def _grads(N, V, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(N, generator=g) for _ in range(3))


def _bwd_check(h, w, t, gl, ge, gs, temperature=None, need_w=True, chunk_vocab=None):
    from kernel_opt import fused_linear_logprob_entropy
    hd = h.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(need_w)
    lp, ent, lse = fused_linear_logprob_entropy(hd, wd, t.to(DEV), temperature, impl="mfma",
                                                chunk_vocab=chunk_vocab)
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


@pytest.mark.parametrize("N,V,D,chunk", [(130, 1000, 256, None), (64, 4099, 192, None),
                                         (300, 2001, 128, None), (64, 4099, 192, 1000),
                                         (33, 2001, 64, 333)])
def test_backward_matches_oracle(N, V, D, chunk):
    """The MFMA head's backward, also over vocabulary chunks whose width is
    not a multiple of four (the padded d_logits rows)."""
    h, w, t = make(N, V, D, seed=20 + N)
    t[::9] = -100
    t[1::13] = V
    _bwd_check(h, w, t, *_grads(N, V, 21), chunk_vocab=chunk)


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
    lp, ent, lse = fused_linear_logprob_entropy_forward(hd, wd, td, impl="mfma")
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


@pytest.mark.parametrize("impl", ["mfma", "chunked"])
def test_backward_matches_unfused_path(impl):
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
            lp, ent, _ = fused_linear_logprob_entropy(hd, wd, td, impl=impl, chunk_vocab=1536)
        else:
            lp, ent, _ = fused_logprob_entropy(hd @ wd.T, td)
        ((lp * gl.to(DEV)).sum() + (ent * ge.to(DEV)).sum()).backward()
        res.append((hd.grad.float(), wd.grad.float()))
    for a, b in zip(res[0], res[1]):
        scale = b.abs().max()
        assert (a - b).abs().max() <= 0.05 * scale


# ---------------------------------------------------------------------------
# Chunked head (library GEMM per vocabulary chunk + klp_fwd_shard / merge)
# ---------------------------------------------------------------------------
SIG_BITS = {torch.bfloat16: 8, torch.float16: 11, torch.float32: 24}


def _chunk_logits(hd, wd, plan):
    """The logits the chunked head computes: the same GEMM call per chunk of
    ``plan`` (a vocab_chunks list, or a width for equal chunks; the GEMM is
    deterministic, so the values are bit-identical to the head's own),
    concatenated."""
    from kernel_opt import lmhead
    h2 = hd.reshape(-1, hd.size(-1))
    N, V = h2.size(0), wd.size(0)
    if isinstance(plan, int):
        plan = [(c0, min(plan, V - c0)) for c0 in range(0, V, plan)]
    parts = []
    for c0, n in plan:
        buf = torch.empty(N * n, dtype=hd.dtype, device=DEV)
        parts.append(lmhead._chunk_logits(buf, h2, wd, c0, n).clone())
    return torch.cat(parts, dim=1)


def _f64(x):
    return x.double().cpu().numpy()


CHUNK_CASES = [  # N, V, D, dtype, chunk_vocab, temperature
    (1, 1, 64, torch.bfloat16, None, None),
    (5, 300, 64, torch.bfloat16, 7, None),
    (130, 1000, 256, torch.bfloat16, None, 0.7),
    (257, 4099, 192, torch.bfloat16, 1000, None),
    (64, 5000, 96, torch.float16, 1024, 1.3),
    (50, 2001, 80, torch.float32, 500, None),
    (300, 20000, 512, torch.bfloat16, None, None),
]


@pytest.mark.parametrize("N,V,D,dtype,chunk,T", CHUNK_CASES)
def test_chunked_forward(N, V, D, dtype, chunk, T, oracle):
    from kernel_opt import fused_linear_logprob_entropy_forward, vocab_chunks
    from klp_testutil import FWD_TOL
    h, w, t = make(N, V, D, seed=40 + N + V, dtype=dtype)
    t[::7] = -100
    t[3::11] = V
    hd, wd, td = h.to(DEV), w.to(DEV), t.to(DEV)
    lp, ent, lse = fused_linear_logprob_entropy_forward(hd, wd, td, T, chunk_vocab=chunk)
    x = _chunk_logits(hd, wd, vocab_chunks(N, V, h.element_size(), chunk))
    # (1) the logprob bar on the logits the chunks computed
    ref = oracle.forward(x.cpu(), t.numpy(), temperature=T)
    for name, o, r in zip(("logp", "entropy", "lse"), (lp, ent, lse), ref):
        err = np.abs(_f64(o) - r).max()
        assert err <= FWD_TOL[dtype], f"{name}: {err:.3g} > {FWD_TOL[dtype]}"
    bad = (t < 0) | (t >= V)
    assert torch.equal(lp.cpu()[bad], -lse.cpu()[bad])
    # (2) the head itself against float64 logits from the inputs
    s = oracle.scale_of(T)
    x64 = (_f64(h) @ _f64(w).T) * s
    p = np.exp(x64 - x64.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    mean = (p * x64).sum(axis=1)
    sd = np.sqrt(np.maximum((p * x64 * x64).sum(axis=1) - mean * mean, 0.0))
    lse64 = np.log(np.exp(x64 - x64.max(axis=1, keepdims=True)).sum(axis=1)) + x64.max(axis=1)
    ent64 = lse64 - mean
    lp64 = np.where(bad.numpy(), -lse64, x64[np.arange(N), np.clip(t.numpy(), 0, V - 1)] - lse64)
    # logit error: one rounding to the input dtype of |x| plus the fp32
    # accumulation of D products (and the fp32 scaling)
    acc = (np.abs(_f64(h)) @ np.abs(_f64(w)).T) * s
    eps = (np.abs(x64).max(axis=1) * 2.0 ** -SIG_BITS[dtype]
           + D * 2.0 ** -24 * acc.max(axis=1) + 2.0 ** -24 * np.abs(x64).max(axis=1))
    for name, o, r, k in (("lse", lse, lse64, eps), ("logp", lp, lp64, 2 * eps),
                          ("entropy", ent, ent64, eps * sd)):
        err = np.abs(_f64(o) - r)
        tol = 2 * k + 2e-5
        assert np.all(err <= tol), f"{name} vs float64 head: {(err / tol).max():.3g}x the bound"


def test_chunked_headline_vocab_and_hidden(oracle):
    """Qwen2.5-7B's head (V = 152064, D = 3584), 300 tokens, default chunks:
    the logprob bar on the chunks' logits."""
    from kernel_opt import fused_linear_logprob_entropy_forward, vocab_chunks
    h, w, t = make(300, 152064, 3584, seed=7, spike=True)
    hd, wd, td = h.to(DEV), w.to(DEV), t.to(DEV)
    outs = fused_linear_logprob_entropy_forward(hd, wd, td)
    x = _chunk_logits(hd, wd, vocab_chunks(300, 152064))
    ref = oracle.forward(x.cpu(), t.numpy())
    for name, o, r in zip(("logp", "entropy", "lse"), outs, ref):
        err = np.abs(_f64(o) - r).max()
        assert err <= 2e-5, f"{name}: {err:.3g}"


def test_chunked_strided_hidden_and_leading_dims(oracle):
    from kernel_opt import fused_linear_logprob_entropy_forward
    g = torch.Generator().manual_seed(9)
    full = torch.randn(3, 41, 128, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(999, 128, generator=g) * 0.25).to(torch.bfloat16).to(DEV)
    t = torch.randint(0, 999, (3, 40), generator=g)
    view = full[:, :-1, :]
    outs = fused_linear_logprob_entropy_forward(view, w, t.to(DEV), chunk_vocab=256)
    assert outs[0].shape == (3, 40)
    x = _chunk_logits(view.reshape(-1, 128), w, 256)
    ref = oracle.forward(x.cpu(), t.reshape(-1).numpy())
    for o, r in zip(outs, ref):
        assert np.abs(_f64(o).reshape(-1) - r).max() <= 2e-5


BWD_CASES = [  # N, V, D, dtype, chunk_vocab, temperature, need_w
    (130, 1000, 256, torch.bfloat16, None, None, True),
    (64, 4099, 192, torch.bfloat16, 1000, 0.7, True),
    (33, 2001, 64, torch.bfloat16, 333, None, False),
    (100, 3000, 128, torch.float16, 1024, 1.3, True),
    (50, 2001, 80, torch.float32, 500, None, True),
]


@pytest.mark.parametrize("N,V,D,dtype,chunk,T,need_w", BWD_CASES)
def test_chunked_backward(N, V, D, dtype, chunk, T, need_w, oracle):
    """d_hidden / d_weight against the float64 closed form on the chunks'
    logits: d_logits within one rounding to the input dtype (plus the fp32
    evaluation noise of its row), carried through the two products, whose
    outputs are rounded once more and accumulate in fp32."""
    from kernel_opt import fused_linear_logprob_entropy, vocab_chunks
    h, w, t = make(N, V, D, seed=60 + N, dtype=dtype)
    t[::9] = -100
    t[1::13] = V
    gl, ge, gs = _grads(N, V, 61)
    hd = h.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(need_w)
    td = t.to(DEV)
    lp, ent, lse = fused_linear_logprob_entropy(hd, wd, td, T, chunk_vocab=chunk)
    ((lp * gl.to(DEV)).sum() + (ent * ge.to(DEV)).sum() + (lse * gs.to(DEV)).sum()).backward()
    x = _chunk_logits(hd.detach(), wd.detach(), vocab_chunks(N, V, h.element_size(), chunk))
    r_lp, r_h, r_l = oracle.forward(x.cpu(), t.numpy(), temperature=T)
    dl = oracle.backward(x.cpu(), t.numpy(), r_l, r_h, gl.double().numpy(), ge.double().numpy(),
                         gs.double().numpy(), temperature=T)
    hf, wf = _f64(h), _f64(w)
    p = SIG_BITS[dtype]
    dl_err = 2.0 ** -(p - 1) * np.abs(dl) + 2.0 ** -20 * np.abs(dl).max(axis=1, keepdims=True)
    ref_dh = dl @ wf
    bound_h = (dl_err @ np.abs(wf) + 2.0 ** -p * np.abs(ref_dh)
               + V * 2.0 ** -24 * (np.abs(dl) @ np.abs(wf)) + 1e-30)
    err_h = np.abs(_f64(hd.grad) - ref_dh)
    assert np.all(err_h <= bound_h), f"d_hidden: {(err_h / bound_h).max():.3g}x the bound"
    if need_w:
        ref_dw = dl.T @ hf
        bound_w = (dl_err.T @ np.abs(hf) + 2.0 ** -p * np.abs(ref_dw)
                   + N * 2.0 ** -24 * (np.abs(dl).T @ np.abs(hf)) + 1e-30)
        err_w = np.abs(_f64(wd.grad) - ref_dw)
        assert np.all(err_w <= bound_w), f"d_weight: {(err_w / bound_w).max():.3g}x the bound"
    else:
        assert wd.grad is None


def test_chunked_holds_no_full_logits():
    """At 1024 tokens of Qwen2.5-7B's vocabulary (V = 152064, with D = 1024
    to keep the weight small) neither pass allocates anything near the
    [N, V] logits (311 MB in bf16): forward and backward stay below half of
    it beyond their outputs and the weight gradient."""
    from kernel_opt import fused_linear_logprob_entropy
    N, V, D = 1024, 152064, 1024
    g = torch.Generator(device=DEV).manual_seed(3)
    h = torch.randn(N, D, device=DEV, generator=g).to(torch.bfloat16).requires_grad_(True)
    w = (torch.randn(V, D, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    w.requires_grad_(True)
    t = torch.randint(0, V, (N,), device=DEV, generator=g)
    full = N * V * 2
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    lp, ent, _ = fused_linear_logprob_entropy(h, w, t)
    torch.cuda.synchronize()
    fwd_extra = torch.cuda.max_memory_allocated() - base
    assert fwd_extra < full // 2, f"forward peak {fwd_extra / 2**20:.0f} MiB beyond the inputs"
    (lp.sum() + ent.sum()).backward()
    torch.cuda.synchronize()
    grads = w.grad.numel() * 2 + h.grad.numel() * 2
    bwd_extra = torch.cuda.max_memory_allocated() - base - grads
    assert bwd_extra < full // 2, f"backward peak {bwd_extra / 2**20:.0f} MiB beyond the grads"
