"""GPU parity of the fused GRPO step (klp_grpo_step.hip), called through the
C ABI (kernel_opt.grpo_step.grpo_step_launch -> klp_grpo_step).

Bars:
  * logprob / entropy / lse against the float64 oracle (klp_oracle.c) within
    the forward tolerance (1e-5 fp32 input, 2e-5 bf16 / fp16 input);
  * the loss against the float64 GRPO oracle evaluated at the kernel's own
    log-probabilities, within 1e-5 relative;
  * d_logits equal, value for value, to klp_bwd's output for the same row
    statistics and upstream gradient (the step uses klp_bwd's formula), that
    upstream gradient being klp_grpo_bwd's d_logp at the kernel's
    log-probabilities; and d_logits within klp_bwd's own bar against the
    float64 oracle's backward (1 ulp of the output dtype, or the fp32 noise of
    cancelling terms: klp_testutil.grad_check);
  * at the C2 size ([4, 256, 152064] bf16) against the unfused composition
    (fused_logprob_entropy + fused_grpo_loss + backward): loss within 1e-5
    relative, logprob / entropy within twice the forward tolerance, d_logits
    within 1 bf16 ulp;
  * repeated calls are bitwise identical.
Inputs are generated on the CPU from fixed seeds and copied to the GPU.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from klp_testutil import FWD_TOL, grad_check, storage_bits, ulp_diff
from oracle.grpo_oracle import grpo_loss

pytestmark = pytest.mark.gpu
DEV = "cuda"
IGNORE = -100


def _ko():
    import kernel_opt
    return kernel_opt


def make_case(B, S, V, dtype, seed, adv_per_token=False, neg_inf=False):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, S, V, generator=g) * 2.0).to(dtype)
    if neg_inf:
        x[0, 0, ::7] = float("-inf")
        x[-1, -1, : V // 2] = float("-inf")
    t = torch.randint(0, V, (B, S), generator=g)
    if S > 1:
        t[0, 1] = IGNORE
    mask = (torch.rand(B, S, generator=g) < 0.75).float()
    mask[0, 0] = 1.0
    adv = torch.randn((B, S) if adv_per_token else (B,), generator=g)
    return x, t, mask, adv


def old_ref(logp_cpu: torch.Tensor, seed: int):
    g = torch.Generator().manual_seed(seed + 1)
    old = logp_cpu + 0.3 * torch.randn(logp_cpu.shape, generator=g)
    ref = logp_cpu + 0.3 * torch.randn(logp_cpu.shape, generator=g)
    return old.float(), ref.float()


def oracle_kw(loss_type, beta, B, L=None, normalizer=None):
    kind = loss_type if loss_type in ("grpo", "bnpo") else "fixed"
    norm = {"dr_grpo": float(B * (L or 1)), "dapo": normalizer}.get(loss_type, 1.0)
    return dict(eps_low=0.2, eps_high=0.28, beta=beta, loss_type=kind, norm_const=norm)


def run_step(x, t, old, adv, mask, ref, loss_type, beta, temperature=None, grad_scale=1.0,
             **extra):
    """klp_grpo_step on the GPU; returns (logp, ent, lse, loss_tok, d) on the GPU."""
    from kernel_opt.grpo_step import grpo_step_launch, grpo_token_weights
    B, S, _ = x.shape
    w = grpo_token_weights(mask.to(DEV), loss_type, **extra).contiguous()
    params = (1.0 if temperature is None else temperature, 0.2, 0.28, beta,
              int(adv.dim() != 1), grad_scale)
    r = ref.to(DEV) if (beta != 0.0 and ref is not None) else None
    return grpo_step_launch(x.to(DEV), t.to(DEV), old.to(DEV), r, adv.to(DEV), w, params)


def unfused_g_logp(logp, old, adv, mask, ref, loss_type, beta, **extra):
    """klp_grpo_bwd's d_logp at the given log-probabilities."""
    lp = logp.detach().clone().requires_grad_(True)
    loss, _ = _ko().fused_grpo_loss(lp, old.to(DEV), adv.to(DEV), mask.to(DEV),
                                    None if ref is None else ref.to(DEV), eps_low=0.2,
                                    eps_high=0.28, beta=beta, loss_type=loss_type, **extra)
    loss.backward()
    return lp.grad


def unfused_bwd(x, t, lse, ent, g, temperature=None):
    from kernel_opt import _C
    d = torch.empty(x.shape, dtype=x.dtype, device=DEV)
    _C.bwd_launch(x, t, lse, ent, g.contiguous(), None, None, d, temperature=temperature)
    return d


CASES = [
    # (dtype, B, S, V)
    (torch.bfloat16, 3, 5, 64),       # fewer vectors than threads
    (torch.bfloat16, 3, 5, 8192),     # exactly one vector per thread, no partial one
    (torch.bfloat16, 2, 4, 12000),    # a partial last vector
    (torch.bfloat16, 1, 3, 152064),   # the C2 vocabulary
    (torch.bfloat16, 1, 2, 155648),   # the row capacity
    (torch.float16, 3, 5, 4096),
    (torch.float16, 1, 3, 152064),
    (torch.float32, 3, 5, 4096),
    (torch.float32, 2, 3, 77824),     # the fp32 row capacity
]


@pytest.mark.parametrize("dtype,B,S,V", CASES)
@pytest.mark.parametrize("loss_type,beta,temperature", [("bnpo", 0.0, None),
                                                        ("grpo", 0.04, 0.7),
                                                        ("dr_grpo", 0.0, 1.3)])
def test_matches_oracle(dtype, B, S, V, loss_type, beta, temperature, oracle):
    seed = 100 + V % 97 + B
    print(f"grpo step: dtype={dtype} shape={(B, S, V)} {loss_type} beta={beta} T={temperature}",
          flush=True)
    x, t, mask, adv = make_case(B, S, V, dtype, seed, adv_per_token=(loss_type == "grpo"))
    e_lp, e_ent, e_lse = oracle.forward(x, t.numpy(), temperature=temperature)
    old, ref = old_ref(torch.tensor(e_lp), seed)
    extra = dict(max_completion_length=S + 3) if loss_type == "dr_grpo" else {}
    logp, ent, lse, loss_tok, d = run_step(x, t, old, adv, mask, ref, loss_type, beta,
                                           temperature, **extra)
    tol = FWD_TOL[dtype]
    for name, ours, e in (("logp", logp, e_lp), ("entropy", ent, e_ent), ("lse", lse, e_lse)):
        err = np.abs(ours.cpu().double().numpy() - e).max()
        assert err <= tol, f"{name}: {err:.3g} > {tol}"

    okw = oracle_kw(loss_type, beta, B, S + 3)
    r = ref.numpy() if beta != 0.0 else None
    k_lp = logp.cpu().double().numpy()
    e_loss, _, e_g = grpo_loss(k_lp, old.numpy(), adv.numpy(), mask.numpy(), r, **okw)
    loss = loss_tok.sum().item()
    assert abs(loss - e_loss) <= 1e-5 * max(1.0, abs(e_loss)), (loss, e_loss)

    g = unfused_g_logp(logp, old, adv, mask, ref if beta != 0.0 else None, loss_type, beta,
                       **extra)
    gmax = np.abs(e_g).max()
    assert np.all(np.abs(g.cpu().double().numpy() - e_g) <= 1e-5 * gmax + 1e-5 * np.abs(e_g))
    d_ref = unfused_bwd(x.to(DEV), t.to(DEV), lse, ent, g, temperature)
    assert torch.equal(d, d_ref), "d_logits differ from klp_bwd with the same inputs"
    worst, detail = grad_check(oracle, x, t, lse, ent, d, g_logp=g, temperature=temperature)
    assert worst <= 1.0, detail


def test_neg_inf_logits_and_masked_rows(oracle):
    """-inf logits (the clamped rescan) get a zero gradient; masked tokens
    get an all-zero d_logits row."""
    B, S, V = 2, 4, 4096
    x, t, mask, adv = make_case(B, S, V, torch.bfloat16, 7, neg_inf=True)
    mask[1, 2] = 0.0
    t[0, 0] = 1        # finite targets in the rows with -inf logits (a -inf
    t[-1, -1] = V - 1  # target logit would make the token's loss NaN)
    e_lp, e_ent, e_lse = oracle.forward(x, t.numpy())
    old, ref = old_ref(torch.tensor(e_lp), 7)
    logp, ent, lse, _, d = run_step(x, t, old, adv, mask, ref, "bnpo", 0.04)
    for ours, e in ((logp, e_lp), (ent, e_ent), (lse, e_lse)):
        assert np.abs(ours.cpu().double().numpy() - e).max() <= 2e-5
    dc = d.cpu().float()
    assert torch.all(dc[torch.isinf(x.float())] == 0)
    assert torch.all(dc[1, 2] == 0)
    g = unfused_g_logp(logp, old, adv, mask, ref, "bnpo", 0.04)
    assert torch.equal(d, unfused_bwd(x.to(DEV), t.to(DEV), lse, ent, g))


def test_sliced_logits_match_contiguous():
    """The shifted slice logits[:, :-1, :] runs in place (row strides) with the
    same results as its contiguous copy."""
    B, L, V = 3, 6, 8192
    x_full, _, _, _ = make_case(B, L, V, torch.bfloat16, 9)
    x_full = x_full.to(DEV)
    view = x_full[:, :-1, :]
    S = L - 1
    _, t, mask, adv = make_case(B, S, V, torch.bfloat16, 10)
    old = torch.full((B, S), -9.0)
    a = run_step(view, t, old, adv, mask, None, "grpo", 0.0)
    b = run_step(view.contiguous(), t, old, adv, mask, None, "grpo", 0.0)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_repeatable():
    x, t, mask, adv = make_case(2, 8, 152064, torch.bfloat16, 11)
    old = torch.full((2, 8), -11.0)
    a = run_step(x, t, old, adv, mask, None, "bnpo", 0.0)
    b = run_step(x, t, old, adv, mask, None, "bnpo", 0.0)
    for u, v in zip(a, b):
        assert torch.equal(u.view(torch.uint8) if u.dtype != torch.float32 else u,
                           v.view(torch.uint8) if v.dtype != torch.float32 else v)


def test_autograd_op():
    """fused_grpo_step: loss.backward() delivers the kernel's d_logits; a
    scaled loss scales it; the backward runs once; logp / entropy carry no
    gradient."""
    ko = _ko()
    B, S, V = 2, 6, 4096
    x, t, mask, adv = make_case(B, S, V, torch.bfloat16, 12)
    old = torch.full((B, S), -8.0)
    _, _, _, lt, d = run_step(x, t, old, adv, mask, None, "bnpo", 0.0)
    xg = x.to(DEV).requires_grad_(True)
    loss, logp, ent = ko.fused_grpo_step(xg, t.to(DEV), old.to(DEV), adv.to(DEV), mask.to(DEV))
    assert not logp.requires_grad and not ent.requires_grad
    assert torch.equal(loss, lt.sum())
    loss.backward()
    assert torch.equal(xg.grad, d)
    with pytest.raises(RuntimeError, match="only once"):
        loss.backward()

    xg2 = x.to(DEV).requires_grad_(True)
    loss2, _, _ = ko.fused_grpo_step(xg2, t.to(DEV), old.to(DEV), adv.to(DEV), mask.to(DEV))
    (loss2 * 0.3).backward()
    assert torch.equal(xg2.grad, (d.float() * torch.tensor(0.3, device=DEV)).to(d.dtype))


def test_host_targets_raise_before_any_launch(monkeypatch):
    """targets in host memory raise RuntimeError before either path is chosen
    (the fused kernel would read the host pointer as device memory).  The
    kernel's entry point is replaced by a stub that fails, so that no kernel
    can launch even if the check regressed."""
    ko = _ko()
    from kernel_opt import grpo_step as gs

    def no_launch(*args, **kwargs):
        raise AssertionError("klp_grpo_step was called with host targets")
    monkeypatch.setattr(gs.lib, "klp_grpo_step", no_launch)
    B, S, V = 2, 3, 4096
    x, t, mask, adv = make_case(B, S, V, torch.bfloat16, 31)
    xg = x.to(DEV).requires_grad_(True)
    old = torch.full((B, S), -9.0, device=DEV)
    with pytest.raises(RuntimeError, match="targets must be on"):
        ko.fused_grpo_step(xg, t, old, adv.to(DEV), mask.to(DEV))


@pytest.mark.parametrize("mode", ["no_grad", "leaf_without_grad"])
def test_call_without_gradient_writes_no_d_logits(mode):
    """Under torch.no_grad(), or for logits that do not require a gradient,
    fused_grpo_step runs the forward composition: peak memory stays below one
    [B, S, V] buffer (the fused kernel would write a full d_logits), and the
    loss equals the composition's."""
    ko = _ko()
    B, S, V = 4, 64, 152064
    print(f"grpo step without gradient: {mode}", flush=True)
    x, t, mask, adv = make_case(B, S, V, torch.bfloat16, 32)
    x, t, mask, adv = x.to(DEV), t.to(DEV), mask.to(DEV), adv.to(DEV)
    if mode == "no_grad":
        x.requires_grad_(True)
    old = torch.full((B, S), -11.0, device=DEV)
    kw = dict(eps_low=0.2, eps_high=0.28, loss_type="grpo")
    ko.fused_grpo_step(x.detach(), t, old, adv, mask, **kw)  # warm caches and workspaces
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    if mode == "no_grad":
        with torch.no_grad():
            loss, lp, _ = ko.fused_grpo_step(x, t, old, adv, mask, **kw)
    else:
        loss, lp, _ = ko.fused_grpo_step(x, t, old, adv, mask, **kw)
    torch.cuda.synchronize()
    extra = torch.cuda.max_memory_allocated() - base
    assert extra < x.numel() * x.element_size() // 4, f"{extra} bytes allocated"
    with torch.no_grad():
        lpb, _, _ = ko.fused_logprob_entropy_forward(x, t)
        lb, _ = ko.fused_grpo_loss(lpb, old, adv, mask, **kw)
    assert torch.equal(loss, lb) and torch.equal(lp, lpb)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_scale_by_upstream(dtype):
    """klp_scale_inplace (through scale_by_upstream), which applies the loss's
    upstream gradient without reading it on the host: t * g multiplied in
    float32 and rounded once, bit for bit as torch's t.float() * g; g == 1
    leaves the bits untouched; every alignment of start and length (the
    kernel's scalar head and tail), and nothing outside the view is written."""
    from kernel_opt.grpo_step import scale_by_upstream
    gen = torch.Generator().manual_seed(21)
    base = (torch.randn(1 << 20, generator=gen) * 3).to(dtype).to(DEV)
    bits = {torch.float32: torch.int32}.get(dtype, torch.int16)
    for off, n in ((0, 0), (0, 1), (1, 7), (3, 8), (0, 4097), (5, (1 << 20) - 9),
                   (0, 1 << 20)):
        for sc in (0.3, -2.5, 0.0, 1.0):
            print(f"scale: dtype={dtype} off={off} n={n} g={sc}", flush=True)
            buf = base.clone()
            view = buf[off:off + n]
            scale_by_upstream(view, torch.tensor(sc, device=DEV))
            src = base[off:off + n]
            exp = src if sc == 1.0 else (src.float() * sc).to(dtype)
            assert torch.equal(view.view(bits), exp.view(bits))
            assert torch.equal(buf[:off], base[:off])
            assert torch.equal(buf[off + n:], base[off + n:])
    # A buffer already scaled by a declared upstream gradient (applied):
    # g == applied writes nothing, any other g multiplies by fp32(g / applied).
    for off, n in ((1, 7), (0, 4097), (5, (1 << 20) - 9)):
        for applied, sc in ((0.125, 0.125), (0.125, 0.3), (0.125, 1.0), (-3.0, -3.0),
                            (-3.0, 0.7), (1.0 / 3.0, 1.0)):
            print(f"rescale: dtype={dtype} off={off} n={n} applied={applied} g={sc}", flush=True)
            buf = base.clone()
            view = buf[off:off + n]
            scale_by_upstream(view, torch.tensor(sc, device=DEV), applied)
            src = base[off:off + n]
            factor = float(np.float32(np.float32(sc) / np.float32(applied)))
            exp = src if np.float32(sc) == np.float32(applied) else (src.float() * factor).to(dtype)
            assert torch.equal(view.view(bits), exp.view(bits))
            assert torch.equal(buf[:off], base[:off])
            assert torch.equal(buf[off + n:], base[off + n:])


@pytest.mark.parametrize("c", [0.125, -2.0, 1.0 / 3.0])
def test_grad_scale_folds_the_upstream_gradient(c):
    """grad_scale c: klp_grpo_step writes d_logits already multiplied by c
    (the loss terms unscaled); through fused_grpo_step, an upstream gradient
    equal to c leaves the forward's d_logits as the gradient (nothing
    written), and any other is applied as the ratio to c."""
    ko = _ko()
    B, S, V = 3, 40, 152064
    print(f"grad_scale {c}", flush=True)
    x, t, mask, adv = make_case(B, S, V, torch.bfloat16, 41)
    old = torch.full((B, S), -8.0)
    lp1, en1, _, lt1, d1 = run_step(x, t, old, adv, mask, None, "grpo", 0.0)
    lpc, enc, _, ltc, dc = run_step(x, t, old, adv, mask, None, "grpo", 0.0, grad_scale=c)
    assert torch.equal(lpc, lp1) and torch.equal(enc, en1) and torch.equal(ltc, lt1)
    ref = (d1.float() * c).to(d1.dtype)
    if c in (0.125, -2.0):  # a power of two: the same bits either way
        assert torch.equal(dc, ref)
    else:  # one rounding against two
        assert int(ulp_diff(storage_bits(dc), storage_bits(ref), 16).max()) <= 1

    xg = x.to(DEV).requires_grad_(True)
    loss, _, _ = ko.fused_grpo_step(xg, t.to(DEV), old.to(DEV), adv.to(DEV), mask.to(DEV),
                                    loss_type="grpo", grad_scale=c)
    assert torch.equal(loss, lt1.sum())
    (loss * c).backward()
    assert torch.equal(xg.grad, dc)

    xg2 = x.to(DEV).requires_grad_(True)
    loss2, _, _ = ko.fused_grpo_step(xg2, t.to(DEV), old.to(DEV), adv.to(DEV), mask.to(DEV),
                                     loss_type="grpo", grad_scale=c)
    loss2.backward()
    factor = float(np.float32(np.float32(1.0) / np.float32(c)))
    assert torch.equal(xg2.grad, (dc.float() * factor).to(dc.dtype))

    for bad in (0.0, float("inf"), float("nan"), 1e-60, 1e60):
        with pytest.raises(ValueError, match="grad_scale"):
            ko.fused_grpo_step(xg2, t.to(DEV), old.to(DEV), adv.to(DEV), mask.to(DEV),
                               grad_scale=bad)


@pytest.mark.parametrize("loss_type", ["grpo", "dr_grpo", "bnpo"])
@pytest.mark.parametrize("mask_kind", ["float", "int32"])
def test_hip_graph_capture_of_loss_and_backward(loss_type, mask_kind):
    """fused_grpo_step's forward and (0.5 * loss).backward() captured in one
    HIP graph: nothing on the way reads a device value on the host (the
    upstream gradient is applied by klp_scale_inplace, the token weights'
    normalisers are host floats).  Every replay, with new logits, eager work
    and synchronisations between replays, equals the eager step on the same
    logits bit for bit.  An int32 mask takes klp_grpo_token_weights into the
    graph (1200 tokens: "bnpo" in two launches through its workspace)."""
    ko = _ko()
    B, S, V = 2, (40 if mask_kind == "float" else 600), 8192
    gen = torch.Generator(device=DEV).manual_seed(17)

    def logits():
        return (torch.randn(B, S, V, generator=gen, device=DEV) * 2).to(torch.bfloat16)
    x = logits().requires_grad_(True)
    t = torch.randint(0, V, (B, S), generator=gen, device=DEV)
    mask = torch.rand(B, S, generator=gen, device=DEV) < 0.9
    mask = mask.float() if mask_kind == "float" else mask.to(torch.int32)
    adv = torch.randn(B, generator=gen, device=DEV)
    old = torch.full((B, S), -9.0, device=DEV)
    kw = dict(eps_low=0.2, eps_high=0.28, loss_type=loss_type)

    def step(inp):
        loss, lp, ent = ko.fused_grpo_step(inp, t, old, adv, mask, **kw)
        (loss * 0.5).backward()
        return loss, lp, ent

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):  # warm-up on the capture stream
            step(x)
            x.grad = None
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = step(x)
    for rep in range(3):
        print(f"graph replay {rep} ({loss_type}, {mask_kind} mask)", flush=True)
        with torch.no_grad():
            x.copy_(logits())
        junk = torch.randn(1000, device=DEV).sum()  # unrelated eager work
        g.replay()
        torch.cuda.synchronize()
        assert junk.isfinite()
        got = [z.detach().clone() for z in out] + [x.grad.clone()]
        xe = x.detach().clone().requires_grad_(True)
        exp = list(step(xe)) + [xe.grad]
        for a, b in zip(got, exp):
            assert torch.equal(a, b.detach()), f"replay {rep} differs from eager"


def test_fallbacks_match_composition():
    """Inputs the fused path does not take (vocab not a whole number of
    16-byte vectors, above the row capacity, sequence-level weights) run the
    unfused composition, with the same results."""
    ko = _ko()
    for V, level in ((1001, "token"), (160000, "token"), (4096, "sequence")):
        print(f"grpo step fallback: V={V} level={level}", flush=True)
        x, t, mask, adv = make_case(2, 3, V, torch.bfloat16, 13)
        old = torch.full((2, 3), -9.0).to(DEV)
        xa = x.to(DEV).requires_grad_(True)
        la, lpa, _ = ko.fused_grpo_step(xa, t.to(DEV), old, adv.to(DEV), mask.to(DEV),
                                        importance_level=level)
        la.backward()
        xb = x.to(DEV).requires_grad_(True)
        lpb, _, _ = ko.fused_logprob_entropy(xb, t.to(DEV))
        lb, _ = ko.fused_grpo_loss(lpb, old, adv.to(DEV), mask.to(DEV), importance_level=level)
        lb.backward()
        assert torch.equal(la, lb) and torch.equal(lpa, lpb)
        assert torch.equal(xa.grad, xb.grad)


@pytest.mark.parametrize("B,S,V,dtype", [(8, 1024, 128256, torch.float16),    # C3
                                          (16, 2048, 151936, torch.bfloat16)])  # C4
def test_full_size_matches_unfused_composition(B, S, V, dtype):
    """C3 and C4 at full size (C4: 4.98e9 elements, 64-bit row offsets): the
    fused step against the unfused composition on the same inputs, loss within
    1e-5 relative, logp / entropy within 4e-5, every d_logits element within
    1 ulp (compared in row blocks to bound memory)."""
    ko = _ko()
    print(f"grpo step full size: {(B, S, V)} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(15)
    x = (torch.randn(B, S, V, generator=g, device=DEV) * 2.0).to(dtype)
    t = torch.randint(0, V, (B, S), generator=g, device=DEV)
    mask = (torch.rand(B, S, generator=g, device=DEV) < 0.9).float()
    adv = torch.randn(B, generator=g, device=DEV)
    with torch.no_grad():
        lp0, _, _ = ko.fused_logprob_entropy_forward(x, t)
    old = lp0 + 0.2 * torch.randn(B, S, generator=g, device=DEV)
    kw = dict(eps_low=0.2, eps_high=0.28, beta=0.0, loss_type="bnpo")
    xa = x.requires_grad_(True)
    la, lpa, enta = ko.fused_grpo_step(xa, t, old, adv, mask, **kw)
    la.backward()
    da = xa.grad
    xa.grad = None
    lpb, entb, _ = ko.fused_logprob_entropy(xa, t)
    lb, _ = ko.fused_grpo_loss(lpb, old, adv, mask, **kw)
    lb.backward()
    db = xa.grad
    assert abs(la.item() - lb.item()) <= 1e-5 * max(1.0, abs(lb.item()))
    assert (lpa - lpb).abs().max().item() <= 4e-5
    assert (enta - entb).abs().max().item() <= 4e-5

    def ordered(v):
        v = v.view(torch.int16).to(torch.int32)
        mag = v & 0x7FFF
        return torch.where(v < 0, -mag, mag)
    a2, b2 = da.view(-1, V), db.view(-1, V)
    worst = 0
    for r0 in range(0, a2.size(0), 2048):
        worst = max(worst, (ordered(a2[r0:r0 + 2048]) - ordered(b2[r0:r0 + 2048]))
                    .abs().max().item())
    assert worst <= 1, f"d_logits up to {worst} ulp from the unfused composition"


def test_c2_matches_unfused_composition():
    """C2 ([4, 256, 152064] bf16): the fused step against the unfused
    composition on the same inputs."""
    ko = _ko()
    B, S, V = 4, 256, 152064
    g = torch.Generator(device=DEV).manual_seed(14)
    x = (torch.randn(B, S, V, generator=g, device=DEV) * 2.0).to(torch.bfloat16)
    t = torch.randint(0, V, (B, S), generator=g, device=DEV)
    mask = (torch.rand(B, S, generator=g, device=DEV) < 0.9).float()
    adv = torch.randn(B, generator=g, device=DEV)
    with torch.no_grad():
        lp0, _, _ = ko.fused_logprob_entropy_forward(x, t)
    old = lp0 + 0.2 * torch.randn(B, S, generator=g, device=DEV)
    ref = lp0 + 0.2 * torch.randn(B, S, generator=g, device=DEV)
    kw = dict(eps_low=0.2, eps_high=0.28, beta=0.04, loss_type="grpo")

    xa = x.clone().requires_grad_(True)
    la, lpa, enta = ko.fused_grpo_step(xa, t, old, adv, mask, ref, **kw)
    la.backward()
    xb = x.clone().requires_grad_(True)
    lpb, entb, _ = ko.fused_logprob_entropy(xb, t)
    lb, _ = ko.fused_grpo_loss(lpb, old, adv, mask, ref, **kw)
    lb.backward()
    assert abs(la.item() - lb.item()) <= 1e-5 * max(1.0, abs(lb.item()))
    assert (lpa - lpb).abs().max().item() <= 4e-5
    assert (enta - entb).abs().max().item() <= 4e-5
    da = xa.grad.view(torch.int16).to(torch.int32)
    db = xb.grad.view(torch.int16).to(torch.int32)

    def ordered(v):
        mag = v & 0x7FFF
        return torch.where(v < 0, -mag, mag)
    ulps = (ordered(da) - ordered(db)).abs().max().item()
    assert ulps <= 1, f"d_logits up to {ulps} bf16 ulp from the unfused composition"


def _step_abi(x, t, old, ref, adv, w, temperature, per_token, sched):
    """klp_grpo_step through the C ABI with an explicit `sched` (None: one
    workgroup per row); returns (logp, ent, lse, loss_tok, d_logits)."""
    from kernel_opt import _C
    from kernel_opt._library import DTYPE_CODES, check_status, lib
    N, V = t.numel(), x.size(-1)
    S = t.size(-1)
    outs = [torch.full(t.shape, float("nan"), device=DEV) for _ in range(4)]
    d = torch.full(x.shape, float("nan"), dtype=x.dtype, device=DEV)
    P = lambda z: None if z is None else z.data_ptr()
    st = torch.cuda.current_stream().cuda_stream
    check_status(lib.klp_grpo_step(P(x), DTYPE_CODES[x.dtype], N, V, *_C.row_layout(x), P(t),
                                   temperature, P(old), P(ref), P(adv), P(w), S, 0.2, 0.28,
                                   0.04 if ref is not None else 0.0, per_token, 1.0,
                                   *map(P, outs), P(d), P(sched), st))
    return (*outs, d)


@pytest.mark.parametrize("dtype,B,S,V,temperature,per_token,with_ref,sliced", [
    (torch.bfloat16, 5, 1024, 152064, 1.0, 0, True, False),    # the C2 vocabulary
    (torch.bfloat16, 5, 1100, 100000, 0.7, 1, True, False),    # 16 vectors, a partial one;
                                                               # temperature, per-token adv
    (torch.bfloat16, 5, 1030, 155648, 1.3, 0, False, True),    # the row capacity, strided
    (torch.bfloat16, 3, 1024, 50000, 1.0, 0, True, True),      # 8 vectors, strided
    (torch.float16, 3, 1024, 128256, 1.0, 0, True, False),     # the C3 vocabulary
    (torch.float16, 3, 1024, 90000, 0.9, 1, False, False),     # 12 vectors
    (torch.float32, 3, 1024, 32000, 0.8, 1, False, False),     # fp32, 8 vectors
    (torch.float32, 3, 1024, 77824, 1.0, 0, True, False),      # fp32 row capacity
])
def test_persistent_rows_match_one_row_per_workgroup(dtype, B, S, V, temperature, per_token,
                                                     with_ref, sliced):
    """With a `sched` counter and at least klp_grpo_step_persistent_min_rows
    rows, klp_grpo_step runs persistent workgroups that claim rows from the
    counter.  Every output equals, bit for bit, the one-workgroup-per-row
    kernel's (sched = NULL) on the same inputs, including rows with -inf
    logits and ignored targets (outputs start as NaN, so a row either kernel
    skipped would show); the counter is left zero, and a second call on it
    (fewer rows) again matches."""
    from kernel_opt._library import KLP_GRPO_STEP_SCHED_BYTES, DTYPE_CODES, lib
    print(f"persistent step: {dtype} {(B, S, V)} T={temperature}", flush=True)
    min_rows = lib.klp_grpo_step_persistent_min_rows(DTYPE_CODES[dtype], V,
                                                     int(temperature != 1.0))
    assert min_rows > 0
    assert B * S >= min_rows, (B * S, min_rows)
    g = torch.Generator(device=DEV).manual_seed(21)
    full = (torch.randn(B, S + int(sliced), V, generator=g, device=DEV) * 2.0).to(dtype)
    x = full[:, :S] if sliced else full
    x[0, 3, ::5] = float("-inf")
    x[1, 7, : V // 3] = float("-inf")
    t = torch.randint(0, V, (B, S), generator=g, device=DEV)
    t[0, 1] = IGNORE
    t[1, 2] = V + 5
    lp0 = torch.randn(B, S, generator=g, device=DEV) - 10.0
    old = lp0 + 0.2 * torch.randn(B, S, generator=g, device=DEV)
    ref = (lp0 + 0.2 * torch.randn(B, S, generator=g, device=DEV)) if with_ref else None
    adv = torch.randn((B, S) if per_token else (B,), generator=g, device=DEV)
    w = (torch.rand(B, S, generator=g, device=DEV) < 0.8).float() / (B * S)
    sched = torch.zeros(KLP_GRPO_STEP_SCHED_BYTES, dtype=torch.uint8, device=DEV)
    for rows in (B, B - 1):  # the second call: fewer rows, still above the threshold
        assert rows * S >= min_rows
        xs, ts = x[:rows], t[:rows]
        olds, refs = old[:rows].contiguous(), None if ref is None else ref[:rows].contiguous()
        advs, ws = adv[:rows].contiguous(), w[:rows].contiguous()
        a = _step_abi(xs, ts, olds, refs, advs, ws, temperature, per_token, None)
        b = _step_abi(xs, ts, olds, refs, advs, ws, temperature, per_token, sched)
        torch.cuda.synchronize()
        assert torch.count_nonzero(sched).item() == 0, "the counter was not left zero"
        for name, u, v in zip(("logp", "entropy", "lse", "loss_tok", "d_logits"), a, b):
            as_int = torch.int32 if u.dtype == torch.float32 else torch.int16
            assert torch.equal(u.view(as_int), v.view(as_int)), name


def test_persistent_rows_only_where_they_pay():
    """The persistent kernel is used for rows of 8 or more 16-byte vectors
    per thread (bf16 / fp16 V > 32768, fp32 V > 16384), from 8 rows per
    resident workgroup on; for shorter rows the one-row kernel fits two
    workgroups per CU and measured faster, and the query reports 0."""
    from kernel_opt._library import KLP_BF16, KLP_FP16, KLP_FP32, lib
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    for scaled in (0, 1):
        for dtype, V in ((KLP_BF16, 32776), (KLP_BF16, 100000), (KLP_BF16, 152064),
                         (KLP_BF16, 155648), (KLP_FP16, 128256), (KLP_FP32, 16388),
                         (KLP_FP32, 32000), (KLP_FP32, 77824)):
            assert lib.klp_grpo_step_persistent_min_rows(dtype, V, scaled) == 8 * n_cu, (dtype, V)
        for dtype, V in ((KLP_BF16, 32000), (KLP_BF16, 32768), (KLP_FP16, 32768),
                         (KLP_FP32, 16384)):
            assert lib.klp_grpo_step_persistent_min_rows(dtype, V, scaled) == 0, (dtype, V)
        assert lib.klp_grpo_step_persistent_min_rows(KLP_BF16, 155656, scaled) == 0


@pytest.mark.parametrize("B,S", [(1, 1), (3, 1000), (4, 256), (16, 2048), (2, 70001),
                                 (64, 8192), (300, 4001), (70001, 3)])
@pytest.mark.parametrize("mask_kind", ["bool", "uint8", "int32", "int64", "none"])
def test_token_weights_kernel_matches_eager(B, S, mask_kind):
    """klp_grpo_token_weights writes the bits of the eager statement
    grpo_step.grpo_token_weights for every loss type: bool / uint8 / int32 /
    int64 0 / 1 masks (one all-zero row, whose normaliser clamps to 1) and no
    mask.  The shapes cover one and many workgroups, grid-wide passes that
    loop (1.2 M tokens over 1024 workgroups) and more rows than the per-row
    grid's 65 535 workgroups; the workspace starts with garbage."""
    import ctypes
    from kernel_opt._library import KLP_GRPO_TOKEN_WEIGHTS_WORKSPACE_BYTES, check_status, lib
    from kernel_opt.grpo_step import grpo_token_weights
    print(f"token weights B={B} S={S} mask={mask_kind}", flush=True)
    g = torch.Generator().manual_seed(B * 7919 + S)
    m01 = (torch.rand(B, S, generator=g) < 0.7)
    if B > 1:
        m01[1] = False
    codes = {"bool": 0, "uint8": 0, "int32": 1, "int64": 2}
    dt = {"bool": torch.bool, "uint8": torch.uint8, "int32": torch.int32, "int64": torch.int64}
    mask = None if mask_kind == "none" else m01.to(dt[mask_kind]).to(DEV)
    st = torch.cuda.current_stream().cuda_stream
    for kind, loss_type, kw in ((0, "grpo", {}), (1, "bnpo", {}), (2, "dr_grpo", {}),
                                (2, "dapo", {"normalizer": 777.0})):
        eager = grpo_token_weights(mask if mask is not None else torch.ones(B, S, device=DEV),
                                   loss_type, **kw)
        scale = 0.0
        if kind == 2:
            den = float(B * S) if loss_type == "dr_grpo" else kw["normalizer"]
            scale = float(np.float32(1.0) / np.float32(den))
        w = torch.full((B, S), -1.0, device=DEV)
        ws = torch.full((KLP_GRPO_TOKEN_WEIGHTS_WORKSPACE_BYTES // 8,), -7, dtype=torch.int64,
                        device=DEV)
        check_status(lib.klp_grpo_token_weights(
            mask.data_ptr() if mask is not None else None, codes.get(mask_kind, 0), B, S, kind,
            ctypes.c_float(scale), w.data_ptr(), ws.data_ptr(), st))
        torch.cuda.synchronize()
        assert torch.equal(w.view(torch.int32), eager.float().contiguous().view(torch.int32)), \
            f"{loss_type}: max |diff| {float((w - eager).abs().max()):.3g}"
