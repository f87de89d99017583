"""GPU checks of the compiled binding (binding/klp_torch.cpp), which the
public logprob, GRPO loss and fused GRPO step entry points go through: each
autograd function against the Python statement of the same op
(ops._FusedLogprobEntropy, grpo._FusedGrpoLoss, grpo_step._FusedGrpoStep over
the same launchers), bit for bit, forward and backward; the split-row
workspaces (one per stream, at most 16 kept); the error behaviour on GPU
tensors.  Under graph capture the binding declines every call before it
allocates or launches anything (binding.CaptureDeclined) and the Python path
runs: the capture tests of test_logprob_gpu.py and test_grpo_step_gpu.py go
through that fallback."""
from __future__ import annotations

import pytest
import torch

from klp_testutil import seeded_logits, seeded_targets

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _grads(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g).to(DEV), torch.randn(shape, generator=g).to(DEV),
            torch.randn(shape, generator=g).to(DEV))


CASES = [  # dtype, shape, temperature, strided, which upstream gradients
    (torch.bfloat16, (4, 33, 5003), None, False, "all"),
    (torch.bfloat16, (2, 65, 4099), 0.7, True, "logp"),
    (torch.float16, (3, 17, 2048), 1.3, False, "ent"),
    (torch.float32, (2, 9, 32000), None, True, "logp+lse"),
    (torch.bfloat16, (8, 152064), None, False, "all"),  # split rows: the workspace
]


@pytest.mark.parametrize("dtype,shape,T,strided,use", CASES)
def test_compiled_op_equals_python_function(dtype, shape, T, strided, use):
    from kernel_opt import fused_logprob_entropy
    from kernel_opt.ops import _FusedLogprobEntropy
    full_shape = shape[:-2] + (shape[-2] + 1, shape[-1]) if strided else shape
    base = seeded_logits(full_shape, dtype, seed=sum(shape)).to(DEV)
    t = seeded_targets(shape[:-1], shape[-1], seed=7).to(DEV)
    t.view(-1)[::11] = -100
    gl, ge, gs = _grads(shape[:-1], 3)
    outs, grads = [], []
    for fn in (lambda x: fused_logprob_entropy(x, t, T),
               lambda x: _FusedLogprobEntropy.apply(x, t, T)):
        leaf = base.clone().requires_grad_(True)
        x = leaf[..., :-1, :] if strided else leaf
        lp, ent, lse = fn(x)
        loss = {"all": (lp * gl).sum() + (ent * ge).sum() + (lse * gs).sum(),
                "logp": (lp * gl).sum(), "ent": (ent * ge).sum(),
                "logp+lse": (lp * gl).sum() + (lse * gs).sum()}[use]
        loss.backward()
        outs.append((lp, ent, lse))
        grads.append(leaf.grad)
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert torch.equal(grads[0], grads[1])
    assert type(outs[0][0].grad_fn).__name__ != type(outs[1][0].grad_fn).__name__


def test_forward_entry_points_equal():
    from kernel_opt import _C, fused_logprob_entropy_forward, fused_logprob_entropy_naive
    from kernel_opt._library import binding
    x = seeded_logits((6, 3001), torch.bfloat16, seed=5).to(DEV)
    t = seeded_targets((6,), 3001, seed=5).to(DEV)
    a = fused_logprob_entropy_forward(x, t)
    b = [torch.empty(6, device=DEV) for _ in range(3)]
    _C.fused_logprob_entropy_v1(x, t, *b)
    c = [torch.empty(6, device=DEV) for _ in range(3)]
    _C.fwd_launch(x, t, *c, config=_C.default_config("fwd", x.dtype, 6, 3001))
    for u, v, w in zip(a, b, c):
        assert torch.equal(u, v) and torch.equal(u, w)
    n = fused_logprob_entropy_naive(x, t)
    m = [torch.empty(6, device=DEV) for _ in range(3)]
    binding.fused_logprob_entropy_naive(x, t, *m)
    for u, v in zip(n, m):
        assert torch.equal(u, v)


def test_split_rows_on_many_streams():
    """Small batches of long rows take split rows (a workspace): 20 streams in
    turn, each result equal to the default stream's; the binding keeps at most
    16 workspaces."""
    from kernel_opt import _C, fused_logprob_entropy_forward
    from kernel_opt._library import binding
    x = seeded_logits((8, 152064), torch.bfloat16, seed=31).to(DEV)
    t = seeded_targets((8,), 152064, seed=31).to(DEV)
    assert _C.default_config("fwd", x.dtype, 8, 152064)[2] > 1
    ref = fused_logprob_entropy_forward(x, t)
    torch.cuda.synchronize()
    for i in range(20):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            out = fused_logprob_entropy_forward(x, t)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        assert binding.workspaces_cached() <= 16
        for a, b in zip(out, ref):
            assert torch.equal(a, b), f"stream {i}"


@pytest.mark.skip(reason="its one run, with the compiled binding under capture, ended in a host "
                         "segmentation fault inside torch.cuda.graph's capture_end whose cause is "
                         "not known; the binding now declines captured calls (CaptureDeclined) "
                         "and they run the Python path, whose capture is tested by "
                         "test_logprob_gpu::test_hip_graph_capture_and_replay and "
                         "test_grpo_step_gpu::test_hip_graph_capture_of_loss_and_backward")
def test_graph_capture_of_split_rows():
    """A split-row forward and the backward captured in a HIP graph: each
    replay, with eager calls on the capture stream in between, equals the
    eager result."""
    from kernel_opt import fused_logprob_entropy
    x0 = seeded_logits((8, 152064), torch.bfloat16, seed=41).to(DEV)
    t = seeded_targets((8,), 152064, seed=41).to(DEV)
    gl, ge, _ = _grads((8,), 42)
    x = x0.clone().requires_grad_(True)

    def step():
        x.grad = None
        lp, ent, lse = fused_logprob_entropy(x, t)
        ((lp * gl).sum() + (ent * ge).sum()).backward()
        return lp, ent, lse, x.grad

    ref = [r.clone() for r in step()]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    x.grad = None
    with torch.cuda.graph(g, stream=s):
        lp, ent, lse = fused_logprob_entropy(x, t)
        ((lp * gl).sum() + (ent * ge).sum()).backward()
    captured = (lp, ent, lse, x.grad)
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(captured, ref):
            assert torch.equal(a, b), f"replay {rep}"
        with torch.cuda.stream(s):
            eager = fused_logprob_entropy(x0, t)
        torch.cuda.synchronize()
        for a, b in zip(eager, ref[:3]):
            assert torch.equal(a, b)


def test_errors_on_gpu_tensors():
    from kernel_opt import _C, fused_logprob_entropy, fused_logprob_entropy_forward
    x = seeded_logits((4, 100), torch.bfloat16, seed=1).to(DEV)
    t = seeded_targets((4,), 100, seed=1).to(DEV)
    with pytest.raises(AssertionError, match=r"logits\[...,V\]="):
        fused_logprob_entropy(x, t[:3])
    with pytest.raises(AssertionError):
        fused_logprob_entropy_forward(x, t.to(torch.int32))
    with pytest.raises(AssertionError):
        fused_logprob_entropy_forward(x.t(), t)  # rows without unit stride
    lse = torch.zeros(4, device=DEV)
    with pytest.raises(RuntimeError, match="d_logits must match"):
        _C.fused_logprob_entropy_v1_backward(x, t, lse, lse, None, None, None,
                                             torch.empty(4, 100, device=DEV))
    with pytest.raises(RuntimeError, match="upstream gradients must be fp32"):
        _C.fused_logprob_entropy_v1_backward(x, t, lse, lse, lse.double(), None, None,
                                             torch.empty_like(x))
    with pytest.raises(RuntimeError, match="temperature"):
        fused_logprob_entropy(x, t, -1.0)
    with pytest.raises(RuntimeError, match="outputs must be float32"):
        _C.fused_logprob_entropy_v1(x, t, lse.half(), lse, lse)


class _PythonPathOnly:
    """Stands in for the binding so that kernel_opt.grpo runs its Python
    statement of the GRPO loss (the path graph capture takes)."""

    class CaptureDeclined(Exception):
        pass

    @staticmethod
    def fused_grpo_loss(*args, **kwargs):
        raise _PythonPathOnly.CaptureDeclined()


GRPO_CASES = [  # loss_type, importance level, beta, per-token advantages, mask, loss scale
    ("bnpo", "token", 0.0, False, "float", 1.0),
    ("grpo", "token", 0.04, True, "bool", 1.0),
    ("dr_grpo", "sequence", 0.04, False, None, 2.5),
    ("dapo", "token", 0.0, True, "int", -0.5),
    ("grpo", "sequence", 0.0, True, "bool", 1.0),
]


@pytest.mark.parametrize("loss_type,level,beta,per_token,mask_kind,scale", GRPO_CASES)
def test_compiled_grpo_loss_equals_python_function(monkeypatch, loss_type, level, beta, per_token,
                                                   mask_kind, scale):
    """fused_grpo_loss through the binding's C++ autograd op and through
    grpo.py's Python autograd.Function: loss, stats and d_logp bit for bit."""
    from kernel_opt import fused_grpo_loss, grpo
    B, S = 6, 37
    g = torch.Generator().manual_seed(B * S + len(loss_type))
    lp0 = (-torch.rand(B, S, generator=g) * 3).to(DEV)
    old = (lp0.cpu() + torch.randn(B, S, generator=g) * 0.1).to(DEV)
    ref = (lp0.cpu() + torch.randn(B, S, generator=g) * 0.2).to(DEV)
    adv = torch.randn((B, S) if per_token else (B,), generator=g).to(DEV)
    m = torch.rand(B, S, generator=g) < 0.8
    mask = None if mask_kind is None else {
        "float": m.float(), "bool": m, "int": m.to(torch.int32), "bf16": m.to(torch.bfloat16),
        "fp16": m.to(torch.float16), "f64": m.to(torch.float64)}[mask_kind].to(DEV)
    kw = dict(beta=beta, loss_type=loss_type, importance_level=level, eps_high=0.28,
              max_completion_length=48 if loss_type == "dr_grpo" else None,
              normalizer=123.0 if loss_type == "dapo" else None)
    results = []
    for python_path in (False, True):
        if python_path:
            monkeypatch.setattr(grpo, "binding", _PythonPathOnly)
        lp = lp0.clone().requires_grad_(True)
        loss, stats = fused_grpo_loss(lp, old, adv, mask, ref, **kw)
        (loss * scale).backward()
        results.append((loss.detach(), stats, lp.grad, type(loss.grad_fn).__name__))
    (l1, s1, d1, n1), (l2, s2, d2, n2) = results
    assert torch.equal(l1, l2) and torch.equal(s1, s2) and torch.equal(d1, d2)
    assert l1.dim() == 0 and l2.dim() == 0
    assert n1 != n2, (n1, n2)


def test_compiled_grpo_loss_edges():
    from kernel_opt import fused_grpo_loss
    lp = torch.zeros(0, 5, device=DEV, requires_grad=True)
    loss, stats = fused_grpo_loss(lp, lp.detach(), torch.zeros(0, device=DEV))
    loss.backward()
    assert loss.item() == 0.0 and torch.equal(stats, torch.zeros(4, device=DEV))
    x = torch.zeros(2, 3, device=DEV)
    with pytest.raises(RuntimeError, match=r"old_logp has shape \(1, 3\), expected \(2, 3\)"):
        fused_grpo_loss(x, x[:1], torch.zeros(2, device=DEV))
    with pytest.raises(RuntimeError, match="advantages must be on cuda:0"):
        fused_grpo_loss(x, x, torch.zeros(2))
    with pytest.raises(RuntimeError, match="eps_low"):
        fused_grpo_loss(x, x, torch.zeros(2, device=DEV), eps_low=-0.1)


class _StepPythonPathOnly:
    """Stands in for the binding so that kernel_opt.grpo_step runs its Python
    statement of the fused step (the path graph capture takes)."""

    class CaptureDeclined(Exception):
        pass

    @staticmethod
    def fused_grpo_step(*args, **kwargs):
        raise _StepPythonPathOnly.CaptureDeclined()


STEP_CASES = [  # dtype, (B, S, V), strided rows, loss_type, beta, per-token adv, mask, T, scale
    (torch.bfloat16, (3, 40, 4096), False, "grpo", 0.0, False, "bool", None, 1.0),
    (torch.bfloat16, (2, 33, 152064), True, "bnpo", 0.04, True, None, 0.7, 1.0),
    (torch.float16, (4, 17, 8200), False, "dr_grpo", 0.04, False, "float", None, 2.5),
    (torch.float32, (2, 9, 32000), True, "dapo", 0.0, True, "int", 1.3, -0.5),
    (torch.bfloat16, (8, 300, 40960), False, "grpo", 0.04, False, "bool", None, 1.0),  # persistent
    # Floating masks other than float32 are taken in float32 (the token
    # weights the kernel reads are float32), for every loss type.
    (torch.bfloat16, (3, 40, 4096), False, "grpo", 0.0, False, "bf16", None, 1.0),
    (torch.bfloat16, (2, 33, 8192), False, "bnpo", 0.04, False, "fp16", None, 1.0),
    (torch.float16, (4, 17, 8200), False, "dr_grpo", 0.04, False, "f64", None, 2.5),
    (torch.bfloat16, (2, 9, 4096), True, "dapo", 0.0, True, "bf16", 1.3, -0.5),
    (torch.float32, (2, 9, 32000), False, "grpo", 0.04, False, "f64", None, 1.0),
    (torch.float16, (3, 12, 4096), False, "bnpo", 0.0, True, "f64", 0.9, 1.0),
    (torch.bfloat16, (2, 21, 4096), False, "dr_grpo", 0.0, False, "bf16", None, 1.0),
    (torch.float32, (2, 9, 4096), False, "dapo", 0.04, False, "fp16", None, 1.0),
]


@pytest.mark.parametrize("dtype,shape,strided,loss_type,beta,per_token,mask_kind,T,scale",
                         STEP_CASES)
def test_compiled_grpo_step_equals_python_function(monkeypatch, dtype, shape, strided, loss_type,
                                                   beta, per_token, mask_kind, T, scale):
    """fused_grpo_step through the binding's C++ autograd op and through
    grpo_step.py's Python statement: loss, logp, entropy, d_logits and the
    stats bit for bit, on the same row counter scheme."""
    from kernel_opt import fused_grpo_step, grpo_step
    B, S, V = shape
    full = (B, S + 1, V) if strided else (B, S, V)
    base = seeded_logits(full, dtype, seed=B * S + V).to(DEV)
    t = seeded_targets((B, S), V, seed=5).to(DEV)
    g = torch.Generator().manual_seed(S)
    old = (-torch.rand(B, S, generator=g) * 3).to(DEV)
    ref = (-torch.rand(B, S, generator=g) * 3).to(DEV)
    adv = torch.randn((B, S) if per_token else (B,), generator=g).to(DEV)
    m = torch.rand(B, S, generator=g) < 0.8
    mask = None if mask_kind is None else {
        "float": m.float(), "bool": m, "int": m.to(torch.int32), "bf16": m.to(torch.bfloat16),
        "fp16": m.to(torch.float16), "f64": m.to(torch.float64)}[mask_kind].to(DEV)
    kw = dict(beta=beta, loss_type=loss_type, eps_high=0.28, temperature=T,
              normalizer=77.0 if loss_type == "dapo" else None, return_stats=True)
    res = []
    for python_path in (False, True):
        if python_path:
            monkeypatch.setattr(grpo_step, "binding", _StepPythonPathOnly)
        leaf = base.clone().requires_grad_(True)
        x = leaf[:, :-1, :] if strided else leaf
        loss, lp, ent, stats = fused_grpo_step(x, t, old, adv, mask, ref, **kw)
        (loss * scale).backward()
        res.append((loss.detach(), lp, ent, stats, leaf.grad, loss.grad_fn.name()))
    for a, b in zip(res[0][:5], res[1][:5]):
        assert torch.equal(a, b)
    assert "CppNode" in res[0][5] and "FusedGrpoStep" in res[0][5], res[0][5]
    assert "CppNode" not in res[1][5], res[1][5]


@pytest.mark.parametrize("normalizer", [-4.0, 0.0])
@pytest.mark.parametrize("mask_kind", ["bool", "int64", None])
def test_compiled_grpo_step_nonpositive_normalizer(monkeypatch, normalizer, mask_kind):
    """A zero or negative "dapo" normaliser: the binding keeps the eager
    statement's weights (negative, or inf / nan), the Python path's bits in
    the loss, logp, entropy and d_logits."""
    from kernel_opt import fused_grpo_step, grpo_step
    B, S, V = 3, 20, 4096
    base = seeded_logits((B, S, V), torch.bfloat16, seed=11).to(DEV)
    t = seeded_targets((B, S), V, seed=12).to(DEV)
    g = torch.Generator().manual_seed(13)
    old = (-torch.rand(B, S, generator=g) * 3).to(DEV)
    adv = torch.randn(B, generator=g).to(DEV)
    m = torch.rand(B, S, generator=g) < 0.8
    mask = None if mask_kind is None else m.to(getattr(torch, mask_kind)).to(DEV)

    def bits(x):
        x = x.detach().contiguous()
        return x.view({4: torch.int32, 2: torch.int16}[x.element_size()])

    res = []
    for python_path in (False, True):
        if python_path:
            monkeypatch.setattr(grpo_step, "binding", _StepPythonPathOnly)
        leaf = base.clone().requires_grad_(True)
        loss, lp, ent = fused_grpo_step(leaf, t, old, adv, mask, loss_type="dapo",
                                        normalizer=normalizer)
        loss.backward()
        res.append([bits(loss), bits(lp), bits(ent), bits(leaf.grad), loss.grad_fn.name()])
    for a, b in zip(res[0][:4], res[1][:4]):
        assert torch.equal(a, b)
    assert "FusedGrpoStep" in res[0][4], res[0][4]
    if normalizer < 0:
        assert torch.isfinite(res[0][0].view(torch.float32)).all()


@pytest.mark.parametrize("upstream", [0.25, 1.0, -3.0])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_compiled_grpo_step_grad_scale(monkeypatch, upstream, dtype):
    """A declared grad_scale of 0.25: the binding's op and the Python
    statement give the same bits for the loss, logp, entropy and d_logits,
    whether the upstream gradient equals it (nothing written in the
    backward) or not (the ratio applied)."""
    from kernel_opt import fused_grpo_step, grpo_step
    B, S, V = 3, 20, 8192
    base = seeded_logits((B, S, V), dtype, seed=21).to(DEV)
    t = seeded_targets((B, S), V, seed=22).to(DEV)
    g = torch.Generator().manual_seed(23)
    old = (-torch.rand(B, S, generator=g) * 3).to(DEV)
    adv = torch.randn(B, generator=g).to(DEV)
    mask = (torch.rand(B, S, generator=g) < 0.8).to(DEV)

    def bits(x):
        x = x.detach().contiguous()
        return x.view({4: torch.int32, 2: torch.int16}[x.element_size()])

    res = []
    for python_path in (False, True):
        if python_path:
            monkeypatch.setattr(grpo_step, "binding", _StepPythonPathOnly)
        leaf = base.clone().requires_grad_(True)
        loss, lp, ent = fused_grpo_step(leaf, t, old, adv, mask, loss_type="grpo",
                                        grad_scale=0.25)
        (loss * upstream).backward()
        res.append([bits(loss), bits(lp), bits(ent), bits(leaf.grad), loss.grad_fn.name()])
    for a, b in zip(res[0][:4], res[1][:4]):
        assert torch.equal(a, b)
    assert "FusedGrpoStep" in res[0][4], res[0][4]


def test_compiled_grpo_step_backward_once_and_fallback():
    from kernel_opt import fused_grpo_step
    x = seeded_logits((2, 5, 4096), torch.bfloat16, seed=3).to(DEV).requires_grad_(True)
    t = seeded_targets((2, 5), 4096, seed=3).to(DEV)
    old = torch.zeros(2, 5, device=DEV)
    adv = torch.ones(2, device=DEV)
    loss, _, _ = fused_grpo_step(x, t, old, adv)
    loss.backward(retain_graph=True)
    with pytest.raises(RuntimeError, match="only once per forward"):
        loss.backward()
    # rows that are not whole 16-byte vectors: the unfused composition
    y = seeded_logits((2, 5, 4099), torch.bfloat16, seed=4).to(DEV).requires_grad_(True)
    t2 = seeded_targets((2, 5), 4099, seed=4).to(DEV)
    loss2, lp2, _ = fused_grpo_step(y, t2, old, adv)
    assert lp2.requires_grad and "FusedGrpoStep" not in loss2.grad_fn.name()
    loss2.backward()
    assert y.grad is not None and torch.isfinite(y.grad.float()).all()


def test_compiled_grpo_step_checks_targets_itself():
    """binding.fused_grpo_step checks targets (device, dtype, layout, shape)
    before any launch, without the Python wrapper's checks in front of it."""
    from kernel_opt._library import binding
    B, S, V = 2, 5, 4096
    x = seeded_logits((B, S, V), torch.bfloat16, seed=11).to(DEV)
    t = seeded_targets((B, S), V, seed=11).to(DEV)
    old = torch.zeros(B, S, device=DEV)
    adv = torch.ones(B, device=DEV)
    args = (old, adv, None, None, 1.0, 0.2, 0.28, 0.0, 1, 1.0)
    assert binding.fused_grpo_step(x, t, *args) is not None
    bad = [
        (t.cpu(), "targets must be on"),
        (t.to(torch.int32), "targets must be int64"),
        (seeded_targets((S, B), V, seed=1).to(DEV).t(), "targets must be contiguous"),
        (t.reshape(-1), "targets has shape"),
    ]
    for tt, msg in bad:
        with pytest.raises(RuntimeError, match=msg):
            binding.fused_grpo_step(x, tt, *args)
