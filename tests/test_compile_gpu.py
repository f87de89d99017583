"""torch.compile round trip (reference tests/test_compile.py:24-65):
compiled forward and backward through ``aot_eager`` equal eager."""
import pytest
import torch

from klp_testutil import seeded_logits, seeded_targets

pytestmark = pytest.mark.gpu
COMPILE_BACKEND = "aot_eager"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_compile_forward_matches_eager(dtype):
    from kernel_opt import fused_logprob_entropy
    B, S, V = 2, 8, 4096
    x = seeded_logits((B, S, V), dtype, seed=0, scale=1.0).cuda()
    t = seeded_targets((B, S), V, seed=0).cuda()

    def fn(x, t):
        return fused_logprob_entropy(x, t)

    eager_out = fn(x, t)
    torch._dynamo.reset()
    comp_out = torch.compile(fn, backend=COMPILE_BACKEND, dynamic=False)(x, t)
    for e, c in zip(eager_out, comp_out):
        atol = 1e-5 if dtype == torch.float32 else 5e-3
        assert torch.allclose(e, c, atol=atol, rtol=atol)


def test_compile_backward_matches_eager():
    from kernel_opt import fused_logprob_entropy
    B, S, V = 2, 4, 2048
    base = seeded_logits((B, S, V), torch.float32, seed=1, scale=1.0).cuda()
    t = seeded_targets((B, S), V, seed=1).cuda()

    def loss_fn(x, t):
        logp, ent, _lse = fused_logprob_entropy(x, t)
        return (logp + 0.1 * ent).sum()

    x_e = base.clone().requires_grad_(True)
    loss_fn(x_e, t).backward()
    x_c = base.clone().requires_grad_(True)
    torch._dynamo.reset()
    torch.compile(loss_fn, backend=COMPILE_BACKEND, dynamic=False)(x_c, t).backward()
    assert torch.allclose(x_c.grad, x_e.grad, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("temperature", [None, 0.75])
def test_compile_fullgraph_no_graph_break(dtype, temperature):
    """With the torch.library registration, fullgraph=True compiles (it would
    raise on a graph break), and forward + backward equal eager."""
    from kernel_opt import fused_logprob_entropy
    B, S, V = 2, 6, 3001
    base = seeded_logits((B, S, V), dtype, seed=3, scale=1.5).cuda()
    t = seeded_targets((B, S), V, seed=3).cuda()

    def loss_fn(x, t):
        logp, ent, lse = fused_logprob_entropy(x, t, temperature=temperature)
        return (logp + 0.1 * ent - 0.01 * lse).sum(), logp, ent, lse

    x_e = base.clone().requires_grad_(True)
    out_e = loss_fn(x_e, t)
    out_e[0].backward()
    torch._dynamo.reset()
    x_c = base.clone().requires_grad_(True)
    out_c = torch.compile(loss_fn, backend=COMPILE_BACKEND, fullgraph=True, dynamic=False)(x_c, t)
    out_c[0].backward()
    for e, c in zip(out_e[1:], out_c[1:]):
        assert torch.equal(e, c)
    assert torch.equal(x_c.grad, x_e.grad)


def test_opcheck_registered_op():
    from kernel_opt import ops  # noqa: F401  (registers the ops)
    x = seeded_logits((3, 5, 777), torch.float32, seed=4).cuda().requires_grad_(True)
    t = seeded_targets((3, 5), 777, seed=4).cuda()
    torch.library.opcheck(torch.ops.kernel_opt.fused_logprob_entropy.default, (x, t, 1.0))
    torch.library.opcheck(torch.ops.kernel_opt.fused_logprob_entropy.default, (x, t, 0.5))
