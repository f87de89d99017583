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
