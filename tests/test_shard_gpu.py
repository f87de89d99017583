"""GPU parity of the vocabulary-shard pieces (klp_fwd_shard, klp_fwd_shard_merge,
the backward on a shard), called through the C ABI (kernel_opt.shard).

P shards are emulated on one GPU as column slices of one logits matrix (each a
strided [N, V_shard] view, as a rank's shard would be its own tensor).  Bars:
  * merged logprob / entropy / lse against the float64 oracle within the
    forward tolerance (1e-5 fp32 input, 2e-5 bf16 / fp16 input), and against
    the unsharded forward within twice that;
  * the shards' d_logits, side by side, equal to the unsharded backward's for
    the same lse / entropy (the per-element formula is the same; the target's
    one-hot term lands in the shard that holds it);
  * a C4-sized 8-way shard ([4096, 151936] bf16 in 8 slices of 18992).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from klp_testutil import FWD_TOL, seeded_logits, seeded_targets

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _shard():
    from kernel_opt import shard
    return shard


def run_sharded(x, t, P, temperature=None):
    sh = _shard()
    V = x.size(-1)
    sv = -(-V // P)
    states = torch.stack([sh.shard_state(x[..., k * sv:min(V, (k + 1) * sv)], t, k * sv,
                                         temperature) for k in range(P)])
    return sh.merge_shard_states(states, t, sv, V), sv


CASES = [(torch.float32, 1, 3000), (torch.float32, 3, 5003), (torch.bfloat16, 2, 8192),
         (torch.bfloat16, 8, 32000), (torch.float16, 5, 4099), (torch.bfloat16, 8, 64)]


@pytest.mark.parametrize("dtype,P,V", CASES)
@pytest.mark.parametrize("temperature", [None, 0.7])
def test_merged_matches_oracle_and_unsharded(dtype, P, V, temperature, oracle):
    from kernel_opt import fused_logprob_entropy_forward
    N = 37
    x = seeded_logits((N, V), dtype, seed=P * 100 + V % 97)
    t = seeded_targets((N,), V, seed=P)
    t[3] = -100
    t[5] = V  # out of range: logp = -lse
    t[6] = V - 1  # in the last (possibly short) shard
    xd, td = x.to(DEV), t.to(DEV)
    (lp, ent, lse), _ = run_sharded(xd, td, P, temperature)
    ref = oracle.forward(x, t.numpy(), temperature=temperature)
    tol = FWD_TOL[dtype]
    for name, o, r in zip(("logp", "entropy", "lse"), (lp, ent, lse), ref):
        err = np.abs(o.cpu().double().numpy() - r).max()
        assert err <= tol, f"{name}: {err:.3g} > {tol}"
    full = fused_logprob_entropy_forward(xd, td, temperature)
    for o, f in zip((lp, ent, lse), full):
        assert (o - f).abs().max().item() <= 2 * tol
    assert torch.equal(lp[5], -lse[5])


@pytest.mark.parametrize("dtype,P,V", CASES)
def test_shard_backward_equals_unsharded(dtype, P, V):
    from kernel_opt import _C
    sh = _shard()
    N = 29
    x = seeded_logits((N, V), dtype, seed=7 + P).to(DEV)
    t = seeded_targets((N,), V, seed=8).to(DEV)
    t[2] = -100
    (lp, ent, lse), sv = run_sharded(x, t, P)
    g = torch.Generator().manual_seed(9)
    gl = torch.randn(N, generator=g).to(DEV)
    ge = torch.randn(N, generator=g).to(DEV)
    gs = torch.randn(N, generator=g).to(DEV)
    parts = [sh.shard_backward(x[:, k * sv:min(V, (k + 1) * sv)], t, k * sv, lse, ent, gl, ge,
                               gs) for k in range(P)]
    full = torch.empty_like(x)
    _C.bwd_launch(x, t, lse, ent, gl, ge, gs, full)
    assert torch.equal(torch.cat(parts, dim=1), full)


def test_c4_shard_shape():
    """C4's vocabulary (151936) over 8 ranks: 18992 columns per shard, 4096 rows."""
    from kernel_opt import fused_logprob_entropy_forward
    N, V, P = 4096, 151936, 8
    g = torch.Generator(device=DEV).manual_seed(10)
    x = (torch.randn(N, V, generator=g, device=DEV) * 2.5).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), generator=g, device=DEV)
    (lp, ent, lse), sv = run_sharded(x, t, P)
    assert sv == 18992
    full = fused_logprob_entropy_forward(x, t)
    for o, f in zip((lp, ent, lse), full):
        assert (o - f).abs().max().item() <= 4e-5
