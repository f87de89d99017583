"""GPU parity of klp_fwd_chunk, the chunked LM head's per-chunk forward whose
last launch merges the chunk states, called through the C ABI.

Bars:
  * equal-width chunks: logprob, entropy and lse bitwise equal to
    klp_fwd_shard on every chunk followed by klp_fwd_shard_merge (the same
    states, merged by the same sequence of combines);
  * chunks of any widths: entropy and lse bitwise equal to those of the same
    shard states merged by klp_fwd_shard_merge (which reads the target logit
    by an equal-width rule, so its logprob is not compared), logprob bitwise
    equal to fp32(target logit * fp32(1 / T)) - lse (0 - lse for a target
    outside the vocabulary), and all three against the float64 oracle within
    the forward tolerance;
  * more than 64 chunks (the merge loads the states 64 at a time), one chunk
    (no state merged), and a target logit of -0.0 in a row whose lse is 0.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from klp_testutil import FWD_TOL, seeded_logits, seeded_targets

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lib():
    from kernel_opt._library import DTYPE_CODES, check_status, lib, ptr, stream_handle
    return DTYPE_CODES, check_status, lib, ptr, stream_handle


def plan_of(V, widths):
    plan, c0 = [], 0
    for w in widths:
        plan.append((c0, w))
        c0 += w
    assert c0 == V
    return plan


def run_chunked(x, t, plan, temperature=None):
    """klp_fwd_chunk over column slices of x (each a strided [N, w] view)."""
    from kernel_opt import _C
    codes, check_status, lib, ptr, stream_handle = _lib()
    N = x.size(0)
    T = 1.0 if temperature is None else float(temperature)
    states = torch.full((len(plan), N, 4), float("nan"), dtype=torch.float32, device=DEV)
    outs = [torch.full((N,), float("nan"), dtype=torch.float32, device=DEV) for _ in range(3)]
    st = stream_handle(x.device.index)
    for c, (c0, n) in enumerate(plan):
        xs = x[:, c0:c0 + n]
        check_status(lib.klp_fwd_chunk(ptr(xs), codes[x.dtype], N, n, *_C.row_layout(xs), ptr(t),
                                       c0, T, ptr(states), c, len(plan), ptr(outs[0]),
                                       ptr(outs[1]), ptr(outs[2]), st))
    return tuple(outs), states


def run_shards(x, t, plan, temperature=None):
    """klp_fwd_shard over the same slices, then klp_fwd_shard_merge."""
    from kernel_opt import shard
    V = x.size(1)
    states = torch.stack([shard.shard_state(x[:, c0:c0 + n], t, c0, temperature)
                          for c0, n in plan])
    # the merge's shard width: the chunks' own when they are equal (the last
    # may be narrower), else any width the merge accepts (its logprob is then
    # not the chunks')
    sv = plan[0][1] if equal_width(plan) else -(-V // len(plan))
    return shard.merge_shard_states(states, t, sv, V), states


def equal_width(plan):
    w = plan[0][1]
    return all(n == w for _, n in plan[:-1]) and plan[-1][1] <= w


CASES = [  # dtype, V, widths (None: equal), temperature
    (torch.bfloat16, 8192, None, None),
    (torch.bfloat16, 152064, [32768] * 4 + [16384, 4608], None),
    (torch.bfloat16, 20000, [16384, 3616], 0.7),
    (torch.float16, 5003, [1000, 3, 2000, 2000], 1.3),
    (torch.float32, 3000, [64, 2936], None),
    (torch.float32, 4099, None, 0.7),
]


@pytest.mark.parametrize("dtype,V,widths,T", CASES)
def test_chunk_merge_matches_shards_and_oracle(dtype, V, widths, T, oracle):
    N = 37
    x = seeded_logits((N, V), dtype, seed=V % 101 + 3)
    t = seeded_targets((N,), V, seed=11)
    t[3] = -100
    t[5] = V
    t[6] = V - 1
    if widths is None:
        P = 4
        sv = -(-V // P)
        widths = [sv] * (P - 1) + [V - sv * (P - 1)]
    plan = plan_of(V, widths)
    xd, td = x.to(DEV), t.to(DEV)
    (lp, ent, lse), states = run_chunked(xd, td, plan, T)
    (s_lp, s_ent, s_lse), s_states = run_shards(xd, td, plan, T)
    # the earlier chunks wrote the shard kernel's states; the last chunk's
    # slot is not written
    assert torch.equal(states[:-1], s_states[:-1])
    assert torch.isnan(states[-1]).all()
    assert torch.equal(ent, s_ent) and torch.equal(lse, s_lse)
    if equal_width(plan):
        assert torch.equal(lp, s_lp)
    # the kernels scale by 1 / T computed in double from the fp32 temperature,
    # rounded to fp32
    scale = np.float32(1.0 / float(np.float32(1.0 if T is None else T)))
    inside = (t >= 0) & (t < V)
    xt = torch.zeros(N, dtype=torch.float32)
    xt[inside] = x[inside.nonzero().squeeze(1), t[inside]].float() * float(scale)
    assert torch.equal(lp.cpu(), xt - lse.cpu())
    ref = oracle.forward(x, t.numpy(), temperature=T)
    tol = FWD_TOL[dtype]
    for name, o, r in zip(("logp", "entropy", "lse"), (lp, ent, lse), ref):
        err = np.abs(o.cpu().double().numpy() - r).max()
        assert err <= tol, f"{name}: {err:.3g} > {tol}"


def test_more_than_64_chunks(oracle):
    N, V = 29, 7000
    x = seeded_logits((N, V), torch.bfloat16, seed=70)
    t = seeded_targets((N,), V, seed=71)
    widths = [97] * 71 + [V - 97 * 71]
    plan = plan_of(V, widths)
    xd, td = x.to(DEV), t.to(DEV)
    (lp, ent, lse), _ = run_chunked(xd, td, plan)
    _, s_ent, s_lse = run_shards(xd, td, plan)[0]
    assert torch.equal(ent, s_ent) and torch.equal(lse, s_lse)
    ref = oracle.forward(x, t.numpy())
    for o, r in zip((lp, ent, lse), ref):
        assert np.abs(o.cpu().double().numpy() - r).max() <= FWD_TOL[torch.bfloat16]


def test_one_chunk_equals_forward():
    """A single chunk merges nothing: the outputs are klp_fwd_shard's state
    finalised, i.e. the forward on the whole row (same launch shape rule)."""
    from kernel_opt import shard
    N, V = 64, 3000
    x = seeded_logits((N, V), torch.bfloat16, seed=80).to(DEV)
    t = seeded_targets((N,), V, seed=81).to(DEV)
    (lp, ent, lse), _ = run_chunked(x, t, [(0, V)])
    s = shard.shard_state(x, t, 0)
    m_lp, m_ent, m_lse = shard.merge_shard_states(s.unsqueeze(0), t, V, V)
    assert torch.equal(lp, m_lp) and torch.equal(ent, m_ent) and torch.equal(lse, m_lse)


def test_negative_zero_target_logit():
    """Row [-0.0, -inf, -inf] in chunks [1, 2]: lse = 0, and the target logit
    -0.0 comes from the first chunk, so logp is -0.0 as the forward gives."""
    from kernel_opt import fused_logprob_entropy_forward
    x = torch.tensor([[-0.0, float("-inf"), float("-inf")]] * 3, dtype=torch.float32, device=DEV)
    t = torch.tensor([0, 1, 5], dtype=torch.int64, device=DEV)
    (lp, ent, lse), _ = run_chunked(x, t, [(0, 1), (1, 2)])
    f_lp, f_ent, f_lse = fused_logprob_entropy_forward(x, t)
    assert torch.equal(lse, f_lse) and torch.equal(ent, f_ent)
    assert torch.equal(lp, f_lp)
    assert torch.signbit(lp[0]).item() and lp[0].item() == 0.0
    assert lp[1].item() == float("-inf")
