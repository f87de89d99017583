"""klp_fwd_noalloc (the forward with no workspace argument; split-row
partial states in the library's per-GPU scratch array) against klp_fwd with
a caller workspace, through the C ABI: two calls in a row, the second on a
smaller input, both in split-row mode (so both go through the scratch),
then one that does not split.  The two entry points run the same kernels
with the same launch shape, so the outputs must be bitwise equal; they are
also checked against the float64 oracle at the forward bar (2e-5 for bf16 /
fp16 input)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(N, V, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(N, V, generator=g) * 2.0).to(dtype)
    t = torch.randint(0, V, (N,), generator=g)
    t[0] = -100  # an ignored target
    return x, t


def _noalloc(x, t):
    from kernel_opt import _C
    from kernel_opt._library import DTYPE_CODES, check_status, lib
    N, V = x.shape
    outs = [torch.full((N,), float("nan"), dtype=torch.float32, device=DEV) for _ in range(3)]
    st = torch.cuda.current_stream().cuda_stream
    check_status(lib.klp_fwd_noalloc(x.data_ptr(), DTYPE_CODES[x.dtype], N, V, *_C.row_layout(x),
                                     t.data_ptr(), *(o.data_ptr() for o in outs), st))
    return outs


def _with_workspace(x, t):
    from kernel_opt import _C
    outs = [torch.full((x.shape[0],), float("nan"), dtype=torch.float32, device=DEV)
            for _ in range(3)]
    _C.fwd_launch(x, t, *outs)
    return outs


@pytest.mark.parametrize("cases", [[(32, 152064, torch.bfloat16), (8, 131075, torch.float16)]])
def test_noalloc_matches_klp_fwd_on_two_calls(cases, oracle):
    from kernel_opt import _C
    for i, (N, V, dtype) in enumerate(cases):
        print(f"klp_fwd_noalloc call {i}: [{N}, {V}] {dtype}", flush=True)
        assert _C.default_config("fwd", dtype, N, V)[2] > 1, "expected a split-row launch"
        x_cpu, t_cpu = _inputs(N, V, dtype, 40 + i)
        x, t = x_cpu.to(DEV), t_cpu.to(DEV)
        got = _noalloc(x, t)
        ref = _with_workspace(x, t)
        torch.cuda.synchronize()
        for name, a, b in zip(("logprob", "entropy", "lse"), got, ref):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32)), name
        e_lp, e_ent, e_lse = oracle.forward(x_cpu, t_cpu.numpy())
        for a, e in zip(got, (e_lp, e_ent, e_lse)):
            assert np.abs(a.cpu().double().numpy() - e).max() <= 2e-5


def test_noalloc_without_split_matches_klp_fwd():
    from kernel_opt import _C
    N, V = 1024, 4096
    assert _C.default_config("fwd", torch.bfloat16, N, V)[2] == 1
    x, t = (z.to(DEV) for z in _inputs(N, V, torch.bfloat16, 44))
    for a, b in zip(_noalloc(x, t), _with_workspace(x, t)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
