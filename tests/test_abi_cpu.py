"""The C-ABI library on the CPU: it loads, exports every symbol the public
headers declare, and rejects bad arguments with the documented status and
message before touching the GPU.  No compute call is made."""
from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from conftest import ROOT

HEADERS = [os.path.join(ROOT, "include", h) for h in ("kernel_opt_hip.h", "kernel_opt_hip_tuning.h")]


def _declared_functions():
    names = []
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(klp_\w+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    from kernel_opt import _library
    declared = _declared_functions()
    assert len(declared) >= 10
    lib = ctypes.CDLL(_library.LIB_PATH)
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    # and the Python loader binds exactly these
    assert sorted(_library.SIGNATURES) == declared


def test_abi_version():
    from kernel_opt import _library
    assert _library.lib.klp_abi_version() == _library.ABI_VERSION == 1


# Fake, suitably aligned addresses: every call below must fail validation (or
# hit the injected failure) before any pointer is dereferenced or any HIP call
# is made.
P = ctypes.c_void_p(0x10000)


def _fwd(lib, dtype=0, n=4, v=100, rows_inner=4, so=0, si=100, logits=P, targets=P, outs=(P, P, P),
         ws=None, ws_bytes=0):
    return lib.klp_fwd(logits, dtype, n, v, rows_inner, so, si, targets, *outs, ws, ws_bytes, None)


def _err():
    from kernel_opt import _library
    return _library.last_error()


def test_validation_errors():
    from kernel_opt._library import KLP_EDTYPE, KLP_EINVAL, KLP_OK, lib
    assert _fwd(lib, dtype=7) == KLP_EDTYPE
    assert _err() == "logits dtype must be bf16, fp16, or fp32"
    assert _fwd(lib, v=0) == KLP_EINVAL and "vocab" in _err()
    assert _fwd(lib, n=-1) == KLP_EINVAL
    assert _fwd(lib, logits=None) == KLP_EINVAL and "non-null" in _err()
    assert _fwd(lib, logits=ctypes.c_void_p(0x10001)) == KLP_EINVAL and "aligned" in _err()
    assert _fwd(lib, targets=ctypes.c_void_p(0x10004)) == KLP_EINVAL and "targets" in _err()
    assert _fwd(lib, rows_inner=0) == KLP_EINVAL
    assert _fwd(lib, si=-5) == KLP_EINVAL
    assert _fwd(lib, outs=(P, None, P)) == KLP_EINVAL and "entropy" in _err()
    # N = 0 is a no-op: succeeds even with null pointers
    assert _fwd(lib, n=0, logits=None, targets=None, outs=(None, None, None)) == KLP_OK
    assert _err() == ""


def test_workspace_and_launch_shape_errors():
    from kernel_opt._library import KLP_EINVAL, KLP_EWORKSPACE, lib
    need = lib.klp_fwd_workspace_bytes_ex(4, 8)
    # one float4 state per (row, split), then a 32-bit arrival counter per
    # row rounded up to 16 bytes
    assert need == 4 * 8 * 16 + 16
    assert lib.klp_fwd_workspace_bytes_ex(5, 2) == 5 * 2 * 16 + 32
    assert lib.klp_fwd_workspace_bytes_ex(4, 1) == 0
    rc = lib.klp_fwd_ex(P, 0, 4, 100, 4, 0, 100, P, P, P, P, P, need - 16, 8, 4, 8, 0, None)
    assert rc == KLP_EWORKSPACE and "workspace" in _err()
    rc = lib.klp_fwd_ex(P, 0, 4, 100, 4, 0, 100, P, P, P, P, ctypes.c_void_p(0x10008), need,
                        8, 4, 8, 0, None)
    assert rc == KLP_EWORKSPACE  # misaligned workspace
    rc = lib.klp_fwd_ex(P, 0, 4, 100, 4, 0, 100, P, P, P, P, None, 0, 5, 4, 1, 0, None)
    assert rc == KLP_EINVAL and "launch shape" in _err()
    rc = lib.klp_fwd_ex(P, 0, 4, 100, 4, 0, 100, P, P, P, P, None, 0, 8, 4, 1, 1, None)
    assert rc == KLP_EINVAL and "flags" in _err()  # forward has no variant flags
    rc = lib.klp_bwd_ex(P, 0, 4, 100, 4, 0, 100, P, P, P, None, None, None, P, 8, 3, 1, 1, None)
    assert rc == KLP_EINVAL and "launch shape" in _err()
    rc = lib.klp_bwd(P, 0, 4, 100, 4, 0, 100, P, P, P, None, None, None, None, None)
    assert rc == KLP_EINVAL and "d_logits" in _err()
    # The backward's row pieces are read with 32-bit buffer offsets: a bf16
    # row of 2^30 logits in one piece is refused, not misread.
    V = 1 << 30
    rc = lib.klp_bwd_ex(P, 0, 1, V, 1, 0, V, P, P, P, None, None, None, P, 16, 2, 1, 1, None)
    assert rc == KLP_EINVAL and "2 GiB" in _err()
    w, u, sp, fl = (ctypes.c_int() for _ in range(4))
    lib.klp_default_config(1, 0, 1, V, ctypes.byref(w), ctypes.byref(u), ctypes.byref(sp),
                           ctypes.byref(fl))
    assert sp.value >= 2  # the default keeps each piece under 2 GiB


def test_injected_launch_failure_reports_elaunch():
    from kernel_opt._library import KLP_ELAUNCH, lib
    lib.klp_debug_fail_next_launches(2)
    try:
        assert _fwd(lib) == KLP_ELAUNCH
        assert "launch failed" in _err() and "injected" in _err()
        rc = lib.klp_bwd(P, 0, 4, 100, 4, 0, 100, P, P, P, None, None, None, P, None)
        assert rc == KLP_ELAUNCH
    finally:
        lib.klp_debug_fail_next_launches(0)


def test_last_error_truncates():
    from kernel_opt._library import lib
    _fwd(lib, dtype=9)
    n = lib.klp_last_error(None, 0)
    buf = ctypes.create_string_buffer(8)
    assert lib.klp_last_error(buf, 8) == n
    assert buf.value == b"logits "


def test_default_launch_shapes():
    from kernel_opt import _C
    # headline config: 1024 rows x 8 waves fill 256 CUs at 8 waves per SIMD,
    # unroll 2 (61 VGPRs), no split
    assert _C.default_config("fwd", torch.bfloat16, 1024, 152064) == (8, 2, 1, 0)
    # several rounds of workgroups: unroll 4; fp32 rows on 4 waves
    assert _C.default_config("fwd", torch.bfloat16, 32768, 151936) == (8, 4, 1, 0)
    assert _C.default_config("fwd", torch.float32, 8192, 262144) == (4, 4, 1, 0)
    # short rows (a vocab shard of C4): 4 waves, unroll 2
    assert _C.default_config("fwd", torch.bfloat16, 32768, 18992) == (4, 2, 1, 0)
    # 256 rows: wider workgroups instead of splitting
    assert _C.default_config("fwd", torch.float32, 256, 32000)[::2] == (16, 1)
    # few rows, long vocab: split rows (needs a workspace), about one
    # workgroup per CU, at least 3 vectors per thread
    w, u, s, f = _C.default_config("fwd", torch.bfloat16, 16, 152064)
    assert (w, u, s) == (8, 2, 8)
    assert _C.default_config("fwd", torch.bfloat16, 1, 152064)[:3] == (8, 2, 8)
    assert _C.default_config("fwd", torch.bfloat16, 128, 152064)[:3] == (8, 2, 2)
    assert _C.default_config("fwd", torch.float32, 64, 262144)[:3] == (8, 2, 4)
    # few rows that are not split: long ones on 8 waves, short ones on 16
    assert _C.default_config("fwd", torch.bfloat16, 256, 152064)[:3] == (8, 2, 1)
    # tiny vocab: never split
    assert _C.default_config("fwd", torch.float32, 4, 64)[2] == 1
    from kernel_opt._library import lib
    assert lib.klp_fwd_workspace_bytes(0, 32768, 151936) == 0
    assert lib.klp_fwd_workspace_bytes(0, 1024, 152064) == 0
    assert lib.klp_fwd_workspace_bytes(0, 16, 152064) == 16 * s * 16 + 64
    # backward splits rows freely (no second pass)
    assert _C.default_config("bwd", torch.bfloat16, 1024, 152064)[2] >= 2
    # bf16 / fp16 logits over the Infinity Cache's size: 4-wave workgroups
    # over pieces of about one iteration (512 vectors): at most one on
    # smaller grids (C2: 19008 vectors in 38 pieces of 504), at most 33/32
    # from 131072 pieces on (C3: 31 of 520, C4: 36 of 528)
    assert _C.default_config("bwd", torch.bfloat16, 1024, 152064)[:3] == (4, 2, 38)
    assert _C.default_config("bwd", torch.float16, 2048, 152064)[:3] == (4, 2, 38)
    assert _C.default_config("bwd", torch.bfloat16, 1536, 128000)[:3] == (4, 2, 32)
    assert _C.default_config("bwd", torch.float16, 8192, 128256)[:3] == (4, 2, 31)
    assert _C.default_config("bwd", torch.bfloat16, 32768, 151936)[:3] == (4, 2, 36)
    assert _C.default_config("bwd", torch.bfloat16, 4096, 152064)[:3] == (4, 2, 36)
    # logits the cache holds: small bf16 / fp16 grids 8-wave workgroups over
    # twice the power-of-two pieces of 16 waves; fp32 rows 4 waves over four
    # times (C1)
    assert _C.default_config("bwd", torch.bfloat16, 256, 152064)[:3] == (8, 2, 16)
    assert _C.default_config("bwd", torch.bfloat16, 1024, 100352)[:3] == (8, 2, 8)
    assert _C.default_config("bwd", torch.float32, 256, 32000)[:3] == (4, 2, 16)
    # rows of fewer than 8 elements (no 16-byte body) over the cache's size:
    # the piece rule has no vectors to cut and leaves the row whole
    assert _C.default_config("bwd", torch.bfloat16, 40_000_000, 4)[2] == 1
    # fp32 rows: 4 waves at every grid size (C5)
    assert _C.default_config("bwd", torch.float32, 8192, 262144)[:3] == (4, 2, 128)


def test_shim_rejects_cpu_tensors_with_reference_messages():
    from kernel_opt import _C
    x = torch.zeros(2, 8)
    t = torch.zeros(2, dtype=torch.int64)
    o = [torch.zeros(2) for _ in range(3)]
    with pytest.raises(RuntimeError, match="logits must be CUDA"):
        _C.fused_logprob_entropy_v1(x, t, *o)
    with pytest.raises(RuntimeError, match="logits must be CUDA"):
        _C.fused_logprob_entropy_naive(x, t, *o)
    with pytest.raises(RuntimeError, match="logits must be contiguous CUDA"):
        _C.fused_logprob_entropy_v1_backward(x, t, o[0], o[1], None, None, None, x)


def test_ops_assert_on_cpu_tensors():
    import kernel_opt
    x = torch.zeros(2, 8)
    t = torch.zeros(2, dtype=torch.int64)
    for f in (kernel_opt.fused_logprob_entropy, kernel_opt.fused_logprob_entropy_forward,
              kernel_opt.fused_logprob_entropy_naive):
        with pytest.raises(AssertionError):
            f(x, t)


def test_row_layout():
    from kernel_opt._C import row_layout
    x = torch.zeros(4, 6, 10)
    assert row_layout(x) == (24, 0, 10)
    assert row_layout(x[:, :-1, :]) == (5, 60, 10)
    assert row_layout(x[:, 1:, :]) == (5, 60, 10)
    assert row_layout(x[1]) == (6, 0, 10)
    assert row_layout(x[:2, :3]) == (3, 60, 10)
    assert row_layout(x[:, :, :5]) == (24, 0, 10)   # narrowed rows keep unit stride
    assert row_layout(x[:, ::2, :]) == (12, 0, 20)   # (b, s) -> (3b + s) * 20
    assert row_layout(x.transpose(0, 1)) == (4, 10, 60)
    assert row_layout(x[::2, ::2, :]) == (3, 120, 20)
    assert row_layout(x[:, :, ::2]) is None          # non-unit element stride
    assert row_layout(torch.zeros(2, 3, 4, 5)[:, :, :-1]) == (3, 20, 5)
    assert row_layout(torch.zeros(2, 3, 4, 5)[:, :-1, :-1]) is None  # three strides
    assert row_layout(torch.zeros(1, 1, 7)) == (1, 0, 0)
    assert row_layout(torch.zeros(7)) == (1, 0, 0)
    assert row_layout(torch.zeros(())) is None


def test_row_layout_fast_path_matches_general_walk():
    """row_layout's contiguous fast path returns what the general stride walk
    returns, for contiguous tensors of every rank up to 4 and every size
    pattern over {0, 1, 2, 3, 7} (size-1 and size-0 dims included)."""
    import itertools
    from kernel_opt._C import _row_layout_walk, row_layout
    for rank in (1, 2, 3, 4):
        for shape in itertools.product((0, 1, 2, 3, 7), repeat=rank):
            t = torch.empty(shape)
            assert row_layout(t) == _row_layout_walk(t), shape


def test_package_surface_matches_reference():
    """reference python/kernel_opt/__init__.py:1-15."""
    import kernel_opt
    for name in ("fused_logprob_entropy", "fused_logprob_entropy_forward",
                 "fused_logprob_entropy_naive", "_C", "__version__"):
        assert hasattr(kernel_opt, name)
    assert kernel_opt.__version__ == "0.0.1"
    for name in ("fused_logprob_entropy_naive", "fused_logprob_entropy_v1",
                 "fused_logprob_entropy_v1_backward"):
        assert callable(getattr(kernel_opt._C, name))
    with pytest.raises(AttributeError):
        kernel_opt.does_not_exist  # noqa: B018


def test_temperature_must_be_finite_and_positive():
    from kernel_opt._library import KLP_EINVAL, lib
    for T in (0.0, -1.0, float("inf"), float("nan")):
        rc = lib.klp_fwd_temp(P, 0, 4, 100, 4, 0, 100, P, T, P, P, P, None, 0, None)
        assert rc == KLP_EINVAL and "temperature" in _err()
        rc = lib.klp_bwd_temp(P, 0, 4, 100, 4, 0, 100, P, T, P, P, None, None, None, P, None)
        assert rc == KLP_EINVAL and "temperature" in _err()


def test_torch_library_ops_registered():
    import kernel_opt  # noqa: F401
    fwd = str(torch.ops.kernel_opt.fused_logprob_entropy.default._schema)
    bwd = str(torch.ops.kernel_opt.fused_logprob_entropy_backward.default._schema)
    assert "float temperature" in fwd and "-> (Tensor, Tensor, Tensor)" in fwd
    assert "Tensor? g_logp" in bwd and bwd.endswith("-> Tensor")


def test_grpo_validation_errors():
    from kernel_opt._library import KLP_EINVAL, KLP_ELAUNCH, KLP_EWORKSPACE, lib
    ws = lib.klp_grpo_workspace_bytes(4)
    assert ws == (4 * 8 + 1) * 4 and lib.klp_grpo_workspace_bytes(0) == 0

    def fwd(**kw):
        a = dict(logp=P, old=P, ref=None, adv=P, mask=None, B=4, S=10, el=0.2, eh=0.2, beta=0.0,
                 norm=1.0, kind=1, level=0, per_tok=0, loss=P, stats=None, ws=P, ws_bytes=ws)
        a.update(kw)
        return lib.klp_grpo_fwd(a["logp"], a["old"], a["ref"], a["adv"], a["mask"], a["B"],
                                a["S"], a["el"], a["eh"], a["beta"], a["norm"], a["kind"],
                                a["level"], a["per_tok"], a["loss"], a["stats"], a["ws"],
                                a["ws_bytes"], None)
    assert fwd(B=0) == KLP_EINVAL and "n_seqs" in _err()
    assert fwd(S=-1) == KLP_EINVAL
    assert fwd(logp=None) == KLP_EINVAL and "logp" in _err()
    assert fwd(el=-0.1) == KLP_EINVAL and "eps_low" in _err()
    assert fwd(beta=float("nan")) == KLP_EINVAL and "beta" in _err()
    assert fwd(kind=7) == KLP_EINVAL and "loss_type" in _err()
    assert fwd(kind=2, norm=0.0) == KLP_EINVAL and "norm_const" in _err()
    assert fwd(level=3) == KLP_EINVAL and "level" in _err()
    assert fwd(ws_bytes=ws - 4) == KLP_EWORKSPACE and "workspace" in _err()
    assert fwd(loss=None) == KLP_EINVAL and "loss" in _err()
    lib.klp_debug_fail_next_launches(1)
    try:
        assert fwd() == KLP_ELAUNCH and "grpo forward" in _err()
    finally:
        lib.klp_debug_fail_next_launches(0)
    rc = lib.klp_grpo_bwd(P, P, None, P, None, 4, 10, 0.2, 0.2, 0.0, 1.0, 1, 0, 0, None, None,
                          P, ws, None)
    assert rc == KLP_EINVAL and "d_logp" in _err()


def test_grpo_step_validation_errors():
    """klp_grpo_step rejects what it cannot run before any launch (no GPU
    needed): the fused path's row-capacity and 16-byte row rules, seq_len,
    null pointers, loss parameters; an injected launch failure is reported."""
    from kernel_opt._library import KLP_EDTYPE, KLP_EINVAL, KLP_ELAUNCH, lib
    assert lib.klp_grpo_step_max_vocab(0) == 19 * 1024 * 8
    assert lib.klp_grpo_step_max_vocab(1) == 19 * 1024 * 8
    assert lib.klp_grpo_step_max_vocab(2) == 19 * 1024 * 4
    assert lib.klp_grpo_step_max_vocab(5) == 0
    A = ctypes.c_void_p(0x100000)  # 16-byte aligned fake device address

    def step(**kw):
        a = dict(logits=A, dtype=0, n=8, v=4096, ri=8, so=0, si=4096, tg=A, temp=1.0, old=A,
                 ref=None, adv=A, w=A, S=4, el=0.2, eh=0.28, beta=0.0, pt=0, gs=1.0, lp=A,
                 ent=A, lse=None, lt=A, d=A, sched=None)
        a.update(kw)
        return lib.klp_grpo_step(a["logits"], a["dtype"], a["n"], a["v"], a["ri"], a["so"],
                                 a["si"], a["tg"], a["temp"], a["old"], a["ref"], a["adv"],
                                 a["w"], a["S"], a["el"], a["eh"], a["beta"], a["pt"], a["gs"],
                                 a["lp"], a["ent"], a["lse"], a["lt"], a["d"], a["sched"], None)
    assert step(n=0) == 0
    assert step(dtype=9) == KLP_EDTYPE
    assert step(temp=0.0) == KLP_EINVAL and "temperature" in _err()
    assert step(S=3) == KLP_EINVAL and "seq_len" in _err()
    assert step(S=0) == KLP_EINVAL and "seq_len" in _err()
    assert step(v=155648 + 8, si=155656) == KLP_EINVAL and "capacity" in _err()
    assert step(dtype=2, v=77824 + 4, si=77828) == KLP_EINVAL and "capacity" in _err()
    assert step(v=4100, si=4100) == KLP_EINVAL and "16-byte" in _err()
    assert step(logits=ctypes.c_void_p(0x100008)) == KLP_EINVAL and "16-byte" in _err()
    assert step(si=4100) == KLP_EINVAL and "16-byte" in _err()
    assert step(ri=4, so=8196) == KLP_EINVAL and "16-byte" in _err()
    assert step(old=None) == KLP_EINVAL and "old_logp" in _err()
    assert step(w=None) == KLP_EINVAL and "tok_weight" in _err()
    assert step(lt=None) == KLP_EINVAL and "loss_tok" in _err()
    assert step(d=None) == KLP_EINVAL and "d_logits" in _err()
    assert step(d=ctypes.c_void_p(0x100004)) == KLP_EINVAL and "d_logits" in _err()
    assert step(el=-1.0) == KLP_EINVAL and "eps_low" in _err()
    assert step(beta=float("inf")) == KLP_EINVAL and "beta" in _err()
    for gs in (0.0, -0.0, float("inf"), float("-inf"), float("nan")):
        assert step(gs=gs) == KLP_EINVAL and "grad_scale" in _err(), gs
    assert step(n=0, gs=0.0) == 0  # no rows: nothing checked past the rows
    assert step(sched=ctypes.c_void_p(0x100004)) == KLP_EINVAL and "sched" in _err()
    lib.klp_debug_fail_next_launches(1)
    try:
        assert step() == KLP_ELAUNCH and "grpo step" in _err()
    finally:
        lib.klp_debug_fail_next_launches(0)


def test_shard_validation_errors():
    """klp_fwd_shard / klp_fwd_shard_merge reject bad arguments before any
    launch; injected launch failures are reported."""
    from kernel_opt._library import KLP_EDTYPE, KLP_EINVAL, KLP_ELAUNCH, lib
    A = ctypes.c_void_p(0x100000)

    def shard(**kw):
        a = dict(x=A, dtype=0, n=8, v=1000, ri=8, so=0, si=1000, t=A, off=0, temp=1.0, st=A)
        a.update(kw)
        return lib.klp_fwd_shard(a["x"], a["dtype"], a["n"], a["v"], a["ri"], a["so"], a["si"],
                                 a["t"], a["off"], a["temp"], a["st"], None)
    assert shard(n=0) == 0
    assert shard(dtype=7) == KLP_EDTYPE
    assert shard(temp=-1.0) == KLP_EINVAL and "temperature" in _err()
    assert shard(off=-1) == KLP_EINVAL and "vocab_offset" in _err()
    assert shard(st=None) == KLP_EINVAL and "state" in _err()
    assert shard(st=ctypes.c_void_p(0x100004)) == KLP_EINVAL and "state" in _err()
    lib.klp_debug_fail_next_launches(1)
    try:
        assert shard() == KLP_ELAUNCH and "shard forward" in _err()
    finally:
        lib.klp_debug_fail_next_launches(0)

    def merge(**kw):
        a = dict(s=A, p=4, n=8, t=A, sv=250, v=1000, lp=A, ent=A, lse=A)
        a.update(kw)
        return lib.klp_fwd_shard_merge(a["s"], a["p"], a["n"], a["t"], a["sv"], a["v"], a["lp"],
                                       a["ent"], a["lse"], None)
    assert merge(n=0) == 0
    assert merge(p=0) == KLP_EINVAL and "n_shards" in _err()
    assert merge(v=1001) == KLP_EINVAL and "vocab" in _err()
    assert merge(v=750) == KLP_EINVAL and "vocab" in _err()
    assert merge(s=ctypes.c_void_p(0x100008)) == KLP_EINVAL and "states" in _err()
    assert merge(t=None) == KLP_EINVAL and "targets" in _err()
    assert merge(lse=None) == KLP_EINVAL and "lse" in _err()
    lib.klp_debug_fail_next_launches(1)
    try:
        assert merge() == KLP_ELAUNCH and "shard merge" in _err()
    finally:
        lib.klp_debug_fail_next_launches(0)


def test_chunk_validation_errors():
    """klp_fwd_chunk rejects bad arguments before any launch: the chunk index
    must lie in [0, n_chunks), the states must be 16-byte aligned, and only
    the last chunk (which writes them) checks the outputs."""
    from kernel_opt._library import KLP_EDTYPE, KLP_EINVAL, KLP_ELAUNCH, lib
    A = ctypes.c_void_p(0x100000)

    def chunk(**kw):
        a = dict(x=A, dtype=0, n=8, v=1000, ri=8, so=0, si=1000, t=A, off=0, temp=1.0, st=A,
                 c=0, nc=3, lp=A, ent=A, lse=A)
        a.update(kw)
        return lib.klp_fwd_chunk(a["x"], a["dtype"], a["n"], a["v"], a["ri"], a["so"], a["si"],
                                 a["t"], a["off"], a["temp"], a["st"], a["c"], a["nc"], a["lp"],
                                 a["ent"], a["lse"], None)
    assert chunk(n=0) == 0
    assert chunk(dtype=7) == KLP_EDTYPE
    assert chunk(temp=0.0) == KLP_EINVAL and "temperature" in _err()
    assert chunk(off=-1) == KLP_EINVAL and "vocab_offset" in _err()
    assert chunk(c=3) == KLP_EINVAL and "chunk_index" in _err()
    assert chunk(c=-1) == KLP_EINVAL and "chunk_index" in _err()
    assert chunk(nc=0) == KLP_EINVAL and "chunk_index" in _err()
    assert chunk(st=None) == KLP_EINVAL and "states" in _err()
    assert chunk(st=ctypes.c_void_p(0x100008)) == KLP_EINVAL and "states" in _err()
    assert chunk(c=2, lse=None) == KLP_EINVAL and "lse" in _err()
    assert chunk(c=2, lp=ctypes.c_void_p(0x100002)) == KLP_EINVAL and "logprob" in _err()
    lib.klp_debug_fail_next_launches(2)
    try:
        # an earlier chunk does not read the outputs
        assert chunk(c=0, lse=None) == KLP_ELAUNCH and "chunk forward" in _err()
        assert chunk(c=2) == KLP_ELAUNCH and "chunk forward" in _err()
    finally:
        lib.klp_debug_fail_next_launches(0)


def test_scale_inplace_validation_errors():
    """klp_scale_inplace rejects bad arguments before any launch; n = 0 is a
    no-op; an injected launch failure is reported."""
    from kernel_opt._library import KLP_EDTYPE, KLP_EINVAL, KLP_ELAUNCH, lib
    A = ctypes.c_void_p(0x100000)

    def scale(**kw):
        a = dict(d=A, dtype=0, n=100, s=A)
        a.update(kw)
        return lib.klp_scale_inplace(a["d"], a["dtype"], a["n"], a["s"], None)
    assert scale(n=0) == 0
    assert scale(n=0, d=None, s=None) == 0
    assert scale(dtype=3) == KLP_EDTYPE
    assert scale(n=-1) == KLP_EINVAL and "n must" in _err()
    assert scale(d=None) == KLP_EINVAL and "data" in _err()
    assert scale(d=ctypes.c_void_p(0x100001)) == KLP_EINVAL and "data" in _err()
    assert scale(dtype=2, d=ctypes.c_void_p(0x100002)) == KLP_EINVAL and "data" in _err()
    assert scale(s=None) == KLP_EINVAL and "scale" in _err()
    assert scale(s=ctypes.c_void_p(0x100002)) == KLP_EINVAL and "scale" in _err()
    lib.klp_debug_fail_next_launches(1)
    try:
        assert scale() == KLP_ELAUNCH and "scale" in _err()
    finally:
        lib.klp_debug_fail_next_launches(0)


def test_rescale_inplace_validation_errors():
    """klp_rescale_inplace checks `applied` (finite, non-zero), then the
    buffer as klp_scale_inplace does; an injected launch failure is
    reported."""
    from kernel_opt._library import KLP_EDTYPE, KLP_EINVAL, KLP_ELAUNCH, lib
    A = ctypes.c_void_p(0x100000)

    def rescale(**kw):
        a = dict(d=A, dtype=0, n=100, s=A, applied=0.125)
        a.update(kw)
        return lib.klp_rescale_inplace(a["d"], a["dtype"], a["n"], a["s"], a["applied"], None)
    for bad in (0.0, -0.0, float("inf"), float("-inf"), float("nan")):
        assert rescale(applied=bad) == KLP_EINVAL and "applied" in _err(), bad
        assert rescale(applied=bad, n=0) == KLP_EINVAL and "applied" in _err(), bad
    assert rescale(n=0) == 0
    assert rescale(applied=-3.0, n=0, d=None, s=None) == 0
    assert rescale(dtype=3) == KLP_EDTYPE
    assert rescale(n=-1) == KLP_EINVAL and "n must" in _err()
    assert rescale(d=ctypes.c_void_p(0x100001)) == KLP_EINVAL and "data" in _err()
    assert rescale(s=None) == KLP_EINVAL and "scale" in _err()
    lib.klp_debug_fail_next_launches(1)
    try:
        assert rescale() == KLP_ELAUNCH and "scale" in _err()
    finally:
        lib.klp_debug_fail_next_launches(0)


def test_header_constants_match_the_python_names():
    """Every #define KLP_<NAME> <int> of include/*.h that kernel_opt._library
    names has the same value there."""
    from kernel_opt import _library
    found = 0
    for name in ("kernel_opt_hip.h", "kernel_opt_hip_tuning.h"):
        with open(os.path.join(ROOT, "include", name)) as f:
            for k, v in re.findall(r"^#define (KLP_[A-Z0-9_]+) (\d+)\s*$", f.read(), re.M):
                if hasattr(_library, k):
                    assert getattr(_library, k) == int(v), k
                    found += 1
    assert found >= 2


def test_grpo_token_weights_validation_errors():
    """klp_grpo_token_weights rejects bad arguments before any launch; an
    empty batch is a no-op; an injected launch failure is reported."""
    from kernel_opt._library import KLP_EDTYPE, KLP_EINVAL, KLP_ELAUNCH, lib
    A = ctypes.c_void_p(0x100000)

    def tw(**kw):
        a = dict(m=A, md=1, B=4, S=8, kind=0, scale=1.0, w=A, ws=None)
        a.update(kw)
        return lib.klp_grpo_token_weights(a["m"], a["md"], a["B"], a["S"], a["kind"],
                                          a["scale"], a["w"], a["ws"], None)
    assert tw(B=0) == 0 and tw(S=0, m=None, w=None) == 0
    assert tw(B=-1) == KLP_EINVAL and "n_seqs" in _err()
    assert tw(kind=3) == KLP_EINVAL and "loss_type" in _err()
    assert tw(md=3) == KLP_EDTYPE and "mask" in _err()
    assert tw(w=None) == KLP_EINVAL and "weights" in _err()
    assert tw(w=ctypes.c_void_p(0x100002)) == KLP_EINVAL and "weights" in _err()
    assert tw(m=ctypes.c_void_p(0x100002)) == KLP_EINVAL and "mask" in _err()       # int32
    assert tw(md=2, m=ctypes.c_void_p(0x100004)) == KLP_EINVAL and "mask" in _err()  # int64
    assert tw(kind=2, scale=0.0) == KLP_EINVAL and "scale" in _err()
    assert tw(kind=2, scale=float("inf")) == KLP_EINVAL and "scale" in _err()
    assert tw(B=1 << 62, S=8) == KLP_EINVAL and "overflows" in _err()
    assert tw(kind=1) == KLP_EINVAL and "workspace" in _err()  # "bnpo" needs one
    assert tw(kind=1, ws=ctypes.c_void_p(0x100004)) == KLP_EINVAL and "workspace" in _err()
    assert tw(kind=1, B=0) == 0
    lib.klp_debug_fail_next_launches(1)
    try:
        assert tw(md=0, m=ctypes.c_void_p(0x100001)) == KLP_ELAUNCH and "token_weights" in _err()
    finally:
        lib.klp_debug_fail_next_launches(0)


def test_ceiling_validation_errors():
    """klp_ceiling_read / _copy / _read_pieces / _write reject bad arguments
    before any launch; n_rows = 0 is a no-op; an injected launch failure is
    reported."""
    from kernel_opt._library import KLP_EINVAL, KLP_ELAUNCH, lib
    A = ctypes.c_void_p(0x100000)

    def read(**kw):
        a = dict(src=A, n=4, rb=4096, w=4, u=4, sp=1, sink=A)
        a.update(kw)
        return lib.klp_ceiling_read(a["src"], a["n"], a["rb"], a["w"], a["u"], a["sp"],
                                    a["sink"], 7, None)

    def copy(**kw):
        a = dict(src=A, dst=A, n=4, rb=4096, w=16, u=2, sp=8)
        a.update(kw)
        return lib.klp_ceiling_copy(a["src"], a["dst"], a["n"], a["rb"], a["w"], a["u"],
                                    a["sp"], None)
    assert read(n=0, src=None, sink=None) == 0 and copy(n=0, src=None, dst=None) == 0
    assert read(n=-1) == KLP_EINVAL and "n_rows" in _err()
    assert read(rb=24) == KLP_EINVAL and "multiple of 16" in _err()
    assert copy(rb=0) == KLP_EINVAL and "multiple of 16" in _err()
    assert read(src=ctypes.c_void_p(0x100008)) == KLP_EINVAL and "src" in _err()
    assert copy(dst=None) == KLP_EINVAL and "dst" in _err()
    assert read(sink=None) == KLP_EINVAL and "sink" in _err()
    assert read(w=3) == KLP_EINVAL and "launch shape" in _err()
    assert copy(u=8) == KLP_EINVAL and "launch shape" in _err()
    assert copy(sp=0) == KLP_EINVAL and "launch shape" in _err()
    assert copy(n=1, rb=(1 << 31) + 16, sp=1) == KLP_EINVAL and "2 GiB" in _err()
    assert read(n=1, rb=(1 << 31) - 16, sp=1) == KLP_EINVAL and "2 GiB" in _err()

    def pieces(**kw):
        a = dict(src=A, n=4, rb=4096, w=8, u=2, sp=16, sink=A)
        a.update(kw)
        return lib.klp_ceiling_read_pieces(a["src"], a["n"], a["rb"], a["w"], a["u"], a["sp"],
                                           a["sink"], 7, None)

    def write(**kw):
        a = dict(dst=A, n=4, rb=4096, w=8, u=2, sp=16)
        a.update(kw)
        return lib.klp_ceiling_write(a["dst"], a["n"], a["rb"], a["w"], a["u"], a["sp"], None)
    assert pieces(n=0, src=None, sink=None) == 0 and write(n=0, dst=None) == 0
    assert pieces(src=None) == KLP_EINVAL and "src" in _err()
    assert pieces(sink=None) == KLP_EINVAL and "sink" in _err()
    assert write(dst=ctypes.c_void_p(0x100004)) == KLP_EINVAL and "dst" in _err()
    assert write(rb=8) == KLP_EINVAL and "multiple of 16" in _err()
    assert write(w=32) == KLP_EINVAL and "launch shape" in _err()
    assert pieces(n=1, rb=(1 << 31) + 16, sp=1) == KLP_EINVAL and "2 GiB" in _err()
    lib.klp_debug_fail_next_launches(1)
    try:
        assert copy() == KLP_ELAUNCH and "ceiling copy" in _err()
    finally:
        lib.klp_debug_fail_next_launches(0)


def test_noalloc_forward_validation_errors():
    """klp_fwd_noalloc checks its arguments before it touches a device, and
    n_rows = 0 is a no-op."""
    from kernel_opt._library import KLP_EDTYPE, KLP_EINVAL, lib
    A = ctypes.c_void_p(0x100000)

    def fwd(**kw):
        a = dict(x=A, dtype=0, n=4, V=100, t=A, o=A)
        a.update(kw)
        return lib.klp_fwd_noalloc(a["x"], a["dtype"], a["n"], a["V"], a["n"], 0, a["V"],
                                   a["t"], a["o"], a["o"], a["o"], None)
    assert fwd(n=0, x=None, t=None) == 0
    assert fwd(dtype=7) == KLP_EDTYPE and "dtype" in _err()
    assert fwd(V=0) == KLP_EINVAL and "vocab" in _err()
    assert fwd(x=None) == KLP_EINVAL and "non-null" in _err()
    assert fwd(t=ctypes.c_void_p(0x100004)) == KLP_EINVAL and "targets" in _err()
