"""Loader for the HIP shared library ``_lib/libkernel_opt_hip.so`` and its
compiled torch binding ``_lib/klp_torch*.so``.

Both are built in-tree by ``__graft_entry__.build()`` (hipcc,
``--offload-arch=gfx950``; the binding by ``setup.py build_ext --inplace``).
There is no fallback: if either is missing or does not load, importing
:mod:`kernel_opt` raises ``ImportError``.  ``lib`` is the library through
ctypes (every entry point of the public headers); ``binding`` is the compiled
module that the logprob op's per-call path goes through.

``torch`` is imported first so that the library's ``libamdhip64.so.7``
dependency resolves (by soname) to the HIP runtime torch already loaded; the
process then holds a single HIP runtime.
"""
from __future__ import annotations

import contextlib
import ctypes
import glob
import importlib.util
import os
import sysconfig

import torch  # noqa: F401  (must precede the dlopen below, see module docstring)

LIB_NAME = "libkernel_opt_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", LIB_NAME)
ABI_VERSION = 1

# klp_dtype values (include/kernel_opt_hip.h)
KLP_BF16, KLP_FP16, KLP_FP32 = 0, 1, 2
DTYPE_CODES = {torch.bfloat16: KLP_BF16, torch.float16: KLP_FP16, torch.float32: KLP_FP32}

# klp_status values
KLP_OK, KLP_EINVAL, KLP_EDTYPE, KLP_ELAUNCH, KLP_EWORKSPACE = 0, 1, 2, 3, 4

# klp_grpo_loss_type / klp_grpo_level values
KLP_GRPO_LOSS_GRPO, KLP_GRPO_LOSS_BNPO, KLP_GRPO_LOSS_FIXED = 0, 1, 2
KLP_GRPO_TOKEN, KLP_GRPO_SEQUENCE = 0, 1
# klp_fwd_noalloc's split-row scratch per GPU (KLP_FWD_NOALLOC_SCRATCH_BYTES).
KLP_FWD_NOALLOC_SCRATCH_BYTES = 65536
# klp_grpo_step's row counter (KLP_GRPO_STEP_SCHED_BYTES).
KLP_GRPO_STEP_SCHED_BYTES = 16
# klp_grpo_token_weights' workspace ("bnpo": per-workgroup partial sums).
KLP_GRPO_TOKEN_WEIGHTS_WORKSPACE_BYTES = 8192

# Every symbol the public headers declare, with its ctypes signature.
_vp, _i32, _i64, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
_ROWS = [_vp, _i32, _i64, _i64, _i64, _i64, _i64]  # logits, dtype, N, V, rows_inner, s_outer, s_inner
SIGNATURES = {
    # include/kernel_opt_hip.h
    "klp_abi_version": (_i32, []),
    "klp_last_error": (_sz, [ctypes.c_char_p, _sz]),
    "klp_fwd_workspace_bytes": (_sz, [_i32, _i64, _i64]),
    "klp_fwd": (_i32, _ROWS + [_vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "klp_fwd_naive": (_i32, _ROWS + [_vp, _vp, _vp, _vp, _vp]),
    "klp_bwd": (_i32, _ROWS + [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "klp_fwd_temp": (_i32, _ROWS + [_vp, ctypes.c_float, _vp, _vp, _vp, _vp, _sz, _vp]),
    "klp_fwd_noalloc": (_i32, _ROWS + [_vp, _vp, _vp, _vp, _vp]),
    "klp_bwd_temp": (_i32, _ROWS + [_vp, ctypes.c_float, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "klp_debug_fail_next_launches": (None, [_i32]),
    "klp_lmh_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "klp_lmh_fwd": (_i32, [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, ctypes.c_float,
                           _vp, _vp, _vp, _vp, _sz, _vp]),
    "klp_lmh_bwd_logits": (_i32, [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, ctypes.c_float,
                                  _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp]),
    "klp_grpo_workspace_bytes": (_sz, [_i64]),
    "klp_grpo_fwd": (_i32, [_vp] * 5 + [_i64, _i64] + [ctypes.c_float] * 4 + [_i32] * 3
                     + [_vp, _vp, _vp, _sz, _vp]),
    "klp_grpo_bwd": (_i32, [_vp] * 5 + [_i64, _i64] + [ctypes.c_float] * 4 + [_i32] * 3
                     + [_vp, _vp, _vp, _sz, _vp]),
    "klp_fwd_shard": (_i32, _ROWS + [_vp, _i64, ctypes.c_float, _vp, _vp]),
    "klp_fwd_shard_merge": (_i32, [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _vp, _vp]),
    "klp_fwd_chunk": (_i32, _ROWS + [_vp, _i64, ctypes.c_float, _vp, _i64, _i64, _vp, _vp, _vp,
                                     _vp]),
    "klp_grpo_step_max_vocab": (_i64, [_i32]),
    "klp_scale_inplace": (_i32, [_vp, _i32, _i64, _vp, _vp]),
    "klp_rescale_inplace": (_i32, [_vp, _i32, _i64, _vp, ctypes.c_float, _vp]),
    "klp_grpo_token_weights": (_i32, [_vp, _i32, _i64, _i64, _i32, ctypes.c_float, _vp, _vp,
                                      _vp]),
    "klp_grpo_step": (_i32, _ROWS + [_vp, ctypes.c_float] + [_vp] * 4 + [_i64]
                      + [ctypes.c_float] * 3 + [_i32, ctypes.c_float] + [_vp] * 7),
    # include/kernel_opt_hip_tuning.h
    "klp_grpo_step_persistent_min_rows": (_i64, [_i32, _i64, _i32]),
    "klp_fwd_workspace_bytes_ex": (_sz, [_i64, _i32]),
    "klp_fwd_ex": (_i32, _ROWS + [_vp, _vp, _vp, _vp, _vp, _sz, _i32, _i32, _i32, _i32, _vp]),
    "klp_bwd_ex": (_i32, _ROWS + [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                                  _vp]),
    "klp_default_config": (None, [_i32, _i32, _i64, _i64] + [ctypes.POINTER(_i32)] * 4),
    "klp_ceiling_read": (_i32, [_vp, _i64, _i64, _i32, _i32, _i32, _vp, ctypes.c_uint32, _vp]),
    "klp_ceiling_copy": (_i32, [_vp, _vp, _i64, _i64, _i32, _i32, _i32, _vp]),
    "klp_ceiling_read_pieces": (_i32, [_vp, _i64, _i64, _i32, _i32, _i32, _vp, ctypes.c_uint32,
                                       _vp]),
    "klp_ceiling_write": (_i32, [_vp, _i64, _i64, _i32, _i32, _i32, _vp]),
}


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"kernel_opt: {LIB_PATH} is not built. Build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` from the repository root.")
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as e:  # pragma: no cover - depends on the machine
        raise ImportError(f"kernel_opt: cannot load {LIB_PATH}: {e}") from e
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.klp_abi_version()
    if version != ABI_VERSION:
        raise ImportError(f"kernel_opt: {LIB_NAME} has ABI version {version}, "
                          f"expected {ABI_VERSION}; rebuild it")
    return lib


lib = _load()


def _load_binding():
    path = os.path.join(os.path.dirname(LIB_PATH),
                        "klp_torch" + sysconfig.get_config_var("EXT_SUFFIX"))
    if not os.path.exists(path):
        found = glob.glob(os.path.join(os.path.dirname(LIB_PATH), "klp_torch*.so"))
        raise ImportError(
            f"kernel_opt: the compiled binding {path} is not built"
            + (f" (found {found[0]}, built for another Python)" if found else "")
            + ". Build it with `python -c 'import __graft_entry__ as g; g.build()'` from "
            "the repository root.")
    spec = importlib.util.spec_from_file_location("kernel_opt._lib.klp_torch", path)
    mod = importlib.util.module_from_spec(spec)
    try:
        spec.loader.exec_module(mod)
    except ImportError as e:  # pragma: no cover - depends on the machine
        raise ImportError(f"kernel_opt: cannot load {path}: {e}") from e
    return mod


binding = _load_binding()


def last_error() -> str:
    n = lib.klp_last_error(None, 0)
    buf = ctypes.create_string_buffer(n + 1)
    lib.klp_last_error(buf, n + 1)
    return buf.value.decode("utf-8", "replace")


# Per-call host helpers of the launch wrappers.  A launch goes onto torch's
# current stream of the tensors' device, with that device current; these
# avoid building a torch.cuda.Stream object and entering a device context
# on every call (together about 3 us of a ~12 us call).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_no_switch = contextlib.nullcontext()


def stream_handle(device_index: int) -> int:
    """The raw hipStream_t of ``device_index``'s current stream."""
    if _raw_stream is not None:
        return _raw_stream(device_index)
    return torch.cuda.current_stream(device_index).cuda_stream


def device_guard(device_index: int):
    """Context manager making ``device_index`` current: a no-op when it
    already is."""
    if torch.cuda.current_device() == device_index:
        return _no_switch
    return torch.cuda.device(device_index)


# Buffers allocated while a stream was being captured into a graph: the
# graph bakes in their addresses, so they must outlive it.  They are kept for
# the life of the process (one small buffer per captured call that needed
# one).
_capture_keepalive: list = []


def capturing() -> bool:
    """True while the current stream is being captured into a graph."""
    return torch.cuda.is_current_stream_capturing()


def keep_for_capture(buf):
    """Keep ``buf`` alive for the life of the process and return it."""
    _capture_keepalive.append(buf)
    return buf


def ptr(t):
    """Data pointer of ``t`` for a ``void*`` argument (``None`` -> NULL)."""
    return None if t is None else t.data_ptr()


def check_status(rc: int) -> None:
    """Raise RuntimeError carrying the native message for a non-zero status
    (the reference raises RuntimeError from TORCH_CHECK)."""
    if rc != KLP_OK:
        raise RuntimeError(last_error() or f"kernel_opt: native call failed with status {rc}")
