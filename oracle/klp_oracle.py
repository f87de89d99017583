"""numpy/ctypes front end of the float64 C oracle (klp_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product never imports it.

Inputs are numpy arrays: logits as their storage bits (uint16 for bf16/fp16,
float32 for fp32) or a torch CPU tensor (converted here), targets as int64.
Outputs are float64.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(HERE, "_build")
BF16, FP16, FP32 = 0, 1, 2
_DTYPE_NAMES = {"bf16": BF16, "fp16": FP16, "fp32": FP32,
                "bfloat16": BF16, "float16": FP16, "float32": FP32}

_dp = ctypes.POINTER(ctypes.c_double)
_vp, _i32, _i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
_ROWS = [_vp, _i32, _i64, _i64, _i64, _i64, _i64]


def lib_path(mutant: int = 0) -> str:
    name = "libklp_oracle.so" if mutant == 0 else f"libklp_oracle_mutant{mutant}.so"
    return os.path.join(BUILD, name)


def build(mutant: int = 0, build_dir: str | None = None) -> str:
    """Compile klp_oracle.c with gcc (optionally with a planted mistake)."""
    bdir = build_dir or BUILD
    cmd = ["make", "-s", "-C", HERE, f"MUTANT={mutant}", f"BUILD={bdir}"]
    subprocess.run(cmd, check=True)
    name = "libklp_oracle.so" if mutant == 0 else f"libklp_oracle_mutant{mutant}.so"
    return os.path.join(bdir, name)


class Oracle:
    def __init__(self, path: str | None = None, mutant: int = 0):
        path = path or lib_path(mutant)
        if not os.path.exists(path):
            path = build(mutant)
        self.path = path
        lib = ctypes.CDLL(path)
        lib.klp_oracle_forward.argtypes = _ROWS + [_vp, ctypes.c_float, _dp, _dp, _dp]
        lib.klp_oracle_forward_naive.argtypes = _ROWS + [_vp, _dp, _dp, _dp]
        lib.klp_oracle_backward.argtypes = _ROWS + [_vp, ctypes.c_float, _dp, _dp, _dp, _dp, _dp,
                                                     _dp]
        lib.klp_oracle_round.argtypes = [_dp, _i32, _i64, _vp]
        lib.klp_oracle_combine.argtypes = [_dp, _dp, _dp]
        lib.klp_oracle_segment_state.argtypes = [_vp, _i32, _i64, _i64, _dp]
        lib.klp_oracle_finalize.argtypes = [_dp, ctypes.c_double, _dp, _dp, _dp]
        lib.klp_oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
        lib.klp_oracle_bf16_to_f32.restype = ctypes.c_float
        lib.klp_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.klp_oracle_f16_to_f32.restype = ctypes.c_float
        lib.klp_oracle_round_bf16.argtypes = [ctypes.c_double]
        lib.klp_oracle_round_bf16.restype = ctypes.c_uint16
        lib.klp_oracle_round_f16.argtypes = [ctypes.c_double]
        lib.klp_oracle_round_f16.restype = ctypes.c_uint16
        self.lib = lib

    # -- helpers -----------------------------------------------------------
    @staticmethod
    def _as_storage(logits, dtype):
        """Returns (contiguous storage array, dtype code)."""
        try:
            import torch
            if isinstance(logits, torch.Tensor):
                t = logits.detach().cpu().contiguous()
                code = {torch.bfloat16: BF16, torch.float16: FP16, torch.float32: FP32}[t.dtype]
                if code == FP32:
                    return t.numpy(), code
                return t.view(torch.int16).numpy().view(np.uint16), code
        except ImportError:  # pragma: no cover
            pass
        code = _DTYPE_NAMES[dtype] if isinstance(dtype, str) else dtype
        arr = np.ascontiguousarray(logits)
        if code == FP32:
            assert arr.dtype == np.float32
        else:
            assert arr.dtype == np.uint16
        return arr, code

    @staticmethod
    def _dptr(a):
        return None if a is None else a.ctypes.data_as(_dp)

    @staticmethod
    def _f64(a, n):
        if a is None:
            return None
        a = np.ascontiguousarray(np.asarray(a, dtype=np.float64).reshape(-1))
        assert a.size == n
        return a

    # -- API ---------------------------------------------------------------
    def forward(self, logits, targets, dtype=None, naive: bool = False, temperature=None):
        """(logp, entropy, lse) float64 for dense [..., V] logits; with a
        temperature T the logits are first multiplied by scale_of(T) in fp32."""
        arr, code = self._as_storage(logits, dtype)
        V = arr.shape[-1]
        n = arr.size // V
        tg = np.ascontiguousarray(np.asarray(targets, dtype=np.int64).reshape(-1))
        assert tg.size == n
        outs = [np.empty(n, np.float64) for _ in range(3)]
        if naive:
            assert temperature is None
            self.lib.klp_oracle_forward_naive(arr.ctypes.data, code, n, V, max(n, 1), 0, V,
                                              tg.ctypes.data, *[self._dptr(o) for o in outs])
        else:
            self.lib.klp_oracle_forward(arr.ctypes.data, code, n, V, max(n, 1), 0, V,
                                        tg.ctypes.data, self.scale_of(temperature),
                                        *[self._dptr(o) for o in outs])
        shape = arr.shape[:-1]
        return tuple(o.reshape(shape) for o in outs)

    @staticmethod
    def scale_of(temperature):
        """The kernels' scale (1.0 for None): the temperature crosses the C ABI
        as a float T32 = fp32(T), and the kernels multiply each logit by the
        float nearest 1/T32.  For some T (1.7, for one) fp32(1/T) is one ulp
        away from it."""
        if temperature is None:
            return 1.0
        return float(np.float32(1.0 / float(np.float32(temperature))))

    def backward(self, logits, targets, lse, ent, g_logp=None, g_ent=None, g_lse=None,
                 dtype=None, temperature=None):
        """float64 d_logits with respect to the unscaled logits, dense, shaped
        like logits."""
        arr, code = self._as_storage(logits, dtype)
        V = arr.shape[-1]
        n = arr.size // V
        tg = np.ascontiguousarray(np.asarray(targets, dtype=np.int64).reshape(-1))
        lse64, ent64 = self._f64(lse, n), self._f64(ent, n)
        gl, ge, gs = self._f64(g_logp, n), self._f64(g_ent, n), self._f64(g_lse, n)
        out = np.empty(arr.shape, np.float64)
        self.lib.klp_oracle_backward(arr.ctypes.data, code, n, V, max(n, 1), 0, V,
                                     tg.ctypes.data, self.scale_of(temperature),
                                     self._dptr(lse64), self._dptr(ent64),
                                     self._dptr(gl), self._dptr(ge), self._dptr(gs),
                                     self._dptr(out))
        return out

    def round_to(self, x, dtype):
        """Round float64 values to dtype storage, nearest-even (uint16 bits
        for bf16/fp16, float32 for fp32)."""
        code = _DTYPE_NAMES[dtype] if isinstance(dtype, str) else dtype
        x = np.ascontiguousarray(np.asarray(x, dtype=np.float64))
        out = np.empty(x.shape, np.float32 if code == FP32 else np.uint16)
        self.lib.klp_oracle_round(self._dptr(x), code, x.size, out.ctypes.data)
        return out

    def combine(self, a, b):
        a = np.ascontiguousarray(a, np.float64)
        b = np.ascontiguousarray(b, np.float64)
        out = np.empty(3, np.float64)
        self.lib.klp_oracle_combine(self._dptr(a), self._dptr(b), self._dptr(out))
        return out

    def segment_state(self, row, v0, v1, dtype=None):
        arr, code = self._as_storage(row, dtype)
        out = np.empty(3, np.float64)
        self.lib.klp_oracle_segment_state(arr.ctypes.data, code, v0, v1, self._dptr(out))
        return out

    def finalize(self, state, x_target):
        st = np.ascontiguousarray(state, np.float64)
        o = [ctypes.c_double() for _ in range(3)]
        self.lib.klp_oracle_finalize(self._dptr(st), float(x_target), *[ctypes.byref(x) for x in o])
        return tuple(x.value for x in o)

    def to_f32(self, bits, dtype):
        code = _DTYPE_NAMES[dtype] if isinstance(dtype, str) else dtype
        fn = self.lib.klp_oracle_bf16_to_f32 if code == BF16 else self.lib.klp_oracle_f16_to_f32
        return np.array([fn(int(b)) for b in np.asarray(bits).reshape(-1)], np.float32)


_default = None


def get() -> Oracle:
    global _default
    if _default is None:
        _default = Oracle()
    return _default
