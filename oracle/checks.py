"""Checkers shared by tests/ and __graft_entry__.smoke(): the gradient bar.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

import numpy as np
import torch

WIDTH = {torch.bfloat16: 16, torch.float16: 16, torch.float32: 32}
DTYPE_NAME = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


def storage_bits(t: torch.Tensor) -> np.ndarray:
    """Storage bits of a bf16/fp16 tensor as int64 (0..65535), or float32 bits."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().astype(np.int64) & 0xFFFFFFFF
    return t.view(torch.int16).numpy().astype(np.int64) & 0xFFFF


def ordered(bits: np.ndarray, width: int) -> np.ndarray:
    """IEEE bit patterns -> integers ordered like the values (+0 == -0), so a
    difference is an ulp count."""
    sign = np.int64(1) << (width - 1)
    mag = bits & (sign - 1)
    return np.where(bits & sign, -mag, mag)


def ulp_diff(a_bits: np.ndarray, b_bits: np.ndarray, width: int) -> np.ndarray:
    return np.abs(ordered(np.asarray(a_bits, np.int64), width)
                  - ordered(np.asarray(b_bits, np.int64), width))


def bits_of(arr: np.ndarray) -> np.ndarray:
    """Bits of an oracle-rounded array (uint16 for bf16/fp16, float32)."""
    if arr.dtype == np.float32:
        return arr.view(np.int32).astype(np.int64) & 0xFFFFFFFF
    return arr.astype(np.int64)


def grad_check(oracle, x_cpu, t_cpu, lse, ent, d_ours, g_logp=None, g_ent=None, g_lse=None,
               temperature=None):
    """Worst normalised gradient error of the kernel against the float64
    oracle's gradient (<= 1 passes); see grad_score for the bar.  `lse` and
    `ent` are the kernel's own saved fp32 values (the oracle's backward takes
    them as inputs, as the kernel does).  Returns (worst, detail string)."""
    n = x_cpu.numel() // x_cpu.shape[-1]

    def np1(g):
        return None if g is None else g.detach().cpu().double().numpy().reshape(-1)

    lse_np, ent_np = np1(lse), np1(ent)
    d_ref = oracle.backward(x_cpu, t_cpu.numpy().reshape(-1), lse_np, ent_np,
                            g_logp=np1(g_logp), g_ent=np1(g_ent), g_lse=np1(g_lse),
                            temperature=temperature)
    return grad_score(oracle, x_cpu, t_cpu, lse_np, ent_np, d_ours, d_ref.reshape(n, -1),
                      np1(g_logp), np1(g_ent), np1(g_lse), temperature=temperature)


def grad_score(oracle, x_cpu, t_cpu, lse_np, ent_np, d_ours, d_ref, gl=None, ge=None, gs=None,
               temperature=None):
    """Bar: every element within 1 ulp of the output dtype of the float64
    reference value d_ref (rounded to nearest-even for bf16/fp16), except
    where that value is the result of cancellation between larger fp32 terms.
    There the bound is the fp32 evaluation noise of the summands,
        noise_v = 2^-22 * (1 + |x_v - lse|) * A_v,
        A_v = p_v (|g_lse| + |g_logp| + |g_ent| (|H| + |x_v - lse|)) + [v == t] |g_logp|,
    i.e. a couple of fp32 ulps of each summand, with exp's argument rounding
    (|x - lse| ulps of p) included.  Any fp32 evaluation of
    p * (g_lse - g_logp - g_ent (log p + H)) + [v == t] g_logp, the
    reference's own fp32 path included, carries errors of that size.  With a
    temperature T, x is the scaled logit fp32(x * s), s = fp32(1/fp32(T)), and the noise
    carries the chain-rule factor 1/T.
    Returns (worst score, detail string); a score <= 1 passes."""
    V = x_cpu.shape[-1]
    n = lse_np.size
    t_np = t_cpu.numpy().reshape(-1)
    x64 = x_cpu.detach().cpu().float().numpy().reshape(n, V)
    scale = 1.0
    if temperature is not None:  # the kernels' scaled logit fp32(x * s)
        scale = oracle.scale_of(temperature)
        x64 = x64 * np.float32(scale)
    x64 = x64.astype(np.float64)
    lp = x64 - lse_np[:, None]
    with np.errstate(invalid="ignore", over="ignore"):
        p = np.where(np.isneginf(x64), 0.0, np.exp(lp))
        lp_abs = np.where(np.isneginf(x64), 0.0, np.abs(lp))
    z = np.zeros(n)
    gl_ = gl if gl is not None else z
    ge_ = ge if ge is not None else z
    gs_ = gs if gs is not None else z
    A = p * (np.abs(gs_)[:, None] + np.abs(gl_)[:, None]
             + np.abs(ge_)[:, None] * (np.abs(ent_np)[:, None] + lp_abs))
    onehot = (np.arange(V)[None, :] == t_np[:, None])
    A = A + onehot * np.abs(gl_)[:, None]
    noise = 2.0 ** -22 * (1.0 + lp_abs) * A * scale

    dt = d_ours.dtype
    d = d_ours.detach().cpu().double().numpy().reshape(n, V)
    abs_err = np.abs(d - d_ref)
    if dt == torch.float32:
        ulp = np.spacing(np.abs(d_ref).astype(np.float32)).astype(np.float64)
        ulps = abs_err / ulp
    else:
        ref_bits = bits_of(oracle.round_to(d_ref, DTYPE_NAME[dt])).reshape(n, V)
        ulps = ulp_diff(storage_bits(d_ours).reshape(n, V), ref_bits, 16).astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        by_noise = np.where(noise > 0, abs_err / noise, np.where(abs_err > 0, np.inf, 0.0))
    score = np.minimum(ulps, by_noise)
    worst = float(score.max()) if score.size else 0.0
    frac = float((ulps <= 1).mean()) if ulps.size else 1.0
    return worst, (f"worst {worst:.3g} (max ulps {float(ulps.max()) if ulps.size else 0:.3g}, "
                   f"{100 * frac:.4f}% of elements within 1 ulp)")
