"""Shared helpers for the tests: ulp distances and small input builders."""
from __future__ import annotations

import numpy as np
import torch


def storage_bits(t: torch.Tensor) -> np.ndarray:
    """Storage bits of a bf16/fp16 tensor as int64 (0..65535), or float32 bits."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().astype(np.int64) & 0xFFFFFFFF
    return t.view(torch.int16).numpy().astype(np.int64) & 0xFFFF


def ordered(bits: np.ndarray, width: int) -> np.ndarray:
    """Map IEEE bit patterns to integers whose order is the values' order
    (+0 and -0 both map to the same point), so a difference is an ulp count."""
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


WIDTH = {torch.bfloat16: 16, torch.float16: 16, torch.float32: 32}
DTYPE_NAME = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}
# North-star forward tolerance (absolute), by input dtype.
FWD_TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-5, torch.float16: 2e-5}


def seeded_logits(shape, dtype, seed, scale=2.0, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    return x.to(dtype).to(device)


def seeded_targets(shape, V, seed, device="cpu"):
    g = torch.Generator().manual_seed(seed + 7919)
    return torch.randint(0, V, shape, generator=g).to(device)
