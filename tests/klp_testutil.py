"""Shared helpers for the tests: ulp distances and small input builders."""
from __future__ import annotations

import torch

from oracle.checks import (DTYPE_NAME, WIDTH, bits_of, grad_check, grad_score,  # noqa: F401
                           ordered, storage_bits, ulp_diff)


# North-star forward tolerance (absolute), by input dtype.
FWD_TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-5, torch.float16: 2e-5}


def seeded_logits(shape, dtype, seed, scale=2.0, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    return x.to(dtype).to(device)


def seeded_targets(shape, V, seed, device="cpu"):
    g = torch.Generator().manual_seed(seed + 7919)
    return torch.randint(0, V, shape, generator=g).to(device)

