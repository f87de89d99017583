"""kernel_opt — fused per-token log-probability + entropy for MI355X (gfx950).

Drop-in for the reference package of the same name
(reference python/kernel_opt/__init__.py:1-15): same public names, the HIP
library ``_lib/libkernel_opt_hip.so`` in place of the CUDA extension.
"""
from . import _C  # noqa: F401  (loads the HIP library; ImportError if it is not built)
from .ops import (  # noqa: F401
    fused_logprob_entropy,
    fused_logprob_entropy_forward,
    fused_logprob_entropy_naive,
)
from .grpo import fused_grpo_loss  # noqa: F401
from .grpo_step import fused_grpo_step  # noqa: F401
from .linear_grpo import fused_linear_grpo_step  # noqa: F401
from .lmhead import (  # noqa: F401
    fused_linear_logprob_entropy,
    fused_linear_logprob_entropy_forward,
    vocab_chunk,
    vocab_chunks,
)


# Lazy import so users without trl can still use the kernels.
def __getattr__(name):
    if name == "KernelOptGRPOTrainer":
        from .trainer import KernelOptGRPOTrainer
        return KernelOptGRPOTrainer
    raise AttributeError(f"module 'kernel_opt' has no attribute {name!r}")


__version__ = "0.0.1"
