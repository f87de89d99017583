"""The reference's eager PyTorch paths, restated (torch ops, any device).

TEST INFRASTRUCTURE ONLY (tests/, smoke(), bench.py's cpu_baseline leg).

* ``ref_fp32``        — the reference's fp32 ground truth
                        (tests/test_logprob.py:17-25): upcast, log_softmax,
                        gather, -(p * log p).sum, logsumexp.
* ``ref_forward_pt``  — the same formulas in the input dtype, differentiable
                        (tests/test_logprob.py:160-167; bench_backward.py:19-26).
* ``trl_selective_log_softmax`` / ``trl_entropy_from_logits`` — TRL 1.4's
  eager path that the fused kernel replaces (trl.trainer.utils, not present
  in this environment).  Restated from the reference's description of it
  (REPORT.md:19-30, notes/stage1_findings.md:38-60): a per-row
  ``log_softmax`` + ``gather`` loop for bf16/fp16 input, gather minus a
  per-row ``logsumexp`` for fp32/fp64 input (hinted at REPORT.md:411-414),
  and a 128-row chunked ``log_softmax -> exp -> mul -> sum`` for entropy.
  Its outputs are not pinned against TRL itself (TRL cannot be imported
  here); it serves as the CPU baseline that is timed, not as a correctness
  oracle.
* ``reference_grpo_loss`` — the reference's GRPO loss, verbatim in meaning
  (examples/compare_one_step.py:232-236).
* ``eager_grpo_loss``     — the generalised GRPO loss of klp_grpo_fwd as a
  chain of eager torch ops (the form TRL's GRPOTrainer writes it in; its
  variants beyond the reference's formula are not pinned against TRL, which
  is absent here).  Differentiated by torch autograd, it pins the gradient
  of oracle/grpo_oracle.py independently of that hand derivation.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def ref_fp32(logits: torch.Tensor, targets: torch.Tensor):
    logits_f = logits.float()
    log_probs = F.log_softmax(logits_f, dim=-1)
    logp = log_probs.gather(-1, targets.unsqueeze(-1)).squeeze(-1)
    p = log_probs.exp()
    ent = -(p * log_probs).sum(-1)
    lse = torch.logsumexp(logits_f, dim=-1)
    return logp, ent, lse


def ref_forward_pt(logits: torch.Tensor, targets: torch.Tensor):
    log_probs = F.log_softmax(logits, dim=-1)
    logp = log_probs.gather(-1, targets.unsqueeze(-1)).squeeze(-1)
    p = log_probs.exp()
    ent = -(p * log_probs).sum(-1)
    lse = torch.logsumexp(logits, dim=-1)
    return logp, ent, lse


def trl_selective_log_softmax(logits: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    if logits.dtype in (torch.float32, torch.float64):
        selected = torch.gather(logits, dim=-1, index=index.unsqueeze(-1)).squeeze(-1)
        lse = torch.stack([torch.logsumexp(lg, dim=-1) for lg in logits])
        return selected - lse
    out = []
    for row_logits, row_labels in zip(logits, index):
        row_logps = F.log_softmax(row_logits, dim=-1)
        out.append(row_logps.gather(dim=-1, index=row_labels.unsqueeze(-1)).squeeze(-1))
    return torch.stack(out)


def trl_entropy_from_logits(logits: torch.Tensor, chunk_size: int = 128) -> torch.Tensor:
    shape = logits.shape[:-1]
    flat = logits.reshape(-1, logits.shape[-1])
    ents = []
    for chunk in flat.split(chunk_size, dim=0):
        logps = F.log_softmax(chunk, dim=-1)
        ents.append(-(torch.exp(logps) * logps).sum(-1))
    return torch.cat(ents, dim=0).reshape(shape)


def trl_eager(logits: torch.Tensor, targets: torch.Tensor):
    """The eager forward the fused kernel replaces: (logp, entropy)."""
    return trl_selective_log_softmax(logits, targets), trl_entropy_from_logits(logits)


def reference_grpo_loss(new_logp, old_logp, advantages, mask, eps_clip=0.2):
    ratio = (new_logp - old_logp).exp()
    surr = -torch.minimum(ratio * advantages,
                          ratio.clamp(1 - eps_clip, 1 + eps_clip) * advantages)
    return (surr * mask).sum() / mask.sum()


def eager_grpo_loss(logp, old_logp, advantages, mask=None, ref_logp=None, eps_low=0.2,
                    eps_high=None, beta=0.0, loss_type="bnpo", level="token", norm_const=1.0):
    eh = eps_low if eps_high is None else eps_high
    m = torch.ones_like(logp) if mask is None else mask
    A = advantages.unsqueeze(1) if advantages.dim() == 1 else advantages
    log_ratio = logp - old_logp
    if level == "sequence":
        w = ((log_ratio * m).sum(-1) / m.sum(-1).clamp(min=1.0)).unsqueeze(-1)
    else:
        w = log_ratio
    coef_1 = torch.exp(w)
    coef_2 = torch.clamp(coef_1, 1 - eps_low, 1 + eh)
    per_token = -torch.min(coef_1 * A, coef_2 * A)
    kl = torch.zeros_like(logp)
    if ref_logp is not None and beta != 0.0:
        kl = torch.exp(ref_logp - logp) - (ref_logp - logp) - 1
        per_token = per_token + beta * kl
    if loss_type == "grpo":
        loss = ((per_token * m).sum(-1) / m.sum(-1).clamp(min=1.0)).mean()
    elif loss_type == "bnpo":
        loss = (per_token * m).sum() / m.sum().clamp(min=1.0)
    else:
        loss = (per_token * m).sum() / norm_const
    den = m.sum().clamp(min=1.0)
    low = ((coef_1 < 1 - eps_low) & (A < 0)).to(logp.dtype)
    high = ((coef_1 > 1 + eh) & (A > 0)).to(logp.dtype)
    stats = torch.stack([(kl * m).sum() / den, (low * m).sum() / den, (high * m).sum() / den,
                         ((low + high) * m).sum() / den])
    return loss, stats.detach()
