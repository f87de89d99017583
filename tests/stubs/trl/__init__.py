"""Minimal stand-in for `trl` (not installable offline), enough to exercise
kernel_opt.trainer.KernelOptGRPOTrainer.

GRPOTrainer here carries only what the override touches: `model_kwarg_keys`,
`temperature`, and the eager `_get_per_token_logps_and_entropies` that the
override defers to for multimodal inputs.  The eager method restates TRL
1.4's text path as the reference describes it (reference
python/kernel_opt/trainer.py:76-131 mirrors it; notes/stage1_findings.md:26-33):
chunked model forward with logits_to_keep + 1, drop the last position, keep
the completion window, divide by the temperature, then
selective_log_softmax + entropy_from_logits.
"""
from __future__ import annotations

import torch


class GRPOTrainer:
    def __init__(self, model_kwarg_keys=("input_ids", "attention_mask", "logits_to_keep"),
                 temperature=1.0):
        self.model_kwarg_keys = tuple(model_kwarg_keys)
        self.temperature = temperature
        self.parent_calls = []

    def _get_per_token_logps_and_entropies(self, model, input_ids, attention_mask,
                                           logits_to_keep, batch_size=None,
                                           compute_entropy=False, **multimodal):
        from oracle.eager_ref import trl_entropy_from_logits, trl_selective_log_softmax

        self.parent_calls.append(dict(multimodal))
        bsz = batch_size or input_ids.size(0)
        all_logps, all_ents = [], []
        for start in range(0, input_ids.size(0), bsz):
            ids = input_ids[start:start + bsz]
            mask = attention_mask[start:start + bsz]
            inputs = {"input_ids": ids, "attention_mask": mask}
            if "logits_to_keep" in self.model_kwarg_keys:
                inputs["logits_to_keep"] = logits_to_keep + 1
            inputs["use_cache"] = False
            logits = model(**inputs).logits
            logits = logits[:, :-1, :]
            logits = logits[:, -logits_to_keep:, :]
            logits = logits / self.temperature
            completion_ids = ids[:, -logits_to_keep:]
            all_logps.append(trl_selective_log_softmax(logits, completion_ids))
            if compute_entropy:
                with torch.no_grad():
                    all_ents.append(trl_entropy_from_logits(logits))
        logps = torch.cat(all_logps, dim=0)
        ents = torch.cat(all_ents, dim=0) if compute_entropy else None
        return logps, ents
