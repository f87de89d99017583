"""KernelOptGRPOTrainer — ``trl.GRPOTrainer`` with the fused kernel in its
logprob/entropy step (reference python/kernel_opt/trainer.py:30-131).

Overrides exactly one method, ``_get_per_token_logps_and_entropies`` — the
single entry point for every logprob computation in TRL's GRPO (policy
logprobs with autograd, old and reference logprobs without; TRL 1.4 call
sites listed at reference trainer.py:3-8).

Multimodal inputs fall back to the parent's eager implementation, as in the
reference (trainer.py:56-74).

Differences from the reference, outputs unchanged up to fp32 rounding:
  - the reference launches the kernel once per batch element because its
    kernel needs contiguous rows (trainer.py:104-124); the HIP kernel
    addresses rows through two strides, so the sliced ``[B, L', V]``
    completion window is passed in one launch, without a copy;
  - the temperature is fused into the kernel instead of a separate in-place
    ``logits.div_(temperature)`` pass (trainer.py:101).  The division then
    happens in fp32 (x * fp32(1/T)) rather than in the logits' dtype, so
    bf16 logits are not re-rounded to bf16 after the division.
"""
from __future__ import annotations

import torch
from trl import GRPOTrainer

from .ops import fused_logprob_entropy

_MULTIMODAL_KWARGS = (
    "pixel_values", "image_grid_thw", "num_images",
    "pixel_attention_mask", "image_sizes",
    "token_type_ids", "mm_token_type_ids", "image_position_ids",
)


class KernelOptGRPOTrainer(GRPOTrainer):
    """trl.GRPOTrainer with the inner logprob+entropy block replaced by the
    fused HIP kernel (fp32 accumulation of bf16/fp16/fp32 logits)."""

    def _get_per_token_logps_and_entropies(
        self,
        model,
        input_ids,
        attention_mask,
        logits_to_keep,
        batch_size=None,
        compute_entropy=False,
        pixel_values=None,
        image_grid_thw=None,
        num_images=None,
        pixel_attention_mask=None,
        image_sizes=None,
        token_type_ids=None,
        mm_token_type_ids=None,
        image_position_ids=None,
    ) -> tuple[torch.Tensor, torch.Tensor | None]:
        mm = dict(
            pixel_values=pixel_values, image_grid_thw=image_grid_thw, num_images=num_images,
            pixel_attention_mask=pixel_attention_mask, image_sizes=image_sizes,
            token_type_ids=token_type_ids, mm_token_type_ids=mm_token_type_ids,
            image_position_ids=image_position_ids,
        )
        if any(v is not None for v in mm.values()):
            return super()._get_per_token_logps_and_entropies(
                model, input_ids, attention_mask, logits_to_keep,
                batch_size=batch_size, compute_entropy=compute_entropy, **mm,
            )

        bsz = batch_size or input_ids.size(0)
        all_logps: list[torch.Tensor] = []
        all_entropies: list[torch.Tensor] = []
        for start in range(0, input_ids.size(0), bsz):
            input_ids_batch = input_ids[start:start + bsz]
            attention_mask_batch = attention_mask[start:start + bsz]
            model_inputs = {"input_ids": input_ids_batch, "attention_mask": attention_mask_batch}
            # `model_kwarg_keys` is TRL's cache of the kwargs the model accepts.
            if "logits_to_keep" in self.model_kwarg_keys:
                # +1 because the last position is dropped below
                model_inputs["logits_to_keep"] = logits_to_keep + 1
            model_inputs["use_cache"] = False

            logits = model(**model_inputs).logits
            logits = logits[:, :-1, :]                 # drop the next-token position
            logits = logits[:, -logits_to_keep:, :]    # keep the completion window
            completion_ids = input_ids_batch[:, -logits_to_keep:]
            if not completion_ids.is_contiguous():
                completion_ids = completion_ids.contiguous()

            # The temperature is applied inside the kernel, where TRL (and the
            # reference, trainer.py:101) first runs logits.div_(temperature)
            # as a separate read + write pass over the logits.
            logps, ents, _lse = fused_logprob_entropy(logits, completion_ids,
                                                      temperature=self.temperature)
            all_logps.append(logps)
            if compute_entropy:
                all_entropies.append(ents.detach())

        logps = torch.cat(all_logps, dim=0)
        entropies = torch.cat(all_entropies, dim=0) if compute_entropy else None
        return logps, entropies
