"""KernelOptGRPOTrainer._get_per_token_logps_and_entropies on the CPU, with
a stub `trl` and the fused op replaced by the eager fp32 formulas (the HIP
kernel needs a GPU; tests/test_trainer_gpu.py runs the real one).  Pins the
override's own logic — chunking, logits_to_keep + 1, the shifted completion
window, temperature, entropy detach and None, multimodal fallback — against
the stub parent's eager TRL path (reference python/kernel_opt/trainer.py:38-131)."""
import os
import sys

import pytest
import torch

from trainer_fixtures import ToyLM, batch

STUBS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "stubs")


@pytest.fixture
def trainer_mod(monkeypatch):
    monkeypatch.syspath_prepend(STUBS)
    sys.modules.pop("trl", None)
    sys.modules.pop("kernel_opt.trainer", None)
    import kernel_opt.trainer as tr
    from oracle.eager_ref import ref_forward_pt

    def cpu_fused(logits, targets, temperature=None):  # the op's contract, eagerly in fp32
        x = logits.float()
        if temperature is not None:
            x = x * torch.tensor(1.0 / temperature, dtype=torch.float32)
        return ref_forward_pt(x, targets)

    monkeypatch.setattr(tr, "fused_logprob_entropy", cpu_fused)
    yield tr
    sys.modules.pop("kernel_opt.trainer", None)
    sys.modules.pop("trl", None)


def test_lazy_attribute(monkeypatch):
    monkeypatch.syspath_prepend(STUBS)
    sys.modules.pop("trl", None)
    sys.modules.pop("kernel_opt.trainer", None)
    import kernel_opt
    cls = kernel_opt.KernelOptGRPOTrainer
    import trl
    assert issubclass(cls, trl.GRPOTrainer)
    sys.modules.pop("kernel_opt.trainer", None)
    sys.modules.pop("trl", None)


@pytest.mark.parametrize("batch_size", [None, 2, 5])
@pytest.mark.parametrize("keep", [1, 4, 11])
@pytest.mark.parametrize("temperature", [1.0, 0.7])
def test_matches_parent_eager_path(trainer_mod, batch_size, keep, temperature):
    model = ToyLM()
    tr = trainer_mod.KernelOptGRPOTrainer(temperature=temperature)
    ids, mask = batch()
    lp, ent = tr._get_per_token_logps_and_entropies(model, ids, mask, keep,
                                                    batch_size=batch_size, compute_entropy=True)
    ref_lp, ref_ent = trainer_mod.GRPOTrainer._get_per_token_logps_and_entropies(
        tr, model, ids, mask, keep, batch_size=batch_size, compute_entropy=True)
    assert lp.shape == ref_lp.shape == (5, keep)
    assert torch.allclose(lp, ref_lp, atol=1e-5, rtol=1e-5)
    assert torch.allclose(ent, ref_ent, atol=1e-5, rtol=1e-5)
    assert not ent.requires_grad and lp.requires_grad
    # the override asked the model for logits_to_keep + 1 positions, no cache
    assert all(c["logits_to_keep"] == keep + 1 and c["use_cache"] is False for c in model.calls)
    n_chunks = -(-5 // (batch_size or 5))
    assert len(model.calls) == 2 * n_chunks  # override + parent


def test_no_entropy_and_no_logits_to_keep_kwarg(trainer_mod):
    model = ToyLM()
    tr = trainer_mod.KernelOptGRPOTrainer(model_kwarg_keys=("input_ids", "attention_mask"))
    ids, mask = batch()
    lp, ent = tr._get_per_token_logps_and_entropies(model, ids, mask, 6)
    assert ent is None and lp.shape == (5, 6)
    assert model.calls[0]["logits_to_keep"] is None
    ref_lp, _ = trainer_mod.GRPOTrainer._get_per_token_logps_and_entropies(tr, model, ids, mask, 6)
    assert torch.allclose(lp, ref_lp, atol=1e-5, rtol=1e-5)


def test_gradient_flows_to_model(trainer_mod):
    model = ToyLM()
    tr = trainer_mod.KernelOptGRPOTrainer(temperature=0.9)
    ids, mask = batch()
    lp, _ = tr._get_per_token_logps_and_entropies(model, ids, mask, 5)
    lp.sum().backward()
    g_ours = model.emb.grad.clone()
    model.emb.grad = None
    ref_lp, _ = trainer_mod.GRPOTrainer._get_per_token_logps_and_entropies(tr, model, ids, mask, 5)
    ref_lp.sum().backward()
    assert torch.allclose(g_ours, model.emb.grad, atol=1e-5, rtol=1e-5)


def test_multimodal_falls_back_to_parent(trainer_mod):
    model = ToyLM()
    tr = trainer_mod.KernelOptGRPOTrainer()
    ids, mask = batch()
    pv = torch.zeros(1)
    tr._get_per_token_logps_and_entropies(model, ids, mask, 3, pixel_values=pv,
                                          compute_entropy=True)
    assert len(tr.parent_calls) == 1 and tr.parent_calls[0]["pixel_values"] is pv
    tr._get_per_token_logps_and_entropies(model, ids, mask, 3, token_type_ids=pv)
    assert len(tr.parent_calls) == 2
