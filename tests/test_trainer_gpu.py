"""KernelOptGRPOTrainer with the real HIP kernel: the override's outputs and
the gradient it sends into the model match the stub parent's eager TRL path
(fp32 model), and the fp32 eager formulas on the same logits (bf16 model,
where TRL's own path is bf16-quantised)."""
import os
import sys

import pytest
import torch

from trainer_fixtures import ToyLM, batch

pytestmark = pytest.mark.gpu
STUBS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "stubs")


@pytest.fixture
def trainer_mod(monkeypatch):
    monkeypatch.syspath_prepend(STUBS)
    sys.modules.pop("trl", None)
    sys.modules.pop("kernel_opt.trainer", None)
    import kernel_opt.trainer as tr
    yield tr
    sys.modules.pop("kernel_opt.trainer", None)
    sys.modules.pop("trl", None)


@pytest.mark.parametrize("batch_size", [None, 2])
@pytest.mark.parametrize("temperature", [1.0, 0.7])
def test_fp32_model_matches_parent(trainer_mod, batch_size, temperature):
    model = ToyLM(vocab_out=5003).cuda()
    tr = trainer_mod.KernelOptGRPOTrainer(temperature=temperature)
    ids, mask = batch(B=6, L=16, device="cuda")
    lp, ent = tr._get_per_token_logps_and_entropies(model, ids, mask, 9, batch_size=batch_size,
                                                    compute_entropy=True)
    lp.sum().backward()
    g_ours = model.emb.grad.clone()
    model.emb.grad = None
    ref_lp, ref_ent = trainer_mod.GRPOTrainer._get_per_token_logps_and_entropies(
        tr, model, ids, mask, 9, batch_size=batch_size, compute_entropy=True)
    ref_lp.sum().backward()
    assert torch.allclose(lp, ref_lp, atol=2e-5, rtol=1e-5)
    assert torch.allclose(ent, ref_ent, atol=2e-5, rtol=1e-5)
    assert torch.allclose(g_ours, model.emb.grad, atol=1e-5, rtol=1e-4)


def test_bf16_model_matches_fp32_formulas(trainer_mod):
    from oracle.eager_ref import ref_fp32
    model = ToyLM(vocab_out=32000, dtype=torch.bfloat16).cuda()
    tr = trainer_mod.KernelOptGRPOTrainer(temperature=1.0)
    ids, mask = batch(B=4, L=20, device="cuda")
    lp, ent = tr._get_per_token_logps_and_entropies(model, ids, mask, 12, compute_entropy=True)
    with torch.no_grad():
        logits = model(ids, mask, logits_to_keep=13).logits[:, :-1, :][:, -12:, :]
        r_lp, r_ent, _ = ref_fp32(logits, ids[:, -12:])
    assert (lp - r_lp).abs().max().item() <= 2e-5
    assert (ent - r_ent).abs().max().item() <= 2e-5
