"""A seeded toy causal LM for the trainer tests: logits depend on the token
and its position, honour `logits_to_keep`, and are differentiable through a
weight tensor."""
from types import SimpleNamespace

import torch


class ToyLM(torch.nn.Module):
    def __init__(self, vocab_in=50, vocab_out=3001, seed=0, dtype=torch.float32):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.emb = torch.nn.Parameter((torch.randn(vocab_in, vocab_out, generator=g) * 2).to(dtype))
        self.pos = torch.nn.Parameter((torch.randn(64, vocab_out, generator=g) * 0.5).to(dtype))
        self.calls = []

    def forward(self, input_ids, attention_mask, logits_to_keep=None, use_cache=True):
        self.calls.append(dict(logits_to_keep=logits_to_keep, use_cache=use_cache,
                               batch=input_ids.size(0)))
        L = input_ids.size(1)
        logits = self.emb[input_ids] + self.pos[:L].unsqueeze(0)
        if logits_to_keep is not None:
            logits = logits[:, -logits_to_keep:, :]
        return SimpleNamespace(logits=logits)


def batch(B=5, L=12, vocab_in=50, seed=1, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, vocab_in, (B, L), generator=g).to(device)
    mask = torch.ones(B, L, dtype=torch.int64, device=device)
    return ids, mask
