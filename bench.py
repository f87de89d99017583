"""bench.py — fused logprob/entropy forward + backward on one MI355X.

Metric: fwd/bwd ms + HBM TB/s (% of peak) at B*S=1024,
V=152064 bf16 (config C2).  A step is one forward and one backward launch of
the fused kernels over that batch, through the library's C ABI (via
kernel_opt._C), with inputs resident in HBM.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C2]
                    [--no-cpu-baseline] [--flush]

Prints ONE JSON line.  `value` = achieved algorithmic HBM bandwidth over the
whole step (fwd bytes + bwd bytes) / (fwd + bwd time), in TB/s.

Algorithmic bytes per launch (s = bytes per logit, N rows, V vocab):
    forward  = N*V*s + 8N (targets) + 12N (logp, entropy, lse)
    backward = 2*N*V*s + 8N (targets) + 16N (lse, entropy, g_logp, g_ent)
(g_lse is None in these workloads, so it is not read.)

Timing (HIP events on the stream the kernels run on): `ms_per_step` is one
event pair around K interleaved forward+backward steps, divided by K; the
per-kernel `fwd_ms` / `bwd_ms` are one event pair around K back-to-back
launches of that kernel, divided by K.  With --flush a 1 GiB buffer is read
(or, with --flush-mode write, overwritten) before every launch and each
launch is timed on its own.  The
roofline object reports the dominant kernel, the backward (it moves twice the
forward's bytes); `traffic` is the HBM bytes per launch that rocprofv3's
FETCH_SIZE / WRITE_SIZE counters measured for that launch shape, scaled by
their readings for a plain copy of known size (MEASURED_TRAFFIC below).

The cpu_baseline leg times the reference's CPU eager path (TRL
selective_log_softmax + entropy_from_logits forward, restated in
oracle/eager_ref.py, plus PyTorch autograd through the eager formulas for
the backward) on the same workload (C2: the whole batch, well under a
second) on this machine's cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "fused-logprob-entropy-cuda-kernel-for-llm-post-training_amd")
for _p in (PKG_DIR, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

HBM_PEAK_TBPS = 8.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA

# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE,
# each scaled by the counter's reading for a plain copy of known size
# (profiles/klp_all_configs_hbm_traffic.md).  Keyed by workload, kernel and
# launch shape (waves, unroll, splits, flags); reported only for that shape.
MEASURED_TRAFFIC = {
    ("C1", "fwd", (16, 4, 1, 0)): 32960385,
    ("C1", "bwd", (16, 2, 4, 1)): 65711874,
    ("C2", "fwd", (4, 4, 1, 0)): 311758388,
    ("C2", "bwd", (16, 2, 8, 1)): 623290575,
    ("C3", "fwd", (4, 4, 1, 0)): 2103303576,
    ("C3", "bwd", (16, 2, 8, 1)): 4205676181,
    ("C4", "fwd", (4, 4, 1, 0)): 9964861906,
    ("C4", "bwd", (16, 2, 10, 1)): 19926260879,
    ("C5", "fwd", (4, 4, 1, 0)): 8592967390,
    ("C5", "bwd", (16, 2, 32, 1)): 17183261794,
}
ROW_BLOCK = 256  # rows per seeded generator block

# BASELINE.json configs.  Seeds are per config; each block of ROW_BLOCK rows
# draws from its own generator seeded with seed * 1_000_003 + block, so any
# row subset can be regenerated on its own.
CONFIGS = {
    "C1": dict(dtype=torch.float32, shape=(2, 128, 32000), sigma=2.0, seed=1001,
               g_logp=1.0 / 256, g_ent=0.01 / 256),
    "C2": dict(dtype=torch.bfloat16, shape=(4, 256, 152064), sigma=2.0, seed=1002,
               g_logp=-1.0 / 1024, g_ent=-0.01 / 1024),
    "C3": dict(dtype=torch.float16, shape=(8, 1024, 128256), sigma=3.0, seed=1003,
               spike=18.0, p_target_spike=0.6, g_logp=-1.0 / 8192, g_ent=-0.01 / 8192),
    "C4": dict(dtype=torch.bfloat16, shape=(16, 2048, 151936), sigma=2.5, seed=1004,
               mask_p=0.7),
    "C5": dict(dtype=torch.float32, shape=(4, 2048, 262144), sigma=1.5, seed=1005,
               parent_len=2049, g_logp=-1.0 / 8192, g_ent=-0.01 / 8192),
}


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def make_inputs(name: str, device="cuda", n_rows: int | None = None):
    """Synthetic inputs of config `name` (first `n_rows` rows if given).

    Returns dict(logits, targets, g_logp, g_ent, parent?) on `device`.
    logits is [B, S, V] (C5: the non-contiguous slice parent[:, :-1, :]);
    when n_rows is given the leading dims collapse to [n_rows, V] (C5 keeps
    its strided layout by slicing whole batch elements).
    """
    cfg = CONFIGS[name]
    B, S, V = cfg["shape"]
    N = B * S
    dtype = cfg["dtype"]
    device = torch.device(device)
    if name == "C5":
        L = cfg["parent_len"]
        b_keep = B if n_rows is None else max(1, math.ceil(n_rows / S))
        parent = torch.zeros(b_keep, L, V, dtype=dtype, device=device)
        rows_view = parent[:, :-1, :]
        flat_rows = [(b, s) for b in range(b_keep) for s in range(S)]
        n = len(flat_rows)
        for blk in range(0, n, ROW_BLOCK):
            g = _gen(device, cfg["seed"] * 1_000_003 + blk // ROW_BLOCK)
            cnt = min(ROW_BLOCK, n - blk)
            vals = torch.randn(cnt, V, generator=g, device=device) * cfg["sigma"]
            for i in range(cnt):
                b, s = flat_rows[blk + i]
                rows_view[b, s].copy_(vals[i])
        logits = rows_view
        tg = _gen(device, cfg["seed"] * 7 + 1)
        targets = torch.randint(0, V, (b_keep, S), generator=tg, device=device)
        if n_rows is not None and n_rows < b_keep * S:
            pass  # whole batch elements are kept so the strided layout stays
        n = b_keep * S
        grads = _grads(cfg, n, device)
        return dict(logits=logits, targets=targets, parent=parent,
                    **{k: (v.view(b_keep, S) if v is not None else None) for k, v in grads.items()})

    n = N if n_rows is None else n_rows
    logits = torch.empty(n, V, dtype=dtype, device=device)
    targets = torch.empty(n, dtype=torch.int64, device=device)
    for blk in range(0, n, ROW_BLOCK):
        cnt = min(ROW_BLOCK, n - blk)
        g = _gen(device, cfg["seed"] * 1_000_003 + blk // ROW_BLOCK)
        vals = torch.randn(cnt, V, generator=g, device=device) * cfg["sigma"]
        tgt = torch.randint(0, V, (cnt,), generator=g, device=device)
        if "spike" in cfg:
            spike_idx = torch.randint(0, V, (cnt,), generator=g, device=device)
            vals[torch.arange(cnt, device=device), spike_idx] += cfg["spike"]
            use_spike = torch.rand(cnt, generator=g, device=device) < cfg["p_target_spike"]
            tgt = torch.where(use_spike, spike_idx, tgt)
        logits[blk:blk + cnt] = vals.to(dtype)
        targets[blk:blk + cnt] = tgt
    grads = _grads(cfg, n, device)
    if n_rows is None:
        logits = logits.view(B, S, V)
        targets = targets.view(B, S)
        grads = {k: (v.view(B, S) if v is not None else None) for k, v in grads.items()}
    return dict(logits=logits, targets=targets, **grads)


def _grads(cfg, n, device):
    if "mask_p" in cfg:
        # loss = -mean(mask * (logp + 0.01 * H)) over all B*S tokens
        B, S, _ = cfg["shape"]
        g = _gen(device, cfg["seed"] * 7 + 2)
        mask = (torch.rand(n, generator=g, device=device) < cfg["mask_p"]).float()
        return dict(g_logp=-mask / (B * S), g_ent=-0.01 * mask / (B * S))
    return dict(g_logp=torch.full((n,), cfg["g_logp"], device=device),
                g_ent=torch.full((n,), cfg["g_ent"], device=device))


def algorithmic_bytes(n_rows: int, vocab: int, elem_bytes: int):
    fwd = n_rows * vocab * elem_bytes + 8 * n_rows + 12 * n_rows
    bwd = 2 * n_rows * vocab * elem_bytes + 8 * n_rows + 16 * n_rows
    return fwd, bwd


# ---------------------------------------------------------------------------
# CPU baseline: the reference's CPU eager path.
# ---------------------------------------------------------------------------
def cpu_baseline(name: str, max_rows: int, logits_gpu, targets_gpu, g_logp, g_ent, reps=3):
    """Times the reference's CPU eager path on the workload (its first
    `max_rows` rows, whole batch elements): the forward as TRL computes it
    (selective_log_softmax + entropy_from_logits, restated in
    oracle/eager_ref.py) and forward + backward as PyTorch autograd of the
    eager formulas.  One warm-up, then the median of `reps` runs."""
    from oracle import eager_ref

    cfg = CONFIGS[name]
    B, S, V = cfg["shape"]
    b_keep = max(1, min(B, max_rows // S))
    x = torch.stack([logits_gpu[b].detach().cpu() for b in range(b_keep)]).contiguous()
    t = targets_gpu[:b_keep].cpu().contiguous()
    gl = g_logp.reshape(B, S)[:b_keep].cpu()
    ge = g_ent.reshape(B, S)[:b_keep].cpu()

    def fwd():
        return eager_ref.trl_selective_log_softmax(x, t), eager_ref.trl_entropy_from_logits(x)

    def fwd_bwd():
        xr = x.clone().requires_grad_(True)
        lp, h, _ = eager_ref.ref_forward_pt(xr, t)
        (lp * gl + h * ge).sum().backward()
        return xr.grad

    def timed(fn):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2]

    t_fwd = timed(fwd)
    t_fb = timed(fwd_bwd)
    scale = B / b_keep
    return dict(fwd_ms=t_fwd * scale * 1e3, fwd_bwd_ms=t_fb * scale * 1e3, rows=b_keep * S,
                threads=torch.get_num_threads(), scaled=b_keep < B)


# ---------------------------------------------------------------------------
# GPU timing
# ---------------------------------------------------------------------------
def _eager_grpo(logp, old, adv, mask, ref, eps_low, eps_high, beta):
    """The GRPO loss as a chain of eager torch ops ("grpo" normaliser, token
    level): the path klp_grpo_* replaces, timed beside it."""
    coef_1 = torch.exp(logp - old)
    coef_2 = torch.clamp(coef_1, 1 - eps_low, 1 + eps_high)
    per_token = -torch.min(coef_1 * adv.unsqueeze(1), coef_2 * adv.unsqueeze(1))
    kl = torch.exp(ref - logp) - (ref - logp) - 1
    per_token = per_token + beta * kl
    return ((per_token * mask).sum(-1) / mask.sum(-1).clamp(min=1.0)).mean()


def grpo_timing(dev, K, B=16, S=2048):
    """Forward + backward of the GRPO loss on [B, S] per-token log-probs
    (C4's batch shape): fused launches against the eager chain."""
    from kernel_opt import fused_grpo_loss
    g = torch.Generator(device="cpu").manual_seed(2024)
    new = (torch.randn(B, S, generator=g) - 2.0).to(dev)
    old = (new.cpu() + 0.3 * torch.randn(B, S, generator=g)).to(dev)
    ref = (new.cpu() + 0.3 * torch.randn(B, S, generator=g)).to(dev)
    adv = torch.randn(B, generator=g).to(dev)
    mask = (torch.rand(B, S, generator=g) < 0.7).float().to(dev)
    lp = new.clone().requires_grad_(True)

    def fused():
        loss, _ = fused_grpo_loss(lp, old, adv, mask, ref, eps_low=0.2, eps_high=0.28,
                                  beta=0.04, loss_type="grpo")
        loss.backward()

    def eager():
        _eager_grpo(lp, old, adv, mask, ref, 0.2, 0.28, 0.04).backward()

    res = {}
    for name, fn in (("fused", fused), ("eager", eager)):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(K):
            fn()
        b.record()
        torch.cuda.synchronize()
        res[name] = a.elapsed_time(b) / K * 1e3
    return {"shape": [B, S], "loss_type": "grpo", "beta": 0.04,
            "fused_fwd_bwd_us": round(res["fused"], 2),
            "eager_fwd_bwd_us": round(res["eager"], 2),
            "note": "loss + loss.backward() per iteration, end to end from Python"}


def grpo_step_timing(dev, K, logits, targets):
    """The fused GRPO step (klp_grpo_step: logprob, GRPO loss gradient and
    d_logits in one read of the logits) against the unfused kernel chain
    klp_fwd -> klp_grpo_fwd -> klp_grpo_bwd -> klp_bwd on the same logits,
    both through the C ABI with preallocated outputs (kernel time only)."""
    import ctypes
    from kernel_opt import _C
    from kernel_opt._library import (DTYPE_CODES, KLP_GRPO_LOSS_GRPO,
                                     KLP_GRPO_STEP_SCHED_BYTES, KLP_GRPO_TOKEN, check_status,
                                     lib)
    from kernel_opt.grpo_step import grpo_token_weights
    B, S, V = logits.shape
    N = B * S
    if V > lib.klp_grpo_step_max_vocab(DTYPE_CODES[logits.dtype]):
        return None
    g = torch.Generator(device="cpu").manual_seed(77)
    f32 = lambda *shape: torch.empty(*shape, dtype=torch.float32, device=dev)
    lp, ent, lse, loss_tok, d_logp = (f32(B, S) for _ in range(5))
    with torch.no_grad():
        _C.fwd_launch(logits, targets, lp, ent, lse)
    old = (lp.cpu() + 0.2 * torch.randn(B, S, generator=g)).to(dev)
    ref = (lp.cpu() + 0.2 * torch.randn(B, S, generator=g)).to(dev)
    adv = torch.randn(B, generator=g).to(dev)
    mask = (torch.rand(B, S, generator=g) < 0.9).float().to(dev)
    w = grpo_token_weights(mask, "grpo").contiguous()
    d = torch.empty(logits.shape, dtype=logits.dtype, device=dev)
    sched = torch.zeros(KLP_GRPO_STEP_SCHED_BYTES, dtype=torch.uint8, device=dev)
    ws = torch.empty(lib.klp_grpo_workspace_bytes(B), dtype=torch.uint8, device=dev)
    loss = f32(1)
    rows = _C.row_layout(logits)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    eps_low, eps_high, beta = 0.2, 0.28, 0.04
    gparams = (eps_low, eps_high, beta, 1.0, KLP_GRPO_LOSS_GRPO, KLP_GRPO_TOKEN, 0)

    def fused():
        check_status(lib.klp_grpo_step(P(logits), DTYPE_CODES[logits.dtype], N, V, *rows,
                                       P(targets), 1.0, P(old), P(ref), P(adv), P(w), S,
                                       eps_low, eps_high, beta, 0, P(lp), P(ent), P(lse),
                                       P(loss_tok), P(d), P(sched), st))

    def unfused():
        _C.fwd_launch(logits, targets, lp, ent, lse)
        check_status(lib.klp_grpo_fwd(P(lp), P(old), P(ref), P(adv), P(mask), B, S, *gparams,
                                      P(loss), None, P(ws), ws.numel(), st))
        check_status(lib.klp_grpo_bwd(P(lp), P(old), P(ref), P(adv), P(mask), B, S, *gparams,
                                      None, P(d_logp), P(ws), ws.numel(), st))
        _C.bwd_launch(logits, targets, lse, ent, d_logp, None, None, d)

    res = {}
    for name, fn in (("fused", fused), ("unfused", unfused)):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(K):
            fn()
        b.record()
        torch.cuda.synchronize()
        res[name] = a.elapsed_time(b) / K * 1e3
    nbytes = 2 * logits.numel() * logits.element_size()  # one read + one write
    tbps = nbytes / (res["fused"] * 1e-6) / 1e12
    del d
    torch.cuda.empty_cache()
    return {"shape": [B, S, V], "loss_type": "grpo", "beta": beta,
            "fused_us": round(res["fused"], 2), "unfused_us": round(res["unfused"], 2),
            "speedup": round(res["unfused"] / res["fused"], 3),
            "fused_algorithmic_bytes": nbytes, "fused_tbps": round(tbps, 4),
            "fused_pct_peak": round(100 * tbps / HBM_PEAK_TBPS, 2),
            "note": "fused = klp_grpo_step (logits read once, d_logits written once); "
                    "unfused = klp_fwd, klp_grpo_fwd, klp_grpo_bwd, klp_bwd (logits read "
                    "twice); both kernel time through the C ABI, outputs preallocated"}


def shard_timing(dev, K, N=32768, V=151936, P=8):
    """One rank's share of C4 under an 8-way vocab-parallel LM head: the
    shard forward (klp_fwd_shard, [N, V/P] bf16 -> 16-byte row states), the
    merge of P states (klp_fwd_shard_merge) and the shard backward (klp_bwd
    with shard-relative targets), through the C ABI with preallocated
    outputs.  The all-gather of the states between them is not part of this
    single-GPU build (16 bytes per row: 512 KB per rank at C4)."""
    import ctypes
    from kernel_opt import _C
    from kernel_opt._library import DTYPE_CODES, check_status, lib
    sv = -(-V // P)
    rank = 3
    g = torch.Generator(device=dev).manual_seed(4)
    x = (torch.randn(N, sv, generator=g, device=dev) * 2.5).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), generator=g, device=dev)
    state = torch.empty(N, 4, dtype=torch.float32, device=dev)
    states = torch.empty(P, N, 4, dtype=torch.float32, device=dev)
    lp, ent, lse = (torch.empty(N, dtype=torch.float32, device=dev) for _ in range(3))
    gl = torch.full((N,), -1.0 / N, device=dev)
    d = torch.empty_like(x)
    t_local = (t - rank * sv).contiguous()
    rows = _C.row_layout(x)
    P_ = lambda z: ctypes.c_void_p(z.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    def fwd():
        check_status(lib.klp_fwd_shard(P_(x), DTYPE_CODES[x.dtype], N, sv, *rows, P_(t),
                                       rank * sv, 1.0, P_(state), st))

    def merge():
        check_status(lib.klp_fwd_shard_merge(P_(states), P, N, P_(t), sv, V, P_(lp), P_(ent),
                                             P_(lse), st))

    def bwd():
        _C.bwd_launch(x, t_local, lse, ent, gl, None, None, d)

    fwd()
    for k in range(P):
        states[k].copy_(state)
    res = {}
    for name, fn in (("fwd", fwd), ("merge", merge), ("bwd", bwd)):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(K):
            fn()
        b.record()
        torch.cuda.synchronize()
        res[name] = a.elapsed_time(b) / K * 1e3
    fb = N * sv * 2 + 8 * N + 16 * N
    bb = 2 * N * sv * 2 + 8 * N + 12 * N
    out = {"shape": {"rows": N, "vocab": V, "shards": P, "shard_columns": sv, "dtype": "bf16"},
           "shard_fwd_us": round(res["fwd"], 2), "merge_us": round(res["merge"], 2),
           "shard_bwd_us": round(res["bwd"], 2),
           "shard_fwd_tbps": round(fb / (res["fwd"] * 1e-6) / 1e12, 4),
           "shard_bwd_tbps": round(bb / (res["bwd"] * 1e-6) / 1e12, 4),
           "note": "per-rank kernels of an 8-way vocab-parallel C4; the exchange of the "
                   "16-byte row states is outside this single-GPU build"}
    del x, d
    torch.cuda.empty_cache()
    return out


def lmhead_timing(dev, N=1024, V=152064, D=3584, K=5):
    """The fused LM head (hidden @ weight^T folded into the logprob/entropy
    reduction, klp_lmh_*) against the unfused path (a bf16 library matmul,
    then the logprob kernels) on Qwen2.5-7B's head shape with C2's 1024
    tokens; random weights.  Forward, and forward + backward with upstream
    gradients on logprob and entropy."""
    from kernel_opt import (fused_linear_logprob_entropy, fused_linear_logprob_entropy_forward,
                            fused_logprob_entropy, fused_logprob_entropy_forward)
    g = torch.Generator(device=dev).manual_seed(3584)
    h = torch.randn(N, D, device=dev, generator=g).to(torch.bfloat16).requires_grad_(True)
    w = (torch.randn(V, D, device=dev, generator=g) / D ** 0.5 * 3).to(torch.bfloat16)
    w.requires_grad_(True)
    t = torch.randint(0, V, (N,), device=dev, generator=g)
    gl = torch.randn(N, device=dev, generator=g)
    ge = torch.randn(N, device=dev, generator=g)

    def fb(fused):
        h.grad = None
        w.grad = None
        if fused:
            lp, ent, _ = fused_linear_logprob_entropy(h, w, t)
        else:
            lp, ent, _ = fused_logprob_entropy(h @ w.T, t)
        ((lp * gl).sum() + (ent * ge).sum()).backward()

    def timed(fn):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(K):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / K

    with torch.no_grad():
        f_fwd = timed(lambda: fused_linear_logprob_entropy_forward(h, w, t))
        u_fwd = timed(lambda: fused_logprob_entropy_forward(h @ w.T, t))
    f_fb = timed(lambda: fb(True))
    u_fb = timed(lambda: fb(False))

    # GRPO on the head: the chunked LM head + fused step (library GEMMs and
    # klp_grpo_step per chunk of tokens) against the unfused path (bf16
    # matmul to the full logits, the logprob op, the GRPO loss, backward), at
    # this token count and at 8x it.
    from kernel_opt import fused_grpo_loss, fused_linear_grpo_step
    kw = dict(eps_low=0.2, eps_high=0.28, loss_type="grpo")

    def grpo_head(n_tok, chunks):
        B, S = 4 * (n_tok // N), N // 4
        hh = torch.randn(B, S, D, device=dev, generator=g).to(torch.bfloat16)
        hh.requires_grad_(True)
        tt = torch.randint(0, V, (B, S), device=dev, generator=g)
        old = -torch.rand(B, S, device=dev, generator=g) * 8 - 4
        adv = torch.randn(B, device=dev, generator=g)
        mask = (torch.rand(B, S, device=dev, generator=g) < 0.9).float()

        def run(chunk):
            hh.grad = None
            w.grad = None
            if chunk:
                loss, _, _ = fused_linear_grpo_step(
                    hh, w, tt, old, adv, mask,
                    chunk_tokens=None if chunk == "default" else chunk, **kw)
            else:
                lp, _, _ = fused_logprob_entropy(torch.matmul(hh, w.T), tt)
                loss, _ = fused_grpo_loss(lp, old, adv, mask, **kw)
            loss.backward()

        def peak_extra(chunk):
            """Peak memory above inputs and weights during one loss +
            backward, the new gradients included."""
            run(chunk)
            hh.grad = None
            w.grad = None
            torch.cuda.synchronize()
            base = torch.cuda.memory_allocated()
            torch.cuda.reset_peak_memory_stats()
            run(chunk)
            torch.cuda.synchronize()
            return round((torch.cuda.max_memory_allocated() - base) / 2 ** 20, 1)

        out = {"tokens": n_tok}
        for chunk in [0] + chunks:
            name = f"chunked_{chunk}" if chunk else "unfused"
            out[name + "_fwd_bwd_ms"] = round(timed(lambda: run(chunk)), 4)
            out[name + "_peak_extra_mib"] = peak_extra(chunk)
        hh.grad = None
        w.grad = None
        return out

    # "default": fused_linear_grpo_step's own chunking (one chunk at 8 * N
    # for this head).
    grpo_heads = [grpo_head(N, [N, N // 4]), grpo_head(8 * N, ["default", 2 * N])]
    torch.cuda.empty_cache()

    flops = 2 * N * V * D
    out = {"shape": {"tokens": N, "vocab": V, "hidden": D}, "dtype": "bf16 in, fp32 accumulate",
           "fused_fwd_ms": round(f_fwd, 4), "unfused_fwd_ms": round(u_fwd, 4),
           "fused_fwd_tflops": round(flops / (f_fwd * 1e-3) / 1e12, 1),
           "fused_fwd_bwd_ms": round(f_fb, 4), "unfused_fwd_bwd_ms": round(u_fb, 4),
           "roofline_fwd": {"bound": "mfma", "achieved": round(flops / (f_fwd * 1e-3) / 1e12, 1),
                            "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                            "frac": round(flops / (f_fwd * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                                          4)},
           "note": "unfused = bf16 library matmul to [N, V] logits, then klp_fwd / klp_bwd",
           "grpo_step": {
               "runs": grpo_heads,
               "note": "fused_linear_grpo_step (chunks of the given token count, 'default' "
                       "its own chunking: library "
                       "GEMMs + klp_grpo_step, d_hidden / d_weight computed in the forward) "
                       "against matmul + fused_logprob_entropy + fused_grpo_loss + backward; "
                       "loss + backward per iteration; peak memory above inputs and weights "
                       "during one iteration, the new gradients included"}}
    del h, w
    torch.cuda.empty_cache()
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="C2", choices=sorted(CONFIGS))
    ap.add_argument("--flush", action="store_true",
                    help="run through a 1 GiB buffer before every launch (cold Infinity Cache)")
    ap.add_argument("--flush-mode", choices=("read", "write"), default="read",
                    help="read: sum the buffer (evicts with clean lines); write: fill it "
                         "(leaves up to the cache size of dirty lines for the next kernel)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=1024,
                    help="rows of the workload the CPU baseline times (whole batch elements)")
    ap.add_argument("--fwd-config", default=None, help="waves,unroll,splits,flags")
    ap.add_argument("--bwd-config", default=None, help="waves,unroll,splits,flags")
    ap.add_argument("--no-lmhead", action="store_true",
                    help="skip the fused LM-head timing (klp_lmh_* against matmul + logprob)")
    ap.add_argument("--no-shard", action="store_true",
                    help="skip the vocab-shard timing (one rank's share of C4 under 8-way "
                         "vocab parallelism)")
    ap.add_argument("--no-grpo", action="store_true",
                    help="skip the GRPO timings (the loss kernels against the eager chain, "
                         "the fused step against the unfused kernels)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run torch's copy of a buffer the size of the logits (known "
                         "traffic, for scaling HBM counters)")
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(rows are independent, so data-parallel ranks would each run this same "
              "kernel on their own batch with no exchange)", file=sys.stderr)
        return 2

    from kernel_opt import _C

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    name = args.config
    cfg = CONFIGS[name]
    inp = make_inputs(name, dev)
    logits, targets = inp["logits"], inp["targets"]
    g_logp, g_ent = inp["g_logp"].contiguous(), inp["g_ent"].contiguous()
    V = logits.size(-1)
    N = logits.numel() // V
    esz = logits.element_size()
    logp = torch.empty(targets.shape, dtype=torch.float32, device=dev)
    ent = torch.empty_like(logp)
    lse = torch.empty_like(logp)
    d_logits = torch.empty(logits.shape, dtype=logits.dtype, device=dev)
    fcfg = tuple(int(v) for v in args.fwd_config.split(",")) if args.fwd_config else None
    bcfg = tuple(int(v) for v in args.bwd_config.split(",")) if args.bwd_config else None
    flush_buf = torch.ones(1 << 30, dtype=torch.uint8, device=dev) if args.flush else None

    def fwd():
        _C.fwd_launch(logits, targets, logp, ent, lse, config=fcfg)

    def bwd():
        _C.bwd_launch(logits, targets, lse, ent, g_logp, g_ent, None, d_logits, config=bcfg)

    stream = torch.cuda.current_stream(dev)
    for _ in range(args.warmup):
        fwd()
        bwd()
    if args.copy_calibration:
        src = logits if logits.is_contiguous() else logits.contiguous()
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        del dst
    torch.cuda.synchronize()

    K = args.steps

    def timed_loop(body):
        """Average ms of `body` over K back-to-back calls: one event pair on
        the stream the kernels run on, around the whole loop."""
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(K):
            body()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / K

    def flush(k):
        if args.flush_mode == "read":
            flush_buf.view(torch.int64).sum()
        else:
            flush_buf.fill_(k & 0xFF)

    def timed_each(fn):
        """Per-launch ms with the Infinity Cache flushed before each launch."""
        ts = []
        for k in range(K):
            flush(k)
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fn()
            b.record(stream)
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        return sum(ts) / K

    t_wall0 = time.perf_counter()
    if flush_buf is None:
        # the step as a training loop runs it: forward then backward, repeated
        step_ms = timed_loop(lambda: (fwd(), bwd()))
        # each kernel on its own, launched back to back
        fwd_avg = timed_loop(fwd)
        bwd_avg = timed_loop(bwd)
    else:
        fwd_avg = timed_each(fwd)
        bwd_avg = timed_each(bwd)
        step_ms = fwd_avg + bwd_avg
    t_wall = time.perf_counter() - t_wall0
    fb, bb = algorithmic_bytes(N, V, esz)
    fwd_tbps = fb / (fwd_avg * 1e-3) / 1e12
    bwd_tbps = bb / (bwd_avg * 1e-3) / 1e12
    step_tbps = (fb + bb) / (step_ms * 1e-3) / 1e12

    cpu = None
    if not args.no_cpu_baseline:
        c = cpu_baseline(name, args.cpu_rows, logits, targets, g_logp, g_ent)
        sample = (f"{c['rows']} of {N} rows of {name} (the whole batch)" if not c["scaled"] else
                  f"{c['rows']} of {N} rows of {name}, scaled by {N}/{c['rows']}")
        cpu = {
            "value": round((fb + bb) / (c["fwd_bwd_ms"] * 1e-3) / 1e12, 6),
            "unit": "TB/s",
            "cores": c["threads"],
            "kind": "port",
            "sample": (f"{sample}; torch CPU, {c['threads']} threads, median of 3 after one "
                       f"warm-up.  Step = eager forward + autograd backward "
                       f"{c['fwd_bwd_ms']:.1f} ms (value = the step's algorithmic bytes over "
                       f"it); the TRL-eager forward alone (restated, oracle/eager_ref.py) "
                       f"takes {c['fwd_ms']:.1f} ms"),
            "fwd_ms": round(c["fwd_ms"], 3),
            "fwd_bwd_ms": round(c["fwd_bwd_ms"], 3),
        }

    grpo = None if args.no_grpo else grpo_timing(dev, K)
    step = None if args.no_grpo else grpo_step_timing(dev, K, logits, targets)
    lmhead = None if args.no_lmhead else lmhead_timing(dev)
    shard = None if args.no_shard else shard_timing(dev, K)

    B, S, _ = cfg["shape"]
    fwd_used = fcfg or _C.default_config("fwd", logits.dtype, N, V)
    bwd_used = bcfg or _C.default_config("bwd", logits.dtype, N, V)
    out = {
        "metric": "fwd/bwd ms + HBM TB/s (% of peak) at B*S=1024, V=152064 bf16",
        "value": round(step_tbps, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[
            logits.dtype],
        "data": "synthetic",
        "config": {"workload": f"{name}: logits [{B},{S},{V}] "
                               f"{str(logits.dtype).replace('torch.', '')}, one forward + one "
                               f"backward launch per step",
                   "global_batch": B, "seq_len": S, "vocab": V, "n_rows": N,
                   "parallelism": "single-gpu",
                   "infinity_cache": (f"flushed ({args.flush_mode} 1 GiB before each launch)"
                                      if args.flush else "warm")},
        "fwd_ms": round(fwd_avg, 5),
        "bwd_ms": round(bwd_avg, 5),
        "fwd_tbps": round(fwd_tbps, 4),
        "bwd_tbps": round(bwd_tbps, 4),
        "fwd_pct_peak": round(100 * fwd_tbps / HBM_PEAK_TBPS, 2),
        "bwd_pct_peak": round(100 * bwd_tbps / HBM_PEAK_TBPS, 2),
        "fwd_launch": dict(zip(("waves", "unroll", "splits", "flags"), fwd_used)),
        "bwd_launch": dict(zip(("waves", "unroll", "splits", "flags"), bwd_used)),
        "wall_s_timed": round(t_wall, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": "klp_bwd_kernel",
            "achieved": round(bb / (bwd_avg * 1e-3) / 1e9, 1),
            "peak": HBM_PEAK_TBPS * 1000,
            "unit": "GB/s",
            "frac": round(bwd_tbps / HBM_PEAK_TBPS, 4),
            "traffic": MEASURED_TRAFFIC.get((name, "bwd", tuple(bwd_used))),
            "algorithmic_bytes": bb,
            "fwd_traffic": MEASURED_TRAFFIC.get((name, "fwd", tuple(fwd_used))),
            "fwd_algorithmic_bytes": fb,
        },
        "cpu_baseline": cpu,
        "grpo_loss": grpo,
        "grpo_step": step,
        "lm_head": lmhead,
        "vocab_shard": shard,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
