"""bench.py — fused logprob/entropy forward + backward on one MI355X.

Metric: fwd/bwd ms + HBM TB/s (% of peak) at B*S=1024,
V=152064 bf16 (config C2).  A step is one forward and one backward launch of
the fused kernels over that batch, through the library's C ABI (via
kernel_opt._C), with inputs resident in HBM.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C2]
                    [--no-cpu-baseline] [--core-only] [--sweep OUT.md]
    python bench.py --trace-from DIR [--config C2]          # rocprofv3 kernel trace -> markdown
    python bench.py --traffic-from FETCH_DIR WRITE_DIR      # rocprofv3 counters -> markdown

Prints ONE JSON line.  `value` = achieved algorithmic HBM bandwidth over the
step (fwd bytes + bwd bytes) / `ms_per_step`, in TB/s.

Algorithmic bytes per launch (s = bytes per logit, N rows, V vocab):
    forward  = N*V*s + 8N (targets) + 12N (logp, entropy, lse)
    backward = 2*N*V*s + 8N (targets) + 16N (lse, entropy, g_logp, g_ent)
(g_lse is None in these workloads, so it is not read.)

Timing, on the stream the kernels run on:
  * `ms_per_step`: one HIP-event pair around K interleaved forward+backward
    steps (the backward re-reads logits the forward has just streamed
    through the 256 MB Infinity Cache, so the step can beat the per-kernel
    rates);
  * `fwd_ms` / `bwd_ms`: one HIP-event pair around max(K, 50) back-to-back
    launches;
  * `fwd_ms_flushed` / `bwd_ms_flushed`: kernel durations from the device's
    own timestamps (torch.profiler over ROCm's tracer, the figures
    rocprofv3 --kernel-trace reports), the median over 24 launches each
    right after a 1 GiB buffer was read (which evicts the logits from the
    cache); `device_timed` gives these and the warm medians with their
    interquartile spread.  Where the profiler sees no GPU (or with
    --no-device-timer) HIP events time them instead: one pair around
    (flush, launch) pairs minus one around the flushes alone;
  * `ceilings`: in the same process, at the same size and launch shapes,
    the library's calibration kernels, warm and flushed: klp_ceiling_read
    (the forward's ring of loads without arithmetic), klp_ceiling_copy (the
    backward's loop of loads and stores), klp_ceiling_read_pieces and
    klp_ceiling_write (that loop's loads alone, its stores alone: their sum
    is the time of a read+write stream whose reads and writes do not
    overlap on the HBM bus), and torch's device copy; `fwd_over_read`,
    `bwd_over_copy` and `bwd_over_read_plus_write` are the kernels' times
    over them;
  * `configs`: C3, C4 and C5 measured the same way at their own sizes.
`roofline` reports the dominant kernel, the backward (it moves twice the
forward's bytes), at the lower of its warm and flushed rates.  `traffic` is
the HBM bytes per launch from a committed rocprofv3 counter summary under
profiles/ (made by --traffic-from) whose build id equals this build's (a hash
of the library sources); null when none matches.

`autograd` times the drop-in path (kernel_opt.fused_logprob_entropy and
loss.backward(), as the reference's bench/bench_backward.py:45-53 does) and
reports the bytes each allocates beyond its outputs (the reference's method,
bench/bench_micro.py:62-78).  `C1` is the BASELINE's CPU-runnable config on
the GPU and on the CPU eager path.

The cpu_baseline leg times the reference's CPU eager path (TRL
selective_log_softmax + entropy_from_logits forward, restated in
oracle/eager_ref.py, plus PyTorch autograd through the eager formulas for
the backward) on the same workload (C2: the whole batch, well under a
second) on this machine's cores.
"""
from __future__ import annotations

import argparse
import csv
import glob
import hashlib
import json
import math
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "fused-logprob-entropy-cuda-kernel-for-llm-post-training_amd")
PROFILES_DIR = os.path.join(ROOT, "profiles")
for _p in (PKG_DIR, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

HBM_PEAK_TBPS = 8.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
FLUSH_BYTES = 1 << 30
SETTLE_S = 0.3          # untimed busy time before the first timed loop
KERNEL_LAUNCHES = 50    # fewest launches behind each per-kernel figure


def build_id() -> str:
    """Hash of the library's sources (kernels, headers, Makefile): the same
    sources build the same kernels, so a profile made from them describes
    this build."""
    paths = (glob.glob(os.path.join(PKG_DIR, "csrc", "*")) +
             glob.glob(os.path.join(ROOT, "include", "*.h")) + [os.path.join(PKG_DIR, "Makefile")])
    h = hashlib.sha256()
    for path in sorted(paths):
        h.update(os.path.relpath(path, ROOT).encode())
        h.update(b"\0")
        with open(path, "rb") as f:
            h.update(f.read())
        h.update(b"\0")
    return h.hexdigest()[:16]


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


def ceiling_row_bytes(vocab: int, elem_bytes: int) -> int:
    """Row size of the calibration kernels' buffer: the logits row rounded up
    to whole 16-byte vectors."""
    return (vocab * elem_bytes + 15) // 16 * 16


# ---------------------------------------------------------------------------
# rocprofv3 output -> committed summaries (profiles/), and back.
#
# A summary is markdown for the reader plus one machine-readable line,
#   <!-- klp-profile {...json...} -->
# carrying the build id, the workload and the per-kernel figures.  The
# default bench run looks up the summaries of its own build id and workload
# for `roofline.traffic` and for the trace cross-check.
# ---------------------------------------------------------------------------
PROFILE_TAG = "klp-profile"


def _rocprof_csv(directory: str, suffix: str):
    hits = sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {directory}")
    rows = []
    for path in hits:
        with open(path, newline="") as f:
            rows.extend(csv.DictReader(f))
    return rows


def short_kernel(name: str) -> str:
    """'void klp::klp_bwd_kernel<0, 16, 2, true, false>(klp::BwdParams)' ->
    'klp_bwd_kernel<0, 16, 2, true, false>' (also through an anonymous
    namespace: 'void klp::(anonymous namespace)::klp_scale_kernel(...)' ->
    'klp_scale_kernel'); other names unchanged up to the argument list."""
    m = re.match(r"(?:void )?(?:klp::)?(?:\(anonymous namespace\)::)?"
                 r"([A-Za-z_0-9]+(?:<[^()]*>)?)", name)
    return m.group(1) if m else name


def _is_klp(name: str) -> bool:
    return "klp::" in name


def _workload_sizes(config: str):
    cfg = CONFIGS[config]
    B, S, V = cfg["shape"]
    esz = torch.empty((), dtype=cfg["dtype"]).element_size()
    return B * S, V, esz


def kernel_bytes(short: str, config: str):
    """Algorithmic bytes of one launch of a klp kernel of `config`'s
    workload, or None for kernels without a stated figure."""
    N, V, esz = _workload_sizes(config)
    fb, bb = algorithmic_bytes(N, V, esz)
    rb = ceiling_row_bytes(V, esz) * N
    if short.startswith("klp_fwd_kernel"):
        return fb
    if short.startswith("klp_bwd_kernel"):
        return bb
    if short.startswith("klp_ceiling_read") or short.startswith("klp_ceiling_write"):
        return rb
    if short.startswith("klp_ceiling_copy"):
        return 2 * rb
    return None


def _profile_line(data: dict) -> str:
    return f"<!-- {PROFILE_TAG} {json.dumps(data, sort_keys=True)} -->"


def load_profiles(kind: str, config: str, bid: str):
    """Machine-readable data of the committed summaries of `kind` ("traffic"
    or "trace") for `config` made from build `bid`."""
    out = []
    for path in sorted(glob.glob(os.path.join(PROFILES_DIR, "*.md"))):
        with open(path) as f:
            for line in f:
                line = line.strip()
                if line.startswith(f"<!-- {PROFILE_TAG} ") and line.endswith("-->"):
                    data = json.loads(line[len(PROFILE_TAG) + 5:-3])
                    if (data.get("kind") == kind and data.get("config") == config
                            and data.get("build_id") == bid):
                        data["file"] = os.path.relpath(path, ROOT)
                        out.append(data)
    return out


def _git_note() -> str:
    """', git `<head>`' where the tree is a git checkout, else '' (a copy of
    the tree without its .git, as on a remote GPU box)."""
    h = _git_head()
    return f", git `{h}`" if h else ""


def _git_head() -> str | None:
    try:
        import subprocess
        return subprocess.run(["git", "-C", ROOT, "rev-parse", "--short=12", "HEAD"],
                              capture_output=True, text=True, check=True).stdout.strip()
    except Exception:
        return None


def summarize_counters(directory: str, config: str, command: str = ""):
    """Per-dispatch averages of every counter in a rocprofv3 --pmc run, for the
    klp forward / backward and calibration kernels (rows of one dispatch and
    counter summed), with SQ_INSTS_* also per element of the workload (x 64
    lanes / N*V: wave instructions times lanes over logits).  Returns
    (markdown, data)."""
    N, V, _ = _workload_sizes(config)
    elems = N * V
    per = {}
    for r in _rocprof_csv(directory, "counter_collection.csv"):
        if not _is_klp(r["Kernel_Name"]):
            continue
        k = short_kernel(r["Kernel_Name"])
        d = per.setdefault(k, {}).setdefault(r["Counter_Name"], {})
        d[r["Dispatch_Id"]] = d.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    names = sorted({c for d in per.values() for c in d})
    kernels = {}
    rows = []
    for k in sorted(per):
        vals = {c: sum(v.values()) / len(v) for c, v in per[k].items()}
        n = max(len(v) for v in per[k].values())
        kernels[k] = {"dispatches": n, "mean": {c: round(v, 2) for c, v in vals.items()}}
        cells = []
        for c in names:
            v = vals.get(c)
            if v is None:
                cells.append("-")
            elif c.startswith("SQ_INSTS_"):
                cells.append(f"{v:.4g} ({v * 64 / elems:.2f}/elem)")
            else:
                cells.append(f"{v:.4g}")
        rows.append(f"| `{k}` | {n} | " + " | ".join(cells) + " |")
    data = {"kind": "counters", "config": config, "build_id": build_id(),
            "git_head": _git_head(), "kernels": kernels}
    md = [f"# rocprofv3 counters: klp kernels, workload {config}", "",
          f"Build id `{data['build_id']}`; summarised by `python bench.py --counters-from DIR "
          f"--config {config}`. Means per dispatch (a dispatch's rows summed over shader "
          f"engines and XCDs); SQ_INSTS_* also per logit element (wave instructions x 64 / "
          f"{elems}).", ""]
    if command:
        md += ["Command (MI355X):", "```", command, "```", ""]
    md += ["| kernel | dispatches | " + " | ".join(names) + " |",
           "|---|---:|" + "---:|" * len(names)]
    md += rows
    md += ["", "<!-- klp-profile " + json.dumps(data, sort_keys=True) + " -->"]
    return "\n".join(md) + "\n", data


def summarize_traffic(fetch_dir: str, write_dir: str, config: str, command: str = ""):
    """Per-dispatch HBM bytes of the klp kernels from two rocprofv3 --pmc
    runs (FETCH_SIZE, WRITE_SIZE; KiB per dispatch), each scaled by what the
    same counter reads for klp_ceiling_copy_kernel, whose reads and writes are
    known (N rows of the logits' size each way).  Returns (markdown, data)."""
    N, V, esz = _workload_sizes(config)
    copy_bytes = ceiling_row_bytes(V, esz) * N
    per = {}
    for counter, directory in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        for r in _rocprof_csv(directory, "counter_collection.csv"):
            if r["Counter_Name"] != counter or not _is_klp(r["Kernel_Name"]):
                continue
            d = per.setdefault(short_kernel(r["Kernel_Name"]), {})
            d.setdefault(counter, []).append(float(r["Counter_Value"]))
    cal = [k for k in per if k.startswith("klp_ceiling_copy")]
    if not cal:
        raise RuntimeError("no klp_ceiling_copy_kernel dispatch: the calibration is missing")
    cd = per[cal[0]]
    f_fetch = copy_bytes / (1024 * sum(cd["FETCH_SIZE"]) / len(cd["FETCH_SIZE"]))
    f_write = copy_bytes / (1024 * sum(cd["WRITE_SIZE"]) / len(cd["WRITE_SIZE"]))
    kernels = {}
    rows = []
    for k in sorted(per):
        d = per[k]
        if "FETCH_SIZE" not in d or "WRITE_SIZE" not in d:
            continue
        fe = sum(d["FETCH_SIZE"]) / len(d["FETCH_SIZE"])
        wr = sum(d["WRITE_SIZE"]) / len(d["WRITE_SIZE"])
        traffic = int(round(1024 * (fe * f_fetch + wr * f_write)))
        alg = kernel_bytes(k, config)
        kernels[k] = {"dispatches": len(d["FETCH_SIZE"]), "fetch_kib": round(fe, 1),
                      "write_kib": round(wr, 1), "traffic_bytes": traffic,
                      "algorithmic_bytes": alg,
                      "ratio": None if not alg else round(traffic / alg, 4)}
        rows.append(f"| `{k}` | {len(d['FETCH_SIZE'])} | {fe:.1f} | {wr:.1f} | {traffic} | "
                    f"{alg if alg else '-'} | {kernels[k]['ratio'] or '-'} |")
    bid = build_id()
    data = {"kind": "traffic", "config": config, "build_id": bid, "git_head": _git_head(),
            "fetch_factor": round(f_fetch, 5), "write_factor": round(f_write, 5),
            "kernels": kernels}
    md = [f"# rocprofv3 HBM counters: klp kernels, workload {config}", "",
          f"Build id `{bid}` (hash of the library sources, as `bench.py` computes it); "
          f"summarised at git `{data['git_head']}` by `python bench.py --traffic-from "
          f"{fetch_dir} {write_dir} --config {config}`.", ""]
    if command:
        md += ["Commands (MI355X):", "```", command, "```", ""]
    md += ["Calibration: `klp_ceiling_copy_kernel` reads and writes exactly "
           f"{copy_bytes} bytes per launch. Scale factors (known bytes / counter bytes): "
           f"FETCH_SIZE x{f_fetch:.5f}, WRITE_SIZE x{f_write:.5f}.", "",
           "| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic bytes | "
           "algorithmic bytes | traffic / algorithmic |", "|---|---:|---:|---:|---:|---:|---:|"]
    md += rows + ["", _profile_line(data), ""]
    return "\n".join(md), data


def _phase(prev: str | None, name: str) -> str:
    if prev is None:
        return "other"
    if "reduce_kernel" in prev:
        return "flushed"
    if prev == name:
        return "back to back"
    if _is_klp(prev):
        return "after another klp kernel"
    return "other"


def summarize_trace(trace_dir: str, config: str, command: str = "", label: str | None = None):
    """Average kernel durations of the klp kernels from a rocprofv3
    --kernel-trace run, overall and per phase of bench.py (a launch right
    after the 1 GiB flush read: "flushed"; after a launch of the same kernel:
    "back to back"; after the other klp kernel: the interleaved step).
    `label` (default: the config) tags the summary; the bench line's
    trace_check reads the summaries tagged with the bare config name, i.e.
    those of a `--core-only` run.  Returns (markdown, data)."""
    rows = _rocprof_csv(trace_dir, "kernel_trace.csv")
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    stats = {}
    prev = None
    for r in rows:
        name = r["Kernel_Name"]
        if _is_klp(name):
            k = short_kernel(name)
            dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            ph = _phase(prev, name)
            stats.setdefault(k, {}).setdefault("all", []).append(dur)
            stats[k].setdefault(ph, []).append(dur)
        prev = name
    kernels = {}
    lines = []
    for k in sorted(stats):
        # A labelled run launches kernels at several shapes (other configs'
        # legs, small batches): no bytes per launch to divide by.
        alg = None if label else kernel_bytes(k, config)
        kernels[k] = {}
        for ph in ("all", "back to back", "flushed", "after another klp kernel", "other"):
            ds = stats[k].get(ph)
            if not ds:
                continue
            avg = sum(ds) / len(ds)
            med = sorted(ds)[len(ds) // 2]
            tb = None if not alg else alg / (avg * 1e-9) / 1e12
            kernels[k][ph] = {"n": len(ds), "avg_ns": round(avg, 1), "median_ns": med,
                              "min_ns": min(ds), "max_ns": max(ds),
                              "tbps": None if tb is None else round(tb, 4)}
            lines.append(f"| `{k}` | {ph} | {len(ds)} | {avg / 1e3:.2f} | {med / 1e3:.2f} | "
                         f"{min(ds) / 1e3:.2f} | {max(ds) / 1e3:.2f} | "
                         f"{'-' if tb is None else f'{tb:.3f} ({100 * tb / HBM_PEAK_TBPS:.1f}%)'} |")
    bid = build_id()
    tag = label or config
    data = {"kind": "trace", "config": tag, "build_id": bid, "git_head": _git_head(),
            "kernels": kernels}
    md = [f"# rocprofv3 kernel trace: klp kernels, workload {tag}", "",
          f"Build id `{bid}` (hash of the library sources, as `bench.py` computes it); "
          f"summarised at git `{data['git_head']}` by `python bench.py --trace-from "
          f"{trace_dir} --config {config}" + (f" --label {label}" if label else "") + "`.",
          ""]
    if command:
        md += ["Command (MI355X):", "```", command, "```", ""]
    md += [("TB/s: not given; this run launches kernels at several shapes (its other "
            "legs), so a kernel's launches are not all of the config's size." if label else
            "TB/s = algorithmic bytes per launch / average duration (forward "
            "N*V*s + 20N, backward 2*N*V*s + 24N, calibration kernels their buffer bytes)."),
           "",
           "| kernel | phase | launches | avg us | median us | min us | max us | TB/s (% of 8) |",
           "|---|---|---:|---:|---:|---:|---:|---:|"]
    md += lines + ["", _profile_line(data), ""]
    return "\n".join(md), data


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
        for queued in (False, True):
            torch.cuda.synchronize()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            if queued:  # long enough to hold K host-issued calls of ~100 us
                torch.cuda._sleep(max(Timer.QUEUE_SPIN_CYCLES, K * 250_000))
            a.record()
            for _ in range(K):
                fn()
            b.record()
            torch.cuda.synchronize()
            res[name + ("_queued" if queued else "")] = a.elapsed_time(b) / K * 1e3
    return {"shape": [B, S], "loss_type": "grpo", "beta": 0.04,
            "fused_fwd_bwd_us": round(res["fused"], 2),
            "eager_fwd_bwd_us": round(res["eager"], 2),
            "fused_fwd_bwd_us_queued": round(res["fused_queued"], 2),
            "eager_fwd_bwd_us_queued": round(res["eager_queued"], 2),
            "note": "loss + loss.backward() per iteration, end to end from Python (the "
                    "fused loss through the compiled binding); *_queued: the same calls "
                    "behind a spin kernel, i.e. GPU time without the host's latency"}


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
                                       eps_low, eps_high, beta, 0, 1.0, P(lp), P(ent),
                                       P(lse), P(loss_tok), P(d), P(sched), st))

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

    # The same step through the public entry points, from Python: the fused
    # step + loss.backward(), against fused_logprob_entropy + fused_grpo_loss
    # + loss.backward(); issued back to back (host-paced) and queued behind a
    # spin kernel (GPU time).
    from kernel_opt import fused_grpo_loss, fused_grpo_step, fused_logprob_entropy
    x = logits.detach().clone().requires_grad_(True)
    kw = dict(eps_low=eps_low, eps_high=eps_high, beta=beta, loss_type="grpo")

    def step_fused():
        loss_, _, _ = fused_grpo_step(x, targets, old, adv, mask, ref, **kw)
        loss_.backward()
        x.grad = None

    mask_i32 = mask.to(torch.int32)

    def step_fused_int32_mask():
        loss_, _, _ = fused_grpo_step(x, targets, old, adv, mask_i32, ref, **kw)
        loss_.backward()
        x.grad = None

    def step_unfused():
        lp_, _, _ = fused_logprob_entropy(x, targets)
        loss_, _ = fused_grpo_loss(lp_, old, adv, mask, ref, **kw)
        loss_.backward()
        x.grad = None

    # A trainer with 8 gradient-accumulation steps backpropagates loss / 8:
    # undeclared, the backward multiplies d_logits by 1/8 (a read and a
    # write of it); declared as grad_scale, the forward applies it.
    def step_fused_ga8():
        loss_, _, _ = fused_grpo_step(x, targets, old, adv, mask_i32, ref, **kw)
        (loss_ / 8).backward()
        x.grad = None

    def step_fused_ga8_declared():
        loss_, _, _ = fused_grpo_step(x, targets, old, adv, mask_i32, ref, grad_scale=0.125,
                                      **kw)
        (loss_ / 8).backward()
        x.grad = None

    e2e = {}
    for name, fn in (("fused", step_fused), ("fused_int32_mask", step_fused_int32_mask),
                     ("fused_loss_over_8", step_fused_ga8),
                     ("fused_loss_over_8_grad_scale", step_fused_ga8_declared),
                     ("unfused", step_unfused)):
        for _ in range(3):
            fn()
        for queued in (False, True):
            torch.cuda.synchronize()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            if queued:  # long enough to hold K host-issued steps
                torch.cuda._sleep(max(Timer.QUEUE_SPIN_CYCLES, K * 500_000))
            a.record()
            for _ in range(K):
                fn()
            b.record()
            torch.cuda.synchronize()
            e2e[name + ("_queued" if queued else "")] = round(a.elapsed_time(b) / K * 1e3, 2)
    del x
    torch.cuda.empty_cache()
    return {"shape": [B, S, V], "loss_type": "grpo", "beta": beta,
            "fused_us": round(res["fused"], 2), "unfused_us": round(res["unfused"], 2),
            "speedup": round(res["unfused"] / res["fused"], 3),
            "fused_algorithmic_bytes": nbytes, "fused_tbps": round(tbps, 4),
            "fused_pct_peak": round(100 * tbps / HBM_PEAK_TBPS, 2),
            "end_to_end_us": e2e,
            "note": "fused = klp_grpo_step (logits read once, d_logits written once); "
                    "unfused = klp_fwd, klp_grpo_fwd, klp_grpo_bwd, klp_bwd (logits read "
                    "twice); both kernel time through the C ABI, outputs preallocated; "
                    "end_to_end_us: the step through the public entry points from Python "
                    "(fused_grpo_step vs fused_logprob_entropy + fused_grpo_loss, loss + "
                    "backward), host-paced and *_queued (GPU time), with a float32 mask "
                    "(token weights in eager torch) and fused_int32_mask with the same mask "
                    "as int32, as TRL's completion_mask comes (token weights in one "
                    "klp_grpo_token_weights launch); fused_loss_over_8: (loss / 8).backward(), "
                    "as under 8 gradient-accumulation steps, without and with grad_scale=1/8 "
                    "declared (undeclared, the backward rescales d_logits)"}


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


def lmhead_timing(dev, N=1024, V=152064, D=3584, K=5, rounds=6):
    """The fused LM head against the unfused path on Qwen2.5-7B's head shape
    with C2's 1024 tokens (and 8x that), random weights.  Three paths:
    "chunked" (the default: a library GEMM per vocabulary chunk, then
    klp_fwd_shard / klp_fwd_shard_merge; the backward recomputes each chunk),
    "mfma" (klp_lmh_fwd, the hand-written GEMM with the reduction as its
    epilogue) and "unfused" (a bf16 library matmul to the [N, V] logits, then
    klp_fwd / klp_bwd).  Forward, and forward + backward with upstream
    gradients on logprob and entropy; medians over interleaved rounds of K
    calls; peak memory beyond the inputs (and, for the backward, beyond the
    new gradients)."""
    from kernel_opt import (fused_linear_logprob_entropy, fused_linear_logprob_entropy_forward,
                            fused_logprob_entropy, fused_logprob_entropy_forward)
    g = torch.Generator(device=dev).manual_seed(3584)
    w = (torch.randn(V, D, device=dev, generator=g) / D ** 0.5 * 3).to(torch.bfloat16)
    w.requires_grad_(True)

    def inputs(n_tok):
        hh = torch.randn(n_tok, D, device=dev, generator=g).to(torch.bfloat16)
        hh.requires_grad_(True)
        return (hh, torch.randint(0, V, (n_tok,), device=dev, generator=g),
                torch.randn(n_tok, device=dev, generator=g),
                torch.randn(n_tok, device=dev, generator=g))

    def fwd(impl, h, t):
        with torch.no_grad():
            if impl == "unfused":
                return fused_logprob_entropy_forward(h @ w.T, t)
            return fused_linear_logprob_entropy_forward(h, w, t, impl=impl)

    def fb(impl, h, t, gl, ge):
        h.grad = None
        w.grad = None
        if impl == "unfused":
            lp, ent, _ = fused_logprob_entropy(h @ w.T, t)
        else:
            lp, ent, _ = fused_linear_logprob_entropy(h, w, t, impl=impl)
        ((lp * gl).sum() + (ent * ge).sum()).backward()

    def timed(fn):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(K):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / K

    def medians(fns):
        for fn in fns.values():
            fn()
            fn()
        times = {k: [] for k in fns}
        order = list(fns)
        for r in range(rounds):
            # the order reverses every round: under sustained GEMM load the
            # clock drifts within a round, and a fixed order would hand the
            # same path the same share of it
            for k in (order if r % 2 == 0 else order[::-1]):
                times[k].append(timed(fns[k]))
        return {k: round(statistics.median(v), 4) for k, v in times.items()}

    def peak_mib(fn, h):
        fn()
        h.grad = None
        w.grad = None
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        fn()
        torch.cuda.synchronize()
        extra = torch.cuda.max_memory_allocated() - base
        if h.grad is not None:
            extra -= h.grad.numel() * h.grad.element_size() + w.grad.numel() * 2
        h.grad = None
        w.grad = None
        return round(extra / 2 ** 20, 1)

    runs = []
    for n_tok, impls in ((N, ("chunked", "mfma", "unfused")), (8 * N, ("chunked", "unfused"))):
        h, t, gl, ge = inputs(n_tok)
        f_ms = medians({i: (lambda i=i: fwd(i, h, t)) for i in impls})
        fb_ms = medians({i: (lambda i=i: fb(i, h, t, gl, ge)) for i in impls})
        run = {"tokens": n_tok}
        for i in impls:
            run[i] = {"fwd_ms": f_ms[i], "fwd_bwd_ms": fb_ms[i],
                      "fwd_tflops": round(2 * n_tok * V * D / (f_ms[i] * 1e-3) / 1e12, 1),
                      "fwd_peak_extra_mib": peak_mib(lambda i=i: fwd(i, h, t), h),
                      "fwd_bwd_peak_beyond_grads_mib":
                          peak_mib(lambda i=i: fb(i, h, t, gl, ge), h)}
        runs.append(run)
        del h, t, gl, ge
        torch.cuda.empty_cache()
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
            if chunk == "head":
                # the vocabulary-chunked LM head, then the GRPO loss (autograd)
                lp, _, _ = fused_linear_logprob_entropy(hh, w, tt)
                loss, _ = fused_grpo_loss(lp, old, adv, mask, **kw)
            elif chunk:
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
        for chunk in [0] + chunks + ["head"]:
            name = ("vocab_chunked_head" if chunk == "head" else f"chunked_{chunk}" if chunk
                    else "unfused")
            run(chunk)
            run(chunk)
            out[name + "_fwd_bwd_ms"] = round(timed(lambda: run(chunk)), 4)
            out[name + "_peak_extra_mib"] = peak_extra(chunk)
        hh.grad = None
        w.grad = None
        return out

    # "default": fused_linear_grpo_step's own chunking (one chunk at 8 * N
    # for this head).
    grpo_heads = [grpo_head(N, [N, N // 4]), grpo_head(8 * N, ["default", 2 * N])]
    torch.cuda.empty_cache()

    c = runs[0]["chunked"]
    out = {"shape": {"tokens": N, "vocab": V, "hidden": D}, "dtype": "bf16",
           "runs": runs,
           "fused_fwd_ms": c["fwd_ms"], "unfused_fwd_ms": runs[0]["unfused"]["fwd_ms"],
           "fused_fwd_bwd_ms": c["fwd_bwd_ms"],
           "unfused_fwd_bwd_ms": runs[0]["unfused"]["fwd_bwd_ms"],
           "roofline_fwd": {"bound": "mfma", "achieved": c["fwd_tflops"],
                            "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                            "frac": round(c["fwd_tflops"] / MFMA_BF16_PEAK_TFLOPS, 4)},
           "note": "fused = the chunked head (default); mfma = klp_lmh_fwd with the "
                   "vocabulary-chunked backward; unfused = bf16 library matmul to [N, V] "
                   "logits, then klp_fwd / klp_bwd; medians of 6 interleaved rounds of 5 "
                   "calls, the order reversed every round",
           "grpo_step": {
               "runs": grpo_heads,
               "note": "fused_linear_grpo_step (chunks of the given token count, 'default' "
                       "its own chunking: library "
                       "GEMMs + klp_grpo_step, d_hidden / d_weight computed in the forward), "
                       "and vocab_chunked_head (fused_linear_logprob_entropy, the "
                       "vocabulary-chunked head, + fused_grpo_loss + backward), "
                       "against matmul + fused_logprob_entropy + fused_grpo_loss + backward; "
                       "loss + backward per iteration; peak memory above inputs and weights "
                       "during one iteration, the new gradients included"}}
    del w
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------
# The core measurement
# ---------------------------------------------------------------------------
class Timer:
    """HIP-event timing on one stream, with an optional Infinity-Cache flush
    (reading, or with mode "write" overwriting, a 1 GiB buffer) before each
    launch."""

    def __init__(self, dev, K, flush_mode="read", buf=None):
        self.stream = torch.cuda.current_stream(dev)
        self.K = K
        self.flush_mode = flush_mode
        self.buf = buf if buf is not None else torch.ones(FLUSH_BYTES, dtype=torch.uint8,
                                                          device=dev)

    QUEUE_SPIN_CYCLES = 4_000_000  # ~2 ms of shader clock

    def b2b(self, body, queued=True):
        """Average ms of `body` over K back-to-back calls: one event pair
        around the whole loop.  With `queued` a spin kernel runs first
        (before the first event), so the host enqueues the K calls while it
        spins and the GPU then runs them without waiting for the host: the
        figure is GPU time even where one call's host issue (~7 us through
        ctypes) exceeds its kernel's duration."""
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        if queued:
            torch.cuda._sleep(self.QUEUE_SPIN_CYCLES)
        a.record(self.stream)
        for _ in range(self.K):
            body()
        b.record(self.stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / self.K

    def flush(self, k=0):
        if self.flush_mode == "read":
            self.buf.view(torch.int64).sum()
        else:
            self.buf.fill_(k & 0xFF)

    FLUSH_ROUNDS = 9

    def flushed(self, body):
        """(ms per launch, ms per launch timed on its own) of `body` right
        after a flush.  The first figure is the median over FLUSH_ROUNDS
        rounds of: one event pair around K / FLUSH_ROUNDS (flush, body)
        pairs minus one around as many flushes alone, so the dispatch gap
        after each flush is not counted (it is what a kernel profiler
        reports), and a round whose flushes ran at another speed than its
        neighbours' (clock changes) does not set the result; one round runs
        first untimed.  The second figure times each launch with its own
        event pair after its flush (includes that gap, about 3 us)."""
        n = max(1, self.K // self.FLUSH_ROUNDS)

        def loop(with_body):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            a.record(self.stream)
            for k in range(n):
                self.flush(k)
                if with_body:
                    body()
            b.record(self.stream)
            torch.cuda.synchronize()
            return a.elapsed_time(b)

        loop(True)
        loop(False)
        diffs = sorted((loop(True) - loop(False)) / n for _ in range(self.FLUSH_ROUNDS))
        ts = []
        for k in range(self.K):
            self.flush(k)
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(self.stream)
            body()
            b.record(self.stream)
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        return diffs[len(diffs) // 2], sum(ts) / len(ts)


class DeviceTimer:
    """Kernel durations from the device's own timestamps: torch.profiler over
    ROCm's tracer, i.e. the begin and end of each dispatch, the figures
    rocprofv3 --kernel-trace reports.  Each figure is the median over
    `n` launches back to back ("warm") or each right after a flush
    ("flushed"), with the interquartile range as the spread.  Unlike a pair
    of HIP events around (flush + launch) minus one around the flush alone,
    it is not the difference of two large, separately noisy times.

    `available` is False where the profiler sees no GPU activity, or when
    disabled (under rocprofv3, whose tracer must not share the process
    with torch's); callers then fall back to HIP events."""

    def __init__(self, timer, enabled=True):
        self.timer = timer
        self.available = False
        if enabled:
            try:
                from torch.profiler import ProfilerActivity
                self.available = ProfilerActivity.CUDA in torch.profiler.supported_activities()
            except Exception:
                self.available = False

    def _durations(self, body, match, n, flushed):
        from torch.profiler import ProfilerActivity, profile
        torch.cuda.synchronize()
        with profile(activities=[ProfilerActivity.CUDA]) as pf:
            for k in range(n):
                if flushed:
                    self.timer.flush(k)
                body()
            torch.cuda.synchronize()
        out = []
        for e in pf.events():
            if e.device_type == torch.autograd.DeviceType.CUDA and match in e.name:
                t = getattr(e, "device_time", None)
                out.append(float(t if t is not None else e.cuda_time))
        return out

    @staticmethod
    def _summary(us):
        us = sorted(us)
        n = len(us)
        med = statistics.median(us)
        q1, q3 = us[n // 4], us[(3 * n) // 4]
        return {"ms": round(med / 1e3, 5), "n": n, "spread_pct": round(100 * (q3 - q1) / med, 2),
                "min_ms": round(us[0] / 1e3, 5), "max_ms": round(us[-1] / 1e3, 5)}

    def stats(self, body, match, n=24):
        """{"warm": {...}, "flushed": {...}} of the kernels named `match` in
        `body` (one such launch per call); the first warm launch, right
        after a flush, is dropped."""
        warm = self._durations(body, match, n + 1, False)[1:]
        flushed = self._durations(body, match, n, True)
        if not warm or not flushed:
            raise RuntimeError(f"profiler saw no kernel named {match!r}")
        return {"warm": self._summary(warm), "flushed": self._summary(flushed)}


def _tbps(nbytes, ms):
    return nbytes / (ms * 1e-3) / 1e12


def core_timing(name, dev, K, warmup, timer, fcfg=None, bcfg=None, dtimer=None):
    """Forward / backward of workload `name` through the C ABI: the timed
    step loop, back-to-back and flushed per-kernel times, and the same-run
    ceilings at the kernels' size and launch shapes: the forward's ring read
    (klp_ceiling_read), the backward's copy (klp_ceiling_copy) and its loads
    and stores alone (klp_ceiling_read_pieces, klp_ceiling_write).  With a
    DeviceTimer the flushed figures (and a warm one beside the events' b2b
    figure) are kernel durations from the device's timestamps; without one,
    HIP events (Timer.flushed)."""
    from kernel_opt import _C
    from kernel_opt._library import check_status, lib

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

    def fwd():
        _C.fwd_launch(logits, targets, logp, ent, lse, config=fcfg)

    def bwd():
        _C.bwd_launch(logits, targets, lse, ent, g_logp, g_ent, None, d_logits, config=bcfg)

    for _ in range(warmup):
        fwd()
        bwd()
    # Untimed: keep the GPU busy for a moment so that its clocks have
    # settled before anything is timed (a few warm-up steps take ~1 ms).
    t_spin = time.perf_counter() + SETTLE_S
    while time.perf_counter() < t_spin:
        for _ in range(8):
            fwd()
            bwd()
        torch.cuda.synchronize()
    torch.cuda.synchronize()

    t_wall0 = time.perf_counter()
    # the timed steps: forward then backward, repeated, as a training loop runs them
    step_ms = timer.b2b(lambda: (fwd(), bwd()))
    t_wall = time.perf_counter() - t_wall0
    # Per-kernel figures over at least KERNEL_LAUNCHES launches each.
    kt = Timer(dev, max(K, KERNEL_LAUNCHES), timer.flush_mode, timer.buf)
    fwd_ms = kt.b2b(fwd)
    bwd_ms = kt.b2b(bwd)

    fwd_used = tuple(fcfg) if fcfg else _C.default_config("fwd", logits.dtype, N, V)
    bwd_used = tuple(bcfg) if bcfg else _C.default_config("bwd", logits.dtype, N, V)

    # Calibration kernels over a buffer of the logits' size (the logits
    # themselves when their rows are whole contiguous 16-byte vectors), with
    # the kernels' launch shapes; the copy and the write go into d_logits.
    rb = ceiling_row_bytes(V, esz)
    if logits.is_contiguous() and (V * esz) % 16 == 0:
        src = logits
    else:
        src = torch.empty(N * rb, dtype=torch.uint8, device=dev)
    dst = d_logits if d_logits.numel() * esz >= N * rb else torch.empty(N * rb, dtype=torch.uint8,
                                                                        device=dev)
    sink = torch.zeros(N * max(fwd_used[2], bwd_used[2], 1), dtype=torch.int32, device=dev)
    st = timer.stream.cuda_stream
    fw, fu, fs, _ = fwd_used
    bw, bu, bs, _ = bwd_used
    magic = 0x9E3779B9

    def ceil_read():
        check_status(lib.klp_ceiling_read(src.data_ptr(), N, rb, fw, fu, fs, sink.data_ptr(),
                                          magic, st))

    def ceil_copy():
        check_status(lib.klp_ceiling_copy(src.data_ptr(), dst.data_ptr(), N, rb, bw, bu, bs,
                                          st))

    def ceil_read_pieces():
        check_status(lib.klp_ceiling_read_pieces(src.data_ptr(), N, rb, bw, bu, bs,
                                                 sink.data_ptr(), magic, st))

    def ceil_write():
        check_status(lib.klp_ceiling_write(dst.data_ptr(), N, rb, bw, bu, bs, st))

    tsrc = src.view(-1)[:N * rb // src.element_size()] if src is logits else src
    tdst = dst.view(-1)[:tsrc.numel()] if dst.dtype == tsrc.dtype else None

    def torch_copy():
        tdst.copy_(tsrc)

    kernels = {"fwd": (fwd, "klp_fwd_kernel"), "bwd": (bwd, "klp_bwd_kernel"),
               "read": (ceil_read, "klp_ceiling_read_kernel"),
               "copy": (ceil_copy, "klp_ceiling_copy_kernel"),
               "read_pieces": (ceil_read_pieces, "klp_ceiling_read_pieces_kernel"),
               "write": (ceil_write, "klp_ceiling_write_kernel")}
    for key in ("read", "copy", "read_pieces", "write"):
        kernels[key][0]()
    warm = {k: (fwd_ms if k == "fwd" else bwd_ms if k == "bwd" else kt.b2b(fn))
            for k, (fn, _) in kernels.items()}
    device = {}
    if dtimer is not None and dtimer.available:
        for k, (fn, match) in kernels.items():
            device[k] = dtimer.stats(fn, match)
        flushed = {k: device[k]["flushed"]["ms"] for k in kernels}
        flushed_each = {}
        method = "device timestamps (torch.profiler): median over the launches, each right " \
                 "after a flush"
    else:
        flushed, flushed_each = {}, {}
        for k, (fn, _) in kernels.items():
            flushed[k], flushed_each[k] = kt.flushed(fn)
        method = "HIP events: (flush + launch) pairs minus flushes alone, median of rounds"
    # The backward's writes restore d_logits for the callers below.
    bwd()
    if tdst is not None:
        torch_copy()
        warm["torch_copy"] = kt.b2b(torch_copy)
        flushed["torch_copy"], _ = kt.flushed(torch_copy)
    bwd()
    del sink
    if dst is not d_logits:
        del dst
    fb, bb = algorithmic_bytes(N, V, esz)
    rbytes = N * rb
    nbytes = {"read": rbytes, "copy": 2 * rbytes, "read_pieces": rbytes, "write": rbytes,
              "torch_copy": 2 * rbytes}
    out_ceil = {
        "read_kernel": f"klp_ceiling_read (the forward's ring), launch "
                       f"{dict(zip(('waves', 'unroll', 'splits'), fwd_used[:3]))}",
        "copy_kernel": f"klp_ceiling_copy, klp_ceiling_read_pieces, klp_ceiling_write (the "
                       f"backward's loop: copy, loads alone, stores alone), launch "
                       f"{dict(zip(('waves', 'unroll', 'splits'), bwd_used[:3]))}",
        "buffer_bytes": rbytes,
        "flushed_method": method,
    }
    for k in nbytes:
        if k not in warm:
            continue
        out_ceil[f"{k}_ms"] = round(warm[k], 5)
        out_ceil[f"{k}_tbps"] = round(_tbps(nbytes[k], warm[k]), 4)
        out_ceil[f"{k}_ms_flushed"] = round(flushed[k], 5)
        out_ceil[f"{k}_tbps_flushed"] = round(_tbps(nbytes[k], flushed[k]), 4)
    out_ceil["fwd_over_read"] = round(fwd_ms / warm["read"], 4)
    out_ceil["bwd_over_copy"] = round(bwd_ms / warm["copy"], 4)
    out_ceil["fwd_over_read_flushed"] = round(flushed["fwd"] / flushed["read"], 4)
    out_ceil["bwd_over_copy_flushed"] = round(flushed["bwd"] / flushed["copy"], 4)
    # A read+write stream whose reads and writes cannot overlap on the HBM
    # bus takes the read-only plus the write-only time.
    out_ceil["read_plus_write_ms"] = round(warm["read_pieces"] + warm["write"], 5)
    out_ceil["read_plus_write_ms_flushed"] = round(flushed["read_pieces"] + flushed["write"], 5)
    out_ceil["read_plus_write_pct_peak"] = round(
        100 * _tbps(2 * rbytes, warm["read_pieces"] + warm["write"]) / HBM_PEAK_TBPS, 2)
    out_ceil["bwd_over_read_plus_write"] = round(bwd_ms / (warm["read_pieces"] + warm["write"]), 4)
    out_ceil["bwd_over_read_plus_write_flushed"] = round(
        flushed["bwd"] / (flushed["read_pieces"] + flushed["write"]), 4)
    return dict(inputs=inp, logits=logits, targets=targets, g_logp=g_logp, g_ent=g_ent,
                N=N, V=V, esz=esz, fb=fb, bb=bb, step_ms=step_ms, wall=t_wall, fwd_ms=fwd_ms,
                bwd_ms=bwd_ms, fwd_fl=flushed["fwd"], fwd_fl_each=flushed_each.get("fwd"),
                bwd_fl=flushed["bwd"], bwd_fl_each=flushed_each.get("bwd"), fwd_used=fwd_used,
                bwd_used=bwd_used, ceilings=out_ceil, device_timed=device, d_logits=d_logits)


_TRACE_ROLES = (("fwd", "klp_fwd_kernel"), ("bwd", "klp_bwd_kernel"),
                ("read", "klp_ceiling_read_kernel"), ("copy", "klp_ceiling_copy_kernel"))


def trace_agreement(profiles, device_timed):
    """The committed kernel-trace summaries' figures for klp_fwd / klp_bwd
    (average us per phase), and this run's device-timed medians divided by
    the trace's medians of the same phase ("back to back" for warm,
    "flushed" for flushed): `bench_over_trace_median`.  The trace is another
    run, usually on another box, whose clock moves both kernels and their
    ceilings; `ratio_over_trace` compares what a box's clock cancels out of:
    this run's forward / read and backward / copy over the same ratios in
    the trace.  None without a summary of this build."""
    out = None
    medians = {}
    for prof in profiles:
        for k, v in prof["kernels"].items():
            for role, prefix in _TRACE_ROLES:
                if k.startswith(prefix):
                    medians.setdefault(role, []).append(v)
    for prof in profiles:
        for k, v in prof["kernels"].items():
            if not (k.startswith("klp_bwd_kernel") or k.startswith("klp_fwd_kernel")):
                continue
            out = out or {"file": prof["file"]}
            out[k] = {ph: round(d["avg_ns"] / 1e3, 3) for ph, d in v.items()}
            role = "bwd" if k.startswith("klp_bwd_kernel") else "fwd"
            dev_t = (device_timed or {}).get(role)
            if dev_t:
                ratio = out.setdefault("bench_over_trace_median", {})
                ratio[role] = {
                    mode: round(dev_t[mode]["ms"] * 1e6 / v[ph]["median_ns"], 4)
                    for mode, ph in (("warm", "back to back"), ("flushed", "flushed"))
                    if ph in v and v[ph].get("median_ns")}
    if out is not None and device_timed:
        for name, num, den in (("fwd_over_read", "fwd", "read"), ("bwd_over_copy", "bwd", "copy")):
            tn, td = medians.get(num, []), medians.get(den, [])
            bn, bd = device_timed.get(num), device_timed.get(den)
            if len(tn) != 1 or len(td) != 1 or not bn or not bd:
                continue  # missing, or several launch shapes of one kernel
            r = {}
            for mode, ph in (("warm", "back to back"), ("flushed", "flushed")):
                a, b = tn[0].get(ph, {}).get("median_ns"), td[0].get(ph, {}).get("median_ns")
                if a and b and bd[mode]["ms"]:
                    r[mode] = round((bn[mode]["ms"] / bd[mode]["ms"]) / (a / b), 4)
            if r:
                out.setdefault("ratio_over_trace", {})[name] = r
    return out


def _device_summary(device):
    """The DeviceTimer figures of core_timing in microseconds: median, the
    interquartile spread in percent, and the count, warm and flushed."""
    if not device:
        return None
    out = {}
    for k, v in device.items():
        out[k] = {mode: {"us": round(v[mode]["ms"] * 1e3, 2), "spread_pct": v[mode]["spread_pct"],
                         "n": v[mode]["n"]} for mode in ("warm", "flushed")}
    return out


def config_legs(names, dev, K, warmup, timer, dtimer):
    """The other BASELINE configs beside the headline, each through
    core_timing at its own size and default launch shapes: forward and
    backward, warm and flushed, with the read / copy / read-only / write-only
    ceilings at that shape.  Inputs are freed before the next config."""
    out = {}
    for name in names:
        print(f"bench.py: config {name}", file=sys.stderr, flush=True)
        core = core_timing(name, dev, min(K, 20), min(warmup, 3), timer, dtimer=dtimer)
        cfg = CONFIGS[name]
        B, S, V = cfg["shape"]
        fb, bb = core["fb"], core["bb"]
        c = core["ceilings"]
        r = {
            "workload": f"{name}: logits [{B},{S},{V}] {str(cfg['dtype']).replace('torch.', '')}"
                        + (", rows strided (parent[:, :-1, :])" if "parent_len" in cfg else ""),
            "fwd_us": round(core["fwd_ms"] * 1e3, 2),
            "bwd_us": round(core["bwd_ms"] * 1e3, 2),
            "step_us": round(core["step_ms"] * 1e3, 2),
            "fwd_us_flushed": round(core["fwd_fl"] * 1e3, 2),
            "bwd_us_flushed": round(core["bwd_fl"] * 1e3, 2),
            "fwd_pct_peak": round(100 * _tbps(fb, core["fwd_ms"]) / HBM_PEAK_TBPS, 2),
            "bwd_pct_peak": round(100 * _tbps(bb, core["bwd_ms"]) / HBM_PEAK_TBPS, 2),
            "fwd_pct_peak_flushed": round(100 * _tbps(fb, core["fwd_fl"]) / HBM_PEAK_TBPS, 2),
            "bwd_pct_peak_flushed": round(100 * _tbps(bb, core["bwd_fl"]) / HBM_PEAK_TBPS, 2),
            "step_tbps": round(_tbps(fb + bb, core["step_ms"]), 4),
            "fwd_launch": dict(zip(("waves", "unroll", "splits", "flags"), core["fwd_used"])),
            "bwd_launch": dict(zip(("waves", "unroll", "splits", "flags"), core["bwd_used"])),
            "ceilings": {k: v for k, v in c.items() if not k.endswith("_kernel")},
            "device_timed": _device_summary(core["device_timed"]),
        }
        out[name] = r
        del core
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out


def autograd_timing(dev, K, logits, targets, g_logp, g_ent):
    """The drop-in path: kernel_opt.fused_logprob_entropy forward and
    loss.backward() through its autograd op, timed and with their
    allocations measured as the reference does (bench/bench_micro.py:62-78:
    peak allocated during the calls minus allocated before;
    bench/bench_backward.py:39-56: events around loss.backward()).
    `*_transient_bytes` is the part of the peak not held after the call
    (intermediates); the backward's held bytes are the gradient's block
    (the caching allocator may round a large block up to its 2 MiB segment
    granularity, so it can exceed the gradient's size by under 2 MiB)."""
    from kernel_opt import fused_logprob_entropy
    x = logits.detach().requires_grad_(True)
    gl, ge = g_logp.view(targets.shape), g_ent.view(targets.shape)

    def loss_of(lp, ent):
        return (lp * gl + ent * ge).sum()

    for _ in range(3):
        x.grad = None
        lp, ent, _ = fused_logprob_entropy(x, targets)
        loss_of(lp, ent).backward()
    x.grad = None
    del lp, ent
    torch.cuda.synchronize()

    # forward: allocation of one call, then timing over K calls
    pre = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    outs = fused_logprob_entropy(x, targets)
    torch.cuda.synchronize()
    fwd_peak = torch.cuda.max_memory_allocated() - pre
    fwd_held = torch.cuda.memory_allocated() - pre
    out_bytes = sum(o.numel() * o.element_size() for o in outs)
    del outs
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(K)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(K)]
    for i in range(K):
        starts[i].record()
        o = fused_logprob_entropy(x, targets)
        ends[i].record()
        del o
    torch.cuda.synchronize()
    fwd_t = sorted(a.elapsed_time(b) for a, b in zip(starts, ends))

    def queued(call):
        """GPU time of one call: a spin kernel first, so that the host has
        issued the call's kernels before the first event's turn comes."""
        torch.cuda.synchronize()
        torch.cuda._sleep(Timer.QUEUE_SPIN_CYCLES)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        call()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b)

    fwd_q = sorted(queued(lambda: fused_logprob_entropy(x, targets)) for _ in range(K))

    # backward: allocation of one call, then timing over K calls
    lp, ent, _ = fused_logprob_entropy(x, targets)
    loss = loss_of(lp, ent)
    torch.cuda.synchronize()
    pre = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    loss.backward()
    torch.cuda.synchronize()
    bwd_peak = torch.cuda.max_memory_allocated() - pre
    bwd_held = torch.cuda.memory_allocated() - pre
    grad_bytes = x.grad.numel() * x.grad.element_size()
    x.grad = None
    bts = []
    for i in range(K):
        lp, ent, _ = fused_logprob_entropy(x, targets)
        loss = loss_of(lp, ent)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        loss.backward()
        b.record()
        x.grad = None
        torch.cuda.synchronize()
        bts.append(a.elapsed_time(b))
    bts.sort()
    bq = []
    for i in range(K):
        lp, ent, _ = fused_logprob_entropy(x, targets)
        loss = loss_of(lp, ent)
        bq.append(queued(loss.backward))
        x.grad = None
    bq.sort()
    return {
        "fwd_ms_median": round(fwd_t[len(fwd_t) // 2], 5),
        "bwd_ms_median": round(bts[len(bts) // 2], 5),
        "fwd_ms_median_queued": round(fwd_q[len(fwd_q) // 2], 5),
        "bwd_ms_median_queued": round(bq[len(bq) // 2], 5),
        "fwd_peak_bytes": fwd_peak, "fwd_output_bytes": out_bytes,
        "fwd_transient_bytes": fwd_peak - fwd_held,
        "bwd_peak_bytes": bwd_peak, "bwd_grad_bytes": grad_bytes,
        "bwd_held_bytes": bwd_held,
        "bwd_transient_bytes": bwd_peak - bwd_held,
        "note": "kernel_opt.fused_logprob_entropy and loss.backward() from Python, events per "
                "call (median of K); loss = sum(logp*g_logp + entropy*g_ent); *_queued: the "
                "same calls behind a spin kernel, i.e. their GPU time without the host's "
                "latency (autograd's engine, the loss's own backward ops, the launch); peak "
                "= max allocated during one call minus allocated before it",
    }


def c1_leg(dev, K, timer, with_cpu):
    """BASELINE config C1 (fp32 [2, 128, 32000]): GPU forward / backward
    (back to back through the C ABI) and the CPU eager path on the whole
    batch."""
    from kernel_opt import _C
    inp = make_inputs("C1", dev)
    x, t = inp["logits"], inp["targets"]
    gl, ge = inp["g_logp"].contiguous(), inp["g_ent"].contiguous()
    lp, ent, lse = (torch.empty(t.shape, dtype=torch.float32, device=dev) for _ in range(3))
    d = torch.empty_like(x)
    V = x.size(-1)
    N = x.numel() // V
    fb, bb = algorithmic_bytes(N, V, 4)

    def fwd():
        _C.fwd_launch(x, t, lp, ent, lse)

    def bwd():
        _C.bwd_launch(x, t, lse, ent, gl, ge, None, d)

    for _ in range(5):
        fwd()
        bwd()
    f_ms, b_ms = timer.b2b(fwd), timer.b2b(bwd)
    f_host, b_host = timer.b2b(fwd, queued=False), timer.b2b(bwd, queued=False)
    out = {"workload": "C1: logits [2,128,32000] float32", "fwd_us": round(f_ms * 1e3, 3),
           "bwd_us": round(b_ms * 1e3, 3), "fwd_tbps": round(_tbps(fb, f_ms), 4),
           "bwd_tbps": round(_tbps(bb, b_ms), 4),
           "fwd_us_host_paced": round(f_host * 1e3, 3), "bwd_us_host_paced": round(b_host * 1e3, 3),
           "timing": "GPU time per launch, launches queued behind a spin kernel; *_host_paced: "
                     "calls issued back to back from Python without it (at this size the "
                     "host's issue rate, ~7 us a call, sets the pace)",
           "fwd_launch": dict(zip(("waves", "unroll", "splits", "flags"),
                                  _C.default_config("fwd", x.dtype, N, V))),
           "bwd_launch": dict(zip(("waves", "unroll", "splits", "flags"),
                                  _C.default_config("bwd", x.dtype, N, V)))}
    if with_cpu:
        c = cpu_baseline("C1", N, x, t, gl, ge)
        out.update({"cpu_fwd_ms": round(c["fwd_ms"], 3), "cpu_fwd_bwd_ms": round(c["fwd_bwd_ms"], 3),
                    "cpu_threads": c["threads"],
                    "cpu_note": "the reference's CPU eager path (TRL-eager forward restated; "
                                "eager forward + autograd backward), whole batch, median of 3"})
    return out


def small_batch_leg(dev, timer):
    """Split-row mode where it is meant to pay: few rows of Qwen2.5-7B's
    vocabulary (bf16 [n, 152064], n = 1, 8, 32), forward GPU time per launch
    (queued), with the dispatcher's shape (rows split), the same rows unsplit
    (8 waves, unroll 2; and 16 waves, unroll 4, the unsplit dispatcher's
    choice before split rows were merged in one launch), and a plain read of
    the same bytes (klp_ceiling_read at the split shape)."""
    from kernel_opt import _C
    from kernel_opt._library import check_status, lib
    V = 152064
    g = torch.Generator(device=dev).manual_seed(152)
    rows = []
    for n in (1, 8, 32):
        x = (torch.randn(n, V, device=dev, generator=g) * 2.0).to(torch.bfloat16)
        t = torch.randint(0, V, (n,), device=dev, generator=g)
        o = [torch.empty(n, device=dev) for _ in range(3)]
        cfg = _C.default_config("fwd", x.dtype, n, V)
        sink = torch.zeros(n * cfg[2], dtype=torch.int32, device=dev)
        st = timer.stream.cuda_stream

        def run(c=None):
            _C.fwd_launch(x, t, *o, config=c)

        def read():
            check_status(lib.klp_ceiling_read(x.data_ptr(), n, V * 2, cfg[0], cfg[1], cfg[2],
                                              sink.data_ptr(), 0x9E3779B9, st))

        res = {}
        for key, fn in (("fwd_us", run), ("unsplit_8w_us", lambda: run((8, 2, 1, 0))),
                        ("unsplit_16w_us", lambda: run((16, 4, 1, 0))), ("read_us", read)):
            fn()
            res[key] = round(statistics.median(timer.b2b(fn) for _ in range(3)) * 1e3, 2)
        rows.append({"rows": n, "launch": dict(zip(("waves", "unroll", "splits"), cfg[:3])),
                     **res})
    return {"shape": "bf16 [rows, 152064]", "runs": rows,
            "note": "GPU time per launch, launches queued behind a spin kernel; a launch this "
                    "small is latency (dispatch, then dependent memory round trips): the read "
                    "of the same bytes bounds it from below"}


def sweep(name, dev, K, timer, out_md, dtimer=None):
    """Launch-shape sweep of the forward and backward at workload `name`,
    back to back and flushed, written as a markdown table: the forward over
    waves x unroll x 1-2 pieces, the backward over waves x unroll x
    power-of-two pieces plus, at 4 and 8 waves, the piece counts of about
    one iteration (the fewest within one, and one on either side).  With a
    DeviceTimer both columns are device-timed medians."""
    from kernel_opt import _C
    inp = make_inputs(name, dev)
    x, t = inp["logits"], inp["targets"]
    gl, ge = inp["g_logp"].contiguous(), inp["g_ent"].contiguous()
    lp, ent, lse = (torch.empty(t.shape, dtype=torch.float32, device=dev) for _ in range(3))
    d = torch.empty(x.shape, dtype=x.dtype, device=dev)
    V = x.size(-1)
    N = x.numel() // V
    fb, bb = algorithmic_bytes(N, V, x.element_size())
    fdef = _C.default_config("fwd", x.dtype, N, V)
    bdef = _C.default_config("bwd", x.dtype, N, V)
    timer = Timer(dev, max(K, KERNEL_LAUNCHES), timer.flush_mode, timer.buf)
    n = timer.K

    def _sweep_times(fn, match):
        if dtimer is not None and dtimer.available:
            st = dtimer.stats(fn, match, n=16)
            return st["warm"]["ms"], st["flushed"]["ms"]
        return timer.b2b(fn), timer.flushed(fn)[0]
    t_spin = time.perf_counter() + SETTLE_S
    while time.perf_counter() < t_spin:
        _C.fwd_launch(x, t, lp, ent, lse)
        _C.bwd_launch(x, t, lse, ent, gl, ge, None, d)
        torch.cuda.synchronize()
    use_dev = dtimer is not None and dtimer.available
    how = ("each shape's kernel duration from the device's timestamps (torch.profiler), the "
           "median over 16 launches back to back and over 16 each right after a 1 GiB read"
           if use_dev else
           f"each shape timed over {n} back-to-back launches queued behind a spin kernel (one "
           "event pair), and right after a 1 GiB read (the median over 9 rounds of one event "
           "pair around K / 9 (read, launch) pairs minus one around as many reads alone, per "
           "launch)")
    lines = [f"# Launch-shape sweep, workload {name} (build `{build_id()}`)", "",
             f"`python bench.py --config {name} --sweep OUT.md --steps {K}`: {how}. "
             "Defaults marked *.", "",
             "| kernel | waves | unroll | splits | b2b us | b2b % of 8 TB/s | flushed us | "
             "flushed % |", "|---|---:|---:|---:|---:|---:|---:|---:|"]
    _C.fwd_launch(x, t, lp, ent, lse)
    for w in (4, 8, 16):
        for u in (2, 4):
            for sp in (1, 2):
                c = (w, u, sp, 0)
                fn = (lambda c=c: _C.fwd_launch(x, t, lp, ent, lse, config=c))
                fn()
                a, f = _sweep_times(fn, "klp_fwd_kernel")
                mark = "*" if c == tuple(fdef) else ""
                lines.append(f"| fwd{mark} | {w} | {u} | {sp} | {a * 1e3:.2f} | "
                             f"{100 * _tbps(fb, a) / HBM_PEAK_TBPS:.1f} | {f * 1e3:.2f} | "
                             f"{100 * _tbps(fb, f) / HBM_PEAK_TBPS:.1f} |")
                print(lines[-1], file=sys.stderr, flush=True)
    nvec = V * x.element_size() // 16
    bcfgs = [(w, u, sp, 1) for w in (4, 8, 16) for u in (2, 4) for sp in (4, 8, 16)]
    for w in (4, 8):
        e = -(-nvec // (w * 64 * 2))
        bcfgs += [(w, 2, sp, 1) for sp in (e - 1, e, e + 1) if 1 <= sp <= 1024]
    if tuple(bdef) not in bcfgs:
        bcfgs.append(tuple(bdef))
    seen = set()
    for c in bcfgs:
        if c in seen:
            continue
        seen.add(c)
        w, u, sp = c[:3]
        fn = (lambda c=c: _C.bwd_launch(x, t, lse, ent, gl, ge, None, d, config=c))
        fn()
        a, f = _sweep_times(fn, "klp_bwd_kernel")
        mark = "*" if c == tuple(bdef) else ""
        lines.append(f"| bwd{mark} | {w} | {u} | {sp} | {a * 1e3:.2f} | "
                     f"{100 * _tbps(bb, a) / HBM_PEAK_TBPS:.1f} | {f * 1e3:.2f} | "
                     f"{100 * _tbps(bb, f) / HBM_PEAK_TBPS:.1f} |")
        print(lines[-1], file=sys.stderr, flush=True)
    with open(out_md, "w") as fh:
        fh.write("\n".join(lines) + "\n")


# ---------------------------------------------------------------------------
# The reference's comparison matrix on this device (bench/bench_micro.py:
# 95-122, shapes of docs/FINAL_REPORT.md:298-314; bench/bench_backward.py;
# traffic multiples of REPORT.md:157-177).  The eager baselines are the
# reference's own, restated here as GPU baselines to be timed (the restatement
# in oracle/eager_ref.py is test infrastructure, used as a checker and by the
# CPU baseline leg only).
# ---------------------------------------------------------------------------
def _trl_selective_log_softmax(logits, index):
    """TRL 1.4's selective_log_softmax as the reference describes it
    (REPORT.md:19-30): gather minus a per-row logsumexp for fp32 / fp64, a
    per-batch-element log_softmax + gather loop otherwise."""
    import torch.nn.functional as F
    if logits.dtype in (torch.float32, torch.float64):
        sel = torch.gather(logits, dim=-1, index=index.unsqueeze(-1)).squeeze(-1)
        return sel - torch.stack([torch.logsumexp(lg, dim=-1) for lg in logits])
    out = []
    for row_logits, row_labels in zip(logits, index):
        lp = F.log_softmax(row_logits, dim=-1)
        out.append(lp.gather(dim=-1, index=row_labels.unsqueeze(-1)).squeeze(-1))
    return torch.stack(out)


def _trl_entropy_from_logits(logits, chunk_size=128):
    """TRL 1.4's entropy_from_logits: 128-row chunks of log_softmax, exp,
    multiply, sum (notes/stage1_findings.md:38-60 of the reference)."""
    import torch.nn.functional as F
    flat = logits.reshape(-1, logits.shape[-1])
    ents = []
    for chunk in flat.split(chunk_size, dim=0):
        lp = F.log_softmax(chunk, dim=-1)
        ents.append(-(torch.exp(lp) * lp).sum(-1))
    return torch.cat(ents, dim=0).reshape(logits.shape[:-1])


def _trl_eager(logits, targets):
    return _trl_selective_log_softmax(logits, targets), _trl_entropy_from_logits(logits)


def _pytorch_separate(logits, targets):
    import torch.nn.functional as F
    lp = F.log_softmax(logits, dim=-1)
    logp = lp.gather(-1, targets.unsqueeze(-1)).squeeze(-1)
    return logp, -(lp.exp() * lp).sum(-1)


def _eager_reference(logits, targets):
    """The differentiable eager forward of the reference's backward bench
    (bench/bench_backward.py:19-26)."""
    import torch.nn.functional as F
    lp = F.log_softmax(logits, dim=-1)
    logp = lp.gather(-1, targets.unsqueeze(-1)).squeeze(-1)
    ent = -(lp.exp() * lp).sum(-1)
    return logp, ent, torch.logsumexp(logits, dim=-1)


MATRIX_SHAPES = ((256, 32000), (1024, 32000), (4096, 32000), (256, 128256), (1024, 128256),
                 (1024, 152064))
MATRIX_BWD_SHAPES = ((256, 32000), (1024, 128256), (1024, 152064), (4096, 32000))
MATRIX_TRAFFIC_SHAPE = (1024, 128256)


def _matrix_inputs(BS, V, dev, seed=0):
    g = _gen(dev, seed)
    x = torch.randn(1, BS, V, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    t = torch.randint(0, V, (1, BS), generator=g, device=dev, dtype=torch.int64)
    return x, t


def _matrix_backends():
    import kernel_opt
    return {
        "ours": lambda x, t: kernel_opt.fused_logprob_entropy(x, t),
        "ours_naive": lambda x, t: kernel_opt.fused_logprob_entropy_naive(x, t),
        "trl_eager": _trl_eager,
        "pytorch_separate": _pytorch_separate,
    }


def _per_call_ms(fn, n_warmup=5, n_iter=30):
    """The reference's timing (bench/bench_micro.py:56-75): an event pair
    around each call, median of n_iter after n_warmup; peak allocation
    during the calls minus before, MB."""
    for _ in range(n_warmup):
        out = fn()
        del out
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    pre = torch.cuda.memory_allocated()
    st = [torch.cuda.Event(enable_timing=True) for _ in range(n_iter)]
    en = [torch.cuda.Event(enable_timing=True) for _ in range(n_iter)]
    for i in range(n_iter):
        st[i].record()
        out = fn()
        en[i].record()
    torch.cuda.synchronize()
    del out
    ts = sorted(a.elapsed_time(b) for a, b in zip(st, en))
    return ts[len(ts) // 2], (torch.cuda.max_memory_allocated() - pre) / 2 ** 20


def matrix(dev, out_md, dtimer):
    """Forward latency of the reference's four backends over its six shapes
    (bf16, B = 1), each the reference's way; our kernels' device time beside
    it; then the backward against eager autograd (bench/bench_backward.py's
    method: events around loss.backward(), median of 20 after 5)."""
    backends = _matrix_backends()
    rows = {}
    for BS, V in MATRIX_SHAPES:
        x, t = _matrix_inputs(BS, V, dev)
        r = {}
        for name, fn in backends.items():
            ms, mb = _per_call_ms(lambda: fn(x, t))
            r[name] = {"ms": round(ms, 4), "alloc_mb": round(mb, 1),
                       "gbps": round(x.numel() * 2 / (ms * 1e-3) / 1e9, 1)}
        if dtimer is not None and dtimer.available:
            dt = dtimer.stats(lambda: backends["ours"](x, t), "klp_fwd_kernel", n=16)
            r["ours"]["kernel_us_warm"] = round(dt["warm"]["ms"] * 1e3, 2)
            r["ours"]["kernel_us_flushed"] = round(dt["flushed"]["ms"] * 1e3, 2)
            dn = dtimer.stats(lambda: backends["ours_naive"](x, t), "klp_fwd_naive_kernel", n=8)
            r["ours_naive"]["kernel_us_warm"] = round(dn["warm"]["ms"] * 1e3, 2)
        rows[(BS, V)] = r
        print(f"bench.py: matrix forward {BS}x{V}: " +
              ", ".join(f"{k} {v['ms']:.3f} ms" for k, v in r.items()), file=sys.stderr,
              flush=True)
        del x, t
        torch.cuda.empty_cache()
    bwd = {}
    import kernel_opt
    for BS, V in MATRIX_BWD_SHAPES:
        base, t = _matrix_inputs(BS, V, dev, seed=1)
        g = _gen(dev, 7)
        gl, ge, gs = (torch.randn(1, BS, generator=g, device=dev) for _ in range(3))
        res = {}
        for name, fwd in (("eager_autograd", _eager_reference),
                          ("ours", kernel_opt.fused_logprob_entropy)):
            times = []
            for i in range(25):
                x = base.clone().requires_grad_(True)
                lp, ent, lse = fwd(x, t)
                loss = (lp * gl + ent * ge + lse * gs).sum()
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                a.record()
                loss.backward()
                b.record()
                torch.cuda.synchronize()
                if i >= 5:
                    times.append(a.elapsed_time(b))
                del x, lp, ent, lse, loss
            res[name] = round(statistics.median(times), 4)
        bwd[(BS, V)] = res
        print(f"bench.py: matrix backward {BS}x{V}: {res}", file=sys.stderr, flush=True)
        del base, t
        torch.cuda.empty_cache()
    bid = build_id()
    md = ["# The reference's comparison matrix on one MI355X", "",
          f"`python bench.py --matrix {out_md}` (build `{bid}`{_git_note()}). bf16 "
          "logits `[1, B*S, V]` ~ N(0, 1), targets uniform, as the reference's "
          "`bench/bench_micro.py:167-169` draws them. Backends as the reference defines them "
          "(`bench/bench_micro.py:95-122`): `ours` = `kernel_opt.fused_logprob_entropy`, "
          "`ours_naive` = `fused_logprob_entropy_naive` (one thread per row), `trl_eager` = "
          "TRL's `selective_log_softmax` + `entropy_from_logits` (restated in `bench.py`; TRL is "
          "not installed), `pytorch_separate` = `F.log_softmax` + gather + `-(p log p).sum`. "
          "Timing as the reference's: a HIP-event pair around each call (host launch "
          "included), median of 30 after 5 warm-ups; `kernel` = our kernel's own duration "
          "from the device's timestamps, back to back and after a 1 GiB flush.", "",
          "Forward, ms (and GB/s of one pass over the logits):", "",
          "| (B*S, V) | TRL eager | PyTorch sep. | naive | **ours** | ours kernel, warm / "
          "flushed | speedup vs TRL | peak alloc MB (TRL / ours) |",
          "|---|---:|---:|---:|---:|---:|---:|---:|"]
    for (BS, V), r in rows.items():
        md.append(f"| ({BS}, {V}) | {r['trl_eager']['ms']:.3f} | "
                  f"{r['pytorch_separate']['ms']:.3f} | {r['ours_naive']['ms']:.3f} | "
                  f"**{r['ours']['ms']:.3f}** ({r['ours']['gbps']:.0f}) | "
                  f"{r['ours'].get('kernel_us_warm', '-')} / "
                  f"{r['ours'].get('kernel_us_flushed', '-')} us | "
                  f"**{r['trl_eager']['ms'] / r['ours']['ms']:.1f}x** | "
                  f"{r['trl_eager']['alloc_mb']:.0f} / {r['ours']['alloc_mb']:.1f} |")
    md += ["", "Backward (`loss.backward()` of `(logp*g_logp + ent*g_ent + lse*g_lse).sum()`, "
           "the reference's `bench/bench_backward.py` method: events around the backward, "
           "median of 20 after 5), ms:", "",
           "| (B*S, V) | eager autograd | **ours** | speedup |", "|---|---:|---:|---:|"]
    for (BS, V), r in bwd.items():
        md.append(f"| ({BS}, {V}) | {r['eager_autograd']:.3f} | **{r['ours']:.3f}** | "
                  f"**{r['eager_autograd'] / r['ours']:.1f}x** |")
    data = {"kind": "matrix", "build_id": bid,
            "forward": {f"{k[0]}x{k[1]}": v for k, v in rows.items()},
            "backward": {f"{k[0]}x{k[1]}": v for k, v in bwd.items()}}
    md += ["", _profile_line(data), ""]
    with open(out_md, "w") as f:
        f.write("\n".join(md))
    print("\n".join(md))


MATRIX_TRAFFIC_BACKENDS = ("ours_fwd", "ours_bwd", "ours_naive", "trl_eager", "pytorch_separate")


def matrix_run(dev):
    """One call of each backend at MATRIX_TRAFFIC_SHAPE for rocprofv3 --pmc
    (FETCH_SIZE, then WRITE_SIZE): first klp_ceiling_copy over the logits'
    bytes (the counters' calibration), then for backend i a marker,
    klp_ceiling_write over one row of 16 * (i + 1) bytes, and the backend's
    call; a last marker closes the sequence.  Warm-up calls run before the
    first marker."""
    from kernel_opt import _C
    from kernel_opt._library import check_status, lib
    BS, V = MATRIX_TRAFFIC_SHAPE
    x, t = _matrix_inputs(BS, V, dev)
    N = BS
    lp, ent, lse = (torch.empty(N, device=dev) for _ in range(3))
    d = torch.empty(x.shape, dtype=x.dtype, device=dev)
    g = torch.full((N,), 1.0 / N, device=dev)
    mk = torch.empty(4096, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    b = _matrix_backends()
    calls = {
        "ours_fwd": lambda: _C.fwd_launch(x, t, lp, ent, lse),
        "ours_bwd": lambda: _C.bwd_launch(x, t, lse, ent, g, g, None, d),
        "ours_naive": lambda: b["ours_naive"](x, t),
        "trl_eager": lambda: b["trl_eager"](x, t),
        "pytorch_separate": lambda: b["pytorch_separate"](x, t),
    }
    for name in MATRIX_TRAFFIC_BACKENDS:
        calls[name]()
    torch.cuda.synchronize()
    check_status(lib.klp_ceiling_copy(x.data_ptr(), d.data_ptr(), N, V * 2, 8, 2, 16, st))
    for i, name in enumerate(MATRIX_TRAFFIC_BACKENDS):
        check_status(lib.klp_ceiling_write(mk.data_ptr(), 1, 16 * (i + 1), 1, 2, 1, st))
        calls[name]()
    check_status(lib.klp_ceiling_write(mk.data_ptr(), 1, 16 * (len(calls) + 1), 1, 2, 1, st))
    torch.cuda.synchronize()
    print(json.dumps({"matrix_run": MATRIX_TRAFFIC_SHAPE, "backends": MATRIX_TRAFFIC_BACKENDS}))


def summarize_matrix_traffic(fetch_dir, write_dir, command=""):
    """Bytes each backend of matrix_run moves: the FETCH_SIZE and WRITE_SIZE
    of every dispatch between its marker and the next, scaled by the
    calibration copy's known bytes.  Returns (markdown, data)."""
    BS, V = MATRIX_TRAFFIC_SHAPE
    logits_bytes = BS * V * 2
    totals, counts, factor = {}, {}, {}
    for counter, directory in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        recs = [r for r in _rocprof_csv(directory, "counter_collection.csv")
                if r["Counter_Name"] == counter]
        recs.sort(key=lambda r: int(r.get("Dispatch_Id") or r.get("Correlation_Id") or 0))
        cal = [r for r in recs if "klp_ceiling_copy_kernel" in r["Kernel_Name"]]
        if not cal:
            raise RuntimeError("no calibration copy in " + directory)
        factor[counter] = logits_bytes / (1024 * float(cal[-1]["Counter_Value"]))
        start = recs.index(cal[-1]) + 1
        cur = None
        for r in recs[start:]:
            if "klp_ceiling_write_kernel" in r["Kernel_Name"]:
                cur = len([k for k in totals if k[0] == counter])
                cur = MATRIX_TRAFFIC_BACKENDS[cur] if cur < len(MATRIX_TRAFFIC_BACKENDS) else None
                if cur is not None:
                    totals[(counter, cur)] = 0.0
                    counts[(counter, cur)] = 0
                continue
            if cur is not None:
                totals[(counter, cur)] += float(r["Counter_Value"]) * 1024 * factor[counter]
                counts[(counter, cur)] += 1
    rows, data = [], {}
    for name in MATRIX_TRAFFIC_BACKENDS:
        fe, wr = totals[("FETCH_SIZE", name)], totals[("WRITE_SIZE", name)]
        need = 2 * logits_bytes if name == "ours_bwd" else logits_bytes
        data[name] = {"dispatches": counts[("FETCH_SIZE", name)], "read_bytes": int(fe),
                      "write_bytes": int(wr), "required_bytes": need,
                      "amplification": round((fe + wr) / need, 3)}
        rows.append(f"| {name} | {counts[('FETCH_SIZE', name)]} | {need / 1e6:.1f} MB | "
                    f"{(fe + wr) / 1e6:.1f} MB (read {fe / 1e6:.1f}, write {wr / 1e6:.1f}) | "
                    f"**{(fe + wr) / need:.2f}x** |")
    md = [f"# Bytes moved per call, (B*S, V) = ({BS}, {V}) bf16, one MI355X", "",
          "rocprofv3 FETCH_SIZE and WRITE_SIZE of every dispatch of each backend "
          "(`bench.py --matrix-run`, dispatches grouped between marker launches), scaled by "
          f"the counters' reading for a copy of known size (FETCH x{factor['FETCH_SIZE']:.5f}, "
          f"WRITE x{factor['WRITE_SIZE']:.5f}); summarised by `python bench.py "
          f"--matrix-traffic-from {fetch_dir} {write_dir}`. The reference's table: "
          "`REPORT.md:157-177` (RTX 4060, ncu).", ""]
    if command:
        md += ["Commands (MI355X):", "```", command, "```", ""]
    md += ["| backend | dispatches | bytes required | bytes moved | amplification |",
           "|---|---:|---:|---:|---:|"] + rows
    data = {"kind": "matrix_traffic", "build_id": build_id(), "backends": data}
    md += ["", _profile_line(data), ""]
    return "\n".join(md), data


def _rng(vals, nd):
    """'a' or 'a–b' (min–max) of the non-None values, nd decimals."""
    v = [x for x in vals if x is not None]
    if not v:
        return "—"
    lo, hi = min(v), max(v)
    return f"{lo:.{nd}f}" if round(lo, nd) == round(hi, nd) else f"{lo:.{nd}f}–{hi:.{nd}f}"


def configs_table(paths, command=""):
    """Markdown table of C1-C5 from bench.py output lines (the default
    command's: the C2 headline, its C1 leg and its C3-C5 `configs` legs),
    one range per cell over the files given."""
    runs = []
    for path in paths:
        with open(path) as f:
            lines = [ln for ln in f.read().splitlines() if ln.strip().startswith("{")]
        runs.append(json.loads(lines[-1]))
    bids = sorted({r.get("build_id") for r in runs})
    per = {c: [] for c in ("C1", "C2", "C3", "C4", "C5")}
    for r in runs:
        c = r["ceilings"]
        per["C2"].append({
            "fwd": r["fwd_ms"] * 1e3, "fwd_fl": r["fwd_ms_flushed"] * 1e3,
            "fwd_pct": r["fwd_pct_peak"], "fwd_pct_fl": r["fwd_pct_peak_flushed"],
            "f_read": c["fwd_over_read"], "f_read_fl": c.get("fwd_over_read_flushed"),
            "bwd": r["bwd_ms"] * 1e3, "bwd_fl": r["bwd_ms_flushed"] * 1e3,
            "bwd_pct": r["bwd_pct_peak"], "bwd_pct_fl": r["bwd_pct_peak_flushed"],
            "b_copy": c["bwd_over_copy"], "b_rw": c.get("bwd_over_read_plus_write"),
            "b_rw_fl": c.get("bwd_over_read_plus_write_flushed"),
            "step": r["ms_per_step"] * 1e3})
        for name, leg in (r.get("configs") or {}).items():
            lc = leg["ceilings"]
            per[name].append({
                "fwd": leg["fwd_us"], "fwd_fl": leg["fwd_us_flushed"],
                "fwd_pct": leg["fwd_pct_peak"], "fwd_pct_fl": leg["fwd_pct_peak_flushed"],
                "f_read": lc["fwd_over_read"], "f_read_fl": lc.get("fwd_over_read_flushed"),
                "bwd": leg["bwd_us"], "bwd_fl": leg["bwd_us_flushed"],
                "bwd_pct": leg["bwd_pct_peak"], "bwd_pct_fl": leg["bwd_pct_peak_flushed"],
                "b_copy": lc["bwd_over_copy"], "b_rw": lc.get("bwd_over_read_plus_write"),
                "b_rw_fl": lc.get("bwd_over_read_plus_write_flushed"), "step": leg["step_us"]})
        c1 = r.get("C1")
        if c1:
            B, S, V = CONFIGS["C1"]["shape"]
            fb = B * S * V * 4 + 20 * B * S
            per["C1"].append({
                "fwd": c1["fwd_us"], "fwd_pct": c1["fwd_tbps"] / 8 * 100,
                "bwd": c1["bwd_us"], "bwd_pct": c1["bwd_tbps"] / 8 * 100,
                "step": None, "fwd_bytes": fb})
    lines = [
        "# Forward / backward at C1–C5 with same-run ceilings (bench.py)", "",
        f"{len(runs)} run(s) of `python bench.py` (the driver's command) on one MI355X each, "
        f"build {', '.join(f'`{b}`' for b in bids)}; each cell is the range over the runs. "
        "C2 is the line's headline, C1 its `C1` leg, C3–C5 its `configs` legs.", "",
        "Warm: launches queued back to back behind a spin kernel (HIP events). Flushed: each "
        "launch's own device duration right after a 1 GiB read (torch.profiler, median of "
        "24). Ceilings, same run, same launch shapes: the forward's ring of loads without "
        "arithmetic (read), the backward's loop as a copy, and that loop's loads alone plus "
        "its stores alone (read-only + write-only). % of 8 TB/s of algorithmic bytes.", ""]
    if command:
        lines += ["Command:", "```", command, "```", ""]
    lines += [
        "| config | fwd µs warm / flushed | fwd % warm / flushed | fwd / read warm, flushed "
        "| bwd µs warm / flushed | bwd % warm / flushed | bwd / copy "
        "| bwd / (read-only + write-only) warm, flushed | step µs |",
        "|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    label = {"C1": "C1 fp32 [2,128,32000]", "C2": "C2 bf16 [4,256,152064]",
             "C3": "C3 fp16 [8,1024,128256]", "C4": "C4 bf16 [16,2048,151936]",
             "C5": "C5 fp32 [4,2048,262144], strided"}
    for name in ("C1", "C2", "C3", "C4", "C5"):
        rs = per[name]
        if not rs:
            continue
        g = lambda k: [x.get(k) for x in rs]  # noqa: E731
        lines.append(
            f"| {label[name]} | {_rng(g('fwd'), 2)} / {_rng(g('fwd_fl'), 2)} "
            f"| {_rng(g('fwd_pct'), 1)} / {_rng(g('fwd_pct_fl'), 1)} "
            f"| {_rng(g('f_read'), 3)}, {_rng(g('f_read_fl'), 3)} "
            f"| {_rng(g('bwd'), 2)} / {_rng(g('bwd_fl'), 2)} "
            f"| {_rng(g('bwd_pct'), 1)} / {_rng(g('bwd_pct_fl'), 1)} "
            f"| {_rng(g('b_copy'), 3)} | {_rng(g('b_rw'), 3)}, {_rng(g('b_rw_fl'), 3)} "
            f"| {_rng(g('step'), 1)} |")
    lines += ["", "C1's figures are GPU time per launch with launches queued (the C1 leg); "
              "at 33 MB it is launch-latency bound and Infinity-Cache resident, and the "
              "leg times no ceilings or flushed launches."]
    return "\n".join(lines) + "\n"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="C2", choices=sorted(CONFIGS))
    ap.add_argument("--flush-mode", choices=("read", "write"), default="read",
                    help="read: sum a 1 GiB buffer before each flushed launch (evicts with "
                         "clean lines); write: fill it (leaves up to the cache size of dirty "
                         "lines for the next kernel)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=1024,
                    help="rows of the workload the CPU baseline times (whole batch elements)")
    ap.add_argument("--fwd-config", default=None, help="waves,unroll,splits,flags")
    ap.add_argument("--bwd-config", default=None, help="waves,unroll,splits,flags")
    ap.add_argument("--core-only", action="store_true",
                    help="only the workload's forward / backward timings and ceilings (for "
                         "profiler runs)")
    ap.add_argument("--no-lmhead", action="store_true",
                    help="skip the fused LM-head timing (klp_lmh_* against matmul + logprob)")
    ap.add_argument("--no-shard", action="store_true",
                    help="skip the vocab-shard timing (one rank's share of C4 under 8-way "
                         "vocab parallelism)")
    ap.add_argument("--no-grpo", action="store_true",
                    help="skip the GRPO timings (the loss kernels against the eager chain, "
                         "the fused step against the unfused kernels)")
    ap.add_argument("--sweep", metavar="OUT_MD", default=None,
                    help="time a grid of launch shapes of the forward and backward and write "
                         "the table to OUT_MD (nothing else runs)")
    ap.add_argument("--trace-from", metavar="DIR", default=None,
                    help="summarise a rocprofv3 --kernel-trace output directory (markdown to "
                         "stdout; no GPU needed)")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"), default=None,
                    help="summarise two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) into HBM "
                         "bytes per launch (markdown to stdout; no GPU needed)")
    ap.add_argument("--command", default="",
                    help="the profiling command, quoted in the --trace-from / --traffic-from "
                         "summary")
    ap.add_argument("--no-device-timer", action="store_true",
                    help="time flushed launches with HIP events instead of the device's "
                         "timestamps through torch.profiler (for runs under rocprofv3)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-config legs (C3, C4, C5 beside the headline C2)")
    ap.add_argument("--matrix", metavar="OUT_MD", default=None,
                    help="the reference's comparison matrix (forward backends over its six "
                         "shapes, backward against eager autograd) into OUT_MD")
    ap.add_argument("--matrix-run", action="store_true",
                    help="one call of each matrix backend between markers, for rocprofv3 "
                         "--pmc runs")
    ap.add_argument("--matrix-traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    default=None, help="bytes moved per backend from two rocprofv3 --pmc runs "
                                       "of --matrix-run (markdown to stdout; no GPU needed)")
    ap.add_argument("--counters-from", metavar="DIR", default=None,
                    help="summarise any rocprofv3 --pmc run's counters per klp kernel "
                         "(markdown to stdout; no GPU needed)")
    ap.add_argument("--configs-table", nargs="+", metavar="BENCH_JSON", default=None,
                    help="C1-C5 table (markdown to stdout) from the output lines of one or "
                         "more default bench.py runs; no GPU needed")
    ap.add_argument("--label", default=None,
                    help="tag of a --trace-from summary other than the config name (a run "
                         "that is not --core-only)")
    args = ap.parse_args(argv)

    if args.trace_from:
        md, _ = summarize_trace(args.trace_from, args.config, args.command, args.label)
        print(md)
        return 0
    if args.traffic_from:
        md, _ = summarize_traffic(*args.traffic_from, args.config, args.command)
        print(md)
        return 0
    if args.matrix_traffic_from:
        md, _ = summarize_matrix_traffic(*args.matrix_traffic_from, args.command)
        print(md)
        return 0
    if args.counters_from:
        md, _ = summarize_counters(args.counters_from, args.config, args.command)
        print(md, end="")
        return 0
    if args.configs_table:
        print(configs_table(args.configs_table, args.command), end="")
        return 0

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(rows are independent, so data-parallel ranks would each run this same "
              "kernel on their own batch with no exchange)", file=sys.stderr)
        return 2

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    name = args.config
    cfg = CONFIGS[name]
    K = args.steps
    timer = Timer(dev, K, args.flush_mode)
    if args.sweep:
        sweep(name, dev, K, timer, args.sweep,
              DeviceTimer(timer, enabled=not args.no_device_timer))
        return 0
    if args.matrix:
        matrix(dev, args.matrix, DeviceTimer(timer, enabled=not args.no_device_timer))
        return 0
    if args.matrix_run:
        matrix_run(dev)
        return 0

    fcfg = tuple(int(v) for v in args.fwd_config.split(",")) if args.fwd_config else None
    bcfg = tuple(int(v) for v in args.bwd_config.split(",")) if args.bwd_config else None
    dtimer = DeviceTimer(timer, enabled=not args.no_device_timer)
    core = core_timing(name, dev, K, args.warmup, timer, fcfg, bcfg, dtimer)
    N, V, fb, bb = core["N"], core["V"], core["fb"], core["bb"]
    step_ms, fwd_ms, bwd_ms = core["step_ms"], core["fwd_ms"], core["bwd_ms"]
    fwd_fl, bwd_fl = core["fwd_fl"], core["bwd_fl"]
    logits, targets = core["logits"], core["targets"]
    del core["d_logits"]

    extra = not args.core_only
    autograd = (autograd_timing(dev, K, logits, targets, core["g_logp"], core["g_ent"])
                if extra else None)
    c1 = c1_leg(dev, K, timer, not args.no_cpu_baseline) if extra and name != "C1" else None
    small = small_batch_leg(dev, timer) if extra else None

    cpu = None
    if extra and not args.no_cpu_baseline:
        c = cpu_baseline(name, args.cpu_rows, logits, targets, core["g_logp"], core["g_ent"])
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
        if c1 is not None and "cpu_fwd_bwd_ms" in c1:
            cpu["C1"] = {"fwd_ms": c1["cpu_fwd_ms"], "fwd_bwd_ms": c1["cpu_fwd_bwd_ms"],
                         "cores": c1["cpu_threads"]}

    per_config = None
    if extra and not args.no_configs and name == "C2":
        per_config = config_legs(("C3", "C4", "C5"), dev, K, args.warmup, timer, dtimer)

    grpo = step = lmhead = shard = None
    if extra:
        grpo = None if args.no_grpo else grpo_timing(dev, K)
        step = None if args.no_grpo else grpo_step_timing(dev, K, logits, targets)
        lmhead = None if args.no_lmhead else lmhead_timing(dev)
        shard = None if args.no_shard else shard_timing(dev, K)

    B, S, _ = cfg["shape"]
    fwd_tbps, bwd_tbps = _tbps(fb, fwd_ms), _tbps(bb, bwd_ms)
    fwd_fl_tbps, bwd_fl_tbps = _tbps(fb, fwd_fl), _tbps(bb, bwd_fl)
    step_tbps = _tbps(fb + bb, step_ms)
    bid = build_id()
    # The dominant kernel at the lower of its warm and flushed rates.
    warm_is_lower = bwd_tbps <= bwd_fl_tbps
    bwd_rate = bwd_tbps if warm_is_lower else bwd_fl_tbps
    bwd_short = None
    traffic = fwd_traffic = None
    traffic_src = None
    for prof in load_profiles("traffic", name, bid):
        for k, v in prof["kernels"].items():
            if k.startswith("klp_bwd_kernel"):
                traffic, bwd_short = v["traffic_bytes"], k
            elif k.startswith("klp_fwd_kernel"):
                fwd_traffic = v["traffic_bytes"]
        traffic_src = prof["file"]
    trace_check = trace_agreement(load_profiles("trace", name, bid), core.get("device_timed"))
    dt = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[logits.dtype]
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
        "dtype": dt,
        "data": "synthetic",
        "config": {"workload": f"{name}: logits [{B},{S},{V}] "
                               f"{str(logits.dtype).replace('torch.', '')}, one forward + one "
                               f"backward launch per step",
                   "global_batch": B, "seq_len": S, "vocab": V, "n_rows": N,
                   "parallelism": "single-gpu",
                   "infinity_cache": "warm for ms_per_step / value / fwd_ms / bwd_ms; "
                                     "*_flushed after a 1 GiB read before each launch"},
        "build_id": bid,
        "fwd_ms": round(fwd_ms, 5),
        "bwd_ms": round(bwd_ms, 5),
        "fwd_ms_flushed": round(fwd_fl, 5),
        "bwd_ms_flushed": round(bwd_fl, 5),
        "device_timed": _device_summary(core["device_timed"]),
        "fwd_tbps": round(fwd_tbps, 4),
        "bwd_tbps": round(bwd_tbps, 4),
        "fwd_pct_peak": round(100 * fwd_tbps / HBM_PEAK_TBPS, 2),
        "bwd_pct_peak": round(100 * bwd_tbps / HBM_PEAK_TBPS, 2),
        "fwd_pct_peak_flushed": round(100 * fwd_fl_tbps / HBM_PEAK_TBPS, 2),
        "bwd_pct_peak_flushed": round(100 * bwd_fl_tbps / HBM_PEAK_TBPS, 2),
        "step_tbps_flushed": round(_tbps(fb + bb, fwd_fl + bwd_fl), 4),
        "fwd_launch": dict(zip(("waves", "unroll", "splits", "flags"), core["fwd_used"])),
        "bwd_launch": dict(zip(("waves", "unroll", "splits", "flags"), core["bwd_used"])),
        "ceilings": core["ceilings"],
        "wall_s_timed": round(core["wall"], 4),
        "roofline": {
            "bound": "hbm",
            "kernel": bwd_short or "klp_bwd_kernel",
            "achieved": round(bwd_rate * 1000, 1),
            "peak": HBM_PEAK_TBPS * 1000,
            "unit": "GB/s",
            "frac": round(bwd_rate / HBM_PEAK_TBPS, 4),
            "timing": ("back to back, warm (lower than flushed)" if warm_is_lower
                       else "flushed per launch (lower than back to back, warm)"),
            "traffic": traffic,
            "algorithmic_bytes": bb,
            "fwd_traffic": fwd_traffic,
            "fwd_algorithmic_bytes": fb,
            "traffic_source": traffic_src or f"no counter summary of build {bid} under profiles/",
            "trace_check": trace_check,
        },
        "autograd": autograd,
        "C1": c1,
        "configs": per_config,
        "small_batch": small,
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
