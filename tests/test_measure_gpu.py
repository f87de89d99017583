"""GPU tests of what bench.py measures with:

* the calibration kernels (klp_ceiling_copy: a bitwise copy of every row
  piece; klp_ceiling_read and klp_ceiling_read_pieces: every 16-byte word of
  every piece reaches its thread's xor fold, pinned by choosing `magic` as
  one thread's fold computed on the host, so that exactly that workgroup
  writes its sink word; klp_ceiling_write: every vector of every row holds
  its index and nothing past the rows is written);
* the drop-in path's allocations at C2 (the reference publishes 0.0 MB of
  intermediates for the forward, notes/stage2_findings.md:30-38, and the
  north star asks for a backward with zero intermediate allocations):
  the forward allocates exactly its three outputs; the backward holds the
  gradient and allocates nothing transient but the loss's own per-row
  gradient tensors.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lib():
    from kernel_opt._library import check_status, lib
    return lib, check_status


@pytest.mark.parametrize("n_rows,row_bytes,waves,unroll,splits", [
    (7, 304128, 4, 2, 38),      # C2 rows, the backward's default shape
    (7, 304128, 16, 2, 8),
    (5, 4096, 4, 4, 3),         # pieces that are not whole 8-vector groups
    (3, 16 * 1000 + 16, 8, 2, 16),
    (2, 16, 1, 2, 1),           # one vector per row
])
def test_ceiling_copy_is_exact(n_rows, row_bytes, waves, unroll, splits):
    lib, check = _lib()
    print(f"ceiling copy {n_rows}x{row_bytes} w{waves} u{unroll} s{splits}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(n_rows * 31 + row_bytes)
    src = torch.randint(0, 256, (n_rows * row_bytes,), dtype=torch.uint8, generator=g,
                        device=DEV)
    # one spare row after dst: it must stay untouched
    dst = torch.full((n_rows * row_bytes + row_bytes,), 0xA5, dtype=torch.uint8, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    check(lib.klp_ceiling_copy(src.data_ptr(), dst.data_ptr(), n_rows, row_bytes, waves,
                               unroll, splits, st))
    torch.cuda.synchronize()
    assert torch.equal(dst[:n_rows * row_bytes], src)
    assert torch.all(dst[n_rows * row_bytes:] == 0xA5)


def _thread_folds(words, n_rows, row_bytes, waves, splits, round8=False):
    """Host model of klp_ceiling_read (and, with round8, of
    klp_ceiling_read_pieces, whose pieces are rounded up to 8 vectors): fold
    of every (workgroup, thread): thread tid of a piece [vb, ve) xors the
    vectors j with (j - vb) % NT == tid, then folds its four 32-bit lanes."""
    NT = waves * 64
    nvec = row_bytes // 16
    per = -(-nvec // splits)
    if round8:
        per = -(-per // 8) * 8
    v = words.reshape(n_rows, nvec, 4)
    folds = {}
    for r in range(n_rows):
        for s in range(splits):
            vb, ve = min(s * per, nvec), min(s * per + per, nvec)
            acc = np.zeros((NT, 4), dtype=np.uint32)
            for j in range(vb, ve):
                acc[(j - vb) % NT] ^= v[r, j]
            folds[r * splits + s] = np.bitwise_xor.reduce(acc, axis=1)
    return folds


@pytest.mark.parametrize("n_rows,row_bytes,waves,unroll,splits", [
    (4, 304128, 4, 4, 1),       # C2 rows, the forward's default shape
    (6, 4096 + 16 * 7, 4, 2, 2),
    (3, 16 * 300, 1, 4, 5),
])
def test_ceiling_read_reads_every_word(n_rows, row_bytes, waves, unroll, splits):
    lib, check = _lib()
    print(f"ceiling read {n_rows}x{row_bytes} w{waves} u{unroll} s{splits}", flush=True)
    rng = np.random.default_rng(row_bytes + splits)
    words = rng.integers(0, 2 ** 32, size=n_rows * row_bytes // 4, dtype=np.uint32)
    folds = _thread_folds(words, n_rows, row_bytes, waves, splits)
    wg = len(folds) // 2
    magic = int(folds[wg][5])
    hits = {b for b, f in folds.items() if np.any(f == magic)}
    assert hits == {wg}, "the chosen fold also occurs elsewhere; pick another seed"
    src = torch.from_numpy(words.view(np.int32)).to(DEV)
    sink = torch.zeros(n_rows * splits, dtype=torch.int32, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    check(lib.klp_ceiling_read(src.data_ptr(), n_rows, row_bytes, waves, unroll, splits,
                               sink.data_ptr(), magic, st))
    torch.cuda.synchronize()
    got = sink.cpu().numpy().view(np.uint32)
    want = np.zeros(n_rows * splits, dtype=np.uint32)
    want[wg] = magic
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n_rows,row_bytes,waves,unroll,splits", [
    (4, 304128, 4, 2, 38),      # C2 rows, the backward's default shape
    (4, 304128, 8, 2, 16),
    (5, 4096 + 16 * 7, 4, 4, 3),
    (3, 16 * 300, 1, 2, 5),
])
def test_ceiling_read_pieces_reads_every_word(n_rows, row_bytes, waves, unroll, splits):
    lib, check = _lib()
    print(f"ceiling read pieces {n_rows}x{row_bytes} w{waves} u{unroll} s{splits}", flush=True)
    rng = np.random.default_rng(row_bytes + 3 * splits)
    words = rng.integers(0, 2 ** 32, size=n_rows * row_bytes // 4, dtype=np.uint32)
    folds = _thread_folds(words, n_rows, row_bytes, waves, splits, round8=True)
    wg = len(folds) // 2 + 1
    magic = int(folds[wg][3])
    hits = {b for b, f in folds.items() if np.any(f == magic)}
    assert hits == {wg}, "the chosen fold also occurs elsewhere; pick another seed"
    src = torch.from_numpy(words.view(np.int32)).to(DEV)
    sink = torch.zeros(n_rows * splits, dtype=torch.int32, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    check(lib.klp_ceiling_read_pieces(src.data_ptr(), n_rows, row_bytes, waves, unroll, splits,
                                      sink.data_ptr(), magic, st))
    torch.cuda.synchronize()
    got = sink.cpu().numpy().view(np.uint32)
    want = np.zeros(n_rows * splits, dtype=np.uint32)
    want[wg] = magic
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n_rows,row_bytes,waves,unroll,splits", [
    (7, 304128, 4, 2, 38),      # C2 rows, the backward's default shape
    (7, 304128, 8, 2, 16),
    (5, 4096, 4, 4, 3),
    (2, 16, 1, 2, 1),
])
def test_ceiling_write_writes_every_vector(n_rows, row_bytes, waves, unroll, splits):
    lib, check = _lib()
    print(f"ceiling write {n_rows}x{row_bytes} w{waves} u{unroll} s{splits}", flush=True)
    dst = torch.full((n_rows * row_bytes + row_bytes,), 0xA5, dtype=torch.uint8, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    check(lib.klp_ceiling_write(dst.data_ptr(), n_rows, row_bytes, waves, unroll, splits, st))
    torch.cuda.synchronize()
    got = dst[:n_rows * row_bytes].cpu().numpy().view(np.uint32).reshape(n_rows, -1, 4)
    idx = np.arange(row_bytes // 16, dtype=np.uint32)
    assert np.array_equal(got, np.broadcast_to(idx[None, :, None], got.shape))
    assert torch.all(dst[n_rows * row_bytes:] == 0xA5)


def test_c2_autograd_path_allocates_no_intermediates():
    """C2 through kernel_opt.fused_logprob_entropy and loss.backward(): the
    forward's peak allocation is its three fp32 outputs, nothing transient;
    the backward's transient allocations are the loss's per-row gradient
    tensors (a few KiB, far below one row of logits), nothing [N, V]-sized."""
    import bench
    inp = bench.make_inputs("C2", DEV)
    r = bench.autograd_timing(torch.device(DEV), 3, inp["logits"], inp["targets"],
                              inp["g_logp"].contiguous(), inp["g_ent"].contiguous())
    print({k: v for k, v in r.items() if k.endswith("bytes")}, flush=True)
    N = inp["targets"].numel()
    assert r["fwd_output_bytes"] == 3 * N * 4
    assert r["fwd_peak_bytes"] == r["fwd_output_bytes"]
    assert r["fwd_transient_bytes"] == 0
    assert r["bwd_grad_bytes"] == inp["logits"].numel() * 2
    # what stays allocated is the gradient's block (the caching allocator
    # may round it up to its 2 MiB segment granularity) ...
    assert 0 <= r["bwd_held_bytes"] - r["bwd_grad_bytes"] < 2 * 1024 * 1024
    # ... and nothing else was allocated on the way but the loss's per-row
    # gradients (8 KiB at C2, below one 304 KB row of logits)
    assert r["bwd_transient_bytes"] <= 64 * 1024
