"""CPU pins of the float64 LM-head oracle (oracle/lmh_oracle.py)."""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import lmh_oracle


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).view(torch.int16) \
        .numpy().view(np.uint16)


def test_matches_c_oracle_on_exact_integer_logits(oracle):
    """Small-integer hidden / weight: every logit is an integer below 2^24,
    exact in fp32, so the C oracle of the logprob forward sees the same
    logits and must agree to float64 rounding."""
    g = np.random.default_rng(1)
    N, V, D = 9, 777, 64
    h = bf16_bits(g.integers(-3, 4, (N, D)))
    w = bf16_bits(g.integers(-2, 3, (V, D)))
    t = g.integers(-2, V + 2, N)
    lp, ent, lse = lmh_oracle.forward(h, w, t)
    x = lmh_oracle.logits(h, w).astype(np.float32)
    assert np.array_equal(x.astype(np.float64), lmh_oracle.logits(h, w))
    r_lp, r_ent, r_lse = oracle.forward(x, t, dtype="fp32")
    np.testing.assert_allclose(lp, r_lp, rtol=0, atol=1e-12)
    np.testing.assert_allclose(ent, r_ent, rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, r_lse, rtol=0, atol=1e-12)


def test_matches_python_loop():
    g = np.random.default_rng(2)
    N, V, D = 3, 7, 64
    h = bf16_bits(g.normal(0, 1, (N, D)))
    w = bf16_bits(g.normal(0, 0.3, (V, D)))
    t = np.array([0, 6, 3])
    lp, ent, lse = lmh_oracle.forward(h, w, t, temperature=0.7)
    hf, wf = lmh_oracle.bf16_to_f64(h), lmh_oracle.bf16_to_f64(w)
    s = float(np.float32(1 / 0.7))
    for n in range(N):
        xs = [math.fsum(hf[n, k] * wf[v, k] for k in range(D)) * s for v in range(V)]
        m = max(xs)
        z = math.fsum(math.exp(x - m) for x in xs)
        l = m + math.log(z)
        e = l - math.fsum(math.exp(x - l) * x for x in xs)
        assert abs(lse[n] - l) < 1e-12 and abs(ent[n] - e) < 1e-12
        assert abs(lp[n] - (xs[t[n]] - l)) < 1e-12


def test_uniform_rows_closed_form():
    g = np.random.default_rng(3)
    N, V, D = 4, 1000, 128
    h = bf16_bits(g.normal(0, 1, (N, D)))
    w = np.tile(bf16_bits(g.normal(0, 0.1, (1, D))), (V, 1))
    lp, ent, lse = lmh_oracle.forward(h, w, np.zeros(N, np.int64))
    np.testing.assert_allclose(ent, math.log(V), rtol=0, atol=1e-12)
    np.testing.assert_allclose(lp, -math.log(V), rtol=0, atol=1e-12)


def test_out_of_range_targets_give_minus_lse():
    g = np.random.default_rng(4)
    h = bf16_bits(g.normal(0, 1, (3, 64)))
    w = bf16_bits(g.normal(0, 0.2, (50, 64)))
    lp, _, lse = lmh_oracle.forward(h, w, np.array([-100, 50, 1000]))
    np.testing.assert_array_equal(lp, -lse)


def test_backward_matches_float64_autograd():
    g = np.random.default_rng(5)
    N, V, D = 6, 40, 64
    h = bf16_bits(g.normal(0, 1, (N, D)))
    w = bf16_bits(g.normal(0, 0.3, (V, D)))
    t = np.array([0, 39, 5, -100, 17, 40])
    gl, ge, gs = (g.normal(0, 1, N) for _ in range(3))
    T = 0.8
    dh, dw, _ = lmh_oracle.backward(h, w, t, gl, ge, gs, temperature=T)
    H = torch.tensor(lmh_oracle.bf16_to_f64(h), requires_grad=True)
    W = torch.tensor(lmh_oracle.bf16_to_f64(w), requires_grad=True)
    x = (H @ W.T) * lmh_oracle.scale_of(T)
    lsm = torch.log_softmax(x, dim=-1)
    tt = torch.tensor(t)
    valid = (tt >= 0) & (tt < V)
    xt = torch.where(valid, x.gather(1, tt.clamp(0, V - 1)[:, None])[:, 0], torch.zeros(N,
                                                                                 dtype=x.dtype))
    lse = torch.logsumexp(x, dim=-1)
    logp = xt - lse
    ent = -(lsm.exp() * lsm).sum(-1)
    loss = (logp * torch.tensor(gl)).sum() + (ent * torch.tensor(ge)).sum() \
        + (lse * torch.tensor(gs)).sum()
    loss.backward()
    np.testing.assert_allclose(dh, H.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, W.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_vocab_chunk_plan():
    """The chunked head's vocabulary plan (host logic): chunks cover the
    vocabulary in order without gaps; small batches take 32768-column chunks
    with a remainder of at least 16384 + 1024 columns cut into 16384 + the
    rest; larger batches take balanced chunks of a multiple of 1024 columns
    within 128 MiB; an explicit width gives equal chunks and no cut."""
    from kernel_opt import vocab_chunk, vocab_chunks

    def check_cover(plan, V):
        c = 0
        for c0, n in plan:
            assert c0 == c and n >= 1
            c += n
        assert c == V

    qwen = vocab_chunks(1024, 152064)
    check_cover(qwen, 152064)
    assert [n for _, n in qwen] == [32768] * 4 + [16384, 4608]
    assert [n for _, n in vocab_chunks(300, 152064)] == [32768] * 4 + [16384, 4608]
    # a remainder below 16384 + 1024 stays whole; 16384 + 1024 is cut
    assert [n for _, n in vocab_chunks(1024, 32768 + 17407)] == [32768, 17407]
    assert [n for _, n in vocab_chunks(1024, 32768 + 17408)] == [32768, 16384, 1024]
    assert [n for _, n in vocab_chunks(1024, 20000)] == [16384, 3616]
    assert [n for _, n in vocab_chunks(1024, 32768)] == [32768]
    assert [n for _, n in vocab_chunks(5, 300)] == [300]
    # larger batches: balanced, whole multiples of 1024 but the last, <= 128 MiB
    for N, V in ((2048, 152064), (8192, 152064), (4096, 151936), (32768, 262144)):
        plan = vocab_chunks(N, V)
        check_cover(plan, V)
        widths = [n for _, n in plan]
        assert all(w == widths[0] for w in widths[:-1]) and widths[-1] <= widths[0]
        assert widths[0] % 1024 == 0 and N * widths[0] * 2 <= 128 << 20
        assert widths[0] == vocab_chunk(N, V)
    # an explicit width: equal chunks, the last the rest, never cut
    assert [n for _, n in vocab_chunks(1024, 152064, chunk_vocab=20000)] == [20000] * 7 + [12064]
    assert [n for _, n in vocab_chunks(1024, 100, chunk_vocab=1000)] == [100]
    # fp32 halves the columns that fit the small-batch rule
    assert vocab_chunk(1024, 152064, elem_bytes=4) != 32768
