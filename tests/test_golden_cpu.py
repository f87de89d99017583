"""The oracle against the committed known-answer fixtures
(tests/golden/klp_golden.npz, written by tests/golden/make_golden.py from
independent numpy two-pass float64 formulas).  CPU only."""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "klp_golden.npz")


def load_cases():
    z = np.load(GOLDEN, allow_pickle=False)
    out = {}
    for name in z["cases"]:
        name = str(name)
        out[name] = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(name + "/")}
    return out


CASES = load_cases()


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_golden(name, oracle):
    c = CASES[name]
    dtype = str(c["dtype"])
    lp, h, l = oracle.forward(c["logits_bits"], c["targets"], dtype=dtype)
    for got, exp, nm in ((lp, c["logp"], "logp"), (h, c["entropy"], "entropy"), (l, c["lse"], "lse")):
        assert np.allclose(got, exp, rtol=1e-12, atol=1e-12), nm
    d = oracle.backward(c["logits_bits"], c["targets"], c["lse32"], c["ent32"],
                        g_logp=c["g_logp"], g_ent=c["g_ent"], g_lse=c["g_lse"], dtype=dtype)
    scale = np.abs(c["d"]).max()
    assert np.abs(d - c["d"]).max() <= 1e-13 * scale


def test_golden_covers_the_edge_cases():
    assert {str(c["dtype"]) for c in CASES.values()} == {"fp32", "bf16", "fp16"}
    assert any(np.isneginf(c["logits_bits"].view(np.float32) if str(c["dtype"]) == "fp32"
                           else np.zeros(1)).any() or str(c["dtype"]) != "fp32"
               for c in CASES.values())
    assert (CASES["fp32_randn"]["targets"] < 0).any()  # an ignore-index target
