"""The oracle pins have teeth: oracle/klp_oracle.c rebuilt with each planted
mistake (-DKLP_MUTANT=k: swapped scale factors, a dropped term, a wrong sign,
an off-by-one target index, truncating rounding, ...) must fail at least one
pin.  Mistakes are planted in the oracle on the CPU only."""
import os
import re

import pytest

import oracle_pins
from conftest import ROOT

MUTANTS = sorted({int(m) for m in re.findall(r"KLP_MUTANT == (\d+)",
                                              open(os.path.join(ROOT, "oracle", "klp_oracle.c")).read())})


def test_mutants_exist():
    assert len(MUTANTS) >= 8


@pytest.mark.parametrize("mutant", MUTANTS)
def test_mutant_is_caught(mutant, tmp_path):
    from oracle import klp_oracle
    path = klp_oracle.build(mutant=mutant, build_dir=str(tmp_path))
    o = klp_oracle.Oracle(path=path)
    caught = []
    for pin in oracle_pins.ALL_PINS:
        try:
            msg = pin(o)
        except Exception as e:  # a crash of a check counts as a catch
            msg = f"raised {type(e).__name__}: {e}"
        if msg is not None:
            caught.append(pin.__name__)
    print(f"mutant {mutant} caught by {caught}")
    assert caught, f"mutant {mutant} passed every pin"
