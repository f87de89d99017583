"""The float64 oracle against independent checks (tests/oracle_pins.py):
brute force, closed forms, invariants, finite differences, the explicit
softmax Jacobian and numpy/torch conversions.  CPU only."""
import pytest

import oracle_pins


@pytest.mark.parametrize("pin", oracle_pins.ALL_PINS, ids=lambda p: p.__name__)
def test_oracle_pin(pin, oracle):
    msg = pin(oracle)
    assert msg is None, msg
