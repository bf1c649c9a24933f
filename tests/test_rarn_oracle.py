"""CPU: the reduce-add RMSNorm oracle (reax_rarn, libreax_howu/reax_rarn_final.cu) against its pins, and each
planted mistake caught by at least one pin (a flat sum-of-squares order, w in place of 1 + w, and d not rounded to
bf16 before the residual)."""
import pytest

import pyoracle
import rarn_cases as RC


@pytest.mark.parametrize("pin", RC.ALL_PINS, ids=lambda f: f.__name__)
def test_pin(pin):
    pin()


@pytest.mark.parametrize("mutant", sorted(pyoracle.RARN_MUTANTS))
def test_mutant_is_caught(mutant):
    failed = []
    for pin in RC.ALL_PINS:
        try:
            pin(mutant=mutant)
        except AssertionError as e:
            failed.append(f"{pin.__name__}: {str(e)[:60]}")
    assert failed, f"mutant {mutant} passed every pin"
