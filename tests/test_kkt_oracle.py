"""CPU: the chunk-solve oracle (reax_kkt, libreax_howu/reax_kkt.cu) against its pins, and each planted mistake
caught by at least one pin (decay direction, the column's beta, the diagonal inside M, the sign of A)."""
import pytest

import kkt_cases as KC
import pyoracle


@pytest.mark.parametrize("pin", KC.ALL_PINS, ids=lambda f: f.__name__)
def test_pin(pin):
    pin()


@pytest.mark.parametrize("mutant", sorted(pyoracle.KKT_MUTANTS))
def test_mutant_is_caught(mutant):
    failed = []
    for pin in KC.ALL_PINS:
        try:
            pin(mutant=mutant)
        except AssertionError as e:
            failed.append(f"{pin.__name__}: {str(e)[:60]}")
    assert failed, f"mutant {mutant} passed every pin"
