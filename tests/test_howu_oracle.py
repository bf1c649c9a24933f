"""CPU: the GDN chunked-forward oracle (reax_howu, libreax_howu/reax_howu.cu) against the token-by-token gated delta
rule and its other pins, and each planted mistake caught (an undecayed inter-chunk term, a strict causal mask, an
undecayed carried state, vdec without its decay)."""
import pytest

import howu_cases as HC
import pyoracle


@pytest.mark.parametrize("pin", HC.ALL_PINS, ids=lambda f: f.__name__)
def test_pin(pin):
    pin()


@pytest.mark.parametrize("mutant", sorted(pyoracle.HOWU_MUTANTS))
def test_mutant_is_caught(mutant):
    failed = []
    for pin in HC.ALL_PINS:
        try:
            pin(mutant=mutant)
        except AssertionError as e:
            failed.append(f"{pin.__name__}: {str(e)[:60]}")
    assert failed, f"mutant {mutant} passed every pin"
