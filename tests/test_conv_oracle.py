"""CPU: the conv + SiLU + L2 oracle (reax_conv_l2 / reax_conv_v, libreax_howu/reax_conv_v2.cu) against its pins,
and each planted mistake caught by at least one pin (reversed taps, the qkv/cache boundary off by one, a plain
L2 sum order, a sign error inside SiLU)."""
import pytest

import conv_cases as CC
import pyoracle


@pytest.mark.parametrize("pin", CC.ALL_PINS, ids=lambda f: f.__name__)
def test_pin(pin):
    pin()


@pytest.mark.parametrize("mutant", sorted(pyoracle.CONV_MUTANTS))
def test_mutant_is_caught(mutant):
    failed = []
    for pin in CC.ALL_PINS:
        try:
            pin(mutant=mutant)
        except AssertionError as e:
            failed.append(f"{pin.__name__}: {str(e)[:60]}")
    assert failed, f"mutant {mutant} passed every pin"
