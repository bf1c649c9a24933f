"""CPU: the oracle against independent facts (see oracle_pins.py) and against the committed golden vectors."""
import glob
import os

import numpy as np
import pytest

import oracle_pins as OP


@pytest.mark.parametrize("pin", OP.ALL_PINS, ids=lambda f: f.__name__)
def test_pin(oracle, pin):
    pin()


GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: os.path.basename(p))
def test_oracle_matches_golden(oracle, path):
    import golden_io

    case, arrays, o_want, lse_want = golden_io.load(path)
    import fmha_cases as FC

    o, lse = FC.oracle_ref(case, arrays)
    OP._close(o, o_want, 1e-9, f"{case.name} O vs golden")
    OP._close(lse, lse_want, 1e-9, f"{case.name} LSE vs golden")


def test_golden_present():
    assert len(GOLDEN) >= 4, "tests/golden/*.npz missing: run tests/golden/make_golden.py"
