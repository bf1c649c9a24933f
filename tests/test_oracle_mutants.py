"""CPU: plant each deliberate mistake in the oracle and check that at least one pin fails.

This shows the pins constrain the oracle: a dropped scale, a wrong GQA head mapping, an off-by-one causal
boundary, a missing normalisation, a wrong LSE base, a sign error in the sigmoid, the wrong half of the gate
tensor, an unweighted split combine, and the drop-in qpos = 0 block rule over tokens instead of rows, on clamped
instead of raw qpos, or left out are each caught.
"""
import pytest

import oracle_pins as OP
import pyoracle

FAST_PINS = [OP.pin_sdpa, OP.pin_closed_forms, OP.pin_gqa_fold, OP.pin_varlen, OP.pin_split_combine, OP.pin_post,
             lambda: OP.pin_sigmoid(step=97), OP.pin_block_rule]


@pytest.mark.parametrize("mutant", sorted(pyoracle.MUTANTS))
def test_mutant_is_caught(oracle, mutant):
    pyoracle.set_mutant(mutant)
    try:
        failed = []
        for pin in FAST_PINS:
            try:
                pin()
            except AssertionError as e:
                failed.append(str(e)[:80])
        assert failed, f"mutant {mutant} passed every pin"
    finally:
        pyoracle.set_mutant(0)
