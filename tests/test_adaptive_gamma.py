"""Adaptive gamma controller vs llm_engine.py:197-208 (runs without a GPU).

Checks hand-worked trajectories: nothing changes before 5 samples, the window
slides over the last 20 rates and is kept across changes, the bounds 1 and 8
hold, steps without proposals add no sample, and the thresholds are strict.
"""
import importlib

import pytest


def _ag():
    return importlib.import_module("hilda-vllm_amd.engine.adaptive_gamma").AdaptiveGamma


def test_needs_five_samples_then_raises_every_step():
    c = _ag()(3)
    got = [c.update(3, 3) for _ in range(8)]
    # samples 1-4: no change; from the 5th on the average (1.0) > 0.8 raises gamma
    assert got == [3, 3, 3, 3, 4, 5, 6, 7]


def test_upper_and_lower_bounds():
    c = _ag()(7)
    got = [c.update(1, 1) for _ in range(7)]
    assert got == [7, 7, 7, 7, 8, 8, 8]
    c = _ag()(2)
    got = [c.update(0, 4) for _ in range(7)]
    assert got == [2, 2, 2, 2, 1, 1, 1]


def test_between_thresholds_holds_and_float_average_as_reference():
    c = _ag()(4)
    for _ in range(25):
        assert c.update(1, 2) == 4  # 0.5 lies between the thresholds
    # the average is sum(window) / len(window) in float, as in the reference:
    # five rates of 0.4 average to exactly 0.4 (not below 0.4), six to 0.3999...
    c = _ag()(4)
    got = [c.update(2, 5) for _ in range(6)]
    assert sum([0.4] * 5) / 5 == 0.4 and sum([0.4] * 6) / 6 < 0.4
    assert got == [4, 4, 4, 4, 4, 3]


def test_window_slides_and_is_kept_across_changes():
    c = _ag()(4)
    # 5 perfect steps: gamma rises on the 5th
    for _ in range(4):
        c.update(1, 1)
    assert c.update(1, 1) == 5
    # the window is kept: after k zeros it is 5 ones + k zeros, average 5 / (5 + k),
    # above 0.8 for k = 1 (raise again) and below 0.4 from k = 8 on
    got = [c.update(0, 5) for _ in range(9)]
    assert got == [6, 6, 6, 6, 6, 6, 6, 5, 4]
    # the window holds at most 20 rates
    for _ in range(30):
        c.update(0, 1)
    assert len(c.rates) == 20 and c.gamma == 1


def test_no_proposal_adds_no_sample():
    c = _ag()(3)
    for _ in range(10):
        assert c.update(0, 0) == 3
    assert c.rates == []


def test_rejects_out_of_range_start():
    with pytest.raises(ValueError):
        _ag()(0)
    with pytest.raises(ValueError):
        _ag()(9)
