"""The overflow floor ladder's next-floor rule (gs_overflow_next_floor), host
code callable without a GPU, against the reference's own checks of that rule
(tests/unit/test_overflow_retry.cpp:27-50, render/host/overflow_retry.h:26-42)."""
import math

import pytest

from gsplat_tt_amd import _lib as L

CAP = 32768
MAX_FLOOR = 0.5


def nf(floor, n, cap=CAP):
    return L.overflow_next_floor(floor, n, cap)


@pytest.mark.parametrize("floor", [1.0 / 16384, 1.0 / 1024, 1.0 / 255, 1.0 / 16, 0.4])
@pytest.mark.parametrize("n", [CAP + 1, 34672, 40000, 2 * CAP, 100 * CAP])
def test_every_step_at_least_doubles_and_stays_below_the_cap(floor, n):
    g = nf(floor, n)
    assert g <= MAX_FLOOR
    assert g >= 2.0 * floor or g == MAX_FLOOR


def test_small_overflow_small_step():
    # one step from 1/16384 at 34672 records lands between 1/8192 and 1/1024
    g = nf(1.0 / 16384, 34672)
    assert 1.0 / 8192 <= g < 1.0 / 1024
    # the bench floor 10 % over stays finer than 1/32
    assert nf(1.0 / 255, 36045) < 1.0 / 32


@pytest.mark.parametrize("floor", [1.0 / 1048576, 1.0 / 16384, 1.0 / 255])
def test_ladder_ends_within_eight_steps(floor):
    g = floor
    for _ in range(8):
        g = nf(g, 10 * CAP)
    assert g == MAX_FLOOR


def test_step_follows_the_log_model_when_it_exceeds_doubling():
    # L = ln(1/floor) scaled by 0.9 cap / n: at n = cap the model floor is
    # floor^0.9, which for a fine floor is more than twice it
    f = 1.0 / 1048576
    assert nf(f, CAP) == pytest.approx(math.exp(math.log(f) * 0.9), rel=1e-6)
    # a count at or below the cap still takes the 0.9 step (the caller only
    # asks when over), and a floor at the cap stays there
    assert nf(MAX_FLOOR, 10 * CAP) == MAX_FLOOR
