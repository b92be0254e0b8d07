"""Device calibration (cvs_calibrate_stream_read): the achievable
streaming-read rate that the HBM-bound kernels are compared with."""
import math

import pytest

pytestmark = pytest.mark.gpu


def test_stream_read_rate_is_positive_and_below_the_nominal_peak(ctx):
    for wg in (256, 2048):
        gbs = ctx.calibrate_stream_read(256 << 20, wg, reps=5)
        assert math.isfinite(gbs) and 1000.0 < gbs < 8500.0, (wg, gbs)


def test_stream_read_rejects_shares_below_one_step(ctx):
    with pytest.raises(ValueError, match="32 KiB"):
        ctx.calibrate_stream_read(1 << 20, 256)


def test_gather_read_rate(ctx):
    """Random 4 KiB-row gathers over a 410 MB set: a finite positive rate;
    over a set that fits the L2 it is faster than over one that does not."""
    big = ctx.calibrate_gather_read(4096, 100_000, 1024, 32, reps=3)
    small = ctx.calibrate_gather_read(4096, 1_000, 1024, 32, reps=3)
    assert math.isfinite(big) and 500.0 < big < 40000.0, big
    assert small > big, (small, big)


def test_gather_read_rejects_bad_rows(ctx):
    with pytest.raises(ValueError):
        ctx.calibrate_gather_read(4100, 1000, 64, 8)
