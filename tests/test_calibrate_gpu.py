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
