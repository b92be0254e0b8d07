"""Device calibration: the achievable streaming-read and gather rates that
the HBM-bound kernels are compared with (cvs_calibrate_stream_read,
cvs_calibrate_gather_read), and the matrix-core rate of the large-batch
scan's register block (cvs_calibrate_mfma)."""
import math

import numpy as np

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


def test_mfma_rate(cvs, ctx):
    """The matrix-core loop: a finite rate below the nominal 2.5 PFLOP/s of
    fp16 dense MFMA, with operands in registers and from LDS; its argument
    checks."""
    data = cvs.DeviceArray.from_host(ctx, np.random.default_rng(0).standard_normal((64, 1024)).astype(np.float16))
    try:
        for lds in (False, True):
            tf = ctx.calibrate_mfma(data.ptr, data.nbytes, 256, 4096, from_lds=lds, reps=2)
            assert math.isfinite(tf) and 100.0 < tf < 2600.0, (lds, tf)
        with pytest.raises(ValueError, match="40 KiB"):
            ctx.calibrate_mfma(data.ptr, 1024, 256, 64)
        with pytest.raises(ValueError):
            ctx.calibrate_mfma(data.ptr, data.nbytes, 0, 64)
    finally:
        data.free()
