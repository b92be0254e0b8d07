"""The synthetic clustered generator: determinism, range independence,
normalisation and the moments of its normal variates."""
import numpy as np


def test_rows_are_unit_norm_and_deterministic(cvs):
    a = cvs.synth_clustered(12345, cvs.STREAM_BASE, 200, 64)
    b = cvs.synth_clustered(12345, cvs.STREAM_BASE, 200, 64)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_allclose(np.linalg.norm(a.astype(np.float64), axis=1), 1.0, rtol=1e-6)


def test_row_ranges_are_independent(cvs):
    whole = cvs.synth_clustered(7, cvs.STREAM_BASE, 100, 32)
    part = cvs.synth_clustered(7, cvs.STREAM_BASE, 40, 32, row0=60)
    np.testing.assert_array_equal(whole[60:], part)


def test_streams_and_seeds_differ(cvs):
    a = cvs.synth_clustered(7, cvs.STREAM_BASE, 10, 32)
    b = cvs.synth_clustered(7, cvs.STREAM_QUERIES, 10, 32)
    c = cvs.synth_clustered(8, cvs.STREAM_BASE, 10, 32)
    assert not np.array_equal(a, b) and not np.array_equal(a, c)


def test_normal_moments(cvs):
    z = np.array([cvs.synth_normal(1, 5, r, c) for r in range(200) for c in range(100)])
    assert abs(z.mean()) < 0.03
    assert abs(z.std() - 1.0) < 0.03
    assert abs((z ** 3).mean()) < 0.08
    assert abs((z ** 4).mean() - 3.0) < 0.2


def test_clusters_are_tight(cvs):
    # sigma = 0.3 noise around 64 N(0, I) centres in 1024-d: rows of the same
    # centre are far closer than rows of different centres.
    x = cvs.synth_clustered(12345, cvs.STREAM_BASE, 300, 1024).astype(np.float64)
    g = x @ x.T
    np.fill_diagonal(g, -1)
    nearest = g.max(1)
    assert np.median(nearest) > 0.8
