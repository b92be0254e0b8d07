"""GPU: the brute force stays exact where fp16 selection alone would not.

The fp16 copy is centred (column mean) and scaled by a power of two, and each
query's candidate selection is certified against a bound on the fp16
arithmetic's error; a query that fails is re-ranked exactly over every row
that could belong to its top k (from the candidate lists, or every row).
Ground truth is the oracle's restatement of the reference's exact CPU loop
(src/cagra.cpp:211-252), with the same gate as tests/test_bf_gpu.py: id sets
equal except at near-ties of the k-th distance (1e-3 relative), distances
within 1e-3 relative.
"""
import numpy as np
import pytest

from test_bf_gpu import assert_parity

pytestmark = pytest.mark.gpu


def clustered(rng, centres, n, sigma=0.3):
    """The benchmark's distribution: a random centre plus noise, L2-normalised."""
    x = centres[rng.integers(0, len(centres), n)] + sigma * rng.standard_normal((n, centres.shape[1])).astype(np.float32)
    return (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)


def search_and_check(ctx, oracle, base, qs, k):
    nbr, dist = ctx.dataset(base).bf_search(qs, k)
    ref_nbr, ref_dist = oracle.bf_exact(base, qs, k + 1, threads=8)
    assert_parity(nbr, dist, ref_nbr, ref_dist, k)
    return nbr, dist


@pytest.mark.parametrize("offset_norm", [30.0, 100.0, 300.0])
def test_offset_data(ctx, oracle, offset_norm):
    """Unit-norm clustered rows and queries shifted by one common offset:
    fp16 inputs without centring lose the neighbours here (a simulation of
    the uncentred selection kept 68% of the true top 10 at offset 100 and
    11% at 300)."""
    rng = np.random.default_rng(int(offset_norm))
    n, d, q, k = 20_000, 1024, 50, 10
    off = rng.standard_normal(d)
    off = (off * offset_norm / np.linalg.norm(off)).astype(np.float32)
    centres = rng.standard_normal((64, d)).astype(np.float32)
    base = clustered(rng, centres, n) + off
    qs = clustered(rng, centres, q) + off
    ctx.bf_escalations(reset=True)
    search_and_check(ctx, oracle, base, qs, k)


@pytest.mark.parametrize("magnitude", [1e6, 1e-9])
def test_values_outside_fp16_range(ctx, oracle, magnitude):
    """Rows of magnitude 1e6 overflow fp16 and rows of 1e-9 are below its
    smallest subnormal; the power-of-two scale brings both into range."""
    rng = np.random.default_rng(7)
    base = (rng.standard_normal((5000, 96)) * magnitude).astype(np.float32)
    qs = (rng.standard_normal((20, 96)) * magnitude).astype(np.float32)
    search_and_check(ctx, oracle, base, qs, 10)


def test_far_queries_overflow_and_rescan(ctx, oracle):
    """Queries 10^6 times farther out than the rows' spread: their fp16 copy
    overflows, no bound holds, and they are re-ranked over every row."""
    rng = np.random.default_rng(11)
    base = rng.standard_normal((3000, 64)).astype(np.float32)
    qs = rng.standard_normal((8, 64)).astype(np.float32)
    qs[:3] *= 1e6
    ctx.bf_escalations(reset=True)
    search_and_check(ctx, oracle, base, qs, 10)
    esc, full = ctx.bf_escalations()
    assert full >= 3 and esc >= full


def test_two_far_clusters_escalate(ctx, oracle):
    """Two tight clusters far apart (offsets +-c, |c| = 400, unit-scale
    spread): the mean sits between them, so centring leaves |x| ~ 400 and the
    fp16 error bound exceeds the gaps between neighbours.  Queries escalate
    and the answer is still exact."""
    rng = np.random.default_rng(3)
    n, d, q, k = 6000, 64, 24, 10
    c = rng.standard_normal(d)
    c = (400.0 * c / np.linalg.norm(c)).astype(np.float32)
    side = np.where(rng.integers(0, 2, n) == 0, 1.0, -1.0).astype(np.float32)[:, None]
    base = side * c + rng.standard_normal((n, d)).astype(np.float32)
    qside = np.where(np.arange(q) % 2 == 0, 1.0, -1.0).astype(np.float32)[:, None]
    qs = qside * c + rng.standard_normal((q, d)).astype(np.float32)
    ctx.bf_escalations(reset=True)
    search_and_check(ctx, oracle, base, qs, k)
    esc, _ = ctx.bf_escalations()
    assert esc > 0


@pytest.mark.parametrize("k", [10, 40, 100])
def test_moderate_conditioning_escalates_from_lists(ctx, oracle, k):
    """Clusters offset by |c| = 12 from the mean with unit spread: some
    queries' fp16 selection cannot be certified at the candidate count, and
    are re-ranked from the candidate lists, which hold every row up to the
    scan's threshold."""
    rng = np.random.default_rng(k)
    n, d, q = 120_000, 64, 64
    cent = rng.standard_normal((8, d)).astype(np.float32)
    cent *= 12.0 / np.linalg.norm(cent, axis=1, keepdims=True)
    base = cent[rng.integers(0, 8, n)] + rng.standard_normal((n, d)).astype(np.float32)
    qs = cent[rng.integers(0, 8, q)] + rng.standard_normal((q, d)).astype(np.float32)
    ctx.bf_escalations(reset=True)
    search_and_check(ctx, oracle, base, qs, k)


def test_benchmark_distribution_needs_no_escalation(ctx, cvs, oracle):
    """N=10,000 D=1024 Q=100 K=10 on the benchmark's distribution: every
    query's selection is certified without re-ranking more rows."""
    base = cvs.synth_clustered(12345, cvs.STREAM_BASE, 10000, 1024)
    qs = cvs.synth_clustered(12345, cvs.STREAM_QUERIES, 100, 1024)
    ctx.bf_escalations(reset=True)
    search_and_check(ctx, oracle, base, qs, 10)
    assert ctx.bf_escalations() == (0, 0)


def test_large_batch_offset(ctx, oracle):
    """The register-blocked large-batch scan (kp = 128 lists) on offset data."""
    rng = np.random.default_rng(21)
    n, d, q, k = 8000, 1024, 1100, 64
    off = rng.standard_normal(d)
    off = (off * 200.0 / np.linalg.norm(off)).astype(np.float32)
    centres = rng.standard_normal((32, d)).astype(np.float32)
    base = clustered(rng, centres, n) + off
    qs = clustered(rng, centres, q) + off
    nbr, dist = ctx.dataset(base).bf_search(qs, k)
    sample = np.arange(0, q, 11)
    ref_nbr, ref_dist = oracle.bf_exact(base, qs[sample], k + 1, threads=8)
    assert_parity(nbr[sample], dist[sample], ref_nbr, ref_dist, k)
