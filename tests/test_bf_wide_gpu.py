"""GPU: brute force beyond the fused scan's limits (d > 1024 or k > 112),
which the reference's CPU loop (src/cagra.cpp:211-252) handles for any d and
k.  These calls run the keys-matrix path (bf_wide.hip): fp16 MFMA keys of
the centred rows, a select of the R-th key (a sampled threshold and the
keys collected below it, or a radix select over every key), the certificate
and the exact re-rank.

Same gate as tests/test_bf_gpu.py against the oracle's restatement of the
reference loop: id sets equal except at near-ties of the k-th distance
(1e-3 relative), distances within 1e-3 relative, rows sorted by
(distance, id), missing slots UINT32_MAX / +inf.
"""
import numpy as np
import pytest

from test_bf_gpu import assert_parity

pytestmark = pytest.mark.gpu


def clustered(rng, n, d, centres, sigma=0.3):
    x = centres[rng.integers(0, len(centres), n)] + sigma * rng.standard_normal((n, d)).astype(np.float32)
    return (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)


def run(ctx, oracle, base, qs, k):
    nbr, dist = ctx.dataset(base).bf_search(qs, k)
    ref_nbr, ref_dist = oracle.bf_exact(base, qs, k + 1, threads=8)
    assert_parity(nbr, dist, ref_nbr, ref_dist, k)
    return nbr, dist


@pytest.mark.parametrize("n,d,q,k", [
    (20000, 1536, 50, 10),
    (12000, 3072, 40, 10),
    (6000, 4096, 20, 100),
    (3000, 3000, 17, 77),      # d padded to 3008
    (4000, 1100, 9, 10),       # d padded to 1152
    (5000, 1531, 7, 10),       # odd d: rows not 16-byte aligned, scalar exact re-rank
    (3000, 130, 5, 150),       # d % 4 == 2 with k above the fused scan's limit
    (30000, 128, 60, 200),     # k above the fused scan's limit, small d
    (20000, 256, 40, 1000),
    (5000, 1536, 30, 200),
    (700, 64, 5, 1000),        # k > n: padded slots
    (10, 2000, 3, 200),        # fewer rows than one tile, k > n
    (3000, 1536, 1, 10),       # a single query
])
def test_wide_shapes(ctx, oracle, n, d, q, k):
    rng = np.random.default_rng(n + d + k)
    centres = rng.standard_normal((64, d)).astype(np.float32)
    base = clustered(rng, n, d, centres)
    qs = clustered(rng, q, d, centres)
    nbr, dist = run(ctx, oracle, base, qs, k)
    if k > n:
        assert (nbr[:, n:] == 0xFFFFFFFF).all() and np.isinf(dist[:, n:]).all()


def test_wide_query_chunks(ctx, oracle):
    """More queries than one chunk (512): three chunks, the last partial."""
    rng = np.random.default_rng(5)
    n, d, q, k = 3000, 1100, 1100, 10
    base = rng.standard_normal((n, d)).astype(np.float32)
    qs = rng.standard_normal((q, d)).astype(np.float32)
    nbr, dist = ctx.dataset(base).bf_search(qs, k)
    sample = np.arange(0, q, 7)
    ref_nbr, ref_dist = oracle.bf_exact(base, qs[sample], k + 1, threads=8)
    assert_parity(nbr[sample], dist[sample], ref_nbr, ref_dist, k)


@pytest.mark.parametrize("offset_norm", [100.0, 300.0])
def test_wide_offset_data(ctx, oracle, offset_norm):
    rng = np.random.default_rng(int(offset_norm) + 1)
    n, d, q, k = 10000, 1536, 30, 10
    centres = rng.standard_normal((64, d)).astype(np.float32)
    off = rng.standard_normal(d)
    off = (off * offset_norm / np.linalg.norm(off)).astype(np.float32)
    run(ctx, oracle, clustered(rng, n, d, centres) + off, clustered(rng, q, d, centres) + off, k)


def test_wide_escalation_and_overflow(ctx, oracle):
    """Two far clusters (the certificate fails, rows up to the bound are
    re-ranked) and queries whose fp16 copy overflows (every row re-ranked),
    at k = 200."""
    rng = np.random.default_rng(9)
    n, d, q, k = 4000, 64, 12, 200
    c = rng.standard_normal(d)
    c = (400.0 * c / np.linalg.norm(c)).astype(np.float32)
    side = np.where(rng.integers(0, 2, n) == 0, 1.0, -1.0).astype(np.float32)[:, None]
    base = side * c + rng.standard_normal((n, d)).astype(np.float32)
    qs = np.where(np.arange(q) % 2 == 0, 1.0, -1.0).astype(np.float32)[:, None] * c + \
        rng.standard_normal((q, d)).astype(np.float32)
    qs[:2] *= 1e6
    ctx.bf_escalations(reset=True)
    run(ctx, oracle, base, qs, k)
    esc, full = ctx.bf_escalations()
    assert full >= 2 and esc > full


def test_wide_integer_ties(ctx, oracle):
    """Integer rows (every quantity exact) with duplicates: ids and distances
    equal the oracle's exactly, ties by id."""
    rng = np.random.default_rng(2)
    uniq = rng.integers(-3, 4, (60, 1200)).astype(np.float32)
    base = np.repeat(uniq, 5, axis=0)
    qs = uniq[:4] + rng.integers(-1, 2, (4, 1200)).astype(np.float32)
    nbr, dist = ctx.dataset(base).bf_search(qs, 150)
    ref_nbr, ref_dist = oracle.bf_exact(base, qs, 150)
    np.testing.assert_array_equal(nbr, ref_nbr)
    np.testing.assert_array_equal(dist, ref_dist)


def test_wide_sample_threshold_short(ctx, oracle):
    """The sampled threshold falls short and the full radix select takes
    over.  With n = 32,768 rows (1,024 tiles of 32) the sample is every second
    tile (16,384 rows); here those are exactly the rows near the queries and
    the rows of odd tiles are far, so the threshold (rank ~286 of the sample
    for R = 400) has only ~286 keys at or below it, fewer than R."""
    rng = np.random.default_rng(31)
    n, d, q, k = 32768, 128, 4, 200
    c = rng.standard_normal(d).astype(np.float32)
    near = (np.arange(n) // 32) % 2 == 0
    base = np.where(near[:, None], c, -30.0 * c).astype(np.float32) + \
        0.5 * rng.standard_normal((n, d)).astype(np.float32)
    qs = c + 0.5 * rng.standard_normal((q, d)).astype(np.float32)
    nbr, _ = run(ctx, oracle, base, qs, k)
    assert near[nbr.astype(np.int64)].all()


def test_wide_sample_threshold_crowded(ctx, oracle):
    """More keys tie at the sampled threshold than the candidate list holds
    (8,192): 10,000 identical integer rows, each at distance 0 from the
    query; the full radix select takes over and ties resolve by id."""
    rng = np.random.default_rng(32)
    n, d, q, k = 20000, 128, 2, 150
    v = rng.integers(-3, 4, d).astype(np.float32)
    base = rng.integers(-3, 4, (n, d)).astype(np.float32)
    base[:10000] = v
    qs = np.stack([v, v])
    nbr, dist = ctx.dataset(base).bf_search(qs, k)
    ref_nbr, ref_dist = oracle.bf_exact(base, qs, k)
    np.testing.assert_array_equal(nbr, ref_nbr)
    np.testing.assert_array_equal(dist, ref_dist)
    assert (nbr == np.arange(k)).all() and (dist == 0).all()


def test_wide_maximum_sizes(ctx, oracle):
    """The largest shapes the entry point accepts: d = CVS_BF_MAX_DIM
    (16,384: 1,024 k-steps per tile) with k = CVS_BF_MAX_K (1,024; R = 2,048
    rows re-ranked), three queries (one partial query tile)."""
    rng = np.random.default_rng(33)
    n, d, q, k = 2500, 16384, 3, 1024
    centres = rng.standard_normal((16, d)).astype(np.float32)
    run(ctx, oracle, clustered(rng, n, d, centres), clustered(rng, q, d, centres), k)


def test_wide_second_pass_in_later_chunk(ctx, oracle):
    """Every query falls back (the construction of
    test_wide_sample_threshold_short) over two query chunks (512 + 88): the
    second pass's per-block flags are indexed within each chunk."""
    rng = np.random.default_rng(34)
    n, d, q, k = 32768, 128, 600, 200
    c = rng.standard_normal(d).astype(np.float32)
    near = (np.arange(n) // 32) % 2 == 0
    base = np.where(near[:, None], c, -30.0 * c).astype(np.float32) + \
        0.5 * rng.standard_normal((n, d)).astype(np.float32)
    qs = c + 0.5 * rng.standard_normal((q, d)).astype(np.float32)
    nbr, dist = ctx.dataset(base).bf_search(qs, k)
    sample = np.r_[0:5, 250:255, 510:520, 590:600]
    ref_nbr, ref_dist = oracle.bf_exact(base, qs[sample], k + 1, threads=8)
    assert_parity(nbr[sample], dist[sample], ref_nbr, ref_dist, k)
    assert near[nbr.astype(np.int64)].all()
