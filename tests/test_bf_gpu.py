"""GPU parity of the fused brute-force path (C ABI: cvs_bf_search) against the
oracle and the reference's golden outputs.

Gate (stated by the target): top-k id sets equal to the reference's except
where the k-th and (k+1)-th reference distances are within 1e-3 relative;
distances within 1e-3 relative.  Integer-valued inputs must match exactly.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
REL_TOL = 1e-3


def assert_parity(nbr, dist, ref_nbr, ref_dist_k1, k):
    """ref_dist_k1: reference distances for k+1 results (sorted)."""
    q = nbr.shape[0]
    ref_dist = ref_dist_k1[:, :k]
    finite = np.isfinite(ref_dist)
    np.testing.assert_array_equal(np.isfinite(dist), finite)
    scale = np.maximum(np.abs(ref_dist), 1e-30)
    err = np.where(finite, np.abs(dist - ref_dist) / scale, 0)
    assert err.max() <= REL_TOL, f"distance error {err.max()}"
    for i in range(q):
        dk = ref_dist_k1[i, k - 1]
        dk1 = ref_dist_k1[i, k] if ref_dist_k1.shape[1] > k else np.inf
        near_tie = np.isfinite(dk1) and abs(dk1 - dk) <= REL_TOL * max(abs(dk), 1e-30)
        if not near_tie:
            assert set(nbr[i].tolist()) == set(ref_nbr[i, :k].tolist()), f"query {i}"
    # rows sorted by (distance, id)
    for i in range(q):
        for j in range(1, k):
            assert dist[i, j - 1] < dist[i, j] or (dist[i, j - 1] == dist[i, j] and nbr[i, j - 1] < nbr[i, j]) \
                or not np.isfinite(dist[i, j])


def check_against_oracle(ctx, oracle, base, queries, k, threads=8):
    ds = ctx.dataset(base)
    nbr, dist = ds.bf_search(queries, k)
    ref_nbr, ref_dist = oracle.bf_exact(base, queries, k + 1, threads=threads)
    assert_parity(nbr, dist, ref_nbr, ref_dist, k)
    return nbr, dist


def test_faiss_known_answers(ctx):
    db = np.array([[0, 0], [10, 0], [0, 10], [2, 2]], np.float32)
    qs = np.array([[0, 0], [9, 1]], np.float32)
    ds = ctx.dataset(db)
    nbr, dist = ds.bf_search(qs, 2)
    assert nbr.tolist() == [[0, 3], [1, 3]]
    assert dist.tolist() == [[0.0, 8.0], [2.0, 50.0]]
    nbr, dist = ds.bf_search(qs[:1], 4)
    assert nbr.tolist() == [[0, 3, 1, 2]] and dist.tolist() == [[0.0, 8.0, 100.0, 100.0]]
    nbr, dist = ds.bf_search(qs, 5)
    assert nbr[:, 4].tolist() == [0xFFFFFFFF] * 2 and np.isinf(dist[:, 4]).all()
    assert nbr[:, :4].tolist() == [[0, 3, 1, 2], [1, 3, 0, 2]]


def test_dispatch_test_inputs_run_on_gpu(ctx, cvs):
    base = np.zeros((64, 8), np.float32)
    for i in range(64):
        base[i, i % 8] = i
    qs = np.zeros((4, 8), np.float32)
    for j in range(4):
        qs[j, j % 8] = 1
    ds = ctx.dataset(base)
    cvs.reset_dispatch_count()
    nbr, dist = ds.bf_search(qs, 4)
    assert cvs.dispatch_count() > 0
    assert nbr.tolist() == [[0, 1, 2, 3], [1, 0, 2, 3], [0, 2, 1, 3], [0, 1, 3, 2]]
    assert dist.tolist() == [[1, 2, 5, 10], [0, 1, 5, 10], [1, 1, 2, 10], [1, 2, 4, 5]]


@pytest.mark.parametrize("name", ["random", "ties", "kbig", "wide"])
def test_reference_golden(ctx, oracle, name):
    g = np.load(os.path.join(GOLDEN, "bf_ref.npz"))
    base, qs, k = g[f"{name}_base"], g[f"{name}_queries"], int(g[f"{name}_k"])
    nbr, dist = ctx.dataset(base).bf_search(qs, k)
    if name in ("ties", "kbig"):
        if name == "ties":  # integer data: every quantity is exact
            np.testing.assert_array_equal(nbr, g[f"{name}_nbr"])
            np.testing.assert_array_equal(dist, g[f"{name}_dist"])
        else:
            np.testing.assert_array_equal(nbr, g[f"{name}_nbr"])
            np.testing.assert_allclose(dist, g[f"{name}_dist"], rtol=REL_TOL)
    else:
        _, ref_dist = oracle.bf_exact(base, qs, k + 1)
        assert_parity(nbr, dist, g[f"{name}_nbr"], ref_dist, k)


@pytest.mark.parametrize("n,d,q,k", [
    (1, 1, 1, 1),
    (7, 5, 3, 10),        # k > n: padded slots
    (100, 64, 130, 10),   # two query blocks
    (1000, 96, 17, 48),   # largest k of the LDS lists
    (1000, 96, 17, 49),   # smallest k of the global-memory lists (kp = 128)
    (20000, 128, 300, 100),
    (3000, 64, 40, 112),  # largest k
    (100, 32, 5, 112),    # k > n with global-memory lists
    (5000, 256, 33, 24),
    (4000, 300, 50, 10),    # 32 k-steps per tile (k-split scan, one stage per tile)
    (2500, 512, 130, 100),  # 32 k-steps, two query blocks, global-memory lists
    (6000, 384, 20, 40),
    (2000, 1024, 5, 1),
    (3333, 1000, 9, 16),  # d not a power of two
    (40000, 128, 129, 10),
])
def test_random_shapes(ctx, oracle, n, d, q, k):
    rng = np.random.default_rng(n * 31 + d)
    base = rng.standard_normal((n, d)).astype(np.float32)
    qs = rng.standard_normal((q, d)).astype(np.float32)
    check_against_oracle(ctx, oracle, base, qs, k)


@pytest.mark.parametrize("n,d,q,k", [
    (30000, 64, 1500, 10),    # > 8 query blocks: range-major launch, LDS lists
    (30000, 64, 1500, 100),   # range-major launch, global-memory lists (8 k-steps or fewer)
    (8000, 1024, 1100, 64),   # register-blocked scan (bf_gemm.hip): 3 query blocks
    (3000, 128, 2000, 100),   # 8 k-steps, one 128-row block per span
    (500, 256, 1200, 100),    # half the spans empty
    (20000, 1000, 1500, 100), # d padded to 1024
    (20000, 512, 5000, 112),  # 10 query blocks: two per XCD for XCDs 0 and 1, largest k
    (12000, 1024, 1300, 10),  # range-major pipelined scan (64 k-steps), kp = 16 LDS lists
    (12000, 512, 1100, 40),   # range-major pipelined scan (32 k-steps), kp = 64 LDS lists
    (7000, 384, 1100, 100),   # d 384 padded to 512: 128 zero columns in every tile
    (5000, 640, 1030, 50),    # d 640 padded to 1024; the last 512-query block holds one 32-query tile
    (9000, 768, 1200, 112),   # d 768 padded to 1024, largest k
    (3000, 896, 2100, 77),    # d 896 padded to 1024, 5 query blocks
])
def test_large_batches(ctx, oracle, n, d, q, k):
    rng = np.random.default_rng(q + k)
    centers = rng.standard_normal((32, d)).astype(np.float32)
    base = centers[rng.integers(0, 32, n)] + 0.3 * rng.standard_normal((n, d)).astype(np.float32)
    qs = centers[rng.integers(0, 32, q)] + 0.3 * rng.standard_normal((q, d)).astype(np.float32)
    check_against_oracle(ctx, oracle, base, qs, k)


def test_duplicate_rows_tie_break_by_id(ctx, oracle):
    rng = np.random.default_rng(5)
    uniq = rng.standard_normal((50, 48)).astype(np.float32)
    base = np.repeat(uniq, 20, axis=0)   # every vector 20 times
    qs = uniq[:6] + 0.01 * rng.standard_normal((6, 48)).astype(np.float32)
    nbr, dist = ctx.dataset(base).bf_search(qs, 25)
    ref_nbr, ref_dist = oracle.bf_exact(base, qs, 25)
    # the 20 copies of the nearest vector come first, in id order
    np.testing.assert_array_equal(nbr[:, :20], ref_nbr[:, :20])
    np.testing.assert_allclose(dist, ref_dist, rtol=REL_TOL)


def test_c1_clustered_config(ctx, cvs, oracle):
    """N=10,000, Q=100, D=1024, K=10 on the clustered distribution."""
    base = cvs.synth_clustered(12345, cvs.STREAM_BASE, 10000, 1024)
    qs = cvs.synth_clustered(12345, cvs.STREAM_QUERIES, 100, 1024)
    check_against_oracle(ctx, oracle, base, qs, 10)


def test_async_matches_sync(ctx, cvs):
    rng = np.random.default_rng(9)
    base = rng.standard_normal((3000, 200)).astype(np.float32)
    qs = rng.standard_normal((40, 200)).astype(np.float32)
    ds = ctx.dataset(base)
    nbr, dist = ds.bf_search(qs, 10)
    dq = cvs.DeviceArray.from_host(ctx, qs)
    dn = cvs.DeviceArray(ctx, (40, 10), np.uint32)
    dd = cvs.DeviceArray(ctx, (40, 10), np.float32)
    ds.bf_search_async(dq, 10, dn, dd)
    ctx.synchronize()
    np.testing.assert_array_equal(dn.to_host(), nbr)
    np.testing.assert_array_equal(dd.to_host(), dist)
    # repeated calls reuse workspaces and give identical results
    for _ in range(3):
        ds.bf_search_async(dq, 10, dn, dd)
    ctx.synchronize()
    np.testing.assert_array_equal(dn.to_host(), nbr)


def test_dataset_from_device_rows(ctx, cvs):
    rng = np.random.default_rng(13)
    base = rng.standard_normal((500, 40)).astype(np.float32)
    qs = rng.standard_normal((3, 40)).astype(np.float32)
    a = ctx.dataset(base).bf_search(qs, 7)
    b = ctx.dataset(cvs.DeviceArray.from_host(ctx, base)).bf_search(qs, 7)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


def test_argument_errors(ctx):
    ds = ctx.dataset(np.ones((10, 4), np.float32))
    with pytest.raises(ValueError):
        ds.bf_search(np.ones((2, 4), np.float32), 0)
    with pytest.raises(ValueError):
        ds.bf_search(np.ones((2, 4), np.float32), 1025)
    with pytest.raises(ValueError):
        ds.bf_search(np.ones((2, 5), np.float32), 3)
    with pytest.raises(ValueError):
        ctx.dataset(np.ones((10, 16385), np.float32)).bf_search(np.ones((1, 16385), np.float32), 3)
    with pytest.raises(ValueError):
        ctx.dataset(np.ones((0, 4), np.float32))


def exact_topk_numpy(base, qs, k, extra=64):
    """fp32 GEMM candidates re-scored in fp64 (ground truth at full size)."""
    cross = qs @ base.T
    norms = np.einsum("ij,ij->i", base, base)
    approx = norms[None, :] - 2 * cross
    cand = np.argpartition(approx, k + extra, axis=1)[:, :k + extra]
    out_i = np.empty((qs.shape[0], k + 1), np.int64)
    out_d = np.empty((qs.shape[0], k + 1), np.float64)
    for i in range(qs.shape[0]):
        c = cand[i]
        d = ((base[c].astype(np.float64) - qs[i].astype(np.float64)) ** 2).sum(1)
        o = np.lexsort((c, d))[:k + 1]
        out_i[i], out_d[i] = c[o], d[o]
    return out_i, out_d


def test_c3_full_size_large_batch(ctx, cvs):
    """N=1,000,000, D=1024, Q=10,000, K=100 in one call: ids and distances
    of 200 sampled queries against the exact ground truth (same gates)."""
    n, d, q, k = 1_000_000, 1024, 10_000, 100
    base = cvs.synth_clustered(12345, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(12345, cvs.STREAM_QUERIES, q, d)
    nbr, dist = ctx.dataset(base).bf_search(qs, k)
    sample = np.random.default_rng(0).choice(q, 200, replace=False)
    gt_i, gt_d = exact_topk_numpy(base, qs[sample], k)
    assert_parity(nbr[sample], dist[sample], gt_i.astype(np.uint32), gt_d, k)
    recall = np.mean([len(set(nbr[s].tolist()) & set(gt_i[j, :k].tolist())) / k for j, s in enumerate(sample)])
    assert recall >= 0.999, recall


def test_c2_full_size_recall(ctx, cvs):
    """N=1,000,000, D=1024, Q=100, K=10: recall@10 = 1.0 vs exact (up to
    near-ties), distances within 1e-3."""
    n, d, q, k = 1_000_000, 1024, 100, 10
    base = cvs.synth_clustered(12345, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(12345, cvs.STREAM_QUERIES, q, d)
    ds = ctx.dataset(base)
    nbr, dist = ds.bf_search(qs, k)
    gt_i, gt_d = exact_topk_numpy(base, qs, k)
    assert_parity(nbr, dist, gt_i.astype(np.uint32), gt_d, k)
    recall = np.mean([len(set(nbr[i]) & set(gt_i[i, :k])) / k for i in range(q)])
    assert recall >= 0.999
