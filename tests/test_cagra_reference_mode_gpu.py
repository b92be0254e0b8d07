"""GPU: the reference's own search route, query by query.

cvs_cagra_entry_points computes each query's entry node as the reference
does (src/cagra.cpp:128-178: the navigation node minimising
|q|^2 - 2 q.v + |v|^2, the first on ties) and cvs_cagra_search_reference runs
the reference's beam search (shaders/cagra_kernels.metal:28-199: one seed, an
unsorted beam with replace-worst insertion, expanded entries marked -d-1).
On integer-valued rows and queries every fp32 sum is exact in any order, so
the GPU's ids and distances must equal the oracle's restatement
(oracle/cagra_oracle.c) for every query, bit for bit.
"""
import numpy as np
import pytest

from search_metrics import assert_recall_not_below, exact_knn, recall

pytestmark = pytest.mark.gpu

K = 10


def integer_rows(cvs, stream, n, d, scale=64.0):
    """The benchmark's clustered unit-norm rows, scaled and rounded to
    integers (|values| <= ~12 at d = 1024, every sum < 2^24)."""
    return np.rint(cvs.synth_clustered(12345, stream, n, d) * scale).astype(np.float32)


@pytest.fixture(scope="module")
def int100k(cvs, oracle):
    n, d = 100_000, 1024
    print("[ref-mode] integer rows and the restated reference graph", flush=True)
    base = integer_rows(cvs, cvs.STREAM_BASE, n, d)
    qs = integer_rows(cvs, cvs.STREAM_QUERIES, 1000, d)
    graph = oracle.cagra_build_reference(base, 64, threads=16)
    nav = cvs.cagra_nav_nodes(n)
    return dict(base=base, qs=qs, graph=graph, nav=nav)


@pytest.fixture(scope="module")
def int100k_index(ctx, int100k):
    idx = ctx.cagra_index(int100k["base"], int100k["graph"], int100k["nav"])
    yield idx
    idx.close()


def test_entry_points_equal_oracle(int100k, int100k_index, oracle):
    b, nav = int100k["base"], int100k["nav"]
    gpu = int100k_index.entry_points(int100k["qs"])
    ref = oracle.cagra_entry_points(int100k["qs"], nav, b[nav])
    np.testing.assert_array_equal(gpu, ref)


@pytest.mark.parametrize("beam,iters", [(64, 200), (128, 200), (32, 50)])
def test_beam_search_equals_oracle_query_by_query(int100k, int100k_index, oracle, beam, iters):
    """N=100,000 D=1024, degree 64 on the restated reference graph: every
    query's ids and distances equal the oracle's."""
    b, g, qs, nav = int100k["base"], int100k["graph"], int100k["qs"], int100k["nav"]
    entry = oracle.cagra_entry_points(qs, nav, b[nav])
    gn, gd = int100k_index.search_reference(qs, K, beam, iters, entry)
    rn, rd = oracle.cagra_search(b, g, qs, K, beam, iters, entry, threads=16)
    np.testing.assert_array_equal(gn, rn)
    np.testing.assert_array_equal(gd, rd)


def test_full_route_small_batch_clamp(int100k, int100k_index, oracle):
    """q = 3 <= 4: the route clamps the beam to 32 (src/cagra.cpp:186-189);
    the oracle's whole route (entry points, policy, search) against the GPU's
    entry points and beam search under the same policy."""
    b, g, nav = int100k["base"], int100k["graph"], int100k["nav"]
    qs = int100k["qs"][:3]
    beam, iters = oracle.cagra_search_policy(64, 0, 3)
    assert (beam, iters) == (32, 200)
    gn, gd = int100k_index.search_reference(qs, K, beam, iters, int100k_index.entry_points(qs))
    rn, rd = oracle.cagra_reference_search(b, g, nav, qs, K, itopk_size=64, threads=16)
    np.testing.assert_array_equal(gn, rn)
    np.testing.assert_array_equal(gd, rd)


def test_hashed_seed_fallback(int100k, int100k_index, oracle):
    """Without entry nodes each query starts from (q * 2654435761) mod n."""
    b, g, qs = int100k["base"], int100k["graph"], int100k["qs"][:200]
    gn, gd = int100k_index.search_reference(qs, K, 64, 200, None)
    rn, rd = oracle.cagra_search(b, g, qs, K, 64, 200, None, threads=16)
    np.testing.assert_array_equal(gn, rn)
    np.testing.assert_array_equal(gd, rd)


def test_global_visited_bitmap(ctx, oracle):
    """n = 600,000 rows (> 2^19): the visited bitmap lives in device memory,
    one slice per query; a random graph with invalid entries."""
    rng = np.random.default_rng(4)
    n, d, g, q = 600_000, 8, 12, 200
    base = rng.integers(-20, 21, (n, d)).astype(np.float32)
    graph = rng.integers(0, n, (n, g)).astype(np.uint32)
    graph[rng.random((n, g)) < 0.05] = 0xFFFFFFFF
    qs = rng.integers(-20, 21, (q, d)).astype(np.float32)
    entry = rng.integers(0, n, q).astype(np.uint32)
    entry[:5] = 0xFFFFFFFF  # hashed fallback for these
    idx = ctx.cagra_index(base, graph)
    gn, gd = idx.search_reference(qs, K, 96, 120, entry)
    idx.close()
    rn, rd = oracle.cagra_search(base, graph, qs, K, 96, 120, entry, threads=16)
    np.testing.assert_array_equal(gn, rn)
    np.testing.assert_array_equal(gd, rd)


def test_float_data_recall_parity(ctx, cvs, oracle):
    """On the benchmark's (non-integer) distribution the sums differ from
    the reference's in rounding only: the paired recall gate holds, and
    almost every query returns the oracle's ids."""
    n, d, q = 20_000, 256, 500
    base = cvs.synth_clustered(777, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(777, cvs.STREAM_QUERIES, q, d)
    graph = oracle.knn_graph(base, 32, threads=16)
    nav = cvs.cagra_nav_nodes(n)
    idx = ctx.cagra_index(base, graph, nav)
    entry = idx.entry_points(qs)
    gn, gd = idx.search_reference(qs, K, 64, 200, entry)
    idx.close()
    rn, rd = oracle.cagra_reference_search(base, graph, nav, qs, K, itopk_size=64, threads=16)
    gt = exact_knn(base, qs, K)
    assert_recall_not_below(gn, rn, gt, K, "reference mode, float data")
    same = np.array([np.array_equal(gn[i], rn[i]) for i in range(q)])
    assert same.mean() >= 0.95, same.mean()
    np.testing.assert_allclose(gd[same], rd[same], rtol=1e-5)
