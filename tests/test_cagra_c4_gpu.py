"""Graph search at the benchmark's configuration, N=100,000 D=1024 fp32,
degree 64, itopk 64, K=10, on the graph the restated reference build makes
(IVF seeding + random bucketing + 5 nn-descent iterations, the reference's
path for 50,000 < N <= 200,000; src/metal_context.mm:289-914) and the
reference's navigation nodes (src/cagra.cpp:63-72).

Each case runs the kernel instance the benchmark runs and is gated against
the restated reference search (oracle.cagra_reference_search: nearest
navigation node entry, beam of itopk; shaders/cagra_kernels.metal:28-199) on
the same graph, navigation nodes and queries, with the paired recall gate of
tests/search_metrics.py, plus the output invariants:
- Q = 10,000 in one call: two waves per query (the throughput kernel), fp32
  and fp16 traversal, search widths 1 and 4;
- Q = 1, 100 separate calls: eight waves per query (the latency kernel);
- 8 teams per query, each with a list of itopk 64, Q = 1,000 and Q = 1.
Ground truth: exact k-NN by numpy (fp64 re-scored), not by this library.
"""
import numpy as np
import pytest

from search_metrics import assert_recall_not_below, exact_knn, recall
from test_cagra_gpu import check_invariants

pytestmark = pytest.mark.gpu

N, D, Q, K, ITOPK, DEGREE = 100_000, 1024, 10_000, 10, 64, 64


@pytest.fixture(scope="module")
def c4(cvs, oracle):
    print("[c4] building the restated reference graph", flush=True)
    base = cvs.synth_clustered(12345, cvs.STREAM_BASE, N, D)
    qs = cvs.synth_clustered(12345, cvs.STREAM_QUERIES, Q, D)
    graph = oracle.cagra_build_reference(base, DEGREE, threads=16)
    nav = cvs.cagra_nav_nodes(N)
    assert np.array_equal(nav, oracle.cagra_nav_nodes(N))
    print("[c4] exact ground truth", flush=True)
    gt = exact_knn(base, qs, K)
    print("[c4] restated reference search", flush=True)
    ref, _ = oracle.cagra_reference_search(base, graph, nav, qs, K, itopk_size=ITOPK, threads=16)
    print(f"[c4] reference recall@10 {recall(ref, gt, K):.4f}", flush=True)
    return dict(base=base, qs=qs, graph=graph, nav=nav, gt=gt, ref=ref)


@pytest.fixture(scope="module")
def c4_index(ctx, c4):
    idx = ctx.cagra_index(c4["base"], c4["graph"], c4["nav"])
    yield idx
    idx.close()


@pytest.mark.parametrize("bits,width", [(32, 1), (32, 4), (16, 1), (16, 4)])
def test_c4_batch_of_10000(c4, c4_index, bits, width):
    print(f"[c4] Q=10,000 bits={bits} width={width}", flush=True)
    c4_index.set_traversal(bits)
    nbr, dist = c4_index.search(c4["qs"], K, itopk_size=ITOPK, search_width=width)
    check_invariants(c4["base"], c4["qs"][::50], nbr[::50], dist[::50])
    assert_recall_not_below(nbr, c4["ref"], c4["gt"], K, f"N=100K Q=10,000 {bits}-bit width {width}")
    assert recall(nbr, c4["gt"], K) >= 0.95


@pytest.mark.parametrize("bits", [32, 16])
def test_c4_single_query_calls(c4, c4_index, bits):
    print(f"[c4] Q=1 x 100 bits={bits}", flush=True)
    c4_index.set_traversal(bits)
    qs = c4["qs"][:100]
    rows = [c4_index.search(qs[i:i + 1], K, itopk_size=ITOPK) for i in range(100)]
    nbr = np.concatenate([r[0] for r in rows])
    dist = np.concatenate([r[1] for r in rows])
    check_invariants(c4["base"], qs, nbr, dist)
    assert_recall_not_below(nbr, c4["ref"][:100], c4["gt"][:100], K, f"N=100K Q=1 x 100 {bits}-bit")


@pytest.mark.parametrize("q", [1000, 1])
def test_c4_teams(c4, c4_index, q):
    print(f"[c4] 8 teams x itopk 64, Q={q}", flush=True)
    c4_index.set_traversal(16)
    qs = c4["qs"][:q] if q > 1 else c4["qs"][:100]
    if q > 1:
        nbr, dist = c4_index.search_teams(qs, K, 8, itopk_size=ITOPK)
    else:
        rows = [c4_index.search_teams(qs[i:i + 1], K, 8, itopk_size=ITOPK) for i in range(len(qs))]
        nbr = np.concatenate([r[0] for r in rows])
        dist = np.concatenate([r[1] for r in rows])
    check_invariants(c4["base"], qs, nbr, dist)
    assert_recall_not_below(nbr, c4["ref"][:len(qs)], c4["gt"][:len(qs)], K, f"N=100K 8 teams, {len(qs)} queries")


def test_c4_own_build_at_least_reference_graph(ctx, c4):
    """This library's graph build (random bucketing + nn-descent + pruning,
    intermediate degree 128 -> 64) at the same size: GPU search on it at
    itopk 64 reaches at least the restated reference search on the restated
    reference graph (equal degree and itopk), 10,000 queries, paired gate."""
    print("[c4] this library's build at N=100K", flush=True)
    graph, st = ctx.cagra_build(c4["base"], intermediate_degree=128, graph_degree=DEGREE)
    idx = ctx.cagra_index(c4["base"], graph, c4["nav"], traversal_bits=32)
    nbr, _ = idx.search(c4["qs"], K, itopk_size=ITOPK)
    idx.close()
    assert_recall_not_below(nbr, c4["ref"], c4["gt"], K,
                            f"N=100K own build ({st['iterations']} nn-descent iterations) vs reference graph")
