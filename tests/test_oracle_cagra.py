"""Pins the CAGRA-search part of the oracle (oracle/cagra_oracle.c) before it
is trusted as the checker of the GPU graph search.

- Navigation nodes, search policy: closed forms of src/cagra.cpp:65-72 and
  :182-189.
- Entry points: exact nearest navigation node on separated data; the
  first-minimum rule on duplicated vectors (src/cagra.cpp:164-177).
- Beam search (shaders/cagra_kernels.metal:28-199):
  * on a complete graph it is exact search, so the FAISS smoke known answers
    (tests/faiss_v1_8_cagra_runtime_smoke.cpp:299-357) must come out;
  * a hand-traced walk along a path graph;
  * invariants on random data (sorted by (d, id), unique, in range,
    distances equal to the exact fp32 distances of the returned ids);
  * a pure-Python copy of the algorithm agrees with the oracle, and each
    planted mistake in that copy changes an answer above.
- Exact kNN graph: equals bf_exact with k = g + 1 minus the row itself.
"""
import math

import numpy as np
import pytest

INV = 0xFFFFFFFF
FAISS_DB = np.array([[0, 0], [10, 0], [0, 10], [2, 2]], np.float32)
FAISS_Q = np.array([[0, 0], [9, 1]], np.float32)


def test_nav_nodes_closed_form(oracle):
    for n in (1, 10, 40_000, 100_000, 1_000_000):
        m = min(200, int(math.sqrt(n)))
        expect = [int(i * (n / m)) for i in range(m)]
        assert oracle.cagra_nav_nodes(n).tolist() == expect
    assert len(oracle.cagra_nav_nodes(100_000)) == 200
    assert oracle.cagra_nav_nodes(10).tolist() == [0, 3, 6]


def test_search_policy_branches(oracle):
    assert oracle.cagra_search_policy(64, 0, 100) == (64, 200)
    assert oracle.cagra_search_policy(0, 0, 100) == (128, 200)
    assert oracle.cagra_search_policy(512, 600, 1000) == (512, 600)
    assert oracle.cagra_search_policy(64, 0, 4) == (32, 200)
    assert oracle.cagra_search_policy(16, 900, 1) == (16, 200)
    assert oracle.cagra_search_policy(64, 0, 5) == (64, 200)


def test_entry_points(oracle):
    nav_vec = np.array([[0, 0], [10, 0], [0, 10], [10, 10]], np.float32)
    nav_ids = np.array([5, 9, 11, 20], np.uint32)
    qs = np.array([[1, 1], [9, 2], [-3, 12], [7, 8]], np.float32)
    assert oracle.cagra_entry_points(qs, nav_ids, nav_vec).tolist() == [5, 9, 11, 20]
    # duplicated navigation vectors: the first minimum wins
    dup = np.array([[1, 1], [1, 1], [5, 5]], np.float32)
    assert oracle.cagra_entry_points(qs[:1], np.array([7, 3, 1], np.uint32), dup).tolist() == [7]


def complete_graph(n):
    return np.array([[j for j in range(n) if j != i] for i in range(n)], np.uint32)


def test_complete_graph_is_exact_search(oracle):
    g = complete_graph(4)
    nbr, dist = oracle.cagra_search(FAISS_DB, g, FAISS_Q, 2, beam=4, max_iter=10)
    assert nbr.tolist() == [[0, 3], [1, 3]]
    assert dist.tolist() == [[0.0, 8.0], [2.0, 50.0]]
    nbr, dist = oracle.cagra_search(FAISS_DB, g, FAISS_Q[:1], 4, beam=4, max_iter=10)
    assert nbr.tolist() == [[0, 3, 1, 2]] and dist.tolist() == [[0.0, 8.0, 100.0, 100.0]]
    nbr, dist = oracle.cagra_search(FAISS_DB, g, FAISS_Q, 5, beam=4, max_iter=10)
    assert nbr[:, 4].tolist() == [INV, INV] and np.isinf(dist[:, 4]).all()


def path_case():
    # points (i, 0), i = 0..19; i links to i-1 and i+1 (missing ends = UINT32_MAX)
    base = np.stack([np.arange(20), np.zeros(20)], 1).astype(np.float32)
    graph = np.array([[i - 1 if i > 0 else INV, i + 1 if i < 19 else INV] for i in range(20)], np.uint32)
    q = np.array([[7, 1]], np.float32)
    return base, graph, q


def fork_case():
    # 0 at the origin links to 1 (1, 0) and 2 (-1, 0); 1 -> 3 (2, 0); 2 -> 4 (-2, 0)
    base = np.array([[0, 0], [1, 0], [-1, 0], [2, 0], [-2, 0]], np.float32)
    graph = np.array([[1, 2], [0, 3], [0, 4], [1, INV], [2, INV]], np.uint32)
    q = np.array([[3, 0]], np.float32)
    return base, graph, q


def test_fork_graph_hand_trace(oracle):
    # Entry 0 (d 9), beam 3.  Iteration 1 expands 0: 1 (d 4) and 2 (d 16)
    # enter.  Iteration 2 expands the closer unexpanded entry, 1: its
    # neighbour 3 (d 1) replaces the worst entry, 2.
    base, graph, q = fork_case()
    nbr, dist = oracle.cagra_search(base, graph, q, 3, beam=3, max_iter=2, entry=np.array([0], np.uint32))
    assert nbr.tolist() == [[3, 1, 0]] and dist.tolist() == [[1.0, 4.0, 9.0]]
    # a beam of 2 evicts 0's replacement slot instead: 2 is never kept
    nbr, dist = oracle.cagra_search(base, graph, q, 3, beam=2, max_iter=10, entry=np.array([0], np.uint32))
    assert nbr.tolist() == [[3, 1, INV]] and dist[0, :2].tolist() == [1.0, 4.0]


def test_path_graph_hand_trace(oracle):
    # Entry 0, beam 3: the walk reaches 7; the beam then holds 7 (d 1),
    # 6 (d 2) and 8 (d 2); 9 (d 5) is not better than the worst (2).
    base, graph, q = path_case()
    nbr, dist = oracle.cagra_search(base, graph, q, 3, beam=3, max_iter=100, entry=np.array([0], np.uint32))
    assert nbr.tolist() == [[7, 6, 8]]
    assert dist.tolist() == [[1.0, 2.0, 2.0]]
    # too few iterations: after 3 expansions (0, 1, 2) the beam holds 1, 2, 3
    nbr, _ = oracle.cagra_search(base, graph, q, 3, beam=3, max_iter=3, entry=np.array([0], np.uint32))
    assert nbr.tolist() == [[3, 2, 1]]


def py_beam_search(base, graph, q, k, beam, max_iter, entry, mistake=None):
    """Pure-Python copy of the reference beam search with optional planted
    mistakes (the checker of the checker)."""
    n = len(base)
    cd = [math.inf] * beam
    cn = [INV] * beam
    seed = entry
    cd[0] = float(((q - base[seed]) ** 2).sum())
    cn[0] = seed
    visited = {seed}
    for _ in range(max_iter):
        bd, bn = math.inf, INV
        for i in range(beam):
            c = cd[i]
            if mistake == "expand_worst":
                if c >= 0 and (bn == INV or c > bd) and c != math.inf:
                    bd, bn = c, cn[i]
            elif c >= 0 and c < bd:
                bd, bn = c, cn[i]
        if bn == INV:
            break
        for i in range(beam):
            if cn[i] == bn:
                cd[i] = -cd[i] - 1
                break
        for nb in graph[bn]:
            nb = int(nb)
            if nb >= n:
                continue
            if nb in visited and mistake != "no_visited":
                continue
            visited.add(nb)
            d = float(((q - base[nb]) ** 2).sum())
            worst, widx = 0.0, beam
            for i in range(beam):
                a = -cd[i] - 1 if cd[i] < 0 else cd[i]
                if a > worst:
                    worst, widx = a, i
            if widx < beam and d < worst:
                cd[widx], cn[widx] = d, nb
    out = sorted(((-c - 1 if c < 0 else c), n_) for c, n_ in zip(cd, cn) if n_ != INV)
    if mistake == "tie_order":
        out = sorted(out, key=lambda t: (t[0], -t[1]))
    out = out[:k]
    return [t[1] for t in out] + [INV] * (k - len(out))


@pytest.mark.parametrize("mistake", [None, "expand_worst", "no_visited", "tie_order"])
def test_python_copy_agrees_and_planted_mistakes_fail(oracle, mistake):
    """The path- and fork-graph known answers reproduce in the Python copy,
    and each planted mistake changes at least one of them."""
    base, graph, q = path_case()
    fb, fg, fq = fork_case()
    got = [py_beam_search(base, graph, q[0], 3, 3, it, 0, mistake) for it in (100, 3)]
    got += [py_beam_search(fb, fg, fq[0], 3, beam, it, 0, mistake) for beam, it in ((3, 2), (2, 10))]
    expect = [[7, 6, 8], [3, 2, 1], [3, 1, 0], [3, 1, INV]]
    if mistake is None:
        assert got == expect
    else:
        assert got != expect


def test_python_copy_matches_oracle_on_random_graphs(oracle):
    rng = np.random.default_rng(5)
    base = rng.integers(-3, 4, size=(60, 5)).astype(np.float32)
    graph = rng.integers(0, 60, size=(60, 6)).astype(np.uint32)
    graph[rng.random(graph.shape) < 0.1] = INV
    qs = rng.integers(-3, 4, size=(10, 5)).astype(np.float32)
    entry = rng.integers(0, 60, size=10).astype(np.uint32)
    nbr, _ = oracle.cagra_search(base, graph, qs, 5, beam=8, max_iter=30, entry=entry)
    for i in range(10):
        assert nbr[i].tolist() == py_beam_search(base, graph, qs[i], 5, 8, 30, int(entry[i]))


def test_invariants_on_random_data(oracle):
    rng = np.random.default_rng(9)
    base = rng.standard_normal((800, 24)).astype(np.float32)
    qs = rng.standard_normal((20, 24)).astype(np.float32)
    graph = oracle.knn_graph(base, 12, threads=4)
    nav = oracle.cagra_nav_nodes(len(base))
    nbr, dist = oracle.cagra_reference_search(base, graph, nav, qs, 10, itopk_size=32, threads=4)
    for i in range(len(qs)):
        ids = nbr[i][nbr[i] != INV]
        assert len(set(ids.tolist())) == len(ids) and (ids < len(base)).all()
        exact = ((base[ids].astype(np.float64) - qs[i]) ** 2).sum(1)
        np.testing.assert_allclose(dist[i][: len(ids)], exact, rtol=1e-5)
        assert all(dist[i][j] <= dist[i][j + 1] for j in range(len(ids) - 1))
    exact_nbr, _ = oracle.bf_exact(base, qs, 10)
    recall = np.mean([len(set(nbr[i]) & set(exact_nbr[i])) / 10 for i in range(len(qs))])
    assert recall > 0.8


def test_knn_graph_matches_brute_force(oracle):
    rng = np.random.default_rng(2)
    base = rng.standard_normal((150, 9)).astype(np.float32)
    g = oracle.knn_graph(base, 7, threads=3)
    nbr, _ = oracle.bf_exact(base, base, 8)
    for i in range(150):
        expect = [j for j in nbr[i].tolist() if j != i][:7]
        assert g[i].tolist() == expect
    tiny = oracle.knn_graph(FAISS_DB, 5)
    assert (tiny[:, 3:] == INV).all() and (tiny[:, :3] != INV).all()


def test_edge_distances_pinned(oracle):
    """recompute_graph_distances restated: numpy fp64 distances on a random
    graph with d a multiple of 4; the reference's D >> 2 loop reads only the
    first 4*floor(d/4) columns (d = 6: columns 4 and 5 are ignored); +inf for
    UINT32_MAX and out-of-range ids."""
    rng = np.random.default_rng(658)
    n, d, g = 300, 64, 12
    rows = rng.standard_normal((n, d)).astype(np.float32)
    graph = rng.integers(0, n, (n, g)).astype(np.uint32)
    graph[3, 5] = 0xFFFFFFFF
    graph[7, 0] = n + 5
    got = oracle.edge_distances(rows, graph, threads=4)
    ok = graph < n
    ref = ((rows.astype(np.float64)[:, None, :] - rows.astype(np.float64)[np.where(ok, graph, 0)]) ** 2).sum(-1)
    np.testing.assert_allclose(got[ok], ref[ok], rtol=2e-6, atol=1e-6)
    assert np.isinf(got[~ok]).all() and (~ok).sum() == 2
    # d = 6: the last two columns do not count
    small = np.array([[0, 0, 0, 0, 5, 5], [1, 2, 2, 0, -7, 9]], np.float32)
    out = oracle.edge_distances(small, np.array([[1], [0]], np.uint32))
    assert out.tolist() == [[9.0], [9.0]]
