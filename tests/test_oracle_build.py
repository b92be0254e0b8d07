"""Pins the restated reference graph build (oracle.cagra_build_reference,
oracle/cagra_build_oracle.c; reference src/metal_context.mm:289-914).

- Exact-seeding path (n <= 50,000, :324-349): on integer-valued data every
  distance is exact, so each row must hold exactly the g nearest other rows
  (ties aside: the data is chosen without ties at the g-th neighbour); the
  20 nn-descent iterations cannot change an exact graph.
- IVF path (50,000 < n <= 200,000): rows full, ids in range, no self edges
  (the reference allows repeated ids from its bucketing merge, so repeats are
  only counted), and most exact neighbours present.
- n > 200,000 is refused (the PQ path is not restated).
"""
import numpy as np
import pytest

INV = 0xFFFFFFFF


def test_exact_path_equals_exact_knn_graph(oracle):
    rng = np.random.default_rng(31)
    # integer points in 4-d (the reference's float4 distance ignores d % 4
    # trailing columns, so d is a multiple of 4)
    x = rng.permutation(np.arange(300))[:120].reshape(-1, 1).astype(np.float32)
    base = np.concatenate([x, (x * 7) % 13, (x * 3) % 5, (x * x) % 11], 1).astype(np.float32)
    g = 6
    got = oracle.cagra_build_reference(base, g, threads=4)
    exact = oracle.knn_graph(base, g + 2, threads=4)
    d = ((base[:, None, :].astype(np.float64) - base[None]) ** 2).sum(-1)
    for i in range(len(base)):
        # compare as sets where the g-th and (g+1)-th exact distances differ
        dk, dk1 = d[i, exact[i, g - 1]], d[i, exact[i, g]]
        if dk != dk1:
            assert set(got[i].tolist()) == set(exact[i, :g].tolist()), i
        assert i not in got[i]


def test_small_n_degree_clamp(oracle):
    base = np.arange(20, dtype=np.float32).reshape(5, 4)
    g = oracle.cagra_build_reference(base, 64)
    assert g.shape == (5, 4)
    for i in range(5):
        assert sorted(g[i].tolist()) == [j for j in range(5) if j != i]


def ivf_case():
    rng = np.random.default_rng(5)
    c = rng.standard_normal((40, 8)).astype(np.float32)
    base = c[rng.integers(0, 40, 50_500)] + 0.2 * rng.standard_normal((50_500, 8)).astype(np.float32)
    return base


def test_ivf_path_quality(oracle):
    base = ivf_case()
    g = oracle.cagra_build_reference(base, 16, threads=8)
    n = len(base)
    assert g.shape == (n, 16)
    assert (g < n).all()
    assert not (g == np.arange(n)[:, None]).any()
    rows = np.random.default_rng(1).choice(n, 400, replace=False)
    exact = oracle.knn_graph(base, 10, threads=8)  # rows only used below
    share = np.mean([len(set(exact[i].tolist()) & set(g[i].tolist())) / 10 for i in rows])
    repeats = np.mean([16 - len(set(g[i].tolist())) for i in rows])
    print(f"share of exact 10-NN: {share:.3f}, mean repeated ids per row {repeats:.3f}")
    assert share > 0.9


def test_refuses_pq_path(oracle):
    with pytest.raises(ValueError):
        oracle.cagra_build_reference(np.zeros((200_001, 1), np.float32), 8)
