"""Pins the restated reference graph build (oracle.cagra_build_reference,
oracle/cagra_build_oracle.c; reference src/metal_context.mm:289-914).

- Exact-seeding path (n <= 50,000, :324-349): on integer-valued data every
  distance is exact, so each row must hold exactly the g nearest other rows
  (ties aside: the data is chosen without ties at the g-th neighbour); the
  20 nn-descent iterations cannot change an exact graph.
- IVF path (50,000 < n <= 200,000): rows full, ids in range, no self edges
  (the reference allows repeated ids from its bucketing merge, so repeats are
  only counted), and most exact neighbours present.
- PQ path (n > 200,000; run here at small n through the size-limit
  arguments): the product quantisation (:437-568) is pinned in closed form
  on data whose 128-dimension slices are drawn from 256 dyadic prototypes
  per subspace laid out so that the evenly strided initial centres are
  exactly the prototypes: k-means converges at once, every code is known,
  and every table entry is an exact fp32 sum.  The PQ seeding graph is in
  range and free of self edges; d < 1024 is refused.
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


def test_pq_path_needs_d1024(oracle):
    """The PQ path reads 8 subspaces of 128 dimensions of every row."""
    with pytest.raises(ValueError):
        oracle.cagra_build_reference(np.zeros((200_001, 1), np.float32), 8)
    with pytest.raises(ValueError):
        oracle.cagra_build_reference(np.zeros((100, 512), np.float32), 8, exact_limit=0, pq_limit=0)


def prototype_rows(seed=3):
    """2048 rows of d = 1024.  Subspace m of row i = 8 c + j holds prototype
    (c + m j) mod 256 of that subspace (256 random multiples of 1/16 in
    [-2, 2]), so each prototype fills exactly 8 rows of each subspace and the
    evenly strided rows 8 c + 4 that seed the centres hold prototypes
    (c + 4 m) mod 256: all 256, once each."""
    rng = np.random.default_rng(seed)
    protos = rng.integers(-32, 33, size=(8, 256, 128)).astype(np.float32) / 16.0
    i = np.arange(2048)
    c, j = i // 8, i % 8
    base = np.empty((2048, 1024), np.float32)
    for m in range(8):
        base[:, 128 * m:128 * (m + 1)] = protos[m][(c + m * j) % 256]
    return base, protos


def test_pq_train_closed_form(oracle):
    """Centres start as the prototypes (centre c = prototype (c + 4 m) mod
    256), every row sits at distance 0 from its own, and each centre's mean
    of 8 identical dyadic slices is that slice exactly, so k-means stops after
    one step: code of row 8 c + j in subspace m = (c + m (j - 4)) mod 256, and
    lut[m][a][b] = |P_m[(a + 4m) % 256] - P_m[(b + 4m) % 256]|^2 exactly."""
    base, protos = prototype_rows()
    codes, lut = oracle.pq_train(base, threads=4)
    i = np.arange(2048)
    c, j = i // 8, i % 8
    for m in range(8):
        assert (codes[:, m] == (c + m * (j - 4)) % 256).all(), m
        p = protos[m][(np.arange(256) + 4 * m) % 256].astype(np.float64)
        want = ((p[:, None, :] - p[None, :, :]) ** 2).sum(-1)
        assert np.array_equal(lut[m].astype(np.float64), want), m


def test_pq_path_graph(oracle, cvs):
    """The PQ seeding (k-means clusters, candidates of the own and 3 nearest
    clusters ranked by table sums, exact distances of the kept entries,
    bucketing, no nn-descent) on clustered data: full rows of in-range ids,
    no self edges, and neighbours well above chance."""
    n, g = 3000, 16
    base = cvs.synth_clustered(11, cvs.STREAM_BASE, n, 1024)
    gr = oracle.cagra_build_reference(base, g, threads=8, exact_limit=0, pq_limit=0)
    assert gr.shape == (n, g) and (gr < n).all()
    assert not (gr == np.arange(n, dtype=np.uint32)[:, None]).any()
    exact = oracle.knn_graph(base, 10, threads=8)
    share = np.mean([len(set(exact[i].tolist()) & set(gr[i].tolist())) / 10 for i in range(0, n, 7)])
    print(f"PQ path: share of exact 10-NN {share:.3f}")
    assert share > 0.3
