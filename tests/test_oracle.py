"""Pins the CPU oracle before it is trusted as the checker of the GPU path.

Checks, in order of strength:
  1. the reference's own known answers (tests/test_l2_distance.cpp:19-49,
     tests/faiss_v1_8_cagra_runtime_smoke.cpp:299-357, and the exact top-4 of
     tests/test_metal_search.cpp:22-28's inputs);
  2. bit-identity with the reference's own CPU code (golden fixtures written
     by tests/golden/make_golden.py from oracle/_ref, and live against
     oracle/_ref where it is built);
  3. fp64 brute force and closed forms on small inputs.
A mistake planted in a copy of the oracle's algorithm must fail these checks
(test_planted_mistakes_are_caught).
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")

# FAISS runtime smoke database and queries (reference test :236-245).
FAISS_DB = np.array([[0, 0], [10, 0], [0, 10], [2, 2]], np.float32)
FAISS_Q = np.array([[0, 0], [9, 1]], np.float32)


def dispatch_test_inputs():
    # tests/test_metal_search.cpp:22-28: base[i, i%8] = i; q[j, j%8] = 1.
    base = np.zeros((64, 8), np.float32)
    for i in range(64):
        base[i, i % 8] = i
    q = np.zeros((4, 8), np.float32)
    for j in range(4):
        q[j, j % 8] = 1
    return base, q


def test_l2_128_known_answers(oracle):
    z = np.zeros(128, np.float32)
    o = np.ones(128, np.float32)
    assert abs(oracle.l2_128(z, o) - 128.0) < 1e-4
    asc = np.arange(128, dtype=np.float32)
    assert abs(oracle.l2_128(asc, asc + 0.5) - 32.0) < 1e-4
    a = np.array([((i % 7) - 3) * 0.25 for i in range(128)], np.float32)
    b = np.array([((i % 5) - 2) * -0.5 for i in range(128)], np.float32)
    expect = float(np.sum((a.astype(np.float64) - b) ** 2))
    assert abs(oracle.l2_128(a, b) - expect) < 1e-4


def test_bf_exact_faiss_known_answers(oracle):
    nbr, dist = oracle.bf_exact(FAISS_DB, FAISS_Q, 2)
    assert nbr.tolist() == [[0, 3], [1, 3]]
    assert dist.tolist() == [[0.0, 8.0], [2.0, 50.0]]
    # Tie at distance 100 resolves to the lower id (reference :326-333).
    nbr, dist = oracle.bf_exact(FAISS_DB, FAISS_Q[:1], 4)
    assert nbr.tolist() == [[0, 3, 1, 2]]
    assert dist.tolist() == [[0.0, 8.0, 100.0, 100.0]]
    # k > N: the last slot is UINT32_MAX / +inf (reference :353-357).
    nbr, dist = oracle.bf_exact(FAISS_DB, FAISS_Q, 5)
    assert nbr[:, 4].tolist() == [0xFFFFFFFF] * 2
    assert np.isinf(dist[:, 4]).all()
    assert nbr[0, 0] == 0 and dist[0, 0] == 0.0


def test_bf_exact_dispatch_test_inputs(oracle):
    base, q = dispatch_test_inputs()
    nbr, dist = oracle.bf_exact(base, q, 4)
    assert nbr.tolist() == [[0, 1, 2, 3], [1, 0, 2, 3], [0, 2, 1, 3], [0, 1, 3, 2]]
    assert dist.tolist() == [[1, 2, 5, 10], [0, 1, 5, 10], [1, 1, 2, 10], [1, 2, 4, 5]]


def test_bf_exact_matches_reference_golden(oracle):
    g = np.load(os.path.join(GOLDEN, "bf_ref.npz"))
    for name in ("random", "ties", "kbig", "wide"):
        nbr, dist = oracle.bf_exact(g[f"{name}_base"], g[f"{name}_queries"], int(g[f"{name}_k"]))
        np.testing.assert_array_equal(nbr, g[f"{name}_nbr"], err_msg=name)
        np.testing.assert_array_equal(dist, g[f"{name}_dist"], err_msg=name)


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(__file__), "..", "oracle", "_ref",
                                                    "libref.so")), reason="oracle/_ref not built here")
def test_bf_exact_bit_identical_to_reference_object(oracle):
    rng = np.random.default_rng(7)
    for n, d, q, k in [(1, 3, 2, 4), (50, 17, 5, 7), (400, 128, 6, 12), (257, 1024, 3, 10)]:
        base = rng.standard_normal((n, d)).astype(np.float32)
        qs = rng.standard_normal((q, d)).astype(np.float32)
        a = oracle.bf_exact(base, qs, k, threads=4)
        b = oracle.ref_bf_search(base, qs, k)
        np.testing.assert_array_equal(a[0], b[0])
        np.testing.assert_array_equal(a[1], b[1])
    for _ in range(3):
        a = rng.standard_normal(128).astype(np.float32)
        b = rng.standard_normal(128).astype(np.float32)
        assert oracle.l2_128(a, b) == oracle.ref().ref_l2_128(a.ctypes.data_as(oracle.c_void_p),
                                                               b.ctypes.data_as(oracle.c_void_p))


def test_bf_exact_against_fp64_brute_force(oracle):
    rng = np.random.default_rng(11)
    base = rng.standard_normal((500, 33)).astype(np.float32)
    qs = rng.standard_normal((8, 33)).astype(np.float32)
    nbr32, d32 = oracle.bf_exact(base, qs, 15)
    full = ((qs.astype(np.float64)[:, None, :] - base.astype(np.float64)[None]) ** 2).sum(-1)
    order = np.lexsort((np.broadcast_to(np.arange(500), full.shape), full), axis=-1)[:, :15]
    np.testing.assert_array_equal(nbr32, order)
    np.testing.assert_allclose(d32, np.take_along_axis(full, order, 1), rtol=1e-5)
    nbr64, d64 = oracle.bf_fp64(base, qs, 15)
    np.testing.assert_array_equal(nbr64, order)
    np.testing.assert_allclose(d64, np.take_along_axis(full, order, 1), rtol=1e-12)


def test_bf_threads_do_not_change_results(oracle):
    rng = np.random.default_rng(3)
    base = rng.standard_normal((300, 20)).astype(np.float32)
    qs = rng.standard_normal((16, 20)).astype(np.float32)
    a = oracle.bf_exact(base, qs, 9, threads=1)
    b = oracle.bf_exact(base, qs, 9, threads=8)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


def _planted_bf(base, qs, k, mistake):
    """A numpy copy of the oracle's algorithm with one planted mistake."""
    diff = qs[:, None, :].astype(np.float64) - base[None].astype(np.float64)
    if mistake == "sign":
        diff = qs[:, None, :].astype(np.float64) + base[None].astype(np.float64)
    d = (diff ** 2).sum(-1)
    if mistake == "dropped_term":
        d = (diff[..., :-1] ** 2).sum(-1)
    ids = np.broadcast_to(np.arange(base.shape[0]), d.shape)
    order = np.lexsort((ids, d), axis=-1)
    if mistake == "tie_order":
        order = np.lexsort((-ids, d), axis=-1)
    return order[:, :k]


@pytest.mark.parametrize("mistake", ["sign", "dropped_term", "tie_order"])
def test_planted_mistakes_are_caught(mistake):
    """The known answers above distinguish each plausible mistake."""
    base, q = dispatch_test_inputs()
    good = [[0, 1, 2, 3], [1, 0, 2, 3], [0, 2, 1, 3], [0, 1, 3, 2]]
    assert _planted_bf(base, q, 4, None).tolist() == good
    assert _planted_bf(base, q, 4, mistake).tolist() != good
