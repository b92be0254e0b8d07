"""Writes the golden fixtures of this directory from the reference's own CPU
code (oracle/_ref/libref.so, compiled in place from the reference's
src/cagra.cpp and src/distance.cpp by oracle/Makefile).

Run from the repository root:  python tests/golden/make_golden.py

Fixtures (inputs and the reference's outputs only):
  bf_ref.npz        exact k-NN cases: random, integer-valued with ties,
                    k > n, d not a multiple of 32
  cgra_ref_v1.bin   CGRA v1 index written by the reference's save_index
                    (dataset + graph + navigation nodes)
  cgra_ref_v1_nods.bin  same without dataset and navigation nodes
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402


def main():
    if not oracle.have_reference():
        oracle.build(with_reference=True)
    rng = np.random.default_rng(20241201)
    cases = {}

    def add(name, base, queries, k):
        nbr, dist = oracle.ref_bf_search(base, queries, k)
        cases[f"{name}_base"] = base
        cases[f"{name}_queries"] = queries
        cases[f"{name}_k"] = np.array(k)
        cases[f"{name}_nbr"] = nbr
        cases[f"{name}_dist"] = dist

    add("random", rng.standard_normal((200, 40)).astype(np.float32),
        rng.standard_normal((9, 40)).astype(np.float32), 10)
    ties_base = rng.integers(-2, 3, size=(128, 6)).astype(np.float32)
    add("ties", ties_base, rng.integers(-2, 3, size=(11, 6)).astype(np.float32), 16)
    add("kbig", rng.standard_normal((5, 33)).astype(np.float32),
        rng.standard_normal((3, 33)).astype(np.float32), 8)
    add("wide", rng.standard_normal((24, 1000)).astype(np.float32),
        rng.standard_normal((3, 1000)).astype(np.float32), 5)
    np.savez_compressed(os.path.join(HERE, "bf_ref.npz"), **cases)

    lib = oracle.ref()
    n, d, g = 6, 3, 2
    ds = (np.arange(n * d, dtype=np.float32) * 0.5 - 2.0).reshape(n, d)
    graph = np.array([[1, 2], [0, 2], [1, 3], [2, 4], [3, 5], [4, 0]], dtype=np.uint32)
    nav = np.array([0, 3], dtype=np.uint32)
    nav_vec = ds[nav].copy()
    p = lambda a: a.ctypes.data_as(oracle.c_void_p)
    rc = lib.ref_save_index(os.path.join(HERE, "cgra_ref_v1.bin").encode(), p(ds), n, d, p(graph), g, p(nav), 2,
                            p(nav_vec))
    assert rc == 0
    rc = lib.ref_save_index(os.path.join(HERE, "cgra_ref_v1_nods.bin").encode(), None, n, d, p(graph), g, None, 0,
                            None)
    assert rc == 0
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
