"""ctypes access to the oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only to check results against it (or, in
bench.py, to time the reference CPU path).

- liboracle.so: the C restatement of the reference search path (oracle.h).
- _ref/libref.so: the reference's own CPU sources compiled in place
  (src/cagra.cpp, src/distance.cpp) behind ref_shim.cpp; present only where
  it was built (it needs the reference sources at build time).
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import subprocess
from ctypes import POINTER, byref, c_char_p, c_float, c_int, c_int64, c_uint32, c_uint64, c_void_p

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(ORACLE_DIR, "liboracle.so")
REF_LIB = os.path.join(ORACLE_DIR, "_ref", "libref.so")
REFERENCE_DIR = os.environ.get("CVS_REFERENCE_DIR", "/root/reference")

_lib = None
_ref = None


def build(with_reference: bool | None = None) -> None:
    """Builds liboracle.so, and _ref/libref.so when the reference sources exist."""
    subprocess.run(["make", "-s", "-C", ORACLE_DIR, "all"], check=True)
    if with_reference is None:
        with_reference = os.path.exists(os.path.join(REFERENCE_DIR, "src", "cagra.cpp"))
    if with_reference:
        subprocess.run(["make", "-s", "-C", ORACLE_DIR, "ref", f"REFERENCE={REFERENCE_DIR}"], check=True)


def build_variant(plant: int, out_dir: str) -> str:
    """Compiles a copy of liboracle.so with mistake number `plant` switched
    on (ORACLE_PLANT in the C sources) into out_dir; returns its path.  For
    the pinning tests, which show that their known answers reject it."""
    out = os.path.join(out_dir, f"liboracle_plant{int(plant)}.so")
    srcs = [os.path.join(ORACLE_DIR, f) for f in ("bf_oracle.c", "cagra_oracle.c", "cagra_build_oracle.c")]
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-ffp-contract=off", "-fopenmp", "-w", "-shared",
                    f"-DORACLE_PLANT={int(plant)}", *srcs, "-lm", "-o", out], check=True)
    return out


@contextlib.contextmanager
def variant(path: str):
    """Routes every oracle call through another build of liboracle.so (a
    planted-mistake copy from build_variant) inside the `with` block."""
    global _lib
    saved = _lib
    _lib = _configure(ctypes.CDLL(path))
    try:
        yield
    finally:
        _lib = saved


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_LIB):
            build(with_reference=False)
        _lib = _configure(ctypes.CDLL(ORACLE_LIB))
    return _lib


def _configure(L: ctypes.CDLL) -> ctypes.CDLL:
    """Declares the C signatures of a loaded liboracle.so."""
    L.oracle_l2_128.restype = c_float
    L.oracle_l2_128.argtypes = [c_void_p, c_void_p]
    for name in ("oracle_bf_exact", "oracle_bf_fp64"):
        fn = getattr(L, name)
        fn.restype = None
        fn.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int]
    L.oracle_cagra_nav_nodes.restype = c_int64
    L.oracle_cagra_nav_nodes.argtypes = [c_int64, c_void_p]
    L.oracle_cagra_entry_points.restype = None
    L.oracle_cagra_entry_points.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_void_p]
    L.oracle_cagra_search_policy.restype = None
    L.oracle_cagra_search_policy.argtypes = [c_uint64, c_uint64, c_int64, POINTER(c_uint32), POINTER(c_uint32)]
    L.oracle_cagra_search.restype = None
    L.oracle_cagra_search.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_uint32, c_void_p, c_int64,
                                      c_void_p, c_int64, c_uint32, c_uint32, c_void_p, c_void_p, c_int]
    L.oracle_cagra_build_ref.restype = c_int
    L.oracle_cagra_build_ref.argtypes = [c_void_p, c_int64, c_int64, c_uint32, c_void_p, c_int]
    L.oracle_cagra_build_ref_ex.restype = c_int
    L.oracle_cagra_build_ref_ex.argtypes = [c_void_p, c_int64, c_int64, c_uint32, c_void_p, c_int, c_int64,
                                            c_int64]
    L.oracle_pq_train.restype = None
    L.oracle_pq_train.argtypes = [c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p]
    L.oracle_kmeans_init.restype = None
    L.oracle_kmeans_init.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_void_p]
    L.oracle_ivf_kmeans.restype = c_int
    L.oracle_ivf_kmeans.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_int, c_void_p, c_void_p, c_int]
    L.oracle_ivf_near_clusters.restype = None
    L.oracle_ivf_near_clusters.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int]
    L.oracle_ivf_seed.restype = None
    L.oracle_ivf_seed.argtypes = [c_void_p, c_int64, c_int64, c_uint32, c_void_p, c_int64, c_void_p, c_int64,
                                  c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int]
    L.oracle_bucketing_perm.restype = None
    L.oracle_bucketing_perm.argtypes = [c_int64, c_void_p]
    L.oracle_bucketing_merge.restype = None
    L.oracle_bucketing_merge.argtypes = [c_void_p, c_int64, c_int64, c_uint32, c_void_p, c_int64, c_void_p,
                                         c_void_p, c_int]
    L.oracle_nn_descent.restype = c_int
    L.oracle_nn_descent.argtypes = [c_void_p, c_int64, c_int64, c_uint32, c_void_p, c_void_p, c_uint32, c_int]
    L.oracle_knn_graph.restype = None
    L.oracle_knn_graph.argtypes = [c_void_p, c_int64, c_int64, c_uint32, c_void_p, c_int]
    L.oracle_edge_distances.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_uint32, c_void_p, c_int]
    return L


def have_reference() -> bool:
    return os.path.exists(REF_LIB)


def ref() -> ctypes.CDLL:
    global _ref
    if _ref is None:
        if not have_reference():
            raise FileNotFoundError(REF_LIB)
        L = ctypes.CDLL(REF_LIB)
        L.ref_bf_search.restype = c_int
        L.ref_bf_search.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p]
        L.ref_l2_128.restype = c_float
        L.ref_l2_128.argtypes = [c_void_p, c_void_p]
        L.ref_save_index.restype = c_int
        L.ref_save_index.argtypes = [c_char_p, c_void_p, c_int64, c_int64, c_void_p, c_uint32, c_void_p, c_uint32,
                                     c_void_p]
        L.ref_load_index.restype = c_int
        L.ref_load_index.argtypes = [c_char_p, POINTER(c_int64), POINTER(c_int64), POINTER(c_uint32),
                                     POINTER(c_int64), c_void_p, c_void_p, c_void_p, c_void_p, POINTER(c_int)]
        _ref = L
    return _ref


def _p(a):
    return a.ctypes.data_as(c_void_p)


def l2_128(a, b) -> float:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return float(lib().oracle_l2_128(_p(a), _p(b)))


def bf_exact(base, queries, k: int, threads: int = 1):
    """Reference CPU search loop restated (src/cagra.cpp:211-252)."""
    base = np.ascontiguousarray(base, np.float32)
    queries = np.ascontiguousarray(queries, np.float32)
    n, d = base.shape
    q = queries.shape[0]
    nbr = np.empty((q, k), np.uint32)
    dist = np.empty((q, k), np.float32)
    lib().oracle_bf_exact(_p(base), n, d, _p(queries), q, k, _p(nbr), _p(dist), int(threads))
    return nbr, dist


def bf_fp64(base, queries, k: int, threads: int = 1):
    base = np.ascontiguousarray(base, np.float32)
    queries = np.ascontiguousarray(queries, np.float32)
    n, d = base.shape
    q = queries.shape[0]
    nbr = np.empty((q, k), np.uint32)
    dist = np.empty((q, k), np.float64)
    lib().oracle_bf_fp64(_p(base), n, d, _p(queries), q, k, _p(nbr), _p(dist), int(threads))
    return nbr, dist


def ref_bf_search(base, queries, k: int):
    """The reference's own CPU path (src/cagra.cpp:211-252), from oracle/_ref."""
    base = np.ascontiguousarray(base, np.float32)
    queries = np.ascontiguousarray(queries, np.float32)
    n, d = base.shape
    q = queries.shape[0]
    nbr = np.empty((q, k), np.uint32)
    dist = np.empty((q, k), np.float32)
    rc = ref().ref_bf_search(_p(base), n, d, _p(queries), q, k, _p(nbr), _p(dist))
    if rc == 1:
        raise ValueError("reference raised std::invalid_argument")
    if rc != 0:
        raise RuntimeError("reference raised an exception")
    return nbr, dist


# ---- CAGRA search (oracle/cagra_oracle.c) ----------------------------------

def cagra_nav_nodes(n: int) -> np.ndarray:
    """Navigation node ids of an n-row index (src/cagra.cpp:65-72)."""
    m = int(lib().oracle_cagra_nav_nodes(int(n), None))
    out = np.empty(m, np.uint32)
    lib().oracle_cagra_nav_nodes(int(n), _p(out))
    return out


def cagra_entry_points(queries, nav_ids, nav_vectors) -> np.ndarray:
    """Per-query entry node: nearest navigation node (src/cagra.cpp:133-177)."""
    queries = np.ascontiguousarray(queries, np.float32)
    nav_ids = np.ascontiguousarray(nav_ids, np.uint32)
    nav_vectors = np.ascontiguousarray(nav_vectors, np.float32)
    q, d = queries.shape
    out = np.empty(q, np.uint32)
    lib().oracle_cagra_entry_points(_p(queries), q, d, _p(nav_ids), _p(nav_vectors), len(nav_ids), _p(out))
    return out


def cagra_search_policy(itopk_size: int, max_iterations: int, q: int):
    """(beam, iterations) chosen by the reference (src/cagra.cpp:182-189)."""
    b, it = c_uint32(0), c_uint32(0)
    lib().oracle_cagra_search_policy(int(itopk_size), int(max_iterations), int(q), byref(b), byref(it))
    return b.value, it.value


def cagra_search(base, graph, queries, k: int, beam: int, max_iter: int, entry=None, threads: int = 1):
    """The reference's beam search (shaders/cagra_kernels.metal:28-199)."""
    base = np.ascontiguousarray(base, np.float32)
    graph = np.ascontiguousarray(graph, np.uint32)
    queries = np.ascontiguousarray(queries, np.float32)
    n, d = base.shape
    q = queries.shape[0]
    g = graph.shape[1] if graph.ndim == 2 else 0
    ent = None if entry is None else np.ascontiguousarray(entry, np.uint32)
    nbr = np.empty((q, k), np.uint32)
    dist = np.empty((q, k), np.float32)
    lib().oracle_cagra_search(_p(base), n, d, _p(graph), g, _p(queries), q, None if ent is None else _p(ent),
                              int(k), int(beam), int(max_iter), _p(nbr), _p(dist), int(threads))
    return nbr, dist


def cagra_reference_search(base, graph, nav_ids, queries, k: int, itopk_size: int = 64,
                           max_iterations: int = 0, threads: int = 1):
    """The reference's whole search route for an index with a graph: entry
    points from the navigation nodes, the beam/iteration policy, beam search
    (src/cagra.cpp:128-196)."""
    base = np.ascontiguousarray(base, np.float32)
    nav_ids = np.ascontiguousarray(nav_ids, np.uint32)
    entry = cagra_entry_points(queries, nav_ids, base[nav_ids]) if len(nav_ids) else None
    beam, iters = cagra_search_policy(itopk_size, max_iterations, len(queries))
    return cagra_search(base, graph, queries, k, beam, iters, entry, threads)


def edge_distances(rows, graph, threads: int = 1) -> np.ndarray:
    """The reference's recompute_graph_distances restated
    (shaders/cagra_kernels.metal:658-681)."""
    rows = np.ascontiguousarray(rows, np.float32)
    graph = np.ascontiguousarray(graph, np.uint32)
    n, d = rows.shape
    g = graph.shape[1]
    out = np.empty((n, g), np.float32)
    lib().oracle_edge_distances(_p(rows), n, d, _p(graph), int(g), _p(out), int(threads))
    return out


def knn_graph(base, g: int, threads: int = 1) -> np.ndarray:
    """Exact degree-g kNN graph without self edges."""
    base = np.ascontiguousarray(base, np.float32)
    n, d = base.shape
    out = np.empty((n, g), np.uint32)
    lib().oracle_knn_graph(_p(base), n, d, int(g), _p(out), int(threads))
    return out


def cagra_build_reference(base, graph_degree: int = 64, threads: int = 1, exact_limit: int = 50000,
                          pq_limit: int = 200000) -> np.ndarray:
    """The reference's graph build restated (src/metal_context.mm:289-914):
    returns n x min(graph_degree, n - 1) uint32 ids.  exact_limit / pq_limit
    are the size limits of its phases (the reference's: 50,000 and 200,000)."""
    base = np.ascontiguousarray(base, np.float32)
    n, d = base.shape
    g = min(int(graph_degree), n - 1)
    out = np.empty((n, max(g, 0)), np.uint32)
    rc = lib().oracle_cagra_build_ref_ex(_p(base), n, d, int(graph_degree), _p(out), int(threads), int(exact_limit),
                                         int(pq_limit))
    if rc == 2:
        raise ValueError("product-quantised seeding needs d >= 1024")
    if rc != 0:
        raise ValueError("invalid arguments")
    return out


def pq_train(base, threads: int = 1):
    """Product quantisation of the build's PQ path (src/metal_context.mm:
    437-568): returns (codes n x 8 uint8, lut 8 x 256 x 256 float32)."""
    base = np.ascontiguousarray(base, np.float32)
    n, d = base.shape
    if d < 1024:
        raise ValueError("product quantisation reads 8 x 128 dimensions")
    codes = np.empty((n, 8), np.uint8)
    lut = np.empty((8, 256, 256), np.float32)
    lib().oracle_pq_train(_p(base), n, d, int(threads), _p(codes), _p(lut))
    return codes, lut


# ---- stages of the restated reference build --------------------------------

def _empty_graph(n: int, g: int):
    return np.full((n, g), 0xFFFFFFFF, np.uint32), np.full((n, g), np.inf, np.float32)


def kmeans_init(base, K: int) -> np.ndarray:
    """Initial IVF centres (src/metal_context.mm:366-375)."""
    base = np.ascontiguousarray(base, np.float32)
    n, d = base.shape
    out = np.empty((K, d), np.float32)
    lib().oracle_kmeans_init(_p(base), n, d, int(K), _p(out))
    return out


def ivf_kmeans(base, centres, max_iter: int = 20, threads: int = 1):
    """Lloyd iterations from `centres` (src/metal_context.mm:381-435):
    returns (centres, assignment, E-steps run)."""
    base = np.ascontiguousarray(base, np.float32)
    cent = np.array(centres, np.float32, copy=True, order="C")
    n, d = base.shape
    assign = np.empty(n, np.uint32)
    it = lib().oracle_ivf_kmeans(_p(base), n, d, cent.shape[0], int(max_iter), _p(cent), _p(assign), int(threads))
    return cent, assign, int(it)


def ivf_near_clusters(centres, n_probe: int = 3, threads: int = 1) -> np.ndarray:
    """The n_probe nearest other centres of each centre (:583-611)."""
    cent = np.ascontiguousarray(centres, np.float32)
    K, d = cent.shape
    out = np.empty((K, n_probe), np.uint32)
    lib().oracle_ivf_near_clusters(_p(cent), K, d, int(n_probe), _p(out), int(threads))
    return out


def ivf_seed(base, g: int, assign, nearc, max_own: int, codes=None, lut=None, graph=None, gdist=None,
             threads: int = 1):
    """Per-cluster seeding (:576-582, :614-681, :712-792) into (graph,
    gdist), fresh (all missing) unless given.  Returns (graph, gdist)."""
    base = np.ascontiguousarray(base, np.float32)
    n, d = base.shape
    assign = np.ascontiguousarray(assign, np.uint32)
    nearc = np.ascontiguousarray(nearc, np.uint32)
    K = nearc.shape[0]
    if graph is None:
        graph, gdist = _empty_graph(n, g)
    graph = np.ascontiguousarray(graph, np.uint32)
    gdist = np.ascontiguousarray(gdist, np.float32)
    cp = None if codes is None else np.ascontiguousarray(codes, np.uint8)
    lp = None if lut is None else np.ascontiguousarray(lut, np.float32)
    lib().oracle_ivf_seed(_p(base), n, d, int(g), _p(assign), K, _p(nearc), nearc.shape[1], int(max_own),
                          None if cp is None else _p(cp), None if lp is None else _p(lp), _p(graph), _p(gdist),
                          int(threads))
    return graph, gdist


def bucketing_perm(n: int) -> np.ndarray:
    """The bucketing permutation (src/metal_context.mm:802-810)."""
    out = np.empty(int(n), np.uint32)
    lib().oracle_bucketing_perm(int(n), _p(out))
    return out


def bucketing_merge(base, g: int, perm, bucket: int = 256, graph=None, gdist=None, threads: int = 1):
    """One random-bucketing pass (shaders/cagra_kernels.metal:403-462)."""
    base = np.ascontiguousarray(base, np.float32)
    n, d = base.shape
    perm = np.ascontiguousarray(perm, np.uint32)
    if graph is None:
        graph, gdist = _empty_graph(n, g)
    graph = np.ascontiguousarray(graph, np.uint32)
    gdist = np.ascontiguousarray(gdist, np.float32)
    lib().oracle_bucketing_merge(_p(base), n, d, int(g), _p(perm), int(bucket), _p(graph), _p(gdist), int(threads))
    return graph, gdist


def nn_descent(base, graph, gdist, max_iter: int, threads: int = 1):
    """nn-descent (shaders/cagra_kernels.metal:334-395): returns (graph,
    gdist, iterations run)."""
    base = np.ascontiguousarray(base, np.float32)
    n, d = base.shape
    graph = np.array(graph, np.uint32, copy=True, order="C")
    gdist = np.array(gdist, np.float32, copy=True, order="C")
    it = lib().oracle_nn_descent(_p(base), n, d, graph.shape[1], _p(graph), _p(gdist), int(max_iter), int(threads))
    return graph, gdist, int(it)
