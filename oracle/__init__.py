"""ctypes access to the oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker.

- liboracle.so: the C restatement of the reference search path (oracle.h).
- _ref/libref.so: the reference's own CPU sources compiled in place
  (src/cagra.cpp, src/distance.cpp) behind ref_shim.cpp; present only where
  it was built (it needs the reference sources at build time).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_uint32, c_void_p

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


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_LIB):
            build(with_reference=False)
        L = ctypes.CDLL(ORACLE_LIB)
        L.oracle_l2_128.restype = c_float
        L.oracle_l2_128.argtypes = [c_void_p, c_void_p]
        for name in ("oracle_bf_exact", "oracle_bf_fp64"):
            fn = getattr(L, name)
            fn.restype = None
            fn.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int]
        _lib = L
    return _lib


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
