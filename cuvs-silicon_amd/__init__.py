"""ctypes binding of libcvs_hip (the C ABI declared in include/cvs_hip.h).

Python host code for tests and benchmarks.  It loads the in-tree shared
library built by ``make -C cuvs-silicon_amd`` and raises if it is missing:
there is no CPU fallback.

Errors map like the C++ front-end does (reference src/cagra.cpp:26-32,
:100-111): CVS_ERR_INVALID_ARGUMENT / CVS_ERR_UNSUPPORTED -> ValueError,
everything else -> RuntimeError.
"""
from __future__ import annotations

import ctypes
import os
import weakref
from ctypes import POINTER, byref, c_char_p, c_double, c_float, c_int, c_int64, c_size_t, c_uint32, c_uint64, c_void_p

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libcvs_hip.so")
CXX_LIB_PATH = os.path.join(LIB_DIR, "libcuvs_silicon.so")
SYNTH_LIB_PATH = os.path.join(LIB_DIR, "libcvs_synth.so")

CVS_OK = 0
CVS_ERR_INVALID_ARGUMENT = 1
CVS_ERR_RUNTIME = 2
CVS_ERR_NO_DEVICE = 3
CVS_ERR_OUT_OF_MEMORY = 4
CVS_ERR_UNSUPPORTED = 5

BF_MAX_DIM = 16384
BF_MAX_K = 1024
CAGRA_MAX_DIM = 8192
CAGRA_MAX_ITOPK = 512
CAGRA_MAX_WIDTH = 16

# Every extern "C" symbol declared in include/cvs_hip.h: name -> (restype, argtypes).
_SIGNATURES = {
    "cvs_last_error": (c_char_p, []),
    "cvs_dispatch_count": (c_uint64, []),
    "cvs_reset_dispatch_count": (None, []),
    "cvs_device_count": (c_int, [POINTER(c_int)]),
    "cvs_context_create": (c_int, [c_int, POINTER(c_void_p)]),
    "cvs_calibrate_stream_read": (c_int, [c_void_p, c_size_t, c_int, c_int, POINTER(c_double)]),
    "cvs_context_destroy": (c_int, [c_void_p]),
    "cvs_context_synchronize": (c_int, [c_void_p]),
    "cvs_context_device_info": (c_int, [c_void_p, c_char_p, c_size_t, POINTER(c_int), POINTER(c_int64)]),
    "cvs_context_set_timing": (c_int, [c_void_p, c_int]),
    "cvs_context_kernel_time": (c_int, [c_void_p, c_char_p, POINTER(c_double), POINTER(c_uint64)]),
    "cvs_device_alloc": (c_int, [c_void_p, c_size_t, POINTER(c_void_p)]),
    "cvs_device_free": (c_int, [c_void_p, c_void_p]),
    "cvs_copy_to_device": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
    "cvs_copy_to_host": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t]),
    "cvs_dataset_create": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int, POINTER(c_void_p)]),
    "cvs_dataset_destroy": (c_int, [c_void_p]),
    "cvs_dataset_shape": (c_int, [c_void_p, POINTER(c_int64), POINTER(c_int64)]),
    "cvs_dataset_rows": (c_int, [c_void_p, POINTER(c_void_p)]),
    "cvs_bf_search": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "cvs_bf_search_async": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "cvs_cagra_index_create": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int, c_void_p, c_uint32, c_int,
                                       c_void_p, c_uint32, POINTER(c_void_p)]),
    "cvs_cagra_index_destroy": (c_int, [c_void_p]),
    "cvs_cagra_index_set_traversal": (c_int, [c_void_p, c_int]),
    "cvs_cagra_build_reference": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int, c_uint32, c_void_p, c_int,
                                          c_void_p]),
    "cvs_cagra_build_reference_ex": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int, c_uint32, c_int64, c_int64,
                                             c_void_p, c_int, c_void_p]),
    "cvs_cagra_index_edge_distances": (c_int, [c_void_p, c_void_p, c_void_p, c_int]),
    "cvs_cagra_search_teams": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_uint32, c_uint32, c_uint32,
                                       c_uint32, c_void_p, c_void_p]),
    "cvs_cagra_search_teams_async": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_uint32, c_uint32,
                                             c_uint32, c_uint32, c_void_p, c_void_p]),
    "cvs_cagra_search": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_uint32, c_uint32, c_uint32,
                                 c_void_p, c_void_p]),
    "cvs_cagra_search_async": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_uint32, c_uint32, c_uint32,
                                       c_void_p, c_void_p, c_void_p]),
}

class RefBuildStats(ctypes.Structure):
    _fields_ = [("graph_degree", c_uint32), ("clusters", c_uint32), ("kmeans_iterations", c_uint32),
                ("descent_iterations", c_uint32), ("descent_changed_nodes", c_uint32),
                ("seconds_kmeans", c_double), ("seconds_seed", c_double), ("seconds_descent", c_double),
                ("seconds_total", c_double), ("pq_iterations", c_uint32), ("seconds_pq", c_double)]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


class BuildStats(ctypes.Structure):
    """cvs_build_stats (include/cvs_hip.h)."""
    _fields_ = [("iterations", c_uint32), ("intermediate_degree", c_uint32), ("graph_degree", c_uint32),
                ("final_update_rate", c_double), ("seconds_seed", c_double), ("seconds_descent", c_double),
                ("seconds_prune", c_double), ("seconds_total", c_double), ("join_ms", c_double),
                ("join_bytes", c_double), ("join_members", c_uint64), ("updates_emitted", c_uint64),
                ("updates_kept", c_uint64), ("insertions", c_uint64), ("seconds_rescore", c_double)]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


_SIGNATURES["cvs_cagra_build"] = (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int, c_uint32, c_uint32, c_uint32,
                                          c_float, c_uint64, c_void_p, c_int, POINTER(BuildStats)])


class BuildOptions(ctypes.Structure):
    """cvs_build_options (include/cvs_hip.h)."""
    _fields_ = [("rescore_fp32", c_int), ("intermediate_out", c_void_p), ("graph_mode", c_int),
                ("reverse_edges", c_uint32)]


GRAPH_DETOUR, GRAPH_KNN = 0, 1


_SIGNATURES["cvs_cagra_build_ex"] = (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int, c_uint32, c_uint32,
                                             c_uint32, c_float, c_uint64, POINTER(BuildOptions), c_void_p, c_int,
                                             POINTER(BuildStats)])

_SIGNATURES["cvs_cagra_optimize"] = (c_int, [c_void_p, c_void_p, c_int64, c_uint32, c_int, c_uint32, c_uint32,
                                             c_void_p, c_int])
_SIGNATURES["cvs_bf_search_noalloc"] = (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p])
_SIGNATURES["cvs_cagra_nav_nodes"] = (c_int, [c_int64, c_void_p, POINTER(c_int64)])
_SIGNATURES["cvs_cagra_entry_points"] = (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p])
_SIGNATURES["cvs_cagra_entry_points_async"] = (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p])
_SIGNATURES["cvs_cagra_search_reference"] = (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_uint32,
                                                     c_uint32, c_void_p, c_void_p, c_void_p])
_SIGNATURES["cvs_cagra_search_reference_async"] = (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_uint32,
                                                           c_uint32, c_void_p, c_void_p, c_void_p])
_SIGNATURES["cvs_calibrate_gather_read"] = (c_int, [c_void_p, c_size_t, c_int64, c_int, c_int, c_int, POINTER(c_double)])
_SIGNATURES["cvs_calibrate_mfma"] = (c_int, [c_void_p, c_void_p, c_size_t, c_int, c_int64, c_int, c_int,
                                             POINTER(c_double)])
_SIGNATURES["cvs_cagra_search_record_async"] = (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_uint32,
                                                        c_uint32, c_uint32, c_void_p, c_void_p, c_void_p, c_void_p,
                                                        c_uint32])
_SIGNATURES["cvs_cagra_replay_gathers"] = (c_int, [c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_int64, c_int,
                                                   c_int, POINTER(c_double)])
_SIGNATURES["cvs_context_bf_escalations"] = (c_int, [c_void_p, POINTER(c_uint64), POINTER(c_uint64), c_int])

# The bucketing permutation seed of the reference (src/metal_context.mm:803).
DEFAULT_BUILD_SEED = 0xFEDCBA9876543210

_lib = None


def library_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Loads libcvs_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C {PKG_DIR}`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def exported_symbols():
    return list(_SIGNATURES)


class CvsError(RuntimeError):
    pass


def _check(status: int) -> None:
    if status == CVS_OK:
        return
    msg = load().cvs_last_error().decode()
    if status in (CVS_ERR_INVALID_ARGUMENT, CVS_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(f"cvs error {status}: {msg}")


def cagra_nav_nodes(n: int) -> np.ndarray:
    """Navigation (seed) node ids of an n-row graph index, as the
    reference's cagra::build picks them (src/cagra.cpp:63-72)."""
    cnt = c_int64(0)
    _check(load().cvs_cagra_nav_nodes(int(n), None, byref(cnt)))
    out = np.empty(cnt.value, np.uint32)
    _check(load().cvs_cagra_nav_nodes(int(n), out.ctypes.data_as(c_void_p), byref(cnt)))
    return out


def device_count() -> int:
    n = c_int(0)
    _check(load().cvs_device_count(byref(n)))
    return n.value


def dispatch_count() -> int:
    return int(load().cvs_dispatch_count())


def reset_dispatch_count() -> None:
    load().cvs_reset_dispatch_count()


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class DeviceArray:
    """A device allocation with numpy shape/dtype bookkeeping."""

    def __init__(self, ctx: "Context", shape, dtype):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = c_void_p()
        _check(load().cvs_device_alloc(ctx.handle, max(self.nbytes, 1), byref(p)))
        self.ptr = p

    @classmethod
    def from_host(cls, ctx: "Context", host: np.ndarray) -> "DeviceArray":
        host = np.ascontiguousarray(host)
        arr = cls(ctx, host.shape, host.dtype)
        if arr.nbytes:
            _check(load().cvs_copy_to_device(ctx.handle, arr.ptr, host.ctypes.data_as(c_void_p), arr.nbytes))
        return arr

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if self.nbytes:
            _check(load().cvs_copy_to_host(self.ctx.handle, out.ctypes.data_as(c_void_p), self.ptr, self.nbytes))
        return out

    def rows(self, lo: int, hi: int) -> "DeviceArray":
        """A view of rows [lo, hi) of this array: same memory, not owned
        (its free() does nothing); it must not outlive this array."""
        if not 0 <= lo <= hi <= self.shape[0]:
            raise ValueError(f"rows [{lo}, {hi}) outside [0, {self.shape[0]})")
        view = DeviceArray.__new__(DeviceArray)
        view.ctx = self.ctx
        view.shape = (hi - lo,) + self.shape[1:]
        view.dtype = self.dtype
        view.nbytes = int(np.prod(view.shape)) * self.dtype.itemsize
        row_bytes = int(np.prod(self.shape[1:])) * self.dtype.itemsize
        view.ptr = c_void_p(self.ptr.value + lo * row_bytes)
        view._view_of = self
        return view

    def free(self) -> None:
        if getattr(self, "_view_of", None) is not None:
            return
        if self.ptr is not None and self.ctx.handle is not None:
            _check(load().cvs_device_free(self.ctx.handle, self.ptr))
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """One device + one HIP stream (C: cvs_context)."""

    def __init__(self, device: int = 0):
        h = c_void_p()
        _check(load().cvs_context_create(int(device), byref(h)))
        self.handle = h
        # Datasets and graph indexes made on this context: the C library
        # refuses to destroy a context that still owns any, so close() closes
        # the live ones first.
        self._children = weakref.WeakSet()

    def _adopt(self, child) -> None:
        self._children.add(child)

    def close(self) -> None:
        if self.handle is not None:
            for child in list(self._children):
                child.close()
            _check(load().cvs_context_destroy(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self) -> None:
        _check(load().cvs_context_synchronize(self.handle))

    def device_info(self):
        name = ctypes.create_string_buffer(256)
        cu = c_int(0)
        mem = c_int64(0)
        _check(load().cvs_context_device_info(self.handle, name, 256, byref(cu), byref(mem)))
        return {"name": name.value.decode(), "compute_units": cu.value, "total_mem_bytes": mem.value}

    def calibrate_stream_read(self, nbytes: int, workgroups: int, reps: int = 20) -> float:
        """Achievable streaming-read rate in GB/s (C: cvs_calibrate_stream_read)."""
        gbs = c_double(0)
        _check(load().cvs_calibrate_stream_read(self.handle, int(nbytes), int(workgroups), int(reps), byref(gbs)))
        return gbs.value

    def calibrate_gather_read(self, row_bytes: int, n_rows: int, workgroups: int, rows_per_team: int,
                              reps: int = 10) -> float:
        """Achievable rate of random whole-row gathers in GB/s (C:
        cvs_calibrate_gather_read)."""
        gbs = c_double(0)
        _check(load().cvs_calibrate_gather_read(self.handle, int(row_bytes), int(n_rows), int(workgroups),
                                                int(rows_per_team), int(reps), byref(gbs)))
        return gbs.value

    def calibrate_mfma(self, data_ptr, nbytes: int, workgroups: int, ksteps: int, from_lds: bool = False,
                       reps: int = 5) -> float:
        """fp16 MFMA rate in TFLOP/s of the large-batch scan's register
        block on the fp16 data at device address data_ptr (an int or a
        c_void_p; C:
        cvs_calibrate_mfma)."""
        tf = c_double(0)
        ptr = data_ptr if isinstance(data_ptr, c_void_p) else c_void_p(int(data_ptr))
        _check(load().cvs_calibrate_mfma(self.handle, ptr, int(nbytes), int(workgroups),
                                         int(ksteps), 1 if from_lds else 0, int(reps), byref(tf)))
        return tf.value

    def set_timing(self, enable: bool) -> None:
        _check(load().cvs_context_set_timing(self.handle, 1 if enable else 0))

    def kernel_time(self, kernel: str):
        """(total_ms, launches) of `kernel` since the last query."""
        ms = c_double(0)
        n = c_uint64(0)
        _check(load().cvs_context_kernel_time(self.handle, kernel.encode(), byref(ms), byref(n)))
        return ms.value, int(n.value)

    def bf_escalations(self, reset: bool = False):
        """(escalated, rescanned): brute-force queries whose fp16 selection
        was not certified and were re-ranked exactly over more rows, and how
        many of those over every row (C: cvs_context_bf_escalations)."""
        esc = c_uint64(0)
        full = c_uint64(0)
        _check(load().cvs_context_bf_escalations(self.handle, byref(esc), byref(full), 1 if reset else 0))
        return int(esc.value), int(full.value)

    def dataset(self, rows) -> "Dataset":
        return Dataset(self, rows)

    def cagra_index(self, rows, graph, seeds=None, traversal_bits: int = 32) -> "CagraIndex":
        return CagraIndex(self, rows, graph, seeds, traversal_bits)

    def cagra_build_reference(self, rows, graph_degree: int = 64, exact_limit: int = None, pq_limit: int = None):
        """The reference's own build algorithm on the GPU (exact seeding for
        n <= 50,000; IVF k-means + per-cluster seeding, random bucketing and
        2-hop nn-descent up to 200,000; product-quantised seeding above).
        exact_limit / pq_limit replace those two sizes (tests).  Returns
        (graph, stats)."""
        st = RefBuildStats()
        rows = _f32(rows)
        n, d = rows.shape
        g = max(min(int(graph_degree), n - 1), 1)
        host = np.empty((n, g), np.uint32)
        if exact_limit is None and pq_limit is None:
            _check(load().cvs_cagra_build_reference(self.handle, rows.ctypes.data_as(c_void_p), n, d, 0,
                                                    int(graph_degree), host.ctypes.data_as(c_void_p), 0, byref(st)))
        else:
            _check(load().cvs_cagra_build_reference_ex(
                self.handle, rows.ctypes.data_as(c_void_p), n, d, 0, int(graph_degree),
                50000 if exact_limit is None else int(exact_limit), 200000 if pq_limit is None else int(pq_limit),
                host.ctypes.data_as(c_void_p), 0, byref(st)))
        return host, st.as_dict()

    def cagra_build(self, rows, intermediate_degree: int = 128, graph_degree: int = 64, max_iterations: int = 20,
                    termination_threshold: float = 0.001, seed: int = DEFAULT_BUILD_SEED, out: "DeviceArray" = None,
                    rescore_fp32: bool = False, intermediate_out: "DeviceArray" = None,
                    graph_mode: int = GRAPH_DETOUR, reverse_edges: int = 0):
        """GPU graph build.  Returns (graph, stats): graph is a host uint32
        array (n, g), or `out` (a device array of that shape) when given.
        rescore_fp32 re-ranks the final intermediate lists by exact fp32
        distances before pruning, intermediate_out (a uint32 device array
        (n, list width)) receives the lists the graph is made from, and
        graph_mode picks how (GRAPH_DETOUR: detour pruning, with the last
        `reverse_edges` kept edges of each row giving way to reverse edges;
        GRAPH_KNN: the nearest graph_degree entries) (cvs_cagra_build_ex)."""
        st = BuildStats()
        if isinstance(rows, DeviceArray):
            n, d = rows.shape
            rptr, rdev = rows.ptr, 1
        else:
            rows = _f32(rows)
            n, d = rows.shape
            rptr, rdev = rows.ctypes.data_as(c_void_p), 0
        g = min(int(graph_degree), max(int(intermediate_degree), int(graph_degree)), n - 1)
        if out is not None:
            if out.shape != (n, g) or out.dtype != np.uint32:
                raise ValueError(f"out must be a uint32 device array of shape {(n, g)}")
            gptr, gdev, host = out.ptr, 1, None
        else:
            host = np.empty((n, max(g, 1)), np.uint32)
            gptr, gdev = host.ctypes.data_as(c_void_p), 0
        if intermediate_out is not None:
            kd = min(max(int(intermediate_degree), int(graph_degree)), n - 1)
            if intermediate_out.shape != (n, kd) or intermediate_out.dtype != np.uint32:
                raise ValueError(f"intermediate_out must be a uint32 device array of shape {(n, kd)}")
        if rescore_fp32 or intermediate_out is not None or graph_mode != GRAPH_DETOUR or reverse_edges:
            opts = BuildOptions(rescore_fp32=int(bool(rescore_fp32)),
                                intermediate_out=intermediate_out.ptr if intermediate_out is not None else None,
                                graph_mode=int(graph_mode), reverse_edges=int(reverse_edges))
            _check(load().cvs_cagra_build_ex(self.handle, rptr, n, d, rdev, int(intermediate_degree),
                                             int(graph_degree), int(max_iterations), float(termination_threshold),
                                             int(seed), byref(opts), gptr, gdev, byref(st)))
        else:
            _check(load().cvs_cagra_build(self.handle, rptr, n, d, rdev, int(intermediate_degree),
                                          int(graph_degree), int(max_iterations), float(termination_threshold),
                                          int(seed), gptr, gdev, byref(st)))
        return (out if out is not None else host), st.as_dict()

    def cagra_optimize(self, knn, graph_degree: int, reverse_edges: int = 0, out: "DeviceArray" = None):
        """Detour pruning of caller k-NN lists (n, width) uint32, nearest
        first, with the last `reverse_edges` kept edges of each row giving way
        to reverse edges (cvs_cagra_optimize).  Returns a host (n,
        graph_degree) uint32 graph, or `out` when given."""
        if isinstance(knn, DeviceArray):
            n, kd = knn.shape
            kptr, kdev = knn.ptr, 1
        else:
            knn = np.ascontiguousarray(knn, np.uint32)
            if knn.ndim != 2:
                raise ValueError("knn must be a 2-D array")
            n, kd = knn.shape
            kptr, kdev = knn.ctypes.data_as(c_void_p), 0
        g = int(graph_degree)
        if out is not None:
            if out.shape != (n, g) or out.dtype != np.uint32:
                raise ValueError(f"out must be a uint32 device array of shape {(n, g)}")
            gptr, gdev, host = out.ptr, 1, None
        else:
            host = np.empty((n, max(g, 1)), np.uint32)
            gptr, gdev = host.ctypes.data_as(c_void_p), 0
        _check(load().cvs_cagra_optimize(self.handle, kptr, int(n), int(kd), kdev, g, int(reverse_edges), gptr,
                                         gdev))
        return out if out is not None else host


class Dataset:
    """Device-resident dataset (C: cvs_dataset)."""

    def __init__(self, ctx: Context, rows):
        self.ctx = ctx
        h = c_void_p()
        if isinstance(rows, DeviceArray):
            n, d = rows.shape
            _check(load().cvs_dataset_create(ctx.handle, rows.ptr, n, d, 1, byref(h)))
        else:
            rows = _f32(rows)
            if rows.ndim != 2:
                raise ValueError("dataset must be a 2-D array")
            n, d = rows.shape
            _check(load().cvs_dataset_create(ctx.handle, rows.ctypes.data_as(c_void_p), n, d, 0, byref(h)))
        self.handle = h
        self.n, self.d = int(n), int(d)
        ctx._adopt(self)

    def close(self) -> None:
        # A dataset dies with its context (Context.close closes it first).
        if self.handle is not None and self.ctx.handle is not None:
            _check(load().cvs_dataset_destroy(self.handle))
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def bf_search(self, queries, k: int):
        """Exact k-NN of host queries; returns (neighbors u32 [q,k], distances f32 [q,k])."""
        queries = _f32(queries)
        if queries.ndim != 2 or queries.shape[1] != self.d:
            raise ValueError("queries must be (q, d)")
        q = queries.shape[0]
        nbr = np.empty((q, k), dtype=np.uint32)
        dist = np.empty((q, k), dtype=np.float32)
        _check(load().cvs_bf_search(self.ctx.handle, self.handle, queries.ctypes.data_as(c_void_p), q, int(k),
                                    nbr.ctypes.data_as(c_void_p), dist.ctypes.data_as(c_void_p)))
        return nbr, dist

    def bf_search_noalloc(self, queries: DeviceArray, k: int, nbr: DeviceArray, dist: DeviceArray) -> None:
        """bf_search_async with the library's per-device scratch array
        (cvs_bf_search_noalloc): no device allocation."""
        _check(load().cvs_bf_search_noalloc(self.ctx.handle, self.handle, queries.ptr, queries.shape[0], int(k),
                                            nbr.ptr, dist.ptr))

    def bf_search_async(self, queries: DeviceArray, k: int, nbr: DeviceArray, dist: DeviceArray) -> None:
        _check(load().cvs_bf_search_async(self.ctx.handle, self.handle, queries.ptr, queries.shape[0], int(k),
                                          nbr.ptr, dist.ptr))


class CagraIndex:
    """Device-resident graph index (C: cvs_cagra_index): rows, neighbour lists
    and seed (navigation) node ids."""

    def __init__(self, ctx: Context, rows, graph, seeds=None, traversal_bits: int = 32):
        self.ctx = ctx
        h = c_void_p()
        graph_dev = isinstance(graph, DeviceArray)
        if graph_dev:
            n_g, degree = graph.shape
            gptr = graph.ptr
        else:
            graph = np.ascontiguousarray(graph, np.uint32)
            if graph.ndim != 2:
                raise ValueError("graph must be a 2-D array")
            n_g, degree = graph.shape
            gptr = graph.ctypes.data_as(c_void_p)
        seeds = np.ascontiguousarray(seeds if seeds is not None else np.zeros(0, np.uint32), np.uint32)
        if isinstance(rows, DeviceArray):
            n, d = rows.shape
            rptr, rdev = rows.ptr, 1
        else:
            rows = _f32(rows)
            if rows.ndim != 2:
                raise ValueError("dataset must be a 2-D array")
            n, d = rows.shape
            rptr, rdev = rows.ctypes.data_as(c_void_p), 0
        if n_g != n:
            raise ValueError("graph must have one row per dataset row")
        _check(load().cvs_cagra_index_create(ctx.handle, rptr, n, d, rdev, gptr, degree, 1 if graph_dev else 0,
                                             seeds.ctypes.data_as(c_void_p) if len(seeds) else None, len(seeds),
                                             byref(h)))
        self.handle = h
        self.n, self.d, self.degree = int(n), int(d), int(degree)
        ctx._adopt(self)
        self.set_traversal(traversal_bits)

    def edge_distances(self, out: "DeviceArray" = None):
        """Exact squared L2 length of every graph edge, (n, degree) float32
        (+inf where the entry is not a row id); into `out` (a device array)
        when given, else returned as a host array."""
        if out is not None:
            if out.shape != (self.n, self.degree) or out.dtype != np.float32:
                raise ValueError(f"out must be a float32 device array of shape {(self.n, self.degree)}")
            _check(load().cvs_cagra_index_edge_distances(self.ctx.handle, self.handle, out.ptr, 1))
            return out
        host = np.empty((self.n, self.degree), np.float32)
        _check(load().cvs_cagra_index_edge_distances(self.ctx.handle, self.handle,
                                                     host.ctypes.data_as(c_void_p), 0))
        return host

    def search_record_async(self, queries: DeviceArray, k: int, nbr: DeviceArray, dist: DeviceArray,
                            stats: DeviceArray, record: DeviceArray, itopk_size: int = 64, search_width: int = 1,
                            max_iterations: int = 0) -> None:
        """search_async that also records each query's evaluated row ids
        (C: cvs_cagra_search_record_async); record is (q, cap) uint32."""
        _check(load().cvs_cagra_search_record_async(self.ctx.handle, self.handle, queries.ptr, queries.shape[0],
                                                    int(k), int(itopk_size), int(search_width), int(max_iterations),
                                                    nbr.ptr, dist.ptr, stats.ptr, record.ptr, record.shape[1]))

    def replay_gathers(self, record: DeviceArray, stats: DeviceArray, bits: int, reps: int = 5) -> float:
        """Mean ms of gathering the recorded rows alone (C:
        cvs_cagra_replay_gathers)."""
        ms = c_double(0)
        _check(load().cvs_cagra_replay_gathers(self.ctx.handle, self.handle, record.ptr, record.shape[1], stats.ptr,
                                               record.shape[0], int(bits), int(reps), byref(ms)))
        return ms.value

    def entry_points(self, queries) -> np.ndarray:
        """Per-query entry node: the nearest seed (navigation) node, as the
        reference picks it (C: cvs_cagra_entry_points)."""
        queries = _f32(queries)
        out = np.empty(queries.shape[0], np.uint32)
        _check(load().cvs_cagra_entry_points(self.ctx.handle, self.handle, queries.ctypes.data_as(c_void_p),
                                             queries.shape[0], out.ctypes.data_as(c_void_p)))
        return out

    def search_reference(self, queries, k: int, beam_size: int, max_iter: int, entry_nodes=None):
        """The reference's own beam search (C: cvs_cagra_search_reference):
        one entry node per query (None: the hashed fallback), beam and
        iteration cap as given."""
        queries = _f32(queries)
        q = queries.shape[0]
        ent = None
        if entry_nodes is not None:
            ent = np.ascontiguousarray(entry_nodes, np.uint32)
            if ent.shape != (q,):
                raise ValueError("entry_nodes must hold one id per query")
        nbr = np.empty((q, k), np.uint32)
        dist = np.empty((q, k), np.float32)
        _check(load().cvs_cagra_search_reference(self.ctx.handle, self.handle, queries.ctypes.data_as(c_void_p), q,
                                                 int(k), int(beam_size), int(max_iter),
                                                 None if ent is None else ent.ctypes.data_as(c_void_p),
                                                 nbr.ctypes.data_as(c_void_p), dist.ctypes.data_as(c_void_p)))
        return nbr, dist

    def search_reference_async(self, queries: DeviceArray, k: int, nbr: DeviceArray, dist: DeviceArray,
                               beam_size: int, max_iter: int, entry_nodes: DeviceArray = None) -> None:
        _check(load().cvs_cagra_search_reference_async(self.ctx.handle, self.handle, queries.ptr, queries.shape[0],
                                                       int(k), int(beam_size), int(max_iter),
                                                       None if entry_nodes is None else entry_nodes.ptr, nbr.ptr,
                                                       dist.ptr))

    def entry_points_async(self, queries: DeviceArray, out: DeviceArray) -> None:
        _check(load().cvs_cagra_entry_points_async(self.ctx.handle, self.handle, queries.ptr, queries.shape[0],
                                                   out.ptr))

    def set_traversal(self, bits: int) -> None:
        """16: candidates evaluated on the fp16 copy, final list re-ranked in
        fp32; 32: every evaluation on the fp32 rows."""
        _check(load().cvs_cagra_index_set_traversal(self.handle, int(bits)))
        self.traversal_bits = int(bits)

    def close(self) -> None:
        # An index dies with its context (Context.close closes it first).
        if self.handle is not None and self.ctx.handle is not None:
            _check(load().cvs_cagra_index_destroy(self.handle))
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def search(self, queries, k: int, itopk_size: int = 64, search_width: int = 1, max_iterations: int = 0):
        """Graph search of host queries; returns (neighbors u32 [q,k], distances f32 [q,k])."""
        queries = _f32(queries)
        if queries.ndim != 2 or queries.shape[1] != self.d:
            raise ValueError("queries must be (q, d)")
        q = queries.shape[0]
        nbr = np.empty((q, k), dtype=np.uint32)
        dist = np.empty((q, k), dtype=np.float32)
        _check(load().cvs_cagra_search(self.ctx.handle, self.handle, queries.ctypes.data_as(c_void_p), q, int(k),
                                       int(itopk_size), int(search_width), int(max_iterations),
                                       nbr.ctypes.data_as(c_void_p), dist.ctypes.data_as(c_void_p)))
        return nbr, dist

    def search_teams(self, queries, k: int, teams: int, itopk_size: int = 32, search_width: int = 1,
                     max_iterations: int = 0):
        """Multi-team graph search of host queries (C: cvs_cagra_search_teams):
        `teams` searches per query with `itopk_size`-entry lists, merged."""
        queries = _f32(queries)
        if queries.ndim != 2 or queries.shape[1] != self.d:
            raise ValueError("queries must be (q, d)")
        q = queries.shape[0]
        nbr = np.empty((q, k), dtype=np.uint32)
        dist = np.empty((q, k), dtype=np.float32)
        _check(load().cvs_cagra_search_teams(self.ctx.handle, self.handle, queries.ctypes.data_as(c_void_p), q, int(k),
                                             int(itopk_size), int(search_width), int(max_iterations), int(teams),
                                             nbr.ctypes.data_as(c_void_p), dist.ctypes.data_as(c_void_p)))
        return nbr, dist

    def search_teams_async(self, queries: DeviceArray, k: int, nbr: DeviceArray, dist: DeviceArray, teams: int,
                           itopk_size: int = 32, search_width: int = 1, max_iterations: int = 0) -> None:
        _check(load().cvs_cagra_search_teams_async(self.ctx.handle, self.handle, queries.ptr, queries.shape[0], int(k),
                                                   int(itopk_size), int(search_width), int(max_iterations),
                                                   int(teams), nbr.ptr, dist.ptr))

    def search_async(self, queries: DeviceArray, k: int, nbr: DeviceArray, dist: DeviceArray, itopk_size: int = 64,
                     search_width: int = 1, max_iterations: int = 0, stats: DeviceArray | None = None) -> None:
        _check(load().cvs_cagra_search_async(self.ctx.handle, self.handle, queries.ptr, queries.shape[0], int(k),
                                             int(itopk_size), int(search_width), int(max_iterations), nbr.ptr,
                                             dist.ptr, stats.ptr if stats is not None else None))


# ---- synthetic data (lib/libcvs_synth.so) ---------------------------------
STREAM_BASE = 1
STREAM_QUERIES = 2
_synth = None


def _synth_lib():
    global _synth
    if _synth is None:
        if not os.path.exists(SYNTH_LIB_PATH):
            raise RuntimeError(f"{SYNTH_LIB_PATH} is missing: build it with `make -C {PKG_DIR}`")
        lib = ctypes.CDLL(SYNTH_LIB_PATH)
        lib.cvs_synth_clustered.restype = None
        lib.cvs_synth_clustered.argtypes = [c_uint64, c_uint32, c_int64, c_int64, c_int64, c_int, c_double, c_void_p]
        lib.cvs_synth_normal.restype = c_double
        lib.cvs_synth_normal.argtypes = [c_uint64, c_uint32, c_uint64, c_uint64]
        _synth = lib
    return _synth


def synth_clustered(seed: int, stream: int, n: int, d: int, n_centers: int = 64, sigma: float = 0.3,
                    row0: int = 0) -> np.ndarray:
    """Rows [row0, row0+n) of the clustered L2-normalised distribution."""
    out = np.empty((int(n), int(d)), dtype=np.float32)
    _synth_lib().cvs_synth_clustered(int(seed), int(stream), int(row0), int(n), int(d), int(n_centers),
                                     float(sigma), out.ctypes.data_as(c_void_p))
    return out


def synth_normal(seed: int, stream: int, row: int, col: int) -> float:
    return float(_synth_lib().cvs_synth_normal(int(seed), int(stream), int(row), int(col)))
