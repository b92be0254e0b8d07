"""Close order of contexts and the datasets / graph indexes made on them.

The C library refuses to destroy a context that still owns a dataset or a
graph index (CVS_ERR_INVALID_ARGUMENT, nothing freed), since their own
destruction uses the context's device and stream.  The Python wrappers close
a context's live children first, and closing a child after its context is a
no-op.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CVS_OK, CVS_ERR_INVALID_ARGUMENT = 0, 1


def test_c_abi_refuses_to_destroy_a_context_with_children(cvs):
    print("[lifetime] C ABI", flush=True)
    lib = cvs.load()
    rows = np.arange(64 * 8, dtype=np.float32).reshape(64, 8)
    ctx, ds, ix = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    assert lib.cvs_context_create(0, ctypes.byref(ctx)) == CVS_OK
    assert lib.cvs_dataset_create(ctx, rows.ctypes.data_as(ctypes.c_void_p), 64, 8, 0, ctypes.byref(ds)) == CVS_OK
    graph = np.zeros((64, 2), np.uint32)
    assert lib.cvs_cagra_index_create(ctx, rows.ctypes.data_as(ctypes.c_void_p), 64, 8, 0,
                                      graph.ctypes.data_as(ctypes.c_void_p), 2, 0, None, 0,
                                      ctypes.byref(ix)) == CVS_OK
    assert lib.cvs_context_destroy(ctx) == CVS_ERR_INVALID_ARGUMENT
    assert b"2 dataset(s) or graph index(es)" in lib.cvs_last_error()
    assert lib.cvs_dataset_destroy(ds) == CVS_OK
    assert lib.cvs_context_destroy(ctx) == CVS_ERR_INVALID_ARGUMENT
    assert lib.cvs_cagra_index_destroy(ix) == CVS_OK
    assert lib.cvs_context_destroy(ctx) == CVS_OK


def test_python_context_closes_its_children_first(cvs):
    print("[lifetime] Python", flush=True)
    rows = np.random.default_rng(0).standard_normal((500, 16)).astype(np.float32)
    with cvs.Context(0) as c:
        ds = c.dataset(rows)
        ix = c.cagra_index(rows, np.zeros((500, 4), np.uint32))
        nbr, _ = ds.bf_search(rows[:3], 2)
        assert nbr[:, 0].tolist() == [0, 1, 2]
    assert c.handle is None and ds.handle is None and ix.handle is None
    ds.close()  # after the context: a no-op, not a use of freed memory
    ix.close()
