"""The allocation-free brute-force entry point (cvs_bf_search_noalloc)
against the allocating one (cvs_bf_search_async) on the same inputs.

Both run the same kernels; the allocation-free one keeps its workspace in
the library's per-device scratch array.  Results must be identical, id for
id and bit for bit, on two calls in a row where the second is smaller (the
scratch keeps the first call's contents), for the in-LDS candidate lists
(k <= 48) and the global ones (k > 48).  A call whose workspace would not
fit fails with CVS_ERR_UNSUPPORTED and leaves the next call working.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CVS_ERR_UNSUPPORTED = 5


def run_both(cvs, ctx, ds, queries, k):
    q = queries.shape[0]
    dq = cvs.DeviceArray.from_host(ctx, queries)
    outs = []
    for noalloc in (False, True):
        dn = cvs.DeviceArray(ctx, (q, k), np.uint32)
        dd = cvs.DeviceArray(ctx, (q, k), np.float32)
        if noalloc:
            ds.bf_search_noalloc(dq, k, dn, dd)
        else:
            ds.bf_search_async(dq, k, dn, dd)
        ctx.synchronize()
        outs.append((dn.to_host(), dd.to_host()))
        dn.free()
        dd.free()
    dq.free()
    return outs


@pytest.mark.parametrize("d,k", [(1024, 10), (1024, 100), (96, 48)])
def test_noalloc_matches_allocating_entry_point(cvs, ctx, oracle, d, k):
    print(f"[no-alloc] d={d} k={k}", flush=True)
    rng = np.random.default_rng(d + k)
    base = cvs.synth_clustered(17, cvs.STREAM_BASE, 20_000, d)
    ds = ctx.dataset(base)
    try:
        for q in (300, 37):  # second call smaller than the first
            queries = cvs.synth_clustered(int(rng.integers(1 << 30)), cvs.STREAM_QUERIES, q, d)
            (n_ref, d_ref), (n_na, d_na) = run_both(cvs, ctx, ds, queries, k)
            assert np.array_equal(n_na, n_ref), (q, k)
            assert np.array_equal(d_na.view(np.uint32), d_ref.view(np.uint32)), (q, k)
            # and both against the oracle: ids equal except at near-ties of
            # the k-th distance, distances within 1e-3 relative
            o_n, o_d = oracle.bf_exact(base, queries, k, threads=8)
            assert np.allclose(d_na, o_d, rtol=1e-3, atol=1e-6)
            for i in range(q):
                if set(n_na[i].tolist()) != set(o_n[i].tolist()):
                    kth, nxt = oracle.bf_exact(base, queries[i:i + 1], k + 1)[1][0, k - 1:k + 1]
                    assert abs(nxt - kth) <= 1e-3 * max(kth, 1e-30), (q, i)
    finally:
        ds.close()


@pytest.mark.parametrize("q", [2000, 7800])
def test_noalloc_large_batch(cvs, ctx, q):
    """Batches of more than 8 query blocks (the range-major launch and its
    32 dataset ranges, the layout that sizes the scratch for k <= 10 at
    D = 1024) through the scratch array, bit for bit against the allocating
    entry point; 7,800 queries is near the largest batch that fits."""
    print(f"[no-alloc] large batch q={q}", flush=True)
    base = cvs.synth_clustered(29, cvs.STREAM_BASE, 30_000, 1024)
    ds = ctx.dataset(base)
    try:
        queries = cvs.synth_clustered(31, cvs.STREAM_QUERIES, q, 1024)
        (n_ref, d_ref), (n_na, d_na) = run_both(cvs, ctx, ds, queries, 10)
        assert np.array_equal(n_na, n_ref)
        assert np.array_equal(d_na.view(np.uint32), d_ref.view(np.uint32))
    finally:
        ds.close()


def test_noalloc_rejects_oversized_call(cvs, ctx):
    print("[no-alloc] oversized", flush=True)
    base = cvs.synth_clustered(3, cvs.STREAM_BASE, 50_000, 1024)
    ds = ctx.dataset(base)
    try:
        q, k = 2000, 100  # needs far more than the 64 MiB scratch
        dq = cvs.DeviceArray(ctx, (q, 1024), np.float32)
        dn = cvs.DeviceArray(ctx, (q, k), np.uint32)
        dd = cvs.DeviceArray(ctx, (q, k), np.float32)
        with pytest.raises(ValueError) as err:
            ds.bf_search_noalloc(dq, k, dn, dd)
        assert "scratch" in str(err.value)
        assert cvs.load().cvs_bf_search_noalloc(ctx.handle, ds.handle, dq.ptr, q, k, dn.ptr, dd.ptr) \
            == CVS_ERR_UNSUPPORTED
        for a in (dq, dn, dd):
            a.free()
        # the scratch still serves a call that fits
        queries = cvs.synth_clustered(5, cvs.STREAM_QUERIES, 64, 1024)
        (n_ref, d_ref), (n_na, d_na) = run_both(cvs, ctx, ds, queries, 10)
        assert np.array_equal(n_na, n_ref) and np.array_equal(d_na, d_ref)
    finally:
        ds.close()
