"""GPU: cvs_cagra_optimize, the build's pruning applied to caller k-NN lists,
and cvs_build_options.intermediate_out, the build's own lists before pruning.

The pruning is checked against a direct numpy statement of the rank-based
detour count (Ootomo et al., CAGRA, 2023): edge u -> v_j (rank j) is
detourable via v_i when i < j and v_j sits at a rank p < j in v_i's list;
each node keeps the g edges of fewest detours, ties by rank, in rank order.
The reverse-edge merge appends in arrival order (device atomics), so it is
checked by what it must hold: the first g/2 entries are the first g/2 kept
edges, every entry is a kept or a reverse edge, no entry repeats, and the
row is as full as those sets allow.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

INVALID = 0xFFFFFFFF


def detour_keep(lists, g):
    """Kept edges per node: lists is (n, kd) of valid ids, nearest first."""
    n, kd = lists.shape
    # rank of w in v's list, as a dict per row
    rank = [dict(zip(row.tolist(), range(kd))) for row in lists]
    kept = np.full((n, g), INVALID, np.uint32)
    for u in range(n):
        row = lists[u]
        det = np.zeros(kd, np.int64)
        for i in range(kd):
            ri = rank[int(row[i])]
            for j in range(i + 1, kd):
                p = ri.get(int(row[j]))
                if p is not None and p < j:
                    det[j] += 1
        order = sorted(range(kd), key=lambda j: (det[j], j))[:g]
        kept[u, :len(order)] = row[sorted(order)]
    return kept


def check_graph(graph, kept, g, r):
    n = graph.shape[0]
    half = g - r
    rev = [set() for _ in range(n)]
    for u in range(n):
        for w in kept[u]:
            if w != INVALID:
                rev[int(w)].add(u)
    for u in range(n):
        row = [int(w) for w in graph[u] if w != INVALID]
        assert len(row) == len(set(row)), u
        assert u not in row, u
        np.testing.assert_array_equal(graph[u, :half], kept[u, :half])
        ks = set(int(w) for w in kept[u] if w != INVALID)
        assert set(row) <= ks | rev[u], u
        if len(rev[u]) <= g:  # every reverse edge arrived: the fill is known
            assert len(row) == min(g, len(ks | rev[u])), u
            fresh = rev[u] - set(int(w) for w in kept[u, :half])
            if len(fresh) <= r:
                assert fresh <= set(row), u


@pytest.fixture(scope="module")
def exact_lists(oracle):
    rng = np.random.default_rng(11)
    n, d, kd = 3000, 48, 40
    centres = rng.standard_normal((30, d)).astype(np.float32)
    base = (centres[rng.integers(0, 30, n)] + 0.4 * rng.standard_normal((n, d))).astype(np.float32)
    return base, oracle.knn_graph(base, kd, threads=8)


@pytest.mark.parametrize("g", [20, 32])
def test_optimize_matches_detour_statement(ctx, exact_lists, g):
    print(f"[optimize] g={g}", flush=True)
    _, lists = exact_lists
    kept = detour_keep(lists, g)
    # without reverse edges the result is the kept edges, exactly
    np.testing.assert_array_equal(ctx.cagra_optimize(lists, g), kept)
    for r in (1, g // 4, g // 2, g):
        check_graph(ctx.cagra_optimize(lists, g, reverse_edges=r), kept, g, r)


def test_optimize_ignores_self_repeats_and_out_of_range(ctx, exact_lists):
    """Lists with the node itself, repeats and ids >= n mixed in give the
    same kept edges as the clean lists."""
    print("[optimize] junk entries", flush=True)
    _, lists = exact_lists
    n, kd = lists.shape
    g = 24
    rng = np.random.default_rng(3)
    width = kd + 12
    noisy = np.full((n, width), INVALID, np.uint32)
    for u in range(n):
        out, junk = [], 0
        for w in lists[u]:
            out.append(int(w))
            if junk < width - kd and rng.random() < 0.2:
                junk += 1
                # the node itself, an id >= n, a padding id, or a repeat of
                # an id already placed (the first occurrence keeps its rank)
                out.append([u, n + int(rng.integers(1000)), INVALID, out[int(rng.integers(len(out)))]][rng.integers(4)])
        assert len(out) <= width
        noisy[u, :len(out)] = out
    np.testing.assert_array_equal(ctx.cagra_optimize(noisy, g), ctx.cagra_optimize(lists, g))
    check_graph(ctx.cagra_optimize(noisy, g, reverse_edges=g // 2), detour_keep(lists, g), g, g // 2)


def test_optimize_device_arrays(cvs, ctx, exact_lists):
    _, lists = exact_lists
    n, kd = lists.shape
    dk = cvs.DeviceArray.from_host(ctx, lists)
    dg = cvs.DeviceArray(ctx, (n, 16), np.uint32)
    ctx.cagra_optimize(dk, 16, out=dg)
    np.testing.assert_array_equal(dg.to_host()[:, :8], ctx.cagra_optimize(lists, 16)[:, :8])
    dk.free()
    dg.free()


@pytest.mark.parametrize("mode", ["knn", "detour", "detour+reverse"])
def test_build_graph_modes_from_intermediate_lists(cvs, ctx, mode):
    """The lists the build exports through intermediate_out give its graph:
    the kept edges of cvs_cagra_optimize on them (the default; the pruning
    reads those lists and nothing else), the first g entries (the
    reference's k-NN graph), or the kept edges merged with g/2 reverse
    edges."""
    print(f"[optimize] build lists, {mode}", flush=True)
    base = cvs.synth_clustered(5, cvs.STREAM_BASE, 20_000, 128)
    n, kd, g = base.shape[0], 64, 32
    gm = cvs.GRAPH_KNN if mode == "knn" else cvs.GRAPH_DETOUR
    r = g // 2 if mode == "detour+reverse" else 0
    inter = cvs.DeviceArray(ctx, (n, kd), np.uint32)
    graph, _ = ctx.cagra_build(base, intermediate_degree=kd, graph_degree=g, intermediate_out=inter, graph_mode=gm,
                               reverse_edges=r)
    lists = inter.to_host()
    inter.free()
    assert (lists != INVALID).all()
    assert not (lists == np.arange(n, dtype=np.uint32)[:, None]).any()
    if mode == "knn":
        np.testing.assert_array_equal(graph, lists[:, :g])
    elif mode == "detour":
        np.testing.assert_array_equal(graph, ctx.cagra_optimize(lists, g))
        # cvs_cagra_build (no options) makes the same kind of graph: kept
        # edges in rank order, so rows sorted by distance (two builds differ
        # slightly: the order in which joins append to the update bins varies)
        default, _ = ctx.cagra_build(base, intermediate_degree=kd, graph_degree=g)
        d = ((base[default[:500]] - base[:500, None, :]) ** 2).sum(-1)
        assert (np.diff(d, axis=1) >= -1e-2 * d[:, 1:]).mean() > 0.99
    else:
        np.testing.assert_array_equal(ctx.cagra_optimize(lists, g)[:, :g - r], graph[:, :g - r])
        check_graph(graph, ctx.cagra_optimize(lists, g), g, r)
    # lists are sorted by exact distance up to the build's fp16 rounding
    d = ((base[lists[:200]] - base[:200, None, :]) ** 2).sum(-1)
    assert (np.diff(d, axis=1) >= -1e-2 * d[:, 1:]).mean() > 0.99


def test_optimize_argument_errors(cvs, ctx):
    lists = np.zeros((10, 8), np.uint32)
    rows = np.random.default_rng(0).standard_normal((100, 8)).astype(np.float32)
    with pytest.raises(ValueError):
        ctx.cagra_build(rows, 16, 8, graph_mode=3)
    with pytest.raises(ValueError):
        ctx.cagra_build(rows, 16, 8, graph_mode=cvs.GRAPH_KNN, reverse_edges=2)
    with pytest.raises(ValueError):
        ctx.cagra_optimize(lists, 9)  # graph_degree > list width
    with pytest.raises(ValueError):
        ctx.cagra_optimize(np.zeros((10, 257), np.uint32), 8)
    with pytest.raises(ValueError):
        ctx.cagra_optimize(np.zeros((1, 8), np.uint32), 4)
    with pytest.raises(ValueError):
        ctx.cagra_optimize(lists, 8, reverse_edges=9)
