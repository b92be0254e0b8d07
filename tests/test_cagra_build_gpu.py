"""GPU graph build (C ABI: cvs_cagra_build).

Gates:
  - invariants of the returned graph: n x min(graph_degree, n - 1) ids, all
    in range, no self edges, no duplicate edges in a row (the reference's
    build allows duplicates; this one must not);
  - neighbour quality: the share of each row's exact 10 nearest neighbours
    that appear in its list (the build keeps the closest half of the pruned
    list first);
  - downstream recall: graph search on the built graph reaches at least the
    recall of the restated reference search on the reference's own graph
    for n <= 50,000 (exact all-pairs seeding, src/metal_context.mm:324-349,
    which the oracle's exact kNN graph stands for) at equal degree and itopk,
    by the paired gate of tests/search_metrics.py;
  - nn-descent convergence: the last iteration's insertion rate is below the
    threshold unless the iteration cap was reached.
"""
import numpy as np
import pytest

from search_metrics import assert_recall_not_below, exact_knn

pytestmark = pytest.mark.gpu

INV = 0xFFFFFFFF


def clustered(rng, n, d, centers=16, sigma=0.5):
    c = rng.standard_normal((centers, d)).astype(np.float32)
    return c[rng.integers(0, centers, n)] + sigma * rng.standard_normal((n, d)).astype(np.float32)


def check_graph(graph, n, g):
    """Every row holds g distinct in-range ids other than its own (n - 1 >= g
    here, so no slot may stay empty)."""
    assert graph.shape == (n, g)
    assert (graph != INV).all(), f"{int((graph == INV).sum())} empty slots"
    assert (graph < n).all()
    assert not (graph == np.arange(n)[:, None]).any()
    for i in range(n):
        assert len(set(graph[i].tolist())) == g, f"row {i} repeats an id"


def recall(nbr, gt, k):
    return float(np.mean([len(set(nbr[i, :k].tolist()) & set(gt[i, :k].tolist())) / k for i in range(len(nbr))]))


@pytest.mark.parametrize("n,d", [(2, 3), (40, 8), (200, 16)])
def test_single_bucket_graphs(ctx, oracle, n, d):
    """n <= 256: one bucket holds every row, so lists start exact."""
    rng = np.random.default_rng(n)
    base = rng.standard_normal((n, d)).astype(np.float32)
    graph, st = ctx.cagra_build(base, intermediate_degree=32, graph_degree=16)
    g = min(16, n - 1)
    check_graph(graph, n, g)
    assert st["graph_degree"] == g and st["intermediate_degree"] == min(32, n - 1)
    # every row holds its exact nearest neighbour
    exact = oracle.knn_graph(base, 1, threads=8)
    assert np.mean([exact[i, 0] in set(graph[i].tolist()) for i in range(n)]) >= 0.97


def test_neighbour_quality_and_convergence(ctx, oracle):
    rng = np.random.default_rng(21)
    n, d = 6000, 64
    base = clustered(rng, n, d)
    graph, st = ctx.cagra_build(base, intermediate_degree=64, graph_degree=32, max_iterations=30)
    check_graph(graph, n, 32)
    print("build stats:", st)
    assert st["iterations"] >= 2
    assert st["iterations"] == 30 or st["final_update_rate"] < 0.001
    exact = oracle.knn_graph(base, 10, threads=16)
    share = np.mean([len(set(exact[i].tolist()) & set(graph[i].tolist())) / 10 for i in range(n)])
    print(f"share of exact 10-NN in the built lists: {share:.4f}")
    assert share > 0.9


@pytest.mark.parametrize("offset_norm", [0.0, 300.0])
def test_neighbour_quality_on_offset_data(ctx, oracle, offset_norm):
    """Unit-norm clustered rows shifted by a common offset: the build's fp16
    copy is centred, so the share of exact neighbours in the lists is the
    same as without the offset (uncentred fp16 rows at offset 300 carry a
    rounding error of ~0.15 per coordinate, far above the neighbour gaps)."""
    rng = np.random.default_rng(77)
    n, d = 6000, 256
    c = rng.standard_normal((32, d)).astype(np.float32)
    x = c[rng.integers(0, 32, n)] + 0.3 * rng.standard_normal((n, d)).astype(np.float32)
    base = x / np.linalg.norm(x, axis=1, keepdims=True)
    off = rng.standard_normal(d)
    base = (base + off * (offset_norm / np.linalg.norm(off))).astype(np.float32)
    graph, _ = ctx.cagra_build(base, intermediate_degree=64, graph_degree=32, max_iterations=30)
    check_graph(graph, n, 32)
    exact = oracle.knn_graph(base, 10, threads=16)
    share = np.mean([len(set(exact[i].tolist()) & set(graph[i].tolist())) / 10 for i in range(n)])
    print(f"offset {offset_norm}: share of exact 10-NN in the built lists: {share:.4f}")
    assert share > 0.9


def test_build_wide_rows(ctx, oracle):
    """d = 1536: the build's fp16 rows, Gram tiles and joins over more than
    1,024 columns."""
    rng = np.random.default_rng(15)
    n, d = 4000, 1536
    base = clustered(rng, n, d)
    graph, _ = ctx.cagra_build(base, intermediate_degree=64, graph_degree=32, max_iterations=20)
    check_graph(graph, n, 32)
    exact = oracle.knn_graph(base, 10, threads=16)
    share = np.mean([len(set(exact[i].tolist()) & set(graph[i].tolist())) / 10 for i in range(n)])
    print(f"d=1536: share of exact 10-NN in the built lists: {share:.4f}")
    assert share > 0.9


@pytest.mark.parametrize("iters", [0, 1, 2, 3])
def test_iteration_limits(ctx, oracle, iters):
    """The join's locality order is made after the first nn-descent
    iteration: 0 iterations prune the bucketing lists in node order, 1 makes
    the order and prunes in it, 2 and more also join in it.  Each graph is
    valid, and joining improves the lists."""
    rng = np.random.default_rng(33)
    n, d = 3000, 48
    base = clustered(rng, n, d)
    graph, st = ctx.cagra_build(base, intermediate_degree=64, graph_degree=32, max_iterations=iters,
                                termination_threshold=0.0)
    check_graph(graph, n, 32)
    assert st["iterations"] == iters
    exact = oracle.knn_graph(base, 10, threads=16)
    share = np.mean([len(set(exact[i].tolist()) & set(graph[i].tolist())) / 10 for i in range(n)])
    print(f"iterations {iters}: share of exact 10-NN in the graph {share:.4f}", flush=True)
    floor = {0: 0.2, 1: 0.95, 2: 0.99, 3: 0.99}[iters]  # measured 0.285, 0.981, 0.9997, 0.9999
    assert share >= floor


@pytest.mark.parametrize("n,d,g,itopk,rescore", [(8000, 128, 32, 64, False), (5000, 1024, 64, 64, False),
                                                 (5000, 1024, 64, 64, True), (6000, 99, 32, 64, True)])
def test_downstream_recall_at_least_reference(ctx, oracle, n, d, g, itopk, rescore):
    """rescore: the final intermediate lists re-ranked by exact fp32
    distances before pruning (cvs_cagra_build_ex; d = 99 takes its
    scalar path)."""
    rng = np.random.default_rng(n + d)
    base = clustered(rng, n, d)
    qs = clustered(np.random.default_rng(7), 300, d)
    graph, st = ctx.cagra_build(base, intermediate_degree=2 * g, graph_degree=g, rescore_fp32=rescore)
    check_graph(graph, n, g)
    assert (st["seconds_rescore"] > 0) == rescore
    nav = oracle.cagra_nav_nodes(n)
    gt, _ = oracle.bf_exact(base, qs, 10, threads=16)
    ours, _ = ctx.cagra_index(base, graph, nav).search(qs, 10, itopk_size=itopk)
    ref_graph = oracle.knn_graph(base, g, threads=16)
    ref, _ = oracle.cagra_reference_search(base, ref_graph, nav, qs, 10, itopk_size=itopk, threads=16)
    assert_recall_not_below(ours, ref, gt, 10, f"n={n} d={d}: built graph + GPU search vs exact graph + "
                                               "restated reference search")


def test_device_output_matches_shape(ctx, cvs):
    rng = np.random.default_rng(3)
    base = rng.standard_normal((1000, 32)).astype(np.float32)
    out = cvs.DeviceArray(ctx, (1000, 24), np.uint32)
    dev = cvs.DeviceArray.from_host(ctx, base)
    g, st = ctx.cagra_build(dev, intermediate_degree=48, graph_degree=24, out=out)
    check_graph(g.to_host(), 1000, 24)


def test_build_argument_errors(ctx):
    with pytest.raises(ValueError):
        ctx.cagra_build(np.ones((1, 4), np.float32))
    with pytest.raises(ValueError):
        ctx.cagra_build(np.ones((10, 4), np.float32), intermediate_degree=300)
    with pytest.raises(ValueError):
        ctx.cagra_build(np.ones((10, 4), np.float32), graph_degree=0)


def test_c5_full_size_build(ctx, cvs, oracle):
    """N=1,000,000, D=1024, intermediate degree 128 -> 64 on the clustered
    distribution: the graph invariants row by row (vectorised), nn-descent
    convergence below 0.1% insertions within the iteration cap, and graph
    search recall@10 at itopk 64 on 500 queries against exact k-NN (numpy):
    at least that of the graph the reference's own algorithm builds at this
    size (its N > 200,000 path: PQ seeding + one bucketing pass, no
    nn-descent; cvs_cagra_build_reference, checked against the oracle's
    restatement at n = 6,000 below) at equal degree and itopk, by the paired
    gate, and above 0.6 (a broken build)."""
    n, d, g = 1_000_000, 1024, 64
    base = cvs.synth_clustered(12345, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(12345, cvs.STREAM_QUERIES, 500, d)
    print("[c5] building N=1M", flush=True)
    graph, st = ctx.cagra_build(base, intermediate_degree=128, graph_degree=g)
    assert graph.shape == (n, g)
    assert (graph < n).all()
    assert not (graph == np.arange(n, dtype=np.uint32)[:, None]).any()
    srt = np.sort(graph, axis=1)
    assert not (srt[:, 1:] == srt[:, :-1]).any(), "a row repeats an id"
    assert st["iterations"] <= 20
    assert st["final_update_rate"] < 0.001 or st["iterations"] == 20
    print("[c5] exact ground truth", flush=True)
    gt = exact_knn(base, qs, 10)
    nav = cvs.cagra_nav_nodes(n)
    idx = ctx.cagra_index(base, graph, nav)
    nbr, _ = idx.search(qs, 10, itopk_size=64)
    idx.close()
    r = recall(nbr, gt, 10)
    print(f"N=1M build: {st['seconds_total']:.2f} s, {st['iterations']} iterations, recall@10 {r:.4f}")
    assert r >= 0.6, r
    print("[c5] the reference's algorithm at N=1M", flush=True)
    rgraph, _ = ctx.cagra_build_reference(base, g)
    ridx = ctx.cagra_index(base, rgraph, nav)
    rnbr, _ = ridx.search(qs, 10, itopk_size=64)
    ridx.close()
    assert_recall_not_below(nbr, rnbr, gt, 10, "N=1M this build vs the reference algorithm's graph, itopk 64")


def neighbour_recall(graph, exact, k):
    """Share of each row's exact k nearest neighbours present in its list."""
    return float(np.mean([len(set(graph[i].tolist()) & set(exact[i, :k].tolist())) / k for i in range(len(graph))]))


@pytest.mark.parametrize("n,d,g", [(3000, 64, 32), (3000, 77, 32), (60_000, 128, 64)])
def test_reference_build_matches_oracle(ctx, cvs, oracle, n, d, g):
    """cvs_cagra_build_reference (the reference's build, src/metal_context.mm:
    289-914, on the GPU) against the oracle's restatement of it on the same
    data: the same graph invariants (no repeated ids, which the reference
    itself allows), and neighbour quality and the restated reference
    search's recall on each graph not below the restated graph's (paired
    gates over rows and queries).
    n = 3000: the exact path (exact kNN graph: all but ties equal); n = 60,000:
    k-means + per-cluster seeding, bucketing and nn-descent."""
    base = cvs.synth_clustered(4242, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(4242, cvs.STREAM_QUERIES, 300, d)
    graph, st = ctx.cagra_build_reference(base, g)
    check_graph(graph, n, g)
    ref = oracle.cagra_build_reference(base, g, threads=16)
    sample = np.random.default_rng(1).choice(n, 500, replace=False)
    gt_rows, _ = oracle.bf_exact(base, base[sample], 11, threads=16)
    exact = np.stack([r[r != s][:10] for r, s in zip(gt_rows, sample)])
    q_gpu = neighbour_recall(graph[sample], exact, 10)
    q_ref = neighbour_recall(ref[sample], exact, 10)
    nav = oracle.cagra_nav_nodes(n)
    gt, _ = oracle.bf_exact(base, qs, 10, threads=16)
    s_gpu, _ = oracle.cagra_reference_search(base, graph, nav, qs, 10, itopk_size=64, threads=16)
    s_ref, _ = oracle.cagra_reference_search(base, ref, nav, qs, 10, itopk_size=64, threads=16)
    r_gpu, r_ref = recall(s_gpu, gt, 10), recall(s_ref, gt, 10)
    print(f"n={n}: stats {st}; neighbour recall@10 gpu {q_gpu:.4f} oracle {q_ref:.4f}; "
          f"search recall gpu graph {r_gpu:.4f} oracle graph {r_ref:.4f}")
    if n <= 50_000:
        assert st["clusters"] == 0 and q_gpu >= 0.999
    else:
        assert st["clusters"] == int(np.sqrt(n)) and 1 <= st["kmeans_iterations"] <= 20
        assert 1 <= st["descent_iterations"] <= 5
    assert_recall_not_below(graph[sample], ref[sample], exact, 10, f"n={n} neighbour recall", whole_rows=True)
    assert_recall_not_below(s_gpu, s_ref, gt, 10, f"n={n} search recall on the GPU graph vs the oracle's graph")


@pytest.mark.gpu
def test_reference_pq_build_matches_oracle(ctx, cvs, oracle):
    """The reference's N > 200,000 build (product-quantised per-cluster
    seeding, src/metal_context.mm:437-709; no nn-descent, src/cagra.cpp:59),
    run at n = 6,000 through the size-limit arguments, against the oracle's
    restatement.  The GPU ranks candidates by the squared distance of the rows
    rebuilt from their codes, the oracle by summing the symmetric PQ table
    (two formulations of the same distance), so graphs agree up to fp32 ties:
    neighbour recall and the restated reference search recall not below the
    oracle graph's (paired gates)."""
    n, d, g = 6000, 1024, 32
    base = cvs.synth_clustered(77, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(77, cvs.STREAM_QUERIES, 300, d)
    print(f"reference PQ build n={n} d={d} g={g} on the GPU", flush=True)
    graph, st = ctx.cagra_build_reference(base, g, exact_limit=0, pq_limit=0)
    check_graph(graph, n, g)
    ref = oracle.cagra_build_reference(base, g, threads=16, exact_limit=0, pq_limit=0)
    sample = np.random.default_rng(2).choice(n, 500, replace=False)
    gt_rows, _ = oracle.bf_exact(base, base[sample], 11, threads=16)
    exact = np.stack([r[r != s][:10] for r, s in zip(gt_rows, sample)])
    q_gpu = neighbour_recall(graph[sample], exact, 10)
    q_ref = neighbour_recall(ref[sample], exact, 10)
    nav = oracle.cagra_nav_nodes(n)
    gt, _ = oracle.bf_exact(base, qs, 10, threads=16)
    s_gpu, _ = oracle.cagra_reference_search(base, graph, nav, qs, 10, itopk_size=64, threads=16)
    s_ref, _ = oracle.cagra_reference_search(base, ref, nav, qs, 10, itopk_size=64, threads=16)
    r_gpu, r_ref = recall(s_gpu, gt, 10), recall(s_ref, gt, 10)
    print(f"stats {st}; neighbour recall@10 gpu {q_gpu:.4f} oracle {q_ref:.4f}; "
          f"search recall gpu graph {r_gpu:.4f} oracle graph {r_ref:.4f}")
    assert st["descent_iterations"] == 0 and 8 <= st["pq_iterations"] <= 80
    assert_recall_not_below(graph[sample], ref[sample], exact, 10, "PQ path neighbour recall", whole_rows=True)
    assert_recall_not_below(s_gpu, s_ref, gt, 10, "PQ path search recall on the GPU graph vs the oracle's graph")
    with pytest.raises(ValueError):  # CVS_ERR_UNSUPPORTED: the PQ path needs d = 1024
        ctx.cagra_build_reference(base[:, :512], g, exact_limit=0, pq_limit=0)
