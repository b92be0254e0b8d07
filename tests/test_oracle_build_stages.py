"""Pins each stage of the restated reference graph build
(oracle/cagra_build_oracle.c; reference src/metal_context.mm:289-914,
shaders/cagra_kernels.metal:334-462) on crafted inputs whose answers are
written out or follow from brute force on a handful of rows, then pins the
composed build against the chain of stages with the reference's constants.

Each known answer is shown to reject a plausible mistake: the oracle is
rebuilt with that mistake switched on (ORACLE_PLANT, oracle.build_variant)
and the same check must fail.

Stages and the mistakes their checks reject:
- kmeans_init (:366-375): centres at rows floor(k s + s/2) - plant 4 drops
  the half stride.
- ivf_kmeans (:381-435): a hand-worked run where two initial centres are the
  same vector; the lower index takes every row, the empty centre becomes the
  zero vector and then captures the rows near the origin - plants 1 (ties to
  the higher index), 2 (an empty centre keeps its old value) and 3 (divides
  by count + 1).
- ivf_near_clusters (:583-611): centres at 0, 1, 3, 7, ..., 127 - plant 5
  (the centre itself is not excluded).
- ivf_seed (:576-582, :712-792): a true neighbour reachable only through the
  third near cluster, a close row in a cluster that is not probed, and the
  max_own cap that leaves the last member unseeded and out of the candidate
  set - plants 6 (two probes) and 7 (no cap); with product-quantisation codes
  (:614-681) it equals the exact form on rows built from the quantisation
  prototypes - plant 8 (seven of the eight subspaces summed).
- bucketing_perm (:802-810): every swap index, recovered from the output by
  inverting the Fisher-Yates shuffle, equals (x_k >> 33) mod (i + 1) with the
  generator state x_k in closed form (jump-ahead) - plants 12 (shift 32), 13
  (ascending i) and 14 (generator advanced after the swap).
- bucketing_merge (kernel :403-462): every row gets its min(g, 64) nearest
  bucket mates, and a mate already in the row is inserted again - plant 9
  (duplicates dropped).
- nn_descent (kernel :334-395, host :853-911): a chain along which each
  iteration moves one hop, and a row where the worst entry must be replaced -
  plants 10 (replaces the first entry) and 11 (miscounts iterations).
"""
import math

import numpy as np
import pytest

INV = 0xFFFFFFFF


@pytest.fixture(scope="module")
def planted(oracle, tmp_path_factory):
    """plant number -> path of a copy of the oracle with that mistake."""
    out = str(tmp_path_factory.mktemp("oracle_plants"))
    cache = {}

    def get(n):
        if n not in cache:
            cache[n] = oracle.build_variant(n, out)
        return cache[n]

    return get


def line_rows(pos, d=4):
    """Rows with the given 1-D positions in column 0 and zeros elsewhere."""
    pos = np.asarray(pos, np.float32)
    out = np.zeros((len(pos), d), np.float32)
    out[:, 0] = pos
    return out


# ---- k-means -----------------------------------------------------------------

def test_kmeans_init_rows(oracle, planted):
    """n = 1000, K = 7: s = 142.857..., centres at rows 71, 214, 357, 500,
    642, 785, 928 (the row index stored in every column)."""
    base = np.repeat(np.arange(1000, dtype=np.float32)[:, None], 4, axis=1)
    want = [71, 214, 357, 500, 642, 785, 928]
    assert oracle.kmeans_init(base, 7)[:, 0].astype(int).tolist() == want
    with oracle.variant(planted(4)):
        assert oracle.kmeans_init(base, 7)[:, 0].astype(int).tolist() != want
    # n / K integral: rows 62, 187, ..., 937
    assert oracle.kmeans_init(base, 8)[:, 0].astype(int).tolist() == [62 + 125 * k for k in range(8)]


KM_ROWS = line_rows([4, 4, 4, 5, 1, 0, 4, 0])
KM_ROWS[7] = [0, 1, 0, 0]


def kmeans_hand_case(oracle):
    init = oracle.kmeans_init(KM_ROWS, 2)
    return oracle.ivf_kmeans(KM_ROWS, init, max_iter=20)


def test_kmeans_hand_worked(oracle, planted):
    """Rows (4,0) x4 (ids 0, 1, 2, 6), (5,0), (1,0), (0,0), (0,1); K = 2
    starts from rows 2 and 6, both (4,0).
    E-step 1: every distance ties, the lower centre takes all rows; M-step 1:
    centre 0 = mean (2.75, 0.125), centre 1 has no rows -> zero.
    E-step 2: (1,0), (0,0), (0,1) are nearer the origin; M-step 2: centre 0 =
    21 / 5 along x, centre 1 = (1/3, 1/3).
    E-step 3: nothing moves -> stop after 3 E-steps."""
    assert np.array_equal(oracle.kmeans_init(KM_ROWS, 2), KM_ROWS[[2, 6]])
    cent, assign, iters = kmeans_hand_case(oracle)
    assert assign.tolist() == [0, 0, 0, 0, 1, 1, 0, 1]
    assert iters == 3
    fifth, third = np.float32(1) / np.float32(5), np.float32(1) / np.float32(3)
    assert cent.tolist() == [[float(np.float32(21) * fifth), 0, 0, 0], [float(third), float(third), 0, 0]]
    for plant in (1, 2, 3):
        with oracle.variant(planted(plant)):
            c2, a2, _ = kmeans_hand_case(oracle)
        assert not (np.array_equal(a2, assign) and np.array_equal(c2, cent)), plant


def test_kmeans_iteration_cap(oracle):
    """The loop stops at max_iter E-steps without a final M-step check."""
    cent, assign, iters = oracle.ivf_kmeans(KM_ROWS, oracle.kmeans_init(KM_ROWS, 2), max_iter=1)
    assert iters == 1
    assert assign.tolist() == [0] * 8  # first E-step: every row ties to centre 0
    assert cent.tolist() == [[2.75, 0.125, 0, 0], [0, 0, 0, 0]]


# ---- near clusters -------------------------------------------------------------

def test_near_clusters_closed_form(oracle, planted):
    """Centres at 0, 1, 3, 7, 15, 31, 63, 127 on a line: gaps double, so the
    nearest three of each are its neighbours on the line, nearest first."""
    cent = line_rows([0, 1, 3, 7, 15, 31, 63, 127])
    want = [[1, 2, 3], [0, 2, 3], [1, 0, 3], [2, 1, 0], [3, 2, 1], [4, 3, 2], [5, 4, 3], [6, 5, 4]]
    assert oracle.ivf_near_clusters(cent, 3).tolist() == want
    with oracle.variant(planted(5)):
        assert oracle.ivf_near_clusters(cent, 3).tolist() != want


# ---- per-cluster seeding ------------------------------------------------------

SEED_POS = [0, 1, 3, 6, 10, 15, 21, 28,  # cluster 0 (ids 0-7)
            100, 102,                   # cluster 1 (ids 8-9)
            200, 203,                   # cluster 2 (ids 10-11)
            23, 50,                     # cluster 3 (ids 12-13)
            20]                         # cluster 4 (id 14)
SEED_ASSIGN = [0] * 8 + [1, 1, 2, 2, 3, 3, 4]
SEED_NEAR = [[1, 2, 3], [2, 0, 3], [1, 0, 3], [0, 4, 1], [3, 0, 1]]
SEED_G, SEED_MAX_OWN = 3, 7


def seed_case(oracle):
    return oracle.ivf_seed(line_rows(SEED_POS), SEED_G, SEED_ASSIGN, SEED_NEAR, SEED_MAX_OWN)


def seed_brute_force():
    """Expected rows from the candidate sets: a cluster's first max_own
    members (row order) then all members of its near clusters in order; each
    of those first members takes its g nearest candidates, nearest first."""
    pos = np.asarray(SEED_POS, np.int64)
    members = {k: [i for i, a in enumerate(SEED_ASSIGN) if a == k] for k in range(len(SEED_NEAR))}
    want = np.full((len(pos), SEED_G), INV, np.int64)
    for k, own in members.items():
        cand = own[:SEED_MAX_OWN] + [i for c in SEED_NEAR[k] for i in members[c]]
        for v in own[:SEED_MAX_OWN]:
            keyed = sorted((int((pos[v] - pos[c]) ** 2), p, c) for p, c in enumerate(cand) if c != v)
            assert len(keyed) <= SEED_G or keyed[SEED_G - 1][0] != keyed[SEED_G][0], "tie at the g-th candidate"
            want[v, :min(SEED_G, len(keyed))] = [c for _, _, c in keyed[:SEED_G]]
    return want


def test_seed_probes_and_cap(oracle, planted):
    graph, gdist = seed_case(oracle)
    # Row 6 (position 21): id 12 (position 23) is reachable only through the
    # third near cluster of cluster 0; id 14 (position 20) sits in cluster 4,
    # which cluster 0 does not probe; id 7 (position 28) is past max_own and
    # is no candidate.
    assert graph[6].tolist() == [12, 5, 4]
    assert gdist[6].tolist() == [4.0, 36.0, 121.0]
    assert graph[7].tolist() == [INV] * 3  # past the cap: seeds nothing
    assert graph[14].tolist() == [6, 12, 5]
    assert np.array_equal(graph, seed_brute_force())
    for plant in (6, 7):
        with oracle.variant(planted(plant)):
            g2, _ = seed_case(oracle)
        assert not np.array_equal(g2, graph), plant


def prototype_rows(seed=3):
    """2048 rows of d = 1024 built from 256 dyadic prototypes per 128-column
    subspace (row 8 c + j holds prototype (c + m j) mod 256 in subspace m);
    every distance between them is an exact fp32 sum."""
    rng = np.random.default_rng(seed)
    protos = rng.integers(-32, 33, size=(8, 256, 128)).astype(np.float32) / 16.0
    i = np.arange(2048)
    c, j = i // 8, i % 8
    base = np.empty((2048, 1024), np.float32)
    for m in range(8):
        base[:, 128 * m:128 * (m + 1)] = protos[m][(c + m * j) % 256]
    return base


def pq_seed_case(oracle, base, with_codes):
    n, g = len(base), 16
    K = 45
    cent, assign, _ = oracle.ivf_kmeans(base, oracle.kmeans_init(base, K), 20, threads=8)
    near = oracle.ivf_near_clusters(cent, 3, threads=8)
    codes = lut = None
    if with_codes:
        codes, lut = oracle.pq_train(base, threads=8)
    return oracle.ivf_seed(base, g, assign, near, (n // K) * 4 + 64, codes, lut, threads=8)


def test_pq_seed_equals_exact_seed_on_prototype_rows(oracle, planted):
    """On rows made of the quantisation prototypes, the rows rebuilt from
    the codes are the rows themselves and every table sum and distance is
    exact, so PQ seeding (table sums, then exact float4 distances of the
    kept entries) gives the exact seeding's graph and distances."""
    base = prototype_rows()
    g_ex, d_ex = pq_seed_case(oracle, base, False)
    g_pq, d_pq = pq_seed_case(oracle, base, True)
    assert (g_ex != INV).any()
    assert np.array_equal(g_pq, g_ex)
    assert np.array_equal(d_pq, d_ex)
    with oracle.variant(planted(8)):
        g8, _ = pq_seed_case(oracle, base, True)
    assert not np.array_equal(g8, g_ex)


# ---- random bucketing --------------------------------------------------------

LCG_A = 6364136223846793005
LCG_C = 1442695040888963407
LCG_X0 = 0xFEDCBA9876543210
M64 = (1 << 64) - 1


def lcg_state(k):
    """State of the reference's generator after k steps (src/metal_context.mm:
    802-810), in closed form: x_k = a^k x_0 + c (1 + a + ... + a^(k-1)) mod
    2^64, with a^k and the geometric sum by repeated squaring (the sum over
    2m terms is the sum over m terms times 1 + a^m), not by stepping."""
    def power_and_sum(m):
        if m == 0:
            return 1, 0
        p, s = power_and_sum(m // 2)
        p2, s2 = (p * p) & M64, (s * (1 + p)) & M64
        if m & 1:
            p2, s2 = (p2 * LCG_A) & M64, (1 + LCG_A * s2) & M64
        return p2, s2
    ak, sk = power_and_sum(k)
    return (ak * LCG_X0 + LCG_C * sk) & M64


def test_lcg_state_closed_form():
    """The repeated-squaring form against direct stepping for the first
    steps, and against the geometric sum (a^k - 1) / (a - 1) taken exactly
    (a^k modulo (a - 1) 2^64, then divided) at large k."""
    x = LCG_X0
    for k in range(1, 200):
        x = (x * LCG_A + LCG_C) & M64
        assert lcg_state(k) == x
    for k in (12345, 100_002, 1 << 40):
        mod = (LCG_A - 1) << 64
        geo = ((pow(LCG_A, k, mod) - 1) % mod) // (LCG_A - 1)
        assert lcg_state(k) == (pow(LCG_A, k, 1 << 64) * LCG_X0 + LCG_C * geo) & M64


def fisher_yates_swaps(perm):
    """Swap indices j_i (i = n-1 down to 1) of a descending Fisher-Yates
    shuffle of the identity that produced `perm`.  Step i swaps positions i
    and j_i and never touches position i again, so perm[i] is the value at
    position j_i just before step i: the steps are replayed forward on an
    index of where each value sits.  Returns None if `perm` is not the output
    of such a shuffle (a recovered index above i)."""
    n = len(perm)
    cur = list(range(n))          # values by position before the next step
    where = list(range(n))        # position of each value
    swaps = {}
    for i in range(n - 1, 0, -1):
        j = where[perm[i]]
        if j > i:
            return None
        swaps[i] = j
        vi, vj = cur[i], cur[j]
        cur[i], cur[j] = vj, vi
        where[vi], where[vj] = j, i
    return swaps


def check_bucketing_perm(perm, sample=None, seed=3):
    """Every recovered swap index (or a sample of them) equals
    (x_(n-i) >> 33) mod (i + 1) with x_k from the closed form."""
    n = len(perm)
    if sorted(perm) != list(range(n)):
        return False
    swaps = fisher_yates_swaps(perm)
    if swaps is None:
        return False
    steps = list(range(n - 1, 0, -1))
    if sample is not None and len(steps) > sample:
        rng = np.random.default_rng(seed)
        steps = sorted(set(rng.choice(steps, sample, replace=False).tolist()) | {n - 1, 1})
    return all(swaps[i] == (lcg_state(n - i) >> 33) % (i + 1) for i in steps)


@pytest.mark.parametrize("n,sample", [(1, None), (2, None), (10, None), (1000, None), (100_003, 400)])
def test_bucketing_perm(oracle, n, sample):
    assert check_bucketing_perm(oracle.bucketing_perm(n).tolist(), sample)


@pytest.mark.parametrize("plant", [12, 13, 14])
def test_bucketing_perm_rejects_planted_mistakes(oracle, planted, plant):
    """Plants: 12 shifts by 32, 13 runs i upwards, 14 advances the generator
    after the swap; each must fail the closed-form check."""
    with oracle.variant(planted(plant)):
        for n in (10, 1000):
            perm = oracle.bucketing_perm(n).tolist()
            assert not check_bucketing_perm(perm)


def bucket_rows(n, seed=9):
    """Distinct integer positions with no repeated pairwise gap: every row's
    neighbours are ordered without ties."""
    rng = np.random.default_rng(seed)
    pos = []
    gaps = set()
    while len(pos) < n:
        x = int(rng.integers(0, 40 * n * n))
        new = {abs(x - y) for y in pos}
        if x in pos or new & gaps or len(new) < len(pos):
            continue
        gaps |= new
        pos.append(x)
    return np.asarray(pos, np.float64)


def bucket_expected(pos, g, bucket):
    n = len(pos)
    take = min(g, 64)
    want = []
    for v in range(n):
        b0 = (v // bucket) * bucket
        mates = [u for u in range(b0, min(b0 + bucket, n)) if u != v]
        mates.sort(key=lambda u: abs(pos[u] - pos[v]))
        want.append(set(mates[:take]))
    return want


@pytest.mark.parametrize("n,g", [(600, 4), (300, 80)])
def test_bucketing_merge_nearest_mates(oracle, n, g):
    """Identity permutation, buckets of 256 positions: every row holds
    exactly its min(g, 64) nearest bucket mates; with g = 80 the remaining
    16 slots stay empty."""
    pos = bucket_rows(n)
    base = line_rows(pos / 1024.0)  # positions < 2^24 / 1024: exact squares
    graph, _ = oracle.bucketing_merge(base, g, np.arange(n, dtype=np.uint32), 256)
    want = bucket_expected(pos, g, 256)
    for v in range(n):
        got = [x for x in graph[v].tolist() if x != INV]
        assert len(got) == len(want[v]) and set(got) == want[v], v


def test_bucketing_merge_keeps_duplicates(oracle, planted):
    """A row that already holds its nearest mate (at its distance) receives
    it again: the reference's merge has no duplicate check."""
    n, g = 300, 4
    pos = bucket_rows(n)
    base = line_rows(pos / 1024.0)
    near1 = [min((u for u in range((v // 256) * 256, min((v // 256) * 256 + 256, n)) if u != v),
                 key=lambda u: abs(pos[u] - pos[v])) for v in range(n)]
    graph = np.full((n, g), INV, np.uint32)
    gdist = np.full((n, g), np.inf, np.float32)
    graph[:, 0] = near1
    gdist[:, 0] = [np.sum((base[v] - base[near1[v]]) ** 2, dtype=np.float32) for v in range(n)]

    def run():
        return oracle.bucketing_merge(base, g, np.arange(n, dtype=np.uint32), 256, graph.copy(), gdist.copy())[0]

    out = run()
    assert all(out[v].tolist().count(near1[v]) == 2 for v in range(n))
    with oracle.variant(planted(9)):
        assert not any(run()[v].tolist().count(near1[v]) == 2 for v in range(n))


# ---- nn-descent ----------------------------------------------------------------

def chain_case(L):
    """Rows at positions 0..L; node 0 points at node L, node j >= 2 at j - 1,
    node 1 at node 2.  Only node 0 can improve, one hop per iteration (the
    neighbour of its neighbour is always one step closer), until it points
    at node 1."""
    base = line_rows(np.arange(L + 1))
    graph = np.zeros((L + 1, 1), np.uint32)
    graph[0, 0] = L
    graph[1, 0] = 2
    graph[2:, 0] = np.arange(1, L)
    gdist = np.array([[float(L * L)], [1.0]] + [[1.0]] * (L - 1), np.float32)
    return base, graph, gdist


def test_nn_descent_chain(oracle, planted):
    L = 9
    base, graph, gdist = chain_case(L)
    g_out, d_out, iters = oracle.nn_descent(base, graph, gdist, 20)
    assert g_out[0, 0] == 1 and d_out[0, 0] == 1.0
    assert np.array_equal(g_out[1:], graph[1:])
    assert iters == L  # L - 1 moves, then one iteration without a change
    g5, d5, it5 = oracle.nn_descent(base, graph, gdist, 5)
    assert it5 == 5 and g5[0, 0] == L - 5 and d5[0, 0] == float((L - 5) ** 2)
    with oracle.variant(planted(11)):
        assert oracle.nn_descent(base, graph, gdist, 20)[2] != L


def test_nn_descent_replaces_worst(oracle, planted):
    """Node 0 (position 0) holds [1 (d 1), 2 (d 100)]; its neighbour 1 holds
    node 3 (position 7, d 49 from node 0), which replaces the worst entry:
    [1, 3].  Nothing else improves, so the second iteration stops."""
    base = line_rows([0, 1, 10, 7])
    graph = np.array([[1, 2], [3, 0], [3, 1], [2, 1]], np.uint32)
    pos = np.array([0, 1, 10, 7], np.float32)
    gdist = (pos[:, None] - pos[graph]) ** 2
    g_out, d_out, iters = oracle.nn_descent(base, graph, gdist.astype(np.float32), 20)
    assert g_out.tolist() == [[1, 3], [3, 0], [3, 1], [2, 1]]
    assert d_out[0].tolist() == [1.0, 49.0]
    assert iters == 2
    with oracle.variant(planted(10)):
        assert oracle.nn_descent(base, graph, gdist.astype(np.float32), 20)[0].tolist() != g_out.tolist()


# ---- the composed build ---------------------------------------------------------

def ivf_data(n=3000, d=16, seed=21):
    """30 centres; 40% of the rows around the first (its cluster overflows
    max_own = (n / K) * 4 + 64), the rest spread over the others."""
    rng = np.random.default_rng(seed)
    cent = rng.standard_normal((30, d)).astype(np.float32) * 3
    which = np.where(rng.random(n) < 0.4, 0, rng.integers(1, 30, n))
    return (cent[which] + 0.5 * rng.standard_normal((n, d))).astype(np.float32)


def ivf_chain(oracle, base, g, K, iters=20, n_probe=3, max_own=None, bucket=256, nd=5, bucketing=True):
    n = len(base)
    cent, assign, _ = oracle.ivf_kmeans(base, oracle.kmeans_init(base, K), iters, threads=8)
    near = oracle.ivf_near_clusters(cent, n_probe, threads=8)
    graph, gdist = oracle.ivf_seed(base, g, assign, near, (n // K) * 4 + 64 if max_own is None else max_own,
                                   threads=8)
    if bucketing:
        graph, gdist = oracle.bucketing_merge(base, g, oracle.bucketing_perm(n), bucket, graph, gdist, threads=8)
    return oracle.nn_descent(base, graph, gdist, nd, threads=8)[0]


def test_composed_ivf_build_is_the_stage_chain(oracle):
    """oracle_cagra_build_ref's IVF path (here at n = 3,000 through
    exact_limit = 0) equals the stages chained with the reference's settings:
    K = clamp(floor(sqrt n), G + 1, 2000), 20 Lloyd iterations, 3 probes,
    max_own = (n / K) * 4 + 64, one bucketing pass over buckets of 256, 5
    nn-descent iterations.  Changing any one of them changes the graph."""
    base = ivf_data()
    n, g = len(base), 16
    K = min(max(int(math.isqrt(n)), g + 1), 2000)
    assert K == 54
    composed = oracle.cagra_build_reference(base, g, threads=8, exact_limit=0, pq_limit=10**9)
    assert np.array_equal(composed, ivf_chain(oracle, base, g, K))
    variants = {
        "K - 1": dict(K=K - 1),
        "2 probes": dict(n_probe=2),
        "max_own without x4": dict(max_own=(n // K) + 64),
        "buckets of 255": dict(bucket=255),
        "no bucketing pass": dict(bucketing=False),
        "3 nn-descent iterations": dict(nd=3),
    }
    for name, kw in variants.items():
        args = dict(K=K)
        args.update(kw)
        assert not np.array_equal(composed, ivf_chain(oracle, base, g, **args)), name


def test_composed_build_k_floor(oracle):
    """With sqrt(n) below G + 1 the centre count is G + 1: n = 100, G = 16
    gives K = 17, not 10."""
    base = ivf_data(n=100, d=8, seed=4)
    composed = oracle.cagra_build_reference(base, 16, threads=4, exact_limit=0, pq_limit=10**9)
    assert np.array_equal(composed, ivf_chain(oracle, base, 16, 17))
    assert not np.array_equal(composed, ivf_chain(oracle, base, 16, 10))


def test_composed_pq_build_is_the_stage_chain(oracle):
    """The PQ path (n > pq_limit): the same IVF stages with the seeding
    ranked by table sums, one bucketing pass and no nn-descent."""
    base = prototype_rows()
    n, g = len(base), 16
    K = min(max(int(math.isqrt(n)), g + 1), 2000)
    composed = oracle.cagra_build_reference(base, g, threads=8, exact_limit=0, pq_limit=0)
    cent, assign, _ = oracle.ivf_kmeans(base, oracle.kmeans_init(base, K), 20, threads=8)
    near = oracle.ivf_near_clusters(cent, 3, threads=8)
    codes, lut = oracle.pq_train(base, threads=8)
    graph, gdist = oracle.ivf_seed(base, g, assign, near, (n // K) * 4 + 64, codes, lut, threads=8)
    graph, gdist = oracle.bucketing_merge(base, g, oracle.bucketing_perm(n), 256, graph, gdist, threads=8)
    assert np.array_equal(composed, graph)
    # no nn-descent on this path: a further iteration would change the graph
    assert not np.array_equal(composed, oracle.nn_descent(base, graph, gdist, 1, threads=8)[0])
