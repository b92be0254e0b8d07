// C++ API checks on the GPU, written the way the reference's callers use the
// API:
//  - the FAISS v1.8 adapter flow of tests/faiss_v1_8_cagra_runtime_smoke.cpp
//    (rebuild on every add, itopk_size = k, UINT32_MAX -> -1) with its known
//    answers (:299-357) and the attach_dataset_on_build = false lifecycle
//    (:247-261), without the FAISS headers;
//  - the dispatch test of tests/test_metal_search.cpp:16-58 (default
//    parameters, dispatch count > 0) plus the exact answers of its inputs;
//  - graph_degree = 0 (exact route, src/cagra.cpp:197-202) and the
//    brute_force namespace (uint32 and int64 ids; D = 1536 with K = 150 beyond
//    the fused scan's limits, bit for bit);
//  - build -> save_index -> load_index -> search on random data against exact
//    search;
//  - the default graph search traverses in fp32 (fp16 traversal is opt-in);
//  - MetalContext::search_brute_force and search_cagra (the reference's
//    backend interface) against the C ABI, with a distinct entry node per
//    query, and the reference_beam search mode of cagra::search.
#include <cuvs/neighbors/brute_force.hpp>
#include <cuvs/neighbors/cagra.hpp>
#include <cuvs_silicon/metal_context.hpp>

#include "cvs_hip.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <random>
#include <set>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "check.hpp"

namespace cagra = cuvs::neighbors::cagra;
namespace bf = cuvs::neighbors::brute_force;
using apitest::expect_throw;

namespace {

constexpr std::uint32_t kNone = std::numeric_limits<std::uint32_t>::max();

// The FAISS-facing adapter of the reference's runtime smoke test, minus FAISS.
struct FaissLikeIndex {
  std::int64_t d;
  std::int64_t ntotal = 0;
  std::vector<float> added;
  raft::resources res;
  cagra::index<float, std::uint32_t> index;

  explicit FaissLikeIndex(std::int64_t dim) : d(dim) {}

  void add(std::int64_t n, const float* v) {
    cagra::index_params params;
    params.metric = cuvs::distance::DistanceType::L2Expanded;
    added.insert(added.end(), v, v + n * d);
    index = cagra::build(res, params,
                         raft::make_device_matrix_view<const float, std::int64_t>(added.data(), ntotal + n, d));
    ntotal += n;
  }

  void search(std::int64_t q, const float* queries, std::int64_t k, float* dist, std::int64_t* labels) {
    if (k <= 0) throw std::invalid_argument("k > 0");
    cagra::search_params sp;
    sp.itopk_size = static_cast<std::uint64_t>(k);
    std::vector<std::uint32_t> ids(static_cast<std::size_t>(q * k));
    cagra::search(res, sp, index, raft::make_device_matrix_view<const float, std::int64_t>(queries, q, d),
                  raft::make_device_matrix_view<std::uint32_t, std::int64_t>(ids.data(), q, k),
                  raft::make_device_matrix_view<float, std::int64_t>(dist, q, k));
    for (std::int64_t i = 0; i < q * k; ++i) labels[i] = ids[i] == kNone ? -1 : static_cast<std::int64_t>(ids[i]);
  }
};

void faiss_smoke() {
  const std::vector<float> db{0, 0, 10, 0, 0, 10, 2, 2};
  const std::vector<float> qs{0, 0, 9, 1};
  {
    raft::resources res;
    cagra::index_params p;
    p.attach_dataset_on_build = false;
    const auto idx = cagra::build(res, p, raft::make_device_matrix_view<const float, std::int64_t>(db.data(), 4, 2));
    CHECK(idx.rows() == 4 && idx.cols() == 2 && idx.dataset().empty());
  }
  FaissLikeIndex index(2);
  index.add(2, db.data());
  index.add(2, db.data() + 4);
  CHECK(index.ntotal == 4 && index.index.rows() == 4);
  CHECK(index.index.graph_degree() == 3);  // min(64, N - 1)
  std::vector<float> dist(4);
  std::vector<std::int64_t> lab(4);
  index.search(2, qs.data(), 2, dist.data(), lab.data());
  CHECK(lab[0] == 0 && dist[0] == 0.f && lab[1] == 3 && dist[1] == 8.f);
  CHECK(lab[2] == 1 && dist[2] == 2.f && lab[3] == 3 && dist[3] == 50.f);
  // tie at distance 100: lower id first
  index.search(1, qs.data(), 4, dist.data(), lab.data());
  CHECK((lab == std::vector<std::int64_t>{0, 3, 1, 2}));
  CHECK((dist == std::vector<float>{0.f, 8.f, 100.f, 100.f}));
  // k > N: last slot -1 / +inf, for one and for two queries
  std::vector<float> d5(10, -7.f);
  std::vector<std::int64_t> l5(10, -7);
  index.search(1, qs.data(), 5, d5.data(), l5.data());
  CHECK(l5[0] == 0 && d5[0] == 0.f && l5[4] == -1 && std::isinf(d5[4]));
  index.search(2, qs.data(), 5, d5.data(), l5.data());
  CHECK(l5[4] == -1 && std::isinf(d5[4]) && l5[9] == -1 && std::isinf(d5[9]) && l5[5] == 1);
  expect_throw<std::invalid_argument>("k = 0", "k > 0", [&] { index.search(2, qs.data(), 0, d5.data(), l5.data()); });
}

void dispatch_test() {
  constexpr int N = 64, Q = 4, D = 8, K = 4;
  std::vector<float> base(N * D, 0.f), queries(Q * D, 0.f);
  for (int i = 0; i < N; ++i) base[i * D + (i % D)] = float(i);
  for (int q = 0; q < Q; ++q) queries[q * D + (q % D)] = 1.f;
  std::vector<std::uint32_t> nbr(Q * K);
  std::vector<float> dist(Q * K);
  raft::resources res;
  cagra::index_params ip;
  cagra::search_params sp;
  auto idx = cagra::build(res, ip, raft::device_matrix_view<const float, std::int64_t>(base.data(), N, D));
  cagra::reset_metal_dispatch_count();
  cagra::search(res, sp, idx, raft::device_matrix_view<const float, std::int64_t>(queries.data(), Q, D),
                raft::device_matrix_view<std::uint32_t, std::int64_t>(nbr.data(), Q, K),
                raft::device_matrix_view<float, std::int64_t>(dist.data(), Q, K));
  CHECK(cagra::metal_dispatch_count() > 0);
  const std::vector<std::uint32_t> en{0, 1, 2, 3, 1, 0, 2, 3, 0, 2, 1, 3, 0, 1, 3, 2};
  const std::vector<float> ed{1, 2, 5, 10, 0, 1, 5, 10, 1, 1, 2, 10, 1, 2, 4, 5};
  CHECK(nbr == en);
  CHECK(dist == ed);
  // The exact route (graph_degree = 0) gives the same answers.
  cagra::index_params exact;
  exact.graph_degree = 0;
  auto eidx = cagra::build(res, exact, raft::device_matrix_view<const float, std::int64_t>(base.data(), N, D));
  CHECK(eidx.graph_degree() == 0 && eidx.knn_graph().empty());
  std::fill(nbr.begin(), nbr.end(), 0u);
  cagra::reset_metal_dispatch_count();
  cagra::search(res, sp, eidx, raft::device_matrix_view<const float, std::int64_t>(queries.data(), Q, D),
                raft::device_matrix_view<std::uint32_t, std::int64_t>(nbr.data(), Q, K),
                raft::device_matrix_view<float, std::int64_t>(dist.data(), Q, K));
  CHECK(cagra::metal_dispatch_count() > 0);
  CHECK(nbr == en && dist == ed);
  // brute_force namespace, uint32 and int64 ids, k > N padding.
  auto bidx = bf::build(res, raft::make_device_matrix_view<const float, std::int64_t>(base.data(), N, D));
  CHECK(bidx.size() == N && bidx.dim() == D);
  bf::search(res, bidx, raft::make_device_matrix_view<const float, std::int64_t>(queries.data(), Q, D),
             raft::make_device_matrix_view<std::uint32_t, std::int64_t>(nbr.data(), Q, K),
             raft::make_device_matrix_view<float, std::int64_t>(dist.data(), Q, K));
  CHECK(nbr == en && dist == ed);
  std::vector<float> small{0, 0, 1, 0, 0, 3, 0, 0};
  auto sidx = bf::build(res, raft::make_device_matrix_view<const float, std::int64_t>(small.data(), 2, 4));
  std::vector<std::int64_t> l64(3);
  std::vector<float> d3(3);
  bf::search(res, sidx, raft::make_device_matrix_view<const float, std::int64_t>(small.data(), 1, 4),
             raft::make_device_matrix_view<std::int64_t, std::int64_t>(l64.data(), 1, 3),
             raft::make_device_matrix_view<float, std::int64_t>(d3.data(), 1, 3));
  CHECK(l64[0] == 0 && l64[1] == 1 && l64[2] == -1 && d3[1] == 10.f && std::isinf(d3[2]));
}

void build_save_load_search(const std::string& scratch) {
  // 20 clusters, each a 4-dimensional Gaussian patch embedded in 48-d:
  // neighbourhoods a graph can navigate (isotropic 48-d noise would leave
  // every point about equally far from all its cluster mates).
  const int N = 3000, D = 48, Q = 50, K = 10, C = 20, R = 4;
  std::mt19937 gen(7);
  std::normal_distribution<float> nd(0.f, 1.f);
  std::vector<float> centers(C * D), basis(C * R * D), base(N * D), qs(Q * D);
  for (auto& v : centers) v = nd(gen);
  for (auto& v : basis) v = 0.5f * nd(gen);
  auto sample = [&](int c, float* out) {
    float z[R];
    for (int r = 0; r < R; ++r) z[r] = nd(gen);
    for (int j = 0; j < D; ++j) {
      float v = centers[c * D + j];
      for (int r = 0; r < R; ++r) v += z[r] * basis[(c * R + r) * D + j];
      out[j] = v;
    }
  };
  // random cluster labels (periodic labels would alias with the evenly
  // spaced navigation nodes)
  std::uniform_int_distribution<int> pick(0, C - 1);
  std::vector<int> base_label(N), query_label(Q);
  for (int i = 0; i < N; ++i) sample(base_label[i] = pick(gen), base.data() + i * D);
  for (int i = 0; i < Q; ++i) sample(query_label[i] = pick(gen), qs.data() + i * D);
  raft::resources res;
  cagra::index_params ip;
  ip.graph_degree = 32;
  ip.intermediate_graph_degree = 64;
  auto idx = cagra::build(res, ip, raft::make_device_matrix_view<const float, std::int64_t>(base.data(), N, D));
  CHECK(idx.graph_degree() == 32 && idx.knn_graph().size() == std::size_t(N) * 32);
  CHECK(idx.nav_nodes().size() == 54 && idx.nav_vectors().size() == 54u * D);  // min(200, sqrt(3000))
  for (std::size_t i = 0; i < idx.knn_graph().size(); ++i) CHECK(idx.knn_graph()[i] < std::uint32_t(N));
  cagra::save_index(idx, scratch + "/built.bin");
  const auto loaded = cagra::load_index(scratch + "/built.bin");
  CHECK(loaded.knn_graph() == idx.knn_graph() && loaded.nav_nodes() == idx.nav_nodes());
  std::vector<std::uint32_t> g(Q * K), e(Q * K);
  std::vector<float> gd(Q * K), ed(Q * K);
  cagra::search_params sp;
  cagra::search(res, sp, loaded, raft::make_device_matrix_view<const float, std::int64_t>(qs.data(), Q, D),
                raft::make_device_matrix_view<std::uint32_t, std::int64_t>(g.data(), Q, K),
                raft::make_device_matrix_view<float, std::int64_t>(gd.data(), Q, K));
  auto bidx = bf::build(res, raft::make_device_matrix_view<const float, std::int64_t>(base.data(), N, D));
  bf::search(res, bidx, raft::make_device_matrix_view<const float, std::int64_t>(qs.data(), Q, D),
             raft::make_device_matrix_view<std::uint32_t, std::int64_t>(e.data(), Q, K),
             raft::make_device_matrix_view<float, std::int64_t>(ed.data(), Q, K));
  // The clusters are far apart and the graph's edges stay inside them, so a
  // query whose cluster holds no navigation node (the search's seeds) is
  // answered from the wrong cluster: the recall gate counts the queries of
  // the clusters the navigation nodes reach.
  std::set<int> seeded;
  for (std::uint32_t v : idx.nav_nodes()) seeded.insert(base_label[v]);
  int hits = 0, hits_seeded = 0, seeded_queries = 0;
  for (int i = 0; i < Q; ++i) {
    std::set<std::uint32_t> s(e.begin() + i * K, e.begin() + (i + 1) * K);
    int h = 0;
    for (int j = 0; j < K; ++j) h += s.count(g[i * K + j]) ? 1 : 0;
    hits += h;
    if (seeded.count(query_label[i])) {
      hits_seeded += h;
      ++seeded_queries;
    }
  }
  const double recall = double(hits) / (Q * K);
  const double recall_seeded = double(hits_seeded) / (std::max(seeded_queries, 1) * K);
  std::printf("graph search recall@10 after save/load: %.3f (%d of %d clusters seeded; %.3f over their %d queries)\n",
              recall, int(seeded.size()), C, recall_seeded, seeded_queries);
  CHECK(seeded_queries >= Q / 2 && recall_seeded >= 0.9);

  // search_algo::MULTI_CTA: teams of workgroups per query, merged; each row
  // sorted by distance with unique ids, distances those of the exact search
  // for the same ids, recall close to the single search's.
  cagra::search_params mp;
  mp.algo = cagra::search_algo::MULTI_CTA;
  mp.itopk_size = 128;  // 4 teams of 32
  std::vector<std::uint32_t> m(Q * K);
  std::vector<float> md(Q * K);
  cagra::search(res, mp, loaded, raft::make_device_matrix_view<const float, std::int64_t>(qs.data(), Q, D),
                raft::make_device_matrix_view<std::uint32_t, std::int64_t>(m.data(), Q, K),
                raft::make_device_matrix_view<float, std::int64_t>(md.data(), Q, K));
  int mhits = 0;
  for (int i = 0; i < Q; ++i) {
    std::set<std::uint32_t> s(e.begin() + i * K, e.begin() + (i + 1) * K);
    std::set<std::uint32_t> row(m.begin() + i * K, m.begin() + (i + 1) * K);
    CHECK(row.size() == std::size_t(K));
    for (int j = 0; j < K; ++j) {
      mhits += s.count(m[i * K + j]) ? 1 : 0;
      if (j > 0) CHECK(md[i * K + j - 1] <= md[i * K + j]);
    }
  }
  const double mrecall = double(mhits) / (Q * K);
  std::printf("multi-team (MULTI_CTA) recall@10: %.3f\n", mrecall);
  CHECK(mrecall >= recall - 0.05);
}

// Changing an index's navigation nodes changes where the next search
// starts (the device copy is refreshed).  The graph has no edges, so a
// search returns its best start candidates: with row B (the query's exact
// nearest row) among the navigation nodes it is found, and after the nodes
// are replaced by a far row it is not (the hashed extra seeds of this query
// do not include B).
void nav_change_reseeds() {
  const std::int64_t N = 100000, D = 8, K = 4;
  const std::uint32_t B = 77777, far_row = 5;
  std::vector<float> base(N * D);
  for (std::int64_t i = 0; i < N; ++i)
    for (std::int64_t j = 0; j < D; ++j) base[i * D + j] = float(100 + (i * 7 + j * 13) % 997);
  for (std::int64_t j = 0; j < D; ++j) base[B * D + j] = 0.f;
  std::vector<float> q(D, 0.5f);
  cagra::index<float, std::uint32_t> idx{base, N, D};
  idx.set_knn_graph(std::vector<std::uint32_t>(N * 4, 0xFFFFFFFFu), 4);
  auto nav_to = [&](std::uint32_t row) {
    idx.set_nav_nodes({row});
    idx.set_nav_vectors(std::vector<float>(base.begin() + row * D, base.begin() + (row + 1) * D));
  };
  raft::resources res;
  cagra::search_params sp;
  std::vector<std::uint32_t> nbr(K);
  std::vector<float> dist(K);
  auto run = [&] {
    cagra::search(res, sp, idx, raft::make_device_matrix_view<const float, std::int64_t>(q.data(), 1, D),
                  raft::make_device_matrix_view<std::uint32_t, std::int64_t>(nbr.data(), 1, K),
                  raft::make_device_matrix_view<float, std::int64_t>(dist.data(), 1, K));
  };
  nav_to(B);
  run();
  CHECK(nbr[0] == B && dist[0] == 2.f);  // 8 x 0.5^2
  nav_to(far_row);
  run();
  CHECK(nbr[0] != B);
  for (int i = 0; i < K; ++i) CHECK(nbr[i] != B);
  nav_to(B);
  run();
  CHECK(nbr[0] == B);
}

// Rows 1, 2 and 3 differ by less than the fp16 copy resolves after
// centring (their centred values 49.99, 50.00, 50.01 all round to 50), so
// an fp16 traversal with a one-entry list keeps the lowest id of the tie
// (row 1) while the fp32 traversal keeps the exact nearest, row 3.
void default_search_is_fp32() {
  const std::int64_t N = 4, D = 4;
  std::vector<float> base(N * D, 0.f);
  base[0] = -200.f;
  base[1 * D] = 0.f;
  base[2 * D] = 0.01f;
  base[3 * D] = 0.02f;
  cagra::index<float, std::uint32_t> idx{base, N, D};
  std::vector<std::uint32_t> g;
  for (std::uint32_t i = 0; i < N; ++i)
    for (std::uint32_t j = 0; j < N; ++j)
      if (j != i) g.push_back(j);
  idx.set_knn_graph(g, N - 1);
  idx.set_nav_nodes({0});
  idx.set_nav_vectors(std::vector<float>(base.begin(), base.begin() + D));
  std::vector<float> q(D, 0.f);
  q[0] = 0.02f;
  raft::resources res;
  std::vector<std::uint32_t> nbr(1);
  std::vector<float> dist(1);
  auto run = [&](const cagra::search_params& sp) {
    cagra::search(res, sp, idx, raft::make_device_matrix_view<const float, std::int64_t>(q.data(), 1, D),
                  raft::make_device_matrix_view<std::uint32_t, std::int64_t>(nbr.data(), 1, 1),
                  raft::make_device_matrix_view<float, std::int64_t>(dist.data(), 1, 1));
    return nbr[0];
  };
  cagra::search_params sp;
  sp.itopk_size = 1;
  CHECK(!sp.fp16_traversal && !sp.reference_beam);
  CHECK(run(sp) == 3u);
  CHECK(dist[0] == 0.f);
  sp.fp16_traversal = true;
  CHECK(run(sp) == 1u);  // the opt-in fp16 copy cannot tell rows 1-3 apart
  sp.fp16_traversal = false;
  CHECK(run(sp) == 3u);
}

// MetalContext (the reference's backend class) against the C ABI.
void metal_context_matches_c_abi() {
  auto& mc = cuvs_silicon::MetalContext::instance();
  CHECK(mc.is_available());
  const std::int64_t N = 3000, D = 48, Q = 40, K = 8;
  std::mt19937 rng(17);
  std::uniform_int_distribution<int> u(-4, 4);  // integer data: every sum exact
  std::vector<float> base(N * D), qs(Q * D);
  for (auto& v : base) v = float(u(rng));
  for (auto& v : qs) v = float(u(rng));

  cvs_context* ctx = nullptr;
  CHECK(cvs_context_create(0, &ctx) == CVS_OK);

  // Exact search.
  std::vector<std::uint32_t> n1(Q * K), n2(Q * K);
  std::vector<float> d1(Q * K), d2(Q * K);
  CHECK(mc.search_brute_force(base.data(), N, D, qs.data(), Q, n1.data(), d1.data(), K) > 0);
  cvs_dataset* ds = nullptr;
  CHECK(cvs_dataset_create(ctx, base.data(), N, D, 0, &ds) == CVS_OK);
  CHECK(cvs_bf_search(ctx, ds, qs.data(), Q, K, n2.data(), d2.data()) == CVS_OK);
  CHECK(n1 == n2 && d1 == d2);
  cvs_dataset_destroy(ds);

  // Graph search with a distinct entry node per query.
  const std::uint32_t G = 16;
  std::vector<std::uint32_t> graph(N * G);
  cvs_build_stats st{};
  CHECK(cvs_cagra_build(ctx, base.data(), N, D, 0, 32, G, 10, 0.001f, 0xFEDCBA9876543210ULL, graph.data(), 0,
                        &st) == CVS_OK);
  std::vector<std::uint32_t> entry(Q);
  for (std::int64_t i = 0; i < Q; ++i) entry[i] = std::uint32_t((i * 977) % N);
  CHECK(mc.search_cagra(base.data(), N, D, graph.data(), G, qs.data(), Q, n1.data(), d1.data(), K, 32, 100,
                        entry.data()) > 0);
  cvs_cagra_index* ix = nullptr;
  CHECK(cvs_cagra_index_create(ctx, base.data(), N, D, 0, graph.data(), G, 0, nullptr, 0, &ix) == CVS_OK);
  CHECK(cvs_cagra_search_reference(ctx, ix, qs.data(), Q, K, 32, 100, entry.data(), n2.data(), d2.data()) ==
        CVS_OK);
  CHECK(n1 == n2 && d1 == d2);
  cvs_cagra_index_destroy(ix);

  // build_knn_graph returns k-NN lists (nearest first), as the reference's
  // does: G distinct ids per row, never the row itself, distances
  // non-decreasing along each row (up to the build's fp16 ranking of near
  // ties), and almost every row holding its exact nearest neighbour.
  {
    const auto knn = mc.build_knn_graph(base.data(), N, D, G, 10, 0);
    CHECK(knn.size() == std::size_t(N) * G);
    auto dist2 = [&](std::int64_t a, std::int64_t b) {
      float s2 = 0.f;
      for (std::int64_t j = 0; j < D; ++j) {
        const float t = base[a * D + j] - base[b * D + j];
        s2 += t * t;
      }
      return s2;
    };
    int nn_held = 0, misordered = 0;
    for (std::int64_t i = 0; i < N; ++i) {
      std::set<std::uint32_t> seen;
      float prev = -1.f;
      for (std::uint32_t g = 0; g < G; ++g) {
        const std::uint32_t v = knn[i * G + g];
        CHECK(v < std::uint32_t(N) && v != std::uint32_t(i) && seen.insert(v).second);
        const float dv = dist2(i, v);
        misordered += dv < prev ? 1 : 0;
        prev = dv;
      }
      float best = 3.0e38f;
      std::int64_t arg = -1;
      for (std::int64_t j = 0; j < N; ++j)
        if (j != i && dist2(i, j) < best) best = dist2(i, j), arg = j;
      nn_held += (seen.count(std::uint32_t(arg)) || dist2(i, knn[i * G]) == best) ? 1 : 0;
    }
    std::printf("build_knn_graph: exact nearest neighbour held by %d of %lld rows, %d misordered steps\n", nn_held,
                (long long)N, misordered);
    CHECK(nn_held >= N * 95 / 100);
    CHECK(misordered <= int(N * G / 100));
  }

  // With no edges each query can only return its own entry node.
  std::vector<std::uint32_t> empty(N * G, kNone);
  CHECK(mc.search_cagra(base.data(), N, D, empty.data(), G, qs.data(), Q, n1.data(), d1.data(), K, 32, 100,
                        entry.data()) > 0);
  for (std::int64_t i = 0; i < Q; ++i) {
    CHECK(n1[i * K] == entry[i]);
    CHECK(n1[i * K + 1] == kNone && std::isinf(d1[i * K + 1]));
  }
  cvs_context_destroy(ctx);
}

// cagra::search with reference_beam: entry nodes from the navigation
// nodes, the beam clamped to 32 for q <= 4, the reference kernel.
void reference_beam_mode() {
  const std::int64_t N = 2500, D = 24, K = 5;
  std::mt19937 rng(23);
  std::uniform_int_distribution<int> u(-5, 5);
  std::vector<float> base(N * D), qs(3 * D);
  for (auto& v : base) v = float(u(rng));
  for (auto& v : qs) v = float(u(rng));
  raft::resources res;
  cagra::index_params ip;
  ip.graph_degree = 16;
  ip.intermediate_graph_degree = 32;
  auto idx = cagra::build(res, ip, raft::make_device_matrix_view<const float, std::int64_t>(base.data(), N, D));
  cagra::search_params sp;
  sp.reference_beam = true;
  sp.itopk_size = 64;
  std::vector<std::uint32_t> nbr(3 * K), n2(3 * K);
  std::vector<float> dist(3 * K), d2(3 * K);
  cagra::search(res, sp, idx, raft::make_device_matrix_view<const float, std::int64_t>(qs.data(), 3, D),
                raft::make_device_matrix_view<std::uint32_t, std::int64_t>(nbr.data(), 3, K),
                raft::make_device_matrix_view<float, std::int64_t>(dist.data(), 3, K));
  // The same through the C ABI: entry points, beam 32 (q = 3 <= 4), 200 iterations.
  cvs_context* ctx = nullptr;
  CHECK(cvs_context_create(0, &ctx) == CVS_OK);
  cvs_cagra_index* ix = nullptr;
  const auto& nav = idx.nav_nodes();
  CHECK(cvs_cagra_index_create(ctx, base.data(), N, D, 0, idx.knn_graph().data(), idx.graph_degree(), 0, nav.data(),
                               std::uint32_t(nav.size()), &ix) == CVS_OK);
  std::vector<std::uint32_t> entry(3);
  CHECK(cvs_cagra_entry_points(ctx, ix, qs.data(), 3, entry.data()) == CVS_OK);
  CHECK(cvs_cagra_search_reference(ctx, ix, qs.data(), 3, K, 32, 200, entry.data(), n2.data(), d2.data()) == CVS_OK);
  CHECK(nbr == n2 && dist == d2);
  cvs_cagra_index_destroy(ix);
  cvs_context_destroy(ctx);
}

}  // namespace

// brute_force beyond the fused scan's limits (D > 1024 and K > 112, the
// reference's CPU loop has neither limit, src/cagra.cpp:211-252): integer
// rows, so every fp32 distance is exact and the answer, ties by id, is fixed.
void wide_brute_force() {
  constexpr std::int64_t N = 600, D = 1536, Q = 3, K = 150;
  std::vector<float> base(N * D), queries(Q * D);
  std::mt19937 gen(17);
  std::uniform_int_distribution<int> val(-3, 3);
  for (auto& v : base) v = float(val(gen));
  for (auto& v : queries) v = float(val(gen));
  raft::resources res;
  auto bidx = bf::build(res, raft::make_device_matrix_view<const float, std::int64_t>(base.data(), N, D));
  std::vector<std::uint32_t> nbr(Q * K);
  std::vector<float> dist(Q * K);
  bf::search(res, bidx, raft::make_device_matrix_view<const float, std::int64_t>(queries.data(), Q, D),
             raft::make_device_matrix_view<std::uint32_t, std::int64_t>(nbr.data(), Q, K),
             raft::make_device_matrix_view<float, std::int64_t>(dist.data(), Q, K));
  for (std::int64_t q = 0; q < Q; ++q) {
    std::vector<std::pair<std::int64_t, std::uint32_t>> all(N);
    for (std::int64_t i = 0; i < N; ++i) {
      std::int64_t acc = 0;
      for (std::int64_t j = 0; j < D; ++j) {
        const std::int64_t t = std::int64_t(queries[q * D + j]) - std::int64_t(base[i * D + j]);
        acc += t * t;
      }
      all[i] = {acc, std::uint32_t(i)};
    }
    std::sort(all.begin(), all.end());
    for (std::int64_t r = 0; r < K; ++r) {
      CHECK(nbr[q * K + r] == all[r].second);
      CHECK(dist[q * K + r] == float(all[r].first));
    }
  }
}

int main(int argc, char** argv) {
  const std::string scratch = argc > 1 ? argv[1] : "/tmp";
  faiss_smoke();
  dispatch_test();
  build_save_load_search(scratch);
  nav_change_reseeds();
  default_search_is_fp32();
  metal_context_matches_c_abi();
  reference_beam_mode();
  wide_brute_force();
  return apitest::finish("test_api_gpu");
}
