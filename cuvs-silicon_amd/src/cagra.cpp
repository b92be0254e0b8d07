// Front-end of the cuVS-style CAGRA API (reference: src/cagra.cpp:20-266).
//
// Validation, exception types, output layout and the graph_degree == 0
// routing follow the reference; all compute is delegated to libcvs_hip.
// There is no CPU search path: without a gfx950 device, build()/search()
// throw std::runtime_error.
#include <cuvs/neighbors/cagra.hpp>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <limits>
#include <stdexcept>
#include <vector>

#include "backend.hpp"

namespace cuvs_silicon_amd {

namespace {
std::atomic<std::uint64_t> g_api_dispatches{0};
}

void add_dispatches(std::uint64_t n) { g_api_dispatches.fetch_add(n); }

Backend::Backend() { check(cvs_context_create(0, &ctx_)); }
Backend::~Backend() {
  if (ctx_) cvs_context_destroy(ctx_);
}
Backend& Backend::instance() {
  static Backend b;
  return b;
}

std::shared_ptr<DatasetHandle> upload_dataset(const float* rows, std::int64_t n, std::int64_t d) {
  cvs_dataset* ds = nullptr;
  counted([&] { return cvs_dataset_create(Backend::instance().ctx(), rows, n, d, 0, &ds); });
  return std::make_shared<DatasetHandle>(ds);
}

}  // namespace cuvs_silicon_amd

namespace cuvs::neighbors::cagra {

namespace detail {
struct device_state {
  std::shared_ptr<cuvs_silicon_amd::DatasetHandle> dataset;          // exact search
  std::shared_ptr<cuvs_silicon_amd::GraphIndexHandle> graph_index;   // graph search
};
std::shared_ptr<device_state> make_device_state() { return std::make_shared<device_state>(); }
}  // namespace detail

using cuvs_silicon_amd::Backend;
using cuvs_silicon_amd::check;
using cuvs_silicon_amd::counted;

template <>
index<float, std::uint32_t> build<float, std::int64_t>(
    const raft::resources& resources, const index_params& params,
    raft::device_matrix_view<const float, std::int64_t> dataset) {
  (void)resources;
  if (params.metric != cuvs::distance::DistanceType::L2Expanded)
    throw std::invalid_argument("CAGRA build supports the L2Expanded metric only");
  if (dataset.data_handle() == nullptr || dataset.extent(0) <= 0 || dataset.extent(1) <= 0)
    throw std::invalid_argument("CAGRA build requires a non-empty dataset");

  const std::int64_t n = dataset.extent(0);
  const std::int64_t d = dataset.extent(1);
  const float* data = dataset.data_handle();

  std::vector<float> storage;
  if (params.attach_dataset_on_build) storage.assign(data, data + n * d);
  index<float, std::uint32_t> idx{std::move(storage), n, d};

  // G = min(graph_degree, N - 1) (src/cagra.cpp:47-48); 0 keeps an exact
  // brute-force index.
  const std::uint32_t degree =
      std::min<std::uint32_t>(params.graph_degree, static_cast<std::uint32_t>(n - 1));
  if (n > 1 && degree > 0) {
    cvs_build_stats stats{};
    std::vector<std::uint32_t> graph(static_cast<std::size_t>(n) * degree);
    counted([&] {
      return cvs_cagra_build(Backend::instance().ctx(), data, n, d, 0,
                             std::max(params.intermediate_graph_degree, degree), degree,
                             params.nn_descent_niter, params.nn_descent_termination_threshold,
                             0xFEDCBA9876543210ULL, graph.data(), 0, &stats);
    });
    if (stats.graph_degree != degree)
      throw std::runtime_error("CAGRA build returned an unexpected graph degree");
    idx.set_knn_graph(std::move(graph), degree);

    // Navigation nodes: min(200, floor(sqrt(N))) evenly spaced rows and
    // their vectors (src/cagra.cpp:63-82); search seeds from them.
    std::int64_t n_nav = 0;
    check(cvs_cagra_nav_nodes(n, nullptr, &n_nav));
    std::vector<std::uint32_t> nav(static_cast<std::size_t>(n_nav));
    check(cvs_cagra_nav_nodes(n, nav.data(), &n_nav));
    std::vector<float> nav_vectors(static_cast<std::size_t>(n_nav * d));
    for (std::int64_t i = 0; i < n_nav; ++i)
      std::copy_n(data + static_cast<std::int64_t>(nav[static_cast<std::size_t>(i)]) * d,
                  static_cast<std::size_t>(d), nav_vectors.data() + i * d);
    idx.set_nav_nodes(std::move(nav));
    idx.set_nav_vectors(std::move(nav_vectors));
  }
  return idx;
}

namespace {

void validate_search(const index<float, std::uint32_t>& index,
                     raft::device_matrix_view<const float, std::int64_t> queries,
                     raft::device_matrix_view<std::uint32_t, std::int64_t> neighbors,
                     raft::device_matrix_view<float, std::int64_t> distances) {
  if (queries.data_handle() == nullptr || neighbors.data_handle() == nullptr ||
      distances.data_handle() == nullptr)
    throw std::invalid_argument("CAGRA search requires valid buffers");
  if (queries.extent(1) != index.cols())
    throw std::invalid_argument("CAGRA search query dimension mismatch");
  if (neighbors.extent(0) != queries.extent(0) || distances.extent(0) != queries.extent(0) ||
      neighbors.extent(1) != distances.extent(1))
    throw std::invalid_argument("CAGRA search output shape mismatch");
}

// Device copies of the index, uploaded on first use: the brute-force layout
// for an index without a graph, the graph index (rows, neighbour lists,
// navigation nodes as seeds) otherwise.
detail::device_state& device_state_of(const index<float, std::uint32_t>& index, bool graph) {
  auto& cache = index.device_cache();
  if (!cache) cache = detail::make_device_state();
  if (index.dataset().empty())
    throw std::invalid_argument("CAGRA search requires an index with an attached dataset");
  if (!graph && !cache->dataset) {
    cache->dataset =
        cuvs_silicon_amd::upload_dataset(index.dataset().data(), index.rows(), index.cols());
  }
  if (graph && !cache->graph_index) {
    if (index.knn_graph().size() !=
        static_cast<std::size_t>(index.rows()) * static_cast<std::size_t>(index.graph_degree()))
      throw std::invalid_argument("CAGRA index graph does not match rows x graph_degree");
    cvs_cagra_index* ix = nullptr;
    const auto& nav = index.nav_nodes();
    counted([&] {
      return cvs_cagra_index_create(Backend::instance().ctx(), index.dataset().data(), index.rows(),
                                    index.cols(), 0, index.knn_graph().data(), index.graph_degree(), 0,
                                    nav.empty() ? nullptr : nav.data(),
                                    static_cast<std::uint32_t>(nav.size()), &ix);
    });
    cache->graph_index = std::make_shared<cuvs_silicon_amd::GraphIndexHandle>(ix);
  }
  return *cache;
}

}  // namespace

template <>
void search<float, std::uint32_t, std::int64_t>(
    const raft::resources& resources, const search_params& params,
    const index<float, std::uint32_t>& index,
    raft::device_matrix_view<const float, std::int64_t> queries,
    raft::device_matrix_view<std::uint32_t, std::int64_t> neighbors,
    raft::device_matrix_view<float, std::int64_t> distances) {
  (void)resources;
  validate_search(index, queries, neighbors, distances);
  const std::int64_t q = queries.extent(0);
  const std::int64_t k = neighbors.extent(1);
  if (q == 0) return;
  if (k <= 0) throw std::invalid_argument("CAGRA search requires k > 0");

  // Routing as in the reference (src/cagra.cpp:125-126): graph search when
  // the index has a graph, exact search otherwise.
  const bool has_graph = index.graph_degree() > 0 && !index.knn_graph().empty();
  detail::device_state& dev = device_state_of(index, has_graph);
  cvs_context* ctx = Backend::instance().ctx();
  if (has_graph) {
    auto clamp32 = [](std::uint64_t v) {
      return static_cast<std::uint32_t>(std::min<std::uint64_t>(v, 0xffffffffu));
    };
    if (params.reference_beam) {
      // The reference's route (src/cagra.cpp:128-196): each query's entry
      // node is its nearest navigation node (on the GPU), beam = itopk_size
      // (0 -> 128), iterations = max_iterations (0 -> 200), and q <= 4
      // clamps the beam to 32.
      std::uint32_t beam = clamp32(params.itopk_size > 0 ? params.itopk_size : 128);
      std::uint32_t iters = clamp32(params.max_iterations > 0 ? params.max_iterations : 200);
      if (q <= 4) {
        beam = std::min<std::uint32_t>(beam, 32u);
        iters = std::min<std::uint32_t>(iters, 200u);
      }
      std::vector<std::uint32_t> entry;
      if (!index.nav_nodes().empty()) {
        entry.resize(static_cast<std::size_t>(q));
        counted([&] {
          return cvs_cagra_entry_points(ctx, dev.graph_index->ix, queries.data_handle(), q, entry.data());
        });
      }
      counted([&] {
        return cvs_cagra_search_reference(ctx, dev.graph_index->ix, queries.data_handle(), q, k, beam, iters,
                                          entry.empty() ? nullptr : entry.data(), neighbors.data_handle(),
                                          distances.data_handle());
      });
      return;
    }
    // itopk_size 0 -> 128 and max_iterations 0 -> the kernel's cap follow
    // src/cagra.cpp:182-185.  The reference's clamp of the beam to 32 for
    // q <= 4 (:186-189) is not applied here: it only lowers recall.
    check(cvs_cagra_index_set_traversal(dev.graph_index->ix, params.fp16_traversal ? 16 : 32));
    if (params.algo == search_algo::MULTI_CTA) {
      // Teams of workgroups per query with 32-entry lists (k if larger), as
      // many teams as cuVS's multi-CTA mode uses CTAs: max(search_width,
      // ceil(itopk_size / 32)), at least 2, within CVS_CAGRA_MAX_TEAMS and
      // CVS_CAGRA_MAX_ITOPK entries in all.  The reference's own multi-team
      // kernel (shaders/cagra_kernels.metal:200-327) is compiled but disabled.
      const std::uint64_t itopk = params.itopk_size ? params.itopk_size : 128;
      const std::uint64_t per_team = std::max<std::uint64_t>(32, static_cast<std::uint64_t>(k));
      std::uint64_t teams = std::max<std::uint64_t>({2, params.search_width, (itopk + 31) / 32});
      teams = std::min<std::uint64_t>({teams, CVS_CAGRA_MAX_TEAMS, std::max<std::uint64_t>(1, CVS_CAGRA_MAX_ITOPK / per_team)});
      counted([&] {
        return cvs_cagra_search_teams(ctx, dev.graph_index->ix, queries.data_handle(), q, k, clamp32(per_team), 1,
                                      clamp32(params.max_iterations), clamp32(teams), neighbors.data_handle(),
                                      distances.data_handle());
      });
      return;
    }
    counted([&] {
      return cvs_cagra_search(ctx, dev.graph_index->ix, queries.data_handle(), q, k,
                              clamp32(params.itopk_size), clamp32(params.search_width),
                              clamp32(params.max_iterations), neighbors.data_handle(),
                              distances.data_handle());
    });
    return;
  }
  counted([&] {
    return cvs_bf_search(ctx, dev.dataset->ds, queries.data_handle(), q, k,
                         neighbors.data_handle(), distances.data_handle());
  });
}

std::uint64_t metal_dispatch_count() noexcept {
  return cuvs_silicon_amd::g_api_dispatches.load();
}
void reset_metal_dispatch_count() noexcept { cuvs_silicon_amd::g_api_dispatches.store(0); }
void increment_metal_dispatch_count() noexcept { cuvs_silicon_amd::add_dispatches(1); }
std::uint64_t gpu_dispatch_count() noexcept { return metal_dispatch_count(); }
void reset_gpu_dispatch_count() noexcept { reset_metal_dispatch_count(); }

}  // namespace cuvs::neighbors::cagra
