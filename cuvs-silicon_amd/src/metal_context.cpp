// cuvs_silicon::MetalContext over the C ABI (reference: the Objective-C++
// singleton in src/metal_context.mm, interface include/cuvs_silicon/
// metal_context.hpp:12-81).  The reference's callers include this class; here
// every member forwards to libcvs_hip on one context (device 0).  Like the
// reference it is not thread-safe: its caches are unsynchronised.
#include <cuvs_silicon/metal_context.hpp>

#include <algorithm>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <vector>

#include "backend.hpp"

namespace cuvs_silicon {

using cuvs_silicon_amd::check;

struct MetalContext::Impl {
  cvs_context* ctx = nullptr;
  // Device copy of the last brute-force dataset, keyed like the reference's
  // fp16 cache (src/metal_context.mm:155-175) by (pointer, N, D).
  const float* bf_ptr = nullptr;
  int64_t bf_n = 0, bf_d = 0;
  cvs_dataset* bf_ds = nullptr;
  // Device copy of the last graph index, keyed by (dataset, graph, N, D, G).
  const float* gi_rows = nullptr;
  const uint32_t* gi_graph = nullptr;
  int64_t gi_n = 0, gi_d = 0;
  uint32_t gi_degree = 0;
  cvs_cagra_index* gi = nullptr;

  void drop_dataset() {
    if (bf_ds) cvs_dataset_destroy(bf_ds);
    bf_ds = nullptr;
    bf_ptr = nullptr;
  }
  void drop_index() {
    if (gi) cvs_cagra_index_destroy(gi);
    gi = nullptr;
    gi_rows = nullptr;
  }
};

MetalContext::MetalContext() : impl_(new Impl) {
  // No device: is_available() reports false and compute members throw.
  if (cvs_context_create(0, &impl_->ctx) != CVS_OK) impl_->ctx = nullptr;
}

MetalContext::~MetalContext() {
  impl_->drop_dataset();
  impl_->drop_index();
  if (impl_->ctx) cvs_context_destroy(impl_->ctx);
  delete impl_;
}

MetalContext& MetalContext::instance() {
  static MetalContext m;
  return m;
}

bool MetalContext::is_available() const noexcept { return impl_->ctx != nullptr; }

std::string MetalContext::chip_model() const {
  if (!impl_->ctx) return {};
  char name[256] = {0};
  int cus = 0;
  int64_t mem = 0;
  if (cvs_context_device_info(impl_->ctx, name, sizeof(name), &cus, &mem) != CVS_OK) return {};
  return name;
}

namespace {
cvs_context* require(cvs_context* ctx) {
  if (!ctx) throw std::runtime_error("no gfx950 device available");
  return ctx;
}
}  // namespace

uint64_t MetalContext::search_brute_force(const float* dataset, int64_t N, int64_t D, const float* queries,
                                          int64_t Q, uint32_t* out_neighbors, float* out_distances, int64_t K) {
  cvs_context* ctx = require(impl_->ctx);
  if (impl_->bf_ds == nullptr || impl_->bf_ptr != dataset || impl_->bf_n != N || impl_->bf_d != D) {
    impl_->drop_dataset();
    check(cvs_dataset_create(ctx, dataset, N, D, 0, &impl_->bf_ds));
    impl_->bf_ptr = dataset;
    impl_->bf_n = N;
    impl_->bf_d = D;
  }
  const uint64_t before = cvs_dispatch_count();
  check(cvs_bf_search(ctx, impl_->bf_ds, queries, Q, K, out_neighbors, out_distances));
  return cvs_dispatch_count() - before;
}

std::vector<uint32_t> MetalContext::build_knn_graph(const float* dataset, int64_t N, int64_t D,
                                                    uint32_t graph_degree, uint32_t n_descent_iters,
                                                    int64_t bucket_size) {
  (void)bucket_size;
  cvs_context* ctx = require(impl_->ctx);
  if (N < 2 || graph_degree == 0) throw std::invalid_argument("graph build needs N >= 2 and a positive degree");
  const uint32_t g = std::min<uint32_t>(graph_degree, static_cast<uint32_t>(N - 1));
  // Intermediate lists twice the output degree, within the build's 128; the
  // result is each row's nearest g list entries, a k-NN graph as the
  // reference's build_knn_graph returns (no pruning).
  const uint32_t inter =
      std::min<uint32_t>(std::max<uint32_t>(g, std::min<uint32_t>(2 * g, 128)), static_cast<uint32_t>(N - 1));
  std::vector<uint32_t> graph(static_cast<size_t>(N) * g);
  cvs_build_stats st{};
  cvs_build_options opts{};
  opts.graph_mode = CVS_GRAPH_KNN;
  check(cvs_cagra_build_ex(ctx, dataset, N, D, 0, inter, g, n_descent_iters, 0.001f, 0xFEDCBA9876543210ULL, &opts,
                           graph.data(), 0, &st));
  return graph;
}

uint64_t MetalContext::search_cagra(const float* dataset, int64_t N, int64_t D, const uint32_t* knn_graph,
                                    uint32_t graph_degree, const float* queries, int64_t Q,
                                    uint32_t* out_neighbors, float* out_distances, int64_t K, uint32_t beam_size,
                                    uint32_t max_iter, const uint32_t* entry_nodes) {
  cvs_context* ctx = require(impl_->ctx);
  Impl& m = *impl_;
  if (m.gi == nullptr || m.gi_rows != dataset || m.gi_graph != knn_graph || m.gi_n != N || m.gi_d != D ||
      m.gi_degree != graph_degree) {
    m.drop_index();
    check(cvs_cagra_index_create(ctx, dataset, N, D, 0, knn_graph, graph_degree, 0, nullptr, 0, &m.gi));
    m.gi_rows = dataset;
    m.gi_graph = knn_graph;
    m.gi_n = N;
    m.gi_d = D;
    m.gi_degree = graph_degree;
  }
  // The reference kernel itself: query q starts from entry_nodes[q] (or the
  // hashed fallback), with the caller's beam and iteration cap
  // (src/metal_context.mm:1041-1110).
  const uint64_t before = cvs_dispatch_count();
  check(cvs_cagra_search_reference(ctx, m.gi, queries, Q, K, beam_size, max_iter, entry_nodes, out_neighbors,
                                   out_distances));
  return cvs_dispatch_count() - before;
}

void MetalContext::run_copy_kernel(const float* src, float* dst, int64_t n) {
  cvs_context* ctx = require(impl_->ctx);
  if (n <= 0) return;
  const size_t bytes = static_cast<size_t>(n) * sizeof(float);
  void* buf = nullptr;
  check(cvs_device_alloc(ctx, bytes, &buf));
  int rc = cvs_copy_to_device(ctx, buf, src, bytes);
  if (rc == CVS_OK) rc = cvs_copy_to_host(ctx, dst, buf, bytes);
  cvs_device_free(ctx, buf);
  check(rc);
}

}  // namespace cuvs_silicon
