// cuVS-style CAGRA API, served by the MI355X backend (libcvs_hip).
//
// Same names, members, defaults and signatures as the reference header
// (include/cuvs/neighbors/cagra.hpp:14-122), so code written against the
// reference (including the FAISS v1.8 cuVS probes) compiles unchanged.
//
// Behaviour (reference src/cagra.cpp):
//  - build(): metric must be L2Expanded and the dataset non-empty, else
//    std::invalid_argument.  graph_degree == 0 (or N == 1) yields an exact
//    brute-force index; otherwise a fixed-degree kNN graph of degree
//    min(graph_degree, N-1) is built on the GPU, plus the navigation entry
//    nodes (min(200, floor(sqrt(N))) evenly spaced rows).
//  - search(): exact brute force when the index has no graph, CAGRA beam
//    search otherwise.  Outputs are row-major Q x K: squared-L2 distances
//    ascending with ties broken by the lower id; slots without a result hold
//    UINT32_MAX / +inf.
//  - All pointers in the raft views are host pointers; calls are blocking.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include <cuvs/distance/distance.hpp>
#include <raft/core/resources.hpp>

namespace cuvs::neighbors::cagra {

enum class search_algo {
  SINGLE_CTA = 0,
  MULTI_CTA = 1,
  MULTI_KERNEL = 2,
  AUTO = 100,
};

enum class hash_mode {
  HASH = 0,
  SMALL = 1,
  AUTO = 100,
};

struct index_params {
  std::uint32_t intermediate_graph_degree = 128;
  std::uint32_t graph_degree = 64;
  bool attach_dataset_on_build = true;
  bool guarantee_connectivity = false;
  cuvs::distance::DistanceType metric = cuvs::distance::DistanceType::L2Expanded;
  // Added after the reference's fields (cuVS names them the same way):
  // nn-descent iteration cap and early-stop threshold on the fraction of
  // list entries replaced in one iteration.
  std::uint32_t nn_descent_niter = 20;
  float nn_descent_termination_threshold = 0.001F;
};

struct search_params {
  std::uint64_t max_queries = 0;
  std::uint64_t itopk_size = 64;
  std::uint64_t max_iterations = 0;
  search_algo algo = search_algo::AUTO;
  std::uint64_t team_size = 0;
  std::uint64_t search_width = 1;
  std::uint64_t min_iterations = 0;
  std::uint64_t thread_block_size = 0;
  hash_mode hashmap_mode = hash_mode::AUTO;
  std::uint64_t hashmap_min_bitlen = 0;
  float hashmap_max_fill_rate = 0.5F;
  std::uint32_t num_random_samplings = 1;
  std::uint64_t rand_xor_mask = 0x128394;
  // Added after the reference's fields:
  // - fp16_traversal: evaluate candidates on an fp16 copy of the rows (the
  //   final list is re-ranked in fp32, so distances stay exact); off: every
  //   evaluation in fp32, as the reference traverses.
  // - reference_beam: run the reference's own beam search (one entry node
  //   per query, the nearest navigation node; an unsorted beam of itopk_size
  //   with replace-worst insertion; the beam clamped to 32 for q <= 4), which
  //   returns what the reference returns query by query; off: the
  //   register-list search seeded from every navigation node.
  bool fp16_traversal = false;
  bool reference_beam = false;
};

namespace detail {
// Device-resident copy of an index's dataset (and graph), created on first
// use and shared between copies of the index.  Opaque to users.
struct device_state;
std::shared_ptr<device_state> make_device_state();
}  // namespace detail

template <typename DataT, typename IndexT = std::uint32_t>
class index {
  static_assert(std::is_same_v<IndexT, std::uint32_t>,
                "the CAGRA index exposes uint32_t graph indices");

 public:
  using value_type = DataT;
  using index_type = IndexT;

  index() = default;
  index(std::vector<DataT> dataset, std::int64_t rows, std::int64_t cols)
      : dataset_(std::move(dataset)), rows_(rows), cols_(cols) {}

  const std::vector<DataT>& dataset() const noexcept { return dataset_; }
  const std::vector<IndexT>& knn_graph() const noexcept { return knn_graph_; }
  std::int64_t rows() const noexcept { return rows_; }
  std::int64_t cols() const noexcept { return cols_; }
  std::uint32_t graph_degree() const noexcept { return graph_degree_; }

  void set_knn_graph(std::vector<IndexT> g, std::uint32_t degree) {
    knn_graph_ = std::move(g);
    graph_degree_ = degree;
    device_.reset();
  }

  // Navigation nodes: evenly spaced dataset rows used to pick each query's
  // entry point; nav_vectors() caches their vectors (n_nav x D).
  const std::vector<IndexT>& nav_nodes() const noexcept { return nav_nodes_; }
  const std::vector<DataT>& nav_vectors() const noexcept { return nav_vectors_; }
  // The device copy seeds searches from the nav nodes, so it is dropped
  // whenever they change (the reference reads them on every search).
  void set_nav_nodes(std::vector<IndexT> n) {
    nav_nodes_ = std::move(n);
    device_.reset();
  }
  void set_nav_vectors(std::vector<DataT> v) {
    nav_vectors_ = std::move(v);
    device_.reset();
  }

  // Backend cache (device copies); filled lazily by search().
  std::shared_ptr<detail::device_state>& device_cache() const noexcept { return device_; }

 private:
  std::vector<DataT> dataset_;
  std::vector<IndexT> knn_graph_;    // N x graph_degree, row-major
  std::vector<IndexT> nav_nodes_;    // entry-point candidates
  std::vector<DataT> nav_vectors_;   // n_nav x D, row-major
  std::uint32_t graph_degree_ = 0;
  std::int64_t rows_ = 0;
  std::int64_t cols_ = 0;
  mutable std::shared_ptr<detail::device_state> device_;
};

template <typename DataT, typename ExtentT>
index<DataT, std::uint32_t> build(const raft::resources& resources, const index_params& params,
                                  raft::device_matrix_view<const DataT, ExtentT> dataset);

template <typename DataT, typename IndexT, typename ExtentT>
void search(const raft::resources& resources, const search_params& params,
            const index<DataT, IndexT>& index,
            raft::device_matrix_view<const DataT, ExtentT> queries,
            raft::device_matrix_view<IndexT, ExtentT> neighbors,
            raft::device_matrix_view<float, ExtentT> distances);

// Index serialization, byte-compatible with the reference's "CGRA" v1 files:
// magic "CGRA", u32 version 1, i64 N, i64 D, u32 G, u32 flags
// (bit0 dataset present, bit1 navigation nodes present), [f32 N*D dataset],
// u32 N*G graph, [u32 n_nav, u32 n_nav ids, f32 n_nav*D vectors].
void save_index(const index<float, std::uint32_t>& idx, const std::string& path);
index<float, std::uint32_t> load_index(const std::string& path);

// Dispatch instrumentation - test hook.  Counts GPU kernel launches made by
// search()/build() since the last reset (0 would mean no GPU work was done).
// The `metal_` names are kept for source compatibility.
std::uint64_t metal_dispatch_count() noexcept;
void reset_metal_dispatch_count() noexcept;
void increment_metal_dispatch_count() noexcept;
std::uint64_t gpu_dispatch_count() noexcept;
void reset_gpu_dispatch_count() noexcept;

}  // namespace cuvs::neighbors::cagra
