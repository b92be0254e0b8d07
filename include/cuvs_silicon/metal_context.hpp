// The reference's device-backend class, cuvs_silicon::MetalContext
// (reference include/cuvs_silicon/metal_context.hpp:12-81), kept under its
// own name and signatures so that code written against it (the reference's
// validation harness tests/test_cohere_wiki_validation.cpp:36 includes this
// header) compiles and links unchanged.  Here it is a thin C++ view of the
// C ABI in cvs_hip.h: one HIP context on device 0, created on first use.
// Implemented in libcuvs_silicon (cuvs-silicon_amd/src/metal_context.cpp).
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace cuvs_silicon {

class MetalContext {
 public:
  // Process-wide instance (created on first call; reference :15).
  static MetalContext& instance();

  // Whether a gfx950 device was found (reference :19).
  bool is_available() const noexcept;

  // Name of the device ("" when none; reference :23).
  std::string chip_model() const;

  // Exact k-NN of Q queries against N rows, squared L2, row-major outputs
  // sorted by (distance, id) (cvs_bf_search; reference :35-40).  The device
  // copy of `dataset` is cached by (pointer, N, D) like the reference's.
  // Returns the number of GPU kernel launches the call made.  Throws
  // std::runtime_error on a device failure.
  uint64_t search_brute_force(const float* dataset, int64_t N, int64_t D, const float* queries, int64_t Q,
                              uint32_t* out_neighbors, float* out_distances, int64_t K);

  // N x graph_degree neighbour lists, row-major (cvs_cagra_build: random
  // bucketing, at most n_descent_iters nn-descent iterations, pruning from
  // an intermediate degree of 2 x graph_degree; reference :47-55).
  // bucket_size is accepted for compatibility; the buckets hold 256 rows.
  std::vector<uint32_t> build_knn_graph(const float* dataset, int64_t N, int64_t D, uint32_t graph_degree = 32,
                                        uint32_t n_descent_iters = 10, int64_t bucket_size = 2048);

  // Graph search with a list of beam_size entries and at most max_iter
  // iterations (cvs_cagra_search; reference :57-73).  The search starts from
  // the distinct entry_nodes (when given) plus hashed rows.  Returns the
  // number of GPU kernel launches the call made.
  uint64_t search_cagra(const float* dataset, int64_t N, int64_t D, const uint32_t* knn_graph,
                        uint32_t graph_degree, const float* queries, int64_t Q, uint32_t* out_neighbors,
                        float* out_distances, int64_t K, uint32_t beam_size = 128, uint32_t max_iter = 200,
                        const uint32_t* entry_nodes = nullptr);

  // Copies n floats from src to dst through device memory (reference :75-77).
  void run_copy_kernel(const float* src, float* dst, int64_t n);

  MetalContext(const MetalContext&) = delete;
  MetalContext& operator=(const MetalContext&) = delete;

 private:
  MetalContext();
  ~MetalContext();
  struct Impl;
  Impl* impl_;
};

}  // namespace cuvs_silicon
