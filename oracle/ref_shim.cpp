// extern "C" wrappers around the reference's own CPU code, compiled from the
// reference sources in place (see oracle/Makefile, target `ref`).  TEST
// INFRASTRUCTURE ONLY: used by tests/ to pin the oracle and by bench.py's
// cpu_baseline leg; never linked into the product.
//
// On Linux the reference's cagra::build() only copies the dataset and
// cagra::search() runs the scalar exact loop (src/cagra.cpp:211-252), so
// ref_bf_search is the reference CPU path itself.
#include <cuvs/neighbors/cagra.hpp>
#include <cuvs_silicon/distance.hpp>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>
#include <vector>

namespace cagra = cuvs::neighbors::cagra;

extern "C" {

// 0 on success, 1 on std::invalid_argument, 2 on any other exception.
int ref_bf_search(const float* base, int64_t n, int64_t d, const float* queries, int64_t q,
                  int64_t k, uint32_t* out_nbr, float* out_dist) {
  try {
    raft::resources res;
    cagra::index_params ip;
    ip.graph_degree = 0;
    auto idx = cagra::build(res, ip, raft::device_matrix_view<const float, int64_t>(base, n, d));
    cagra::search_params sp;
    cagra::search(res, sp, idx, raft::device_matrix_view<const float, int64_t>(queries, q, d),
                  raft::device_matrix_view<uint32_t, int64_t>(out_nbr, q, k),
                  raft::device_matrix_view<float, int64_t>(out_dist, q, k));
    return 0;
  } catch (const std::invalid_argument&) {
    return 1;
  } catch (...) {
    return 2;
  }
}

float ref_l2_128(const float* a, const float* b) {
  try {
    return cuvs_silicon::squared_l2_distance_128(a, b);
  } catch (...) {
    return NAN;
  }
}

// Writes a CGRA v1 file with the reference's save_index.
int ref_save_index(const char* path, const float* dataset, int64_t n, int64_t d,
                   const uint32_t* graph, uint32_t degree, const uint32_t* nav, uint32_t n_nav,
                   const float* nav_vectors) {
  try {
    std::vector<float> ds;
    if (dataset) ds.assign(dataset, dataset + n * d);
    cagra::index<float, uint32_t> idx(std::move(ds), n, d);
    idx.set_knn_graph(std::vector<uint32_t>(graph, graph + (size_t)n * degree), degree);
    if (n_nav) {
      idx.set_nav_nodes(std::vector<uint32_t>(nav, nav + n_nav));
      idx.set_nav_vectors(std::vector<float>(nav_vectors, nav_vectors + (size_t)n_nav * d));
    }
    cagra::save_index(idx, path);
    return 0;
  } catch (...) {
    return 2;
  }
}

// Loads a CGRA file with the reference's load_index; copies fields out when
// the destination pointers are non-null.  Returns 0, or 2 on an exception.
int ref_load_index(const char* path, int64_t* n, int64_t* d, uint32_t* degree, int64_t* n_nav,
                   float* dataset, uint32_t* graph, uint32_t* nav, float* nav_vectors,
                   int* has_dataset) {
  try {
    auto idx = cagra::load_index(path);
    *n = idx.rows();
    *d = idx.cols();
    *degree = idx.graph_degree();
    *n_nav = (int64_t)idx.nav_nodes().size();
    *has_dataset = idx.dataset().empty() ? 0 : 1;
    if (dataset && !idx.dataset().empty())
      std::memcpy(dataset, idx.dataset().data(), idx.dataset().size() * sizeof(float));
    if (graph && !idx.knn_graph().empty())
      std::memcpy(graph, idx.knn_graph().data(), idx.knn_graph().size() * sizeof(uint32_t));
    if (nav && !idx.nav_nodes().empty())
      std::memcpy(nav, idx.nav_nodes().data(), idx.nav_nodes().size() * sizeof(uint32_t));
    if (nav_vectors && !idx.nav_vectors().empty())
      std::memcpy(nav_vectors, idx.nav_vectors().data(), idx.nav_vectors().size() * sizeof(float));
    return 0;
  } catch (...) {
    return 2;
  }
}

}  // extern "C"
