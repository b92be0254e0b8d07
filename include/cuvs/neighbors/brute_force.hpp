// cuVS-style exact brute-force k-NN.
//
// The reference reaches exact search only through cagra::build() with
// graph_degree = 0 (src/cagra.cpp:47-50, :197-202); that route keeps
// working.  This namespace is the direct entry point of the same fused GPU
// kernel, shaped like cuVS's cuvs::neighbors::brute_force API: build() uploads
// the dataset once, search() runs exact squared-L2 k-NN.  Pointers in the raft
// views are host pointers; calls are blocking.  Missing results (k > N) are
// UINT32_MAX / +inf for uint32 ids and -1 / +inf for int64 ids.
#pragma once

#include <cstdint>
#include <memory>

#include <cuvs/distance/distance.hpp>
#include <raft/core/resources.hpp>

namespace cuvs::neighbors::brute_force {

namespace detail {
struct device_dataset;
}

template <typename T>
class index {
 public:
  index() = default;
  std::int64_t size() const noexcept { return rows_; }
  std::int64_t dim() const noexcept { return cols_; }
  cuvs::distance::DistanceType metric() const noexcept { return metric_; }
  const std::shared_ptr<detail::device_dataset>& device() const noexcept { return device_; }

  index(std::shared_ptr<detail::device_dataset> dev, std::int64_t rows, std::int64_t cols,
        cuvs::distance::DistanceType metric)
      : device_(std::move(dev)), rows_(rows), cols_(cols), metric_(metric) {}

 private:
  std::shared_ptr<detail::device_dataset> device_;
  std::int64_t rows_ = 0;
  std::int64_t cols_ = 0;
  cuvs::distance::DistanceType metric_ = cuvs::distance::DistanceType::L2Expanded;
};

// Throws std::invalid_argument for an empty dataset or a metric other than
// L2Expanded.
index<float> build(const raft::resources& resources,
                   raft::device_matrix_view<const float, std::int64_t> dataset,
                   cuvs::distance::DistanceType metric = cuvs::distance::DistanceType::L2Expanded);

void search(const raft::resources& resources, const index<float>& index,
            raft::device_matrix_view<const float, std::int64_t> queries,
            raft::device_matrix_view<std::uint32_t, std::int64_t> neighbors,
            raft::device_matrix_view<float, std::int64_t> distances);

void search(const raft::resources& resources, const index<float>& index,
            raft::device_matrix_view<const float, std::int64_t> queries,
            raft::device_matrix_view<std::int64_t, std::int64_t> neighbors,
            raft::device_matrix_view<float, std::int64_t> distances);

}  // namespace cuvs::neighbors::brute_force
