// cuvs::neighbors::brute_force front-end: the direct route to the fused
// brute-force kernel (the reference reaches it only via graph_degree = 0,
// src/cagra.cpp:197-202).
#include <cuvs/neighbors/brute_force.hpp>

#include <stdexcept>
#include <vector>

#include "backend.hpp"

namespace cuvs::neighbors::brute_force {

namespace detail {
struct device_dataset {
  std::shared_ptr<cuvs_silicon_amd::DatasetHandle> handle;
};
}  // namespace detail

index<float> build(const raft::resources& resources,
                   raft::device_matrix_view<const float, std::int64_t> dataset,
                   cuvs::distance::DistanceType metric) {
  (void)resources;
  if (metric != cuvs::distance::DistanceType::L2Expanded)
    throw std::invalid_argument("brute_force supports the L2Expanded metric only");
  if (dataset.data_handle() == nullptr || dataset.extent(0) <= 0 || dataset.extent(1) <= 0)
    throw std::invalid_argument("brute_force build requires a non-empty dataset");
  auto dev = std::make_shared<detail::device_dataset>();
  dev->handle = cuvs_silicon_amd::upload_dataset(dataset.data_handle(), dataset.extent(0),
                                                 dataset.extent(1));
  return index<float>(std::move(dev), dataset.extent(0), dataset.extent(1), metric);
}

namespace {
void validate(const index<float>& idx, std::int64_t q, std::int64_t qd, std::int64_t nr,
              std::int64_t nc, std::int64_t dr, std::int64_t dc, const void* qp, const void* np,
              const void* dp) {
  if (!idx.device()) throw std::invalid_argument("brute_force index is not built");
  if (!qp || !np || !dp) throw std::invalid_argument("brute_force search requires valid buffers");
  if (qd != idx.dim()) throw std::invalid_argument("brute_force query dimension mismatch");
  if (nr != q || dr != q || nc != dc)
    throw std::invalid_argument("brute_force output shape mismatch");
  if (nc <= 0) throw std::invalid_argument("brute_force search requires k > 0");
}
}  // namespace

void search(const raft::resources& resources, const index<float>& idx,
            raft::device_matrix_view<const float, std::int64_t> queries,
            raft::device_matrix_view<std::uint32_t, std::int64_t> neighbors,
            raft::device_matrix_view<float, std::int64_t> distances) {
  (void)resources;
  validate(idx, queries.extent(0), queries.extent(1), neighbors.extent(0), neighbors.extent(1),
           distances.extent(0), distances.extent(1), queries.data_handle(),
           neighbors.data_handle(), distances.data_handle());
  if (queries.extent(0) == 0) return;
  cvs_context* ctx = cuvs_silicon_amd::Backend::instance().ctx();
  cuvs_silicon_amd::counted([&] {
    return cvs_bf_search(ctx, idx.device()->handle->ds, queries.data_handle(), queries.extent(0),
                         neighbors.extent(1), neighbors.data_handle(), distances.data_handle());
  });
}

void search(const raft::resources& resources, const index<float>& idx,
            raft::device_matrix_view<const float, std::int64_t> queries,
            raft::device_matrix_view<std::int64_t, std::int64_t> neighbors,
            raft::device_matrix_view<float, std::int64_t> distances) {
  const std::int64_t q = queries.extent(0), k = neighbors.extent(1);
  validate(idx, q, queries.extent(1), neighbors.extent(0), k, distances.extent(0),
           distances.extent(1), queries.data_handle(), neighbors.data_handle(),
           distances.data_handle());
  std::vector<std::uint32_t> ids(static_cast<std::size_t>(q * k));
  search(resources, idx, queries,
         raft::make_device_matrix_view<std::uint32_t, std::int64_t>(ids.data(), q, k), distances);
  for (std::size_t i = 0; i < ids.size(); ++i)
    neighbors.data_handle()[i] =
        ids[i] == 0xffffffffu ? std::int64_t{-1} : static_cast<std::int64_t>(ids[i]);
}

}  // namespace cuvs::neighbors::brute_force
