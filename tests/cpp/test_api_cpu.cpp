// C++ API checks that need no GPU: the CGRA v1 file format against files
// written by the reference's own save_index (tests/golden/cgra_ref_v1*.bin,
// reference src/cagra.cpp:305-366), the index type, and the argument
// validation that happens before any device work (src/cagra.cpp:26-32,
// :100-111, :332-364).
//
// Usage: test_api_cpu <golden dir> <scratch dir>
#include <cuvs/neighbors/brute_force.hpp>
#include <cuvs/neighbors/cagra.hpp>

#include <cstdint>
#include <fstream>
#include <iterator>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

#include "check.hpp"

namespace cagra = cuvs::neighbors::cagra;
using apitest::expect_throw;

static std::vector<char> slurp(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  return std::vector<char>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

int main(int argc, char** argv) {
  if (argc < 3) {
    std::fprintf(stderr, "usage: %s <golden dir> <scratch dir>\n", argv[0]);
    return 2;
  }
  const std::string golden = argv[1], scratch = argv[2];

  // Reference-written index with dataset and navigation nodes (n=6, d=3, g=2).
  {
    const auto idx = cagra::load_index(golden + "/cgra_ref_v1.bin");
    CHECK(idx.rows() == 6 && idx.cols() == 3 && idx.graph_degree() == 2);
    CHECK(idx.dataset().size() == 18);
    for (int i = 0; i < 18; ++i) CHECK(idx.dataset()[i] == float(i) * 0.5f - 2.0f);
    const std::vector<std::uint32_t> graph{1, 2, 0, 2, 1, 3, 2, 4, 3, 5, 4, 0};
    CHECK(idx.knn_graph() == graph);
    CHECK((idx.nav_nodes() == std::vector<std::uint32_t>{0, 3}));
    CHECK(idx.nav_vectors().size() == 6);
    CHECK(idx.nav_vectors()[3] == idx.dataset()[9]);
    // Saving it again reproduces the reference's bytes.
    cagra::save_index(idx, scratch + "/roundtrip.bin");
    CHECK(slurp(scratch + "/roundtrip.bin") == slurp(golden + "/cgra_ref_v1.bin"));
  }
  // Without dataset and navigation nodes.
  {
    const auto idx = cagra::load_index(golden + "/cgra_ref_v1_nods.bin");
    CHECK(idx.rows() == 6 && idx.cols() == 3 && idx.graph_degree() == 2);
    CHECK(idx.dataset().empty() && idx.nav_nodes().empty() && idx.nav_vectors().empty());
    cagra::save_index(idx, scratch + "/roundtrip_nods.bin");
    CHECK(slurp(scratch + "/roundtrip_nods.bin") == slurp(golden + "/cgra_ref_v1_nods.bin"));
  }
  // Errors of load_index (src/cagra.cpp:330-366).
  expect_throw<std::runtime_error>("missing file", "cannot open",
                                   [&] { cagra::load_index(scratch + "/does_not_exist.bin"); });
  {
    std::ofstream(scratch + "/bad_magic.bin", std::ios::binary) << "XXXX\x01\x00\x00\x00";
    expect_throw<std::runtime_error>("bad magic", "invalid magic",
                                     [&] { cagra::load_index(scratch + "/bad_magic.bin"); });
    auto bytes = slurp(golden + "/cgra_ref_v1.bin");
    bytes[4] = 2;  // version 2
    std::ofstream(scratch + "/bad_version.bin", std::ios::binary).write(bytes.data(), std::streamsize(bytes.size()));
    expect_throw<std::runtime_error>("bad version", "unsupported version",
                                     [&] { cagra::load_index(scratch + "/bad_version.bin"); });
    bytes[4] = 1;
    std::ofstream(scratch + "/truncated.bin", std::ios::binary).write(bytes.data(), std::streamsize(bytes.size() - 9));
    expect_throw<std::runtime_error>("truncated", "read failed",
                                     [&] { cagra::load_index(scratch + "/truncated.bin"); });
  }

  // Validation before any device work.
  raft::resources res;
  const std::vector<float> data{0, 0, 10, 0, 0, 10, 2, 2};
  const auto view = raft::make_device_matrix_view<const float, std::int64_t>(data.data(), 4, 2);
  {
    cagra::index_params ip;
    ip.metric = cuvs::distance::DistanceType::InnerProduct;
    expect_throw<std::invalid_argument>("inner product", "L2Expanded", [&] { cagra::build(res, ip, view); });
    cagra::index_params ok;
    expect_throw<std::invalid_argument>("empty dataset", "non-empty", [&] {
      cagra::build(res, ok, raft::make_device_matrix_view<const float, std::int64_t>(data.data(), 0, 2));
    });
    expect_throw<std::invalid_argument>("null dataset", "non-empty", [&] {
      cagra::build(res, ok, raft::make_device_matrix_view<const float, std::int64_t>(nullptr, 4, 2));
    });
    expect_throw<std::invalid_argument>("brute force inner product", "L2Expanded", [&] {
      cuvs::neighbors::brute_force::build(res, view, cuvs::distance::DistanceType::InnerProduct);
    });
  }
  {
    cagra::index<float, std::uint32_t> idx(std::vector<float>(data), 4, 2);
    std::vector<float> q(6), d(4);
    std::vector<std::uint32_t> n(4);
    cagra::search_params sp;
    expect_throw<std::invalid_argument>("null queries", "valid buffers", [&] {
      cagra::search(res, sp, idx, raft::make_device_matrix_view<const float, std::int64_t>(nullptr, 2, 2),
                    raft::make_device_matrix_view<std::uint32_t, std::int64_t>(n.data(), 2, 2),
                    raft::make_device_matrix_view<float, std::int64_t>(d.data(), 2, 2));
    });
    expect_throw<std::invalid_argument>("dimension mismatch", "dimension", [&] {
      cagra::search(res, sp, idx, raft::make_device_matrix_view<const float, std::int64_t>(q.data(), 2, 3),
                    raft::make_device_matrix_view<std::uint32_t, std::int64_t>(n.data(), 2, 2),
                    raft::make_device_matrix_view<float, std::int64_t>(d.data(), 2, 2));
    });
    expect_throw<std::invalid_argument>("output shape", "shape", [&] {
      cagra::search(res, sp, idx, raft::make_device_matrix_view<const float, std::int64_t>(q.data(), 2, 2),
                    raft::make_device_matrix_view<std::uint32_t, std::int64_t>(n.data(), 1, 2),
                    raft::make_device_matrix_view<float, std::int64_t>(d.data(), 2, 2));
    });
  }
  // Dispatch counter API (include/cuvs/neighbors/cagra.hpp:119-122).
  cagra::reset_metal_dispatch_count();
  CHECK(cagra::metal_dispatch_count() == 0);
  cagra::increment_metal_dispatch_count();
  CHECK(cagra::metal_dispatch_count() == 1 && cagra::gpu_dispatch_count() == 1);
  cagra::reset_gpu_dispatch_count();
  CHECK(cagra::metal_dispatch_count() == 0);
  return apitest::finish("test_api_cpu");
}
