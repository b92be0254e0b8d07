// Vector-file loaders (no GPU): the cases of the reference's
// tests/test_sift_loader.cpp:150-500 for include/cuvs_silicon/sift_loader.hpp,
// the error precedence of its sequential reader on multi-threaded loads, and
// the Cohere .bin format of include/cuvs_silicon/bin_io.hpp.
#include <cuvs_silicon/bin_io.hpp>
#include <cuvs_silicon/sift_loader.hpp>

#include <cstdint>
#include <cstdio>
#include <fstream>
#include <string>
#include <vector>

#include "check.hpp"

namespace cs = cuvs_silicon;
using apitest::expect_throw;

namespace {

std::string g_dir;

std::string path_of(const std::string& name) { return g_dir + "/" + name; }

// Writes records of (int32 count, values); count_override >= 0 replaces
// every row's count field.
template <typename V>
void write_vecs(const std::string& path, const std::vector<std::vector<V>>& rows, std::int32_t count_override = -1) {
  std::ofstream out(path, std::ios::binary);
  for (const auto& r : rows) {
    const std::int32_t n = count_override >= 0 ? count_override : std::int32_t(r.size());
    out.write(reinterpret_cast<const char*>(&n), 4);
    out.write(reinterpret_cast<const char*>(r.data()), std::streamsize(r.size() * sizeof(V)));
  }
}

void append_bytes(const std::string& path, std::size_t n) {
  std::ofstream out(path, std::ios::binary | std::ios::app);
  for (std::size_t i = 0; i < n; ++i) out.put('\x7f');
}

void truncate_by(const std::string& path, std::size_t n) {
  std::ifstream in(path, std::ios::binary);
  std::vector<char> bytes((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
  bytes.resize(bytes.size() - n);
  std::ofstream(path, std::ios::binary).write(bytes.data(), std::streamsize(bytes.size()));
}

// rows x cols with value(r, c) = r * cols + c.
std::vector<std::vector<float>> counting_rows(std::size_t rows, std::size_t cols) {
  std::vector<std::vector<float>> v(rows, std::vector<float>(cols));
  for (std::size_t r = 0; r < rows; ++r)
    for (std::size_t c = 0; c < cols; ++c) v[r][c] = float(r * cols + c);
  return v;
}

void fvecs_cases() {
  {
    const auto p = path_of("valid.fvecs");
    write_vecs<float>(p, {{1.f, 2.f, 3.f}, {4.f, 5.f, 6.f}});
    const auto ds = cs::load_fvecs(p, 2, 3);
    CHECK(ds.rows == 2 && ds.cols == 3);
    CHECK((ds.values == std::vector<float>{1.f, 2.f, 3.f, 4.f, 5.f, 6.f}));
  }
  {
    const auto p = path_of("d128.fvecs");
    write_vecs<float>(p, counting_rows(2, 128));
    const auto ds = cs::load_fvecs(p, 2, 128);
    CHECK(ds.values.size() == 256);
    for (std::size_t i = 0; i < ds.values.size(); ++i) CHECK(ds.values[i] == float(i));
  }
  {
    const auto p = path_of("wrong_dim.fvecs");
    write_vecs<float>(p, {{1.f, 2.f, 3.f}}, 4);
    expect_throw<cs::SiftLoadError>("wrong dimension", "dimension does not match",
                                    [&] { cs::load_fvecs(p, 1, 3); });
  }
  {
    const auto p = path_of("short.fvecs");
    write_vecs<float>(p, {{1.f, 2.f, 3.f}});
    expect_throw<cs::SiftLoadError>("too few rows", "ended before row dimension header",
                                    [&] { cs::load_fvecs(p, 2, 3); });
  }
  {
    const auto p = path_of("extra.fvecs");
    write_vecs<float>(p, {{1.f, 2.f, 3.f}, {4.f, 5.f, 6.f}});
    expect_throw<cs::SiftLoadError>("trailing row", "extra trailing bytes", [&] { cs::load_fvecs(p, 1, 3); });
    append_bytes(p, 1);
    expect_throw<cs::SiftLoadError>("trailing byte", "extra trailing bytes", [&] { cs::load_fvecs(p, 2, 3); });
  }
  {
    const auto p = path_of("cut.fvecs");
    write_vecs<float>(p, {{1.f, 2.f, 3.f}, {4.f, 5.f, 6.f}});
    truncate_by(p, 2);
    expect_throw<cs::SiftLoadError>("cut payload", "ended before row vector payload",
                                    [&] { cs::load_fvecs(p, 2, 3); });
    // Strict shape check: a short last payload is an error here as well.
    expect_throw<cs::SiftLoadError>("validate cut payload", "ended before row vector payload",
                                    [&] { cs::validate_fvecs_shape(p, 2, 3); });
  }
  {
    expect_throw<cs::SiftLoadError>("missing file", "failed to open fvecs file",
                                    [&] { cs::load_fvecs(path_of("absent.fvecs"), 1, 3); });
    expect_throw<cs::SiftLoadError>("directory", "failed to open fvecs file", [&] { cs::load_fvecs(g_dir, 1, 3); });
    expect_throw<cs::SiftLoadError>("shape overflow", "overflows",
                                    [&] { cs::load_fvecs(path_of("valid.fvecs"), SIZE_MAX / 2, 3); });
  }
  {
    // Zero rows: an empty file loads, any byte is trailing.
    const auto p = path_of("empty.fvecs");
    std::ofstream(p, std::ios::binary).close();
    const auto ds = cs::load_fvecs(p, 0, 7);
    CHECK(ds.rows == 0 && ds.cols == 7 && ds.values.empty());
    append_bytes(p, 3);
    expect_throw<cs::SiftLoadError>("bytes after zero rows", "extra trailing bytes",
                                    [&] { cs::load_fvecs(p, 0, 7); });
  }
  {
    // 120,000 rows of 96 floats (46 MB, several copy threads).  Row 100,000
    // has a wrong header and the file is also cut short: the row error comes
    // first, as from a sequential reader.
    const std::size_t rows = 120000, cols = 96;
    const auto p = path_of("big.fvecs");
    write_vecs<float>(p, counting_rows(rows, cols));
    const auto ds = cs::load_fvecs(p, rows, cols);
    bool same = ds.values.size() == rows * cols;
    for (std::size_t i = 0; same && i < ds.values.size(); ++i) same = ds.values[i] == float(i);
    CHECK(same);
    {
      std::fstream f(p, std::ios::binary | std::ios::in | std::ios::out);
      f.seekp(std::streamoff(100000 * (4 + 4 * cols)));
      const std::int32_t bad = 95;
      f.write(reinterpret_cast<const char*>(&bad), 4);
    }
    truncate_by(p, 10);
    expect_throw<cs::SiftLoadError>("late wrong header", "dimension does not match",
                                    [&] { cs::load_fvecs(p, rows, cols); });
    expect_throw<cs::SiftLoadError>("rows before the bad one", "extra trailing bytes",
                                    [&] { cs::load_fvecs(p, 99999, cols); });
  }
}

void sift1m_cases() {
  CHECK(cs::kSift1MBaseVectorCount == 1000000);
  CHECK(cs::kSift1MQueryVectorCount == 10000);
  CHECK(cs::kSift1MVectorDimension == 128);
  CHECK(cs::kSift1MGroundTruthNeighborCount == 100);
  {
    const auto p = path_of("sift_query.fvecs");
    write_vecs<float>(p, counting_rows(cs::kSift1MQueryVectorCount, cs::kSift1MVectorDimension));
    const auto ds = cs::load_sift1m_queries(p);
    CHECK(ds.rows == 10000 && ds.cols == 128 && ds.values.size() == 1280000);
    CHECK(ds.values.front() == 0.f && ds.values.back() == float(ds.values.size() - 1));
  }
  {
    const auto one = path_of("one_row.fvecs");
    write_vecs<float>(one, {std::vector<float>(128, 1.f)});
    const auto narrow = path_of("narrow_row.fvecs");
    write_vecs<float>(narrow, {std::vector<float>(127, 1.f)});
    expect_throw<cs::SiftLoadError>("query count", "ended before", [&] { cs::load_sift1m_queries(one); });
    expect_throw<cs::SiftLoadError>("query width", "dimension", [&] { cs::load_sift1m_queries(narrow); });
    expect_throw<cs::SiftLoadError>("base count", "ended before", [&] { cs::load_sift1m_base(one); });
    expect_throw<cs::SiftLoadError>("base width", "dimension", [&] { cs::load_sift1m_base(narrow); });
  }
  {
    // 1M headers with sparse (unwritten) payloads.
    const auto p = path_of("sparse_base.fvecs");
    {
      std::ofstream out(p, std::ios::binary);
      const std::int32_t dim = 128;
      for (std::size_t r = 0; r < cs::kSift1MBaseVectorCount; ++r) {
        out.write(reinterpret_cast<const char*>(&dim), 4);
        out.seekp(128 * 4 - 1, std::ios::cur);
        out.put('\0');
      }
    }
    cs::validate_sift1m_base_shape(p);
    std::remove(p.c_str());
  }
  {
    const auto p = path_of("sift_gt.ivecs");
    std::vector<std::vector<std::int32_t>> rows(10000, std::vector<std::int32_t>(100));
    for (std::size_t r = 0; r < rows.size(); ++r)
      for (std::size_t c = 0; c < 100; ++c) rows[r][c] = std::int32_t(r * 100 + c);
    write_vecs<std::int32_t>(p, rows);
    const auto gt = cs::load_sift1m_groundtruth(p);
    CHECK(gt.query_count == 10000 && gt.neighbor_count == 100 && gt.neighbors.size() == 1000000);
    CHECK(gt.neighbors.front() == 0 && gt.neighbors.back() == 999999);
    const auto one = path_of("gt_one.ivecs");
    write_vecs<std::int32_t>(one, {std::vector<std::int32_t>(100, 1)});
    expect_throw<cs::SiftLoadError>("gt count", "ended before", [&] { cs::load_sift1m_groundtruth(one); });
    const auto narrow = path_of("gt_narrow.ivecs");
    write_vecs<std::int32_t>(narrow, {std::vector<std::int32_t>(99, 1)});
    expect_throw<cs::SiftLoadError>("gt width", "neighbor count does not match",
                                    [&] { cs::load_sift1m_groundtruth(narrow); });
  }
}

void ivecs_cases() {
  {
    const auto p = path_of("valid.ivecs");
    write_vecs<std::int32_t>(p, {{7, 8, 9}, {10, 11, 12}});
    const auto gt = cs::load_ivecs(p, 2, 3);
    CHECK(gt.query_count == 2 && gt.neighbor_count == 3);
    CHECK((gt.neighbors == std::vector<std::uint32_t>{7, 8, 9, 10, 11, 12}));
  }
  {
    const auto p = path_of("wrong_n.ivecs");
    write_vecs<std::int32_t>(p, {{1, 2, 3}}, 4);
    expect_throw<cs::SiftLoadError>("ivecs width", "neighbor count does not match", [&] { cs::load_ivecs(p, 1, 3); });
  }
  {
    const auto p = path_of("short.ivecs");
    write_vecs<std::int32_t>(p, {{1, 2, 3}});
    expect_throw<cs::SiftLoadError>("ivecs rows", "neighbor-count header", [&] { cs::load_ivecs(p, 2, 3); });
  }
  {
    const auto p = path_of("negative.ivecs");
    write_vecs<std::int32_t>(p, {{1, -2, 3}});
    expect_throw<cs::SiftLoadError>("negative id", "non-negative", [&] { cs::load_ivecs(p, 1, 3); });
    // A negative id ahead of the cut is met first by a sequential reader.
    truncate_by(p, 2);
    expect_throw<cs::SiftLoadError>("negative then cut", "non-negative", [&] { cs::load_ivecs(p, 1, 3); });
    const auto q = path_of("cut.ivecs");
    write_vecs<std::int32_t>(q, {{1, 2, -3}});
    truncate_by(q, 2);
    expect_throw<cs::SiftLoadError>("cut before negative", "ended before row neighbor payload",
                                    [&] { cs::load_ivecs(q, 1, 3); });
  }
  {
    const auto p = path_of("extra.ivecs");
    write_vecs<std::int32_t>(p, {{1, 2}, {3, 4}});
    expect_throw<cs::SiftLoadError>("ivecs trailing", "extra trailing bytes", [&] { cs::load_ivecs(p, 1, 2); });
    expect_throw<cs::SiftLoadError>("missing ivecs", "failed to open ivecs file",
                                    [&] { cs::load_ivecs(path_of("absent.ivecs"), 1, 2); });
  }
}

void combined_cases() {
  const auto b = path_of("c_base.fvecs"), q = path_of("c_query.fvecs"), g = path_of("c_gt.ivecs");
  write_vecs<float>(b, {{1.f, 2.f}, {3.f, 4.f}, {5.f, 6.f}});
  write_vecs<float>(q, {{7.f, 8.f}, {9.f, 10.f}});
  write_vecs<std::int32_t>(g, {{0, 2}, {1, 0}});
  const auto ds = cs::load_sift_dataset(b, q, g, 3, 2, 2, 2);
  CHECK(ds.base.rows == 3 && ds.base.cols == 2 && ds.queries.rows == 2 && ds.queries.cols == 2);
  CHECK(ds.groundtruth.query_count == 2 && ds.groundtruth.neighbor_count == 2);
  CHECK((ds.base.values == std::vector<float>{1.f, 2.f, 3.f, 4.f, 5.f, 6.f}));
  CHECK((ds.queries.values == std::vector<float>{7.f, 8.f, 9.f, 10.f}));
  CHECK((ds.groundtruth.neighbors == std::vector<std::uint32_t>{0, 2, 1, 0}));

  write_vecs<float>(b, {{1.f, 2.f}, {3.f, 4.f}});
  write_vecs<float>(q, {{5.f, 6.f}});
  write_vecs<std::int32_t>(g, {{0, 2}});
  expect_throw<cs::SiftLoadError>("gt outside base", "outside base",
                                  [&] { cs::load_sift_dataset(b, q, g, 2, 1, 2, 2); });
}

void bin_cases() {
  {
    // Header (3, 5) then 15 floats, as scripts/download_cohere_wiki.py:57-63 writes.
    const auto p = path_of("base.bin");
    std::vector<float> v(15);
    for (int i = 0; i < 15; ++i) v[std::size_t(i)] = 0.25f * float(i) - 1.f;
    cs::save_bin(p, v.data(), 3, 5);
    std::ifstream in(p, std::ios::binary);
    std::int32_t hdr[2];
    in.read(reinterpret_cast<char*>(hdr), 8);
    CHECK(hdr[0] == 3 && hdr[1] == 5);
    std::int32_t r = -1, c = -1;
    const auto back = cs::load_bin<float>(p, r, c);
    CHECK(r == 3 && c == 5 && back == v);
    // Bytes after the payload are ignored, as by the harness's reader.
    append_bytes(p, 5);
    CHECK(cs::load_bin<float>(p, r, c) == v);
  }
  {
    const auto p = path_of("gt.bin");
    const std::vector<std::int32_t> ids{4, 0, 7, 1, 9, 2};
    cs::save_bin(p, ids.data(), 2, 3);
    std::int32_t r = 0, c = 0;
    CHECK(cs::load_bin<std::int32_t>(p, r, c) == ids);
    CHECK(r == 2 && c == 3);
    const auto u = cs::load_bin<std::uint32_t>(p, r, c);
    CHECK(u.size() == 6 && u[2] == 7u);
    truncate_by(p, 1);
    expect_throw<std::runtime_error>("cut payload", "Truncated file", [&] { cs::load_bin<std::int32_t>(p, r, c); });
    truncate_by(p, 24 + 8 - 1 - 5);
    expect_throw<std::runtime_error>("cut header", "Truncated file", [&] { cs::load_bin<std::int32_t>(p, r, c); });
    expect_throw<std::runtime_error>("missing bin", "Cannot open",
                                     [&] { cs::load_bin<float>(path_of("absent.bin"), r, c); });
    const std::int32_t neg[2] = {-1, 4};
    std::ofstream(p, std::ios::binary).write(reinterpret_cast<const char*>(neg), 8);
    expect_throw<std::runtime_error>("negative rows", "Invalid shape", [&] { cs::load_bin<float>(p, r, c); });
  }
  {
    // 5,000 x 1,024 floats (20 MB): several 1 MiB slices, a partial last one.
    const std::int32_t rows = 5000, cols = 1024;
    std::vector<float> v(std::size_t(rows) * cols);
    for (std::size_t i = 0; i < v.size(); ++i) v[i] = float(i % 8191) * 0.5f;
    const auto p = path_of("big.bin");
    cs::save_bin(p, v.data(), rows, cols);
    std::int32_t r = 0, c = 0;
    CHECK(cs::load_bin<float>(p, r, c) == v);
    CHECK(r == rows && c == cols);
    // Empty matrix.
    cs::save_bin<float>(path_of("empty.bin"), nullptr, 0, 1024);
    CHECK(cs::load_bin<float>(path_of("empty.bin"), r, c).empty() && r == 0 && c == 1024);
  }
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: %s <scratch dir>\n", argv[0]);
    return 2;
  }
  g_dir = argv[1];
  fvecs_cases();
  sift1m_cases();
  ivecs_cases();
  combined_cases();
  bin_cases();
  return apitest::finish("test_loaders");
}
