// "CGRA" v1 index files, byte-compatible with the reference's
// save_index/load_index (src/cagra.cpp:305-366).  Field order follows the
// reference's code (dataset before graph), little-endian, no padding:
//   char[4] "CGRA" | u32 version=1 | i64 N | i64 D | u32 G | u32 flags
//   | flags&1: f32[N*D] dataset | u32[N*G] graph
//   | flags&2: u32 n_nav, u32[n_nav] ids, f32[n_nav*D] vectors
#include <cuvs/neighbors/cagra.hpp>

#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>

namespace cuvs::neighbors::cagra {

namespace {

struct File {
  std::FILE* f = nullptr;
  ~File() {
    if (f) std::fclose(f);
  }
};

template <typename T>
void put(std::FILE* f, const T& v, bool& ok) {
  ok = ok && std::fwrite(&v, sizeof(T), 1, f) == 1;
}
template <typename T>
void put_array(std::FILE* f, const std::vector<T>& v, bool& ok) {
  if (!v.empty()) ok = ok && std::fwrite(v.data(), sizeof(T), v.size(), f) == v.size();
}
template <typename T>
bool get(std::FILE* f, T& v) {
  return std::fread(&v, sizeof(T), 1, f) == 1;
}
template <typename T>
bool get_array(std::FILE* f, std::vector<T>& v, std::size_t n) {
  v.resize(n);
  return n == 0 || std::fread(v.data(), sizeof(T), n, f) == n;
}

}  // namespace

void save_index(const index<float, std::uint32_t>& idx, const std::string& path) {
  File file;
  file.f = std::fopen(path.c_str(), "wb");
  if (!file.f) throw std::runtime_error("save_index: cannot open " + path);
  const bool has_dataset = !idx.dataset().empty();
  const bool has_nav = !idx.nav_nodes().empty();
  const std::uint32_t flags = (has_dataset ? 0x1u : 0u) | (has_nav ? 0x2u : 0u);
  bool ok = std::fwrite("CGRA", 1, 4, file.f) == 4;
  put(file.f, std::uint32_t{1}, ok);
  put(file.f, idx.rows(), ok);
  put(file.f, idx.cols(), ok);
  put(file.f, idx.graph_degree(), ok);
  put(file.f, flags, ok);
  if (has_dataset) put_array(file.f, idx.dataset(), ok);
  put_array(file.f, idx.knn_graph(), ok);
  if (has_nav) {
    put(file.f, static_cast<std::uint32_t>(idx.nav_nodes().size()), ok);
    put_array(file.f, idx.nav_nodes(), ok);
    put_array(file.f, idx.nav_vectors(), ok);
  }
  ok = ok && std::fflush(file.f) == 0;
  if (!ok) throw std::runtime_error("save_index: write failed");
}

index<float, std::uint32_t> load_index(const std::string& path) {
  File file;
  file.f = std::fopen(path.c_str(), "rb");
  if (!file.f) throw std::runtime_error("load_index: cannot open " + path);
  char magic[4] = {0, 0, 0, 0};
  if (std::fread(magic, 1, 4, file.f) != 4 || std::memcmp(magic, "CGRA", 4) != 0)
    throw std::runtime_error("load_index: invalid magic");
  std::uint32_t version = 0;
  if (!get(file.f, version) || version != 1)
    throw std::runtime_error("load_index: unsupported version");
  std::int64_t n = 0, d = 0;
  std::uint32_t g = 0, flags = 0;
  if (!get(file.f, n) || !get(file.f, d) || !get(file.f, g) || !get(file.f, flags))
    throw std::runtime_error("load_index: read failed");
  if (n < 0 || d < 0) throw std::runtime_error("load_index: read failed");

  std::vector<float> dataset;
  bool ok = true;
  if (flags & 0x1u) ok = get_array(file.f, dataset, static_cast<std::size_t>(n * d));
  if (!ok) throw std::runtime_error("load_index: read failed");
  index<float, std::uint32_t> idx(std::move(dataset), n, d);

  std::vector<std::uint32_t> graph;
  if (!get_array(file.f, graph, static_cast<std::size_t>(n) * g))
    throw std::runtime_error("load_index: read failed");
  idx.set_knn_graph(std::move(graph), g);

  if (flags & 0x2u) {
    std::uint32_t n_nav = 0;
    std::vector<std::uint32_t> nav;
    std::vector<float> nav_vectors;
    if (!get(file.f, n_nav) || !get_array(file.f, nav, n_nav) ||
        !get_array(file.f, nav_vectors, static_cast<std::size_t>(n_nav) * static_cast<std::size_t>(d)))
      throw std::runtime_error("load_index: read failed");
    idx.set_nav_nodes(std::move(nav));
    idx.set_nav_vectors(std::move(nav_vectors));
  }
  return idx;
}

}  // namespace cuvs::neighbors::cagra
