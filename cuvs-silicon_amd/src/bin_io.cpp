// Cohere ".bin" row matrices: int32 rows, int32 cols, rows*cols 4-byte
// values.  Reader semantics of the reference harness's load_bin<T>
// (tests/test_cohere_wiki_validation.cpp:40-52): the header and the payload
// must be present, bytes after the payload are ignored.  Writer layout of
// scripts/download_cohere_wiki.py:57-71.
#include <cuvs_silicon/bin_io.hpp>

#include <cstdio>
#include <limits>
#include <stdexcept>

#include "file_map.hpp"

namespace cuvs_silicon {

template <typename T>
std::vector<T> load_bin(const std::string& path, std::int32_t& rows, std::int32_t& cols) {
  static_assert(sizeof(T) == 4, "4-byte element types only");
  detail::MappedFile file;
  if (!file.open(path)) throw std::runtime_error("Cannot open: " + path);
  if (file.size() < 8) throw std::runtime_error("Truncated file: " + path);
  rows = detail::read_i32(file.data());
  cols = detail::read_i32(file.data() + 4);
  if (rows < 0 || cols < 0) throw std::runtime_error("Invalid shape in: " + path);
  const std::size_t count = std::size_t(rows) * std::size_t(cols);
  const std::size_t bytes = count * sizeof(T);
  if (file.size() - 8 < bytes) throw std::runtime_error("Truncated file: " + path);
  std::vector<T> out(count);
  // Copied in 1 MiB-aligned slices by up to 16 threads.
  constexpr std::size_t kSlice = std::size_t(1) << 20;
  const std::size_t slices = (bytes + kSlice - 1) / kSlice;
  const unsigned char* src = file.data() + 8;
  unsigned char* dst = reinterpret_cast<unsigned char*>(out.data());
  detail::parallel_ranges(slices, detail::copy_threads(slices, kSlice), [&](std::size_t b, std::size_t e, unsigned) {
    const std::size_t lo = b * kSlice, hi = std::min(bytes, e * kSlice);
    if (hi > lo) std::memcpy(dst + lo, src + lo, hi - lo);
  });
  return out;
}

template <typename T>
void save_bin(const std::string& path, const T* values, std::int32_t rows, std::int32_t cols) {
  static_assert(sizeof(T) == 4, "4-byte element types only");
  if (rows < 0 || cols < 0) throw std::invalid_argument("save_bin: negative shape");
  const std::size_t count = std::size_t(rows) * std::size_t(cols);
  if (count != 0 && values == nullptr) throw std::invalid_argument("save_bin: null values");
  std::FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) throw std::runtime_error("Cannot open: " + path);
  const std::int32_t header[2] = {rows, cols};
  bool ok = std::fwrite(header, sizeof(header), 1, f) == 1;
  if (ok && count != 0) ok = std::fwrite(values, sizeof(T), count, f) == count;
  ok = (std::fclose(f) == 0) && ok;
  if (!ok) throw std::runtime_error("Write failed: " + path);
}

template std::vector<float> load_bin<float>(const std::string&, std::int32_t&, std::int32_t&);
template std::vector<std::int32_t> load_bin<std::int32_t>(const std::string&, std::int32_t&, std::int32_t&);
template std::vector<std::uint32_t> load_bin<std::uint32_t>(const std::string&, std::int32_t&, std::int32_t&);
template void save_bin<float>(const std::string&, const float*, std::int32_t, std::int32_t);
template void save_bin<std::int32_t>(const std::string&, const std::int32_t*, std::int32_t, std::int32_t);
template void save_bin<std::uint32_t>(const std::string&, const std::uint32_t*, std::int32_t, std::int32_t);

}  // namespace cuvs_silicon
