// Read-only whole-file mappings and a threaded copy out of them, shared by
// the vector-file loaders (sift_loader.cpp, bin_io.cpp).
#pragma once

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

namespace cuvs_silicon::detail {

class MappedFile {
 public:
  MappedFile() = default;
  MappedFile(const MappedFile&) = delete;
  MappedFile& operator=(const MappedFile&) = delete;
  ~MappedFile() {
    if (base_) ::munmap(const_cast<unsigned char*>(base_), size_);
    if (fd_ >= 0) ::close(fd_);
  }

  // Maps a regular file; false when it cannot be opened or mapped.  An
  // empty file maps to size() == 0 and data() == nullptr.
  bool open(const std::string& path) {
    fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd_ < 0) return false;
    struct stat st;
    if (::fstat(fd_, &st) != 0 || !S_ISREG(st.st_mode)) return false;
    size_ = static_cast<std::size_t>(st.st_size);
    if (size_ == 0) return true;
    void* p = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (p == MAP_FAILED) {
      size_ = 0;
      return false;
    }
    ::madvise(p, size_, MADV_SEQUENTIAL);
    base_ = static_cast<const unsigned char*>(p);
    return true;
  }

  const unsigned char* data() const { return base_; }
  std::size_t size() const { return size_; }

 private:
  int fd_ = -1;
  const unsigned char* base_ = nullptr;
  std::size_t size_ = 0;
};

// Threads for work over `items` units of `bytes_per_item` bytes: one per
// 32 MiB, at most 16 and at most the hardware's.
inline unsigned copy_threads(std::size_t items, std::size_t bytes_per_item) {
  const std::size_t total = items * bytes_per_item;
  const std::size_t by_size = total / (std::size_t(32) << 20) + 1;
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  return unsigned(std::min<std::size_t>({by_size, std::size_t(16), std::size_t(hw), std::max<std::size_t>(items, 1)}));
}

// Runs fn(begin, end, t) over [0, items) split into contiguous ranges, one
// per thread (t = the range's index).
template <typename Fn>
void parallel_ranges(std::size_t items, unsigned threads, Fn&& fn) {
  if (threads <= 1) {
    fn(std::size_t(0), items, 0u);
    return;
  }
  std::vector<std::thread> pool;
  pool.reserve(threads);
  for (unsigned t = 0; t < threads; ++t) {
    const std::size_t b = items * t / threads, e = items * (t + 1) / threads;
    pool.emplace_back([&fn, b, e, t] { fn(b, e, t); });
  }
  for (auto& th : pool) th.join();
}

inline std::int32_t read_i32(const unsigned char* p) {
  std::int32_t v;
  std::memcpy(&v, p, sizeof(v));
  return v;
}

}  // namespace cuvs_silicon::detail
