// Host-side glue between the cuVS-style C++ API and the C ABI of libcvs_hip.
#pragma once

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>

#include "cvs_hip.h"

namespace cuvs_silicon_amd {

// Converts a C-ABI status into the reference's exception types:
// argument/shape problems -> std::invalid_argument, everything else ->
// std::runtime_error (reference: src/cagra.cpp:26-32, :100-111;
// src/metal_context.mm:146-147, :245-246).
inline void check(int status) {
  if (status == CVS_OK) return;
  const std::string msg = cvs_last_error();
  if (status == CVS_ERR_INVALID_ARGUMENT || status == CVS_ERR_UNSUPPORTED)
    throw std::invalid_argument(msg);
  throw std::runtime_error(msg);
}

// Process-wide context on device 0 (the reference's MetalContext::instance(),
// src/metal_context.mm:96-99).  Throws std::runtime_error when no gfx950
// device is present: there is no CPU fallback.
class Backend {
 public:
  static Backend& instance();
  cvs_context* ctx() const noexcept { return ctx_; }
  Backend(const Backend&) = delete;
  Backend& operator=(const Backend&) = delete;

 private:
  Backend();
  ~Backend();
  cvs_context* ctx_ = nullptr;
};

// Owning handle of a device dataset.
struct DatasetHandle {
  cvs_dataset* ds = nullptr;
  DatasetHandle() = default;
  explicit DatasetHandle(cvs_dataset* d) : ds(d) {}
  DatasetHandle(const DatasetHandle&) = delete;
  DatasetHandle& operator=(const DatasetHandle&) = delete;
  ~DatasetHandle() {
    if (ds) cvs_dataset_destroy(ds);
  }
};

// Owning handle of a device graph index.
struct GraphIndexHandle {
  cvs_cagra_index* ix = nullptr;
  GraphIndexHandle() = default;
  explicit GraphIndexHandle(cvs_cagra_index* i) : ix(i) {}
  GraphIndexHandle(const GraphIndexHandle&) = delete;
  GraphIndexHandle& operator=(const GraphIndexHandle&) = delete;
  ~GraphIndexHandle() {
    if (ix) cvs_cagra_index_destroy(ix);
  }
};

// Uploads host rows (n x d) to the device.
std::shared_ptr<DatasetHandle> upload_dataset(const float* rows, std::int64_t n, std::int64_t d);

// Adds to the API-level dispatch counter (defined in cagra.cpp).
void add_dispatches(std::uint64_t n);

// Runs one C-ABI call that launches kernels and adds the number of launches
// it made to the API-level dispatch counter.
template <typename Fn>
void counted(Fn&& fn) {
  const std::uint64_t before = cvs_dispatch_count();
  check(fn());
  add_dispatches(cvs_dispatch_count() - before);
}

}  // namespace cuvs_silicon_amd
