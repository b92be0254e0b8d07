// Internal definitions shared by the HIP translation units of libcvs_hip.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <map>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "cvs_hip.h"

namespace cvs {

// Exception carrying a C-ABI status code; converted at the extern "C" edge.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] inline void fail(int code, const std::string& msg) { throw Error(code, msg); }

inline void check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return;
  const int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
                       ? CVS_ERR_OUT_OF_MEMORY
                       : CVS_ERR_RUNTIME;
  fail(code, std::string(what) + ": " + hipGetErrorString(e));
}

#define CVS_HIP(call) ::cvs::check_hip((call), #call)

void set_last_error(const std::string& msg);
void count_dispatch(uint64_t n = 1);

// Runs `fn`, mapping exceptions to status codes + thread-local message.
template <typename Fn>
int guarded(Fn&& fn) {
  try {
    fn();
    set_last_error("");
    return CVS_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return CVS_ERR_OUT_OF_MEMORY;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return CVS_ERR_RUNTIME;
  }
}

// A growable device allocation owned by a context (workspaces).
struct DeviceBuffer {
  void* ptr = nullptr;
  size_t bytes = 0;
  void reserve(size_t need);
  void release();
  template <typename T>
  T* as() const { return static_cast<T*>(ptr); }
};

// Event pairs bracketing the launches of one kernel family.
struct KernelTimer {
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
  std::vector<hipEvent_t> pool;
};

}  // namespace cvs

struct cvs_context {
  int device = 0;
  // Datasets and graph indexes created on this context and not yet
  // destroyed; cvs_context_destroy refuses while any is alive, since each
  // of them uses the context's stream and device at its own destruction.
  int live_children = 0;
  hipStream_t stream = nullptr;
  int compute_units = 0;
  int64_t total_mem = 0;
  std::string name;
  bool timing = false;
  std::map<std::string, cvs::KernelTimer> timers;
  // Workspaces reused across calls (never shrink).
  cvs::DeviceBuffer ws_search;    // brute force: query tiles, thresholds, candidate lists
  cvs::DeviceBuffer ws_io;        // staging of host queries / results
  cvs::DeviceBuffer ws_teams;     // per-team lists of multi-team graph search
  // Brute-force escalation counters (device, allocated with the context):
  // [0] queries whose fp16 selection could not be certified and were
  // re-ranked exactly over more rows, [1] of them over every row.
  unsigned long long* bf_counters = nullptr;
};

struct cvs_dataset {
  cvs_context* ctx = nullptr;
  int64_t n = 0;          // rows
  int64_t d = 0;          // dimensions
  int64_t dp = 0;         // padded dimensions (padded_dim)
  int64_t n_tiles = 0;    // 32-row tiles, padded to a multiple of kTilePad
  float* rows = nullptr;          // n x d fp32, row-major
  uint16_t* tiles = nullptr;      // n_tiles x (dp/16) x 64 lanes x 8 fp16 of scale * (row - mu)
  float* norms = nullptr;         // n_tiles*32 squared norms of the fp16 rows (+inf pad)
  // The fp16 copy is centred and scaled: tiles hold fp16(scale * fl(x - mu))
  // with mu the fp32 column mean (L2 distances are translation invariant,
  // and the fp16 rounding error then scales with the rows' spread, not their
  // offset) and scale a power of two that puts the largest centred value in
  // [128, 256), so that queries up to 256 times farther out stay finite and
  // small values stay normal.
  float* mu = nullptr;            // dp fp32 column means, zero-padded (device)
  float scale = 1.f;
  // Bounds for the per-query certificate of the fp16 selection, in scaled
  // units: every row has |x~| <= cert_rmax and |x~ - scale (x - mu)| <= cert_dx
  // (measured at creation, rounded up).  Infinite when the rows are not
  // finite, which sends every query to the exact fallback.
  float cert_rmax = 0.f;
  float cert_dx = 0.f;
};

struct cvs_cagra_index {
  cvs_context* ctx = nullptr;
  int64_t n = 0;
  int64_t d = 0;
  int64_t dpad = 0;        // row stride in elements (d rounded up to 128)
  uint32_t degree = 0;
  uint32_t n_seeds = 0;
  int traversal_bits = 32;   // 32: rows only; 16: traverse rows16, re-rank the list from rows
  float* rows = nullptr;     // n x dpad fp32, zero-padded
  void* rows16 = nullptr;    // n x dpad fp16 copy of scale * (rows - mu), zero-padded
  float* mu = nullptr;       // dpad column means (zero-padded)
  float scale = 1.f;         // power of two of the fp16 copy (see cvs_dataset)
  uint32_t* graph = nullptr; // n x degree
  uint32_t* seeds = nullptr; // n_seeds ids
};

namespace cvs {

// Makes the context's device current for the calling thread.
void bind(cvs_context* ctx);

// Copies n rows of d floats (contiguous, host or device memory) into dst
// with a row pitch of `pitch` floats (pitch >= d; the pad columns are left as
// they are), enqueued on the context stream.  A host source moves in one
// contiguous transfer (staged through a device buffer when pitch != d):
// row-by-row transfers from pageable host memory are slow.
void upload_rows(cvs_context* ctx, float* dst, int64_t pitch, const float* src, int64_t n, int64_t d,
                 int src_on_device);

// Kernel timing.  While a context's timing is on, timer_span() hands out a
// start and a stop event for one kernel family: the family's first launch
// takes `start` and its last launch `stop` (hipExtLaunchKernelGGL), and the
// runtime fills them from those dispatches' own timestamps.  No marker
// packets go between kernels, so timing can stay on inside a timed loop
// without changing it.  Both events are null while timing is off, which
// makes the launches plain ones.
struct TimerSpan {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
TimerSpan timer_span(cvs_context* ctx, const char* kernel);

// Launch-site helper: checks the launch, counts the dispatch.
inline void after_launch(const char* what) {
  check_hip(hipGetLastError(), what);
  count_dispatch(1);
}

// fp16 tile layout (shared by dataset and query tiles): tile t holds rows
// [32t, 32t+32); k-step s holds columns [16s, 16s+16); lane l of a 64-lane
// wave holds row 32t + (l % 32), columns 16s + 8*(l/32) + [0, 8).  One k-step
// of one tile is therefore 1 KiB contiguous, loaded by one wave with one
// 16-byte access per lane, and is exactly the per-lane A (or B) operand of
// v_mfma_f32_32x32x16_f16.  The tile count is padded to a multiple of
// kTilePad so that the scan can always stream whole 64 KiB units.
constexpr int kTileRows = 32;
constexpr int kStepCols = 16;
constexpr int kStepBytes = 1024;
constexpr int kTilePad = 64;
constexpr int kNormSlack = 256;  // floats allocated past the last tile's norms

// Padded dimensions of a dataset's tiles: 32 times a power of two up to 1024
// (the fused scan is instantiated per k-step count), a multiple of 64 beyond
// (only the keys-matrix path reads those, four k-steps at a time).
inline int64_t padded_dim(int64_t d) {
  if (d > 1024) return (d + 63) / 64 * 64;
  int64_t p = 32;
  while (p < d) p *= 2;
  return p;
}

// Launches the fp32 -> fp16-tile conversion of scale * (row - mu) (rows n x
// d with row stride d; mu d floats, or null for zero); writes n_tiles tiles
// and n_tiles*32 norms.  With `stats` (3 floats, zeroed beforehand, read as
// non-negative bit patterns) it also raises stats[1] to the largest squared
// norm and stats[2] to the largest squared rounding error |x~ - s (x - mu)|^2
// of a row.
void launch_to_tiles(cvs_context* ctx, const float* rows, int64_t n, int64_t d, int64_t dp, int64_t n_tiles,
                     uint16_t* tiles, float* norms, const float* mu = nullptr, float scale = 1.f,
                     uint32_t* stats = nullptr);

// Centring and scaling of an fp16 copy (the brute-force tiles, the graph
// build's rows, the graph search's traversal copy): computes mu (dp floats,
// the fp32 column means of the n x d rows, zero past d) on the device and
// returns the power-of-two scale that puts the largest |x - mu| in
// [128, 256) (1 if the rows are all equal or not finite).  Synchronizes.
float centre_rows(cvs_context* ctx, const float* rows, int64_t n, int64_t d, int64_t dp, float* mu);

}  // namespace cvs
