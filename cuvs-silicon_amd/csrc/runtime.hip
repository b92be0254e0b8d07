// Context, error, memory, timing and dataset-layout parts of the C ABI.
//
// Replaces the reference's MetalContext singleton and its buffer caches
// (src/metal_context.mm:22-117, :155-175): one explicit context per device
// with a single HIP stream, explicit dataset handles instead of a cache keyed
// by host pointer, and a device-side fp32 -> fp16 conversion in place of the
// host loop at src/metal_context.mm:161-167.
#include <atomic>
#include <cmath>
#include <cstring>
#include <string>

#include "cvs_internal.hpp"

namespace cvs {

namespace {
thread_local std::string g_last_error;
std::atomic<uint64_t> g_dispatches{0};
}  // namespace

void set_last_error(const std::string& msg) { g_last_error = msg; }
void count_dispatch(uint64_t n) { g_dispatches.fetch_add(n, std::memory_order_relaxed); }

void DeviceBuffer::reserve(size_t need) {
  if (need <= bytes) return;
  release();
  size_t want = need + need / 4;  // headroom for slightly larger calls
  check_hip(hipMalloc(&ptr, want), "hipMalloc(workspace)");
  bytes = want;
}

void DeviceBuffer::release() {
  if (ptr) (void)hipFree(ptr);
  ptr = nullptr;
  bytes = 0;
}

void bind(cvs_context* ctx) {
  if (!ctx) fail(CVS_ERR_INVALID_ARGUMENT, "null context");
  CVS_HIP(hipSetDevice(ctx->device));
}

void upload_rows(cvs_context* ctx, float* dst, int64_t pitch, const float* src, int64_t n, int64_t d,
                 int src_on_device) {
  const size_t row = size_t(d) * sizeof(float);
  if (pitch == d) {
    CVS_HIP(hipMemcpyAsync(dst, src, row * size_t(n), src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                           ctx->stream));
    return;
  }
  const float* dsrc = src;
  void* staging = nullptr;
  if (!src_on_device) {
    CVS_HIP(hipMalloc(&staging, row * size_t(n)));
    const hipError_t e = hipMemcpyAsync(staging, src, row * size_t(n), hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) {
      (void)hipFree(staging);
      check_hip(e, "hipMemcpyAsync");
    }
    dsrc = static_cast<const float*>(staging);
  }
  const hipError_t e = hipMemcpy2DAsync(dst, size_t(pitch) * sizeof(float), dsrc, row, row, size_t(n),
                                        hipMemcpyDeviceToDevice, ctx->stream);
  if (staging) {
    // The staging buffer is released once the copy out of it has finished.
    const hipError_t es = hipStreamSynchronize(ctx->stream);
    (void)hipFree(staging);
    check_hip(es, "hipStreamSynchronize");
  }
  check_hip(e, "hipMemcpy2DAsync");
}

TimerSpan timer_span(cvs_context* ctx, const char* kernel) {
  if (!ctx->timing) return {};
  KernelTimer& t = ctx->timers[kernel];
  hipEvent_t e[2];
  for (auto& ev : e) {
    if (!t.pool.empty()) {
      ev = t.pool.back();
      t.pool.pop_back();
    } else {
      CVS_HIP(hipEventCreate(&ev));
    }
  }
  t.pending.emplace_back(e[0], e[1]);
  return {e[0], e[1]};
}

// ---------------------------------------------------------------------------
// fp32 rows -> fp16 32-row tiles + squared norms of the fp16-rounded rows.
// One 256-thread workgroup per tile; wave w converts k-steps w, w+4, ...
// Lane l owns row 32t + l%32 and, in k-step s, the 8 columns
// 16s + 8*(l/32) + [0,8).  Partial norms are combined across the two lanes of
// a row with one xor-shuffle and across the waves in a fixed order through
// LDS, so the result does not depend on scheduling.  Rows >= n and columns
// >= d are written as zeros; padding rows get norm +inf so that no distance
// involving them can pass a candidate filter.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void to_tiles_kernel(const float* __restrict__ rows,
                                                       int64_t n, int64_t d, int ksteps,
                                                       uint4* __restrict__ tiles,
                                                       float* __restrict__ norms) {
  __shared__ float s_part[4][32];
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t r = t * kTileRows + (lane & 31);
  const int cgrp = lane >> 5;
  const bool row_ok = r < n;
  const float* src = rows + (row_ok ? r : 0) * d;
  const bool vec = (d & 3) == 0 && (reinterpret_cast<uintptr_t>(rows) & 15) == 0;
  float acc = 0.f;
#pragma unroll 4
  for (int s = wave; s < ksteps; s += 4) {
    const int64_t c0 = int64_t(s) * kStepCols + cgrp * 8;
    float v[8];
    if (vec && row_ok && c0 + 8 <= d) {
      const float4 a = *reinterpret_cast<const float4*>(src + c0);
      const float4 b = *reinterpret_cast<const float4*>(src + c0 + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (row_ok && c0 + i < d) ? src[c0 + i] : 0.f;
    }
    _Float16 h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      h[i] = static_cast<_Float16>(v[i]);
      const float hv = static_cast<float>(h[i]);
      acc += hv * hv;
    }
    uint4 packed;
    __builtin_memcpy(&packed, h, sizeof(packed));
    tiles[(t * ksteps + s) * 64 + lane] = packed;
  }
  acc += __shfl_xor(acc, 32);
  if (cgrp == 0) s_part[wave][lane] = acc;
  __syncthreads();
  if (threadIdx.x < 32) {
    const float sum = ((s_part[0][threadIdx.x] + s_part[1][threadIdx.x]) + s_part[2][threadIdx.x]) +
                      s_part[3][threadIdx.x];
    norms[t * kTileRows + threadIdx.x] = (t * kTileRows + threadIdx.x < n) ? sum : INFINITY;
  }
}

void launch_to_tiles(cvs_context* ctx, const float* rows, int64_t n, int64_t d, int64_t dp,
                     int64_t n_tiles, uint16_t* tiles, float* norms) {
  if (n_tiles <= 0) return;
  hipLaunchKernelGGL(to_tiles_kernel, dim3(static_cast<unsigned>(n_tiles)), dim3(256), 0,
                     ctx->stream, rows, n, d, static_cast<int>(dp / kStepCols),
                     reinterpret_cast<uint4*>(tiles), norms);
  after_launch("to_tiles_kernel");
}

// ---------------------------------------------------------------------------
// Device calibration: the achievable HBM streaming-read rate, the bound a
// streaming kernel is measured against next to the nominal 8 TB/s.  Each
// workgroup reads one contiguous share of the buffer (as the brute-force
// scan reads its row range) in steps of 32 KiB, 8 non-temporal 16-byte loads
// per thread, with two steps in flight (two register sets, each reloaded two
// steps ahead as soon as it is consumed, as the scan keeps its stages).
// Loads are buffer loads over the share, so a step past its end reads zeros
// without a memory access and no load sits behind a branch.  The XOR of the
// data decides a store that never happens in practice but keeps every load.
// ---------------------------------------------------------------------------
typedef uint32_t stream_vec __attribute__((ext_vector_type(4)));
constexpr int kStreamLoads = 8;
constexpr uint64_t kStreamStepVecs = uint64_t(kStreamLoads) * 256;  // 16-byte vectors per step

__global__ __launch_bounds__(256) void stream_read_kernel(const stream_vec* __restrict__ src, uint64_t steps_per_wg,
                                                          uint32_t* __restrict__ sink) {
  const uint32_t step_bytes = uint32_t(kStreamStepVecs * 16);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<stream_vec*>(src + uint64_t(blockIdx.x) * steps_per_wg * kStreamStepVecs), 0,
      int(uint32_t(steps_per_wg) * step_bytes), 0x00020000);
  auto load = [&](stream_vec (&v)[kStreamLoads], uint64_t step) {
    const uint32_t off = uint32_t(step) * step_bytes + threadIdx.x * 16u;
#pragma unroll
    for (int i = 0; i < kStreamLoads; ++i)
      v[i] = __builtin_bit_cast(stream_vec, __builtin_amdgcn_raw_buffer_load_b128(rs, off + uint32_t(i) * 4096u, 0, 2));
  };
  uint32_t acc = 0;
  auto consume = [&](const stream_vec (&v)[kStreamLoads]) {
#pragma unroll
    for (int i = 0; i < kStreamLoads; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  };
  stream_vec a[kStreamLoads], b[kStreamLoads];
  load(a, 0);
  load(b, 1);
  for (uint64_t s = 0; s < steps_per_wg; s += 2) {
    consume(a);
    load(a, s + 2);
    consume(b);
    load(b, s + 3);
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x * 256 + threadIdx.x] = acc;
}

}  // namespace cvs

using namespace cvs;

extern "C" {

const char* cvs_last_error(void) { return g_last_error.c_str(); }
uint64_t cvs_dispatch_count(void) { return g_dispatches.load(); }
void cvs_reset_dispatch_count(void) { g_dispatches.store(0); }

int cvs_device_count(int* out_count) {
  return guarded([&] {
    if (!out_count) fail(CVS_ERR_INVALID_ARGUMENT, "null out_count");
    int c = 0;
    if (hipGetDeviceCount(&c) != hipSuccess) c = 0;
    *out_count = c;
  });
}

int cvs_context_create(int device, cvs_context** out_ctx) {
  return guarded([&] {
    if (!out_ctx) fail(CVS_ERR_INVALID_ARGUMENT, "null out_ctx");
    *out_ctx = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
      fail(CVS_ERR_NO_DEVICE, "no HIP device available");
    if (device < 0 || device >= count)
      fail(CVS_ERR_INVALID_ARGUMENT, "device index out of range");
    hipDeviceProp_t prop;
    CVS_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
      fail(CVS_ERR_NO_DEVICE, std::string("kernels are built for gfx950, device is ") +
                                  prop.gcnArchName);
    auto* ctx = new cvs_context();
    ctx->device = device;
    ctx->compute_units = prop.multiProcessorCount;
    ctx->total_mem = static_cast<int64_t>(prop.totalGlobalMem);
    ctx->name = prop.name[0] ? std::string(prop.name) + " (" + prop.gcnArchName + ")"
                             : std::string(prop.gcnArchName);
    try {
      CVS_HIP(hipSetDevice(device));
      CVS_HIP(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
    } catch (...) {
      delete ctx;
      throw;
    }
    *out_ctx = ctx;
  });
}

int cvs_context_destroy(cvs_context* ctx) {
  return guarded([&] {
    if (!ctx) return;
    if (ctx->live_children > 0)
      fail(CVS_ERR_INVALID_ARGUMENT, "context still owns " + std::to_string(ctx->live_children) +
                                         " dataset(s) or graph index(es): destroy them first");
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (auto& kv : ctx->timers) {
      for (auto& p : kv.second.pending) {
        (void)hipEventDestroy(p.first);
        (void)hipEventDestroy(p.second);
      }
      for (auto e : kv.second.pool) (void)hipEventDestroy(e);
    }
    ctx->ws_search.release();
    ctx->ws_io.release();
    ctx->ws_teams.release();
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
  });
}

int cvs_context_synchronize(cvs_context* ctx) {
  return guarded([&] {
    bind(ctx);
    CVS_HIP(hipStreamSynchronize(ctx->stream));
  });
}

int cvs_context_device_info(cvs_context* ctx, char* name, size_t name_len, int* compute_units,
                            int64_t* total_mem_bytes) {
  return guarded([&] {
    if (!ctx) fail(CVS_ERR_INVALID_ARGUMENT, "null context");
    if (name && name_len) {
      std::strncpy(name, ctx->name.c_str(), name_len - 1);
      name[name_len - 1] = '\0';
    }
    if (compute_units) *compute_units = ctx->compute_units;
    if (total_mem_bytes) *total_mem_bytes = ctx->total_mem;
  });
}

int cvs_context_set_timing(cvs_context* ctx, int enable) {
  return guarded([&] {
    if (!ctx) fail(CVS_ERR_INVALID_ARGUMENT, "null context");
    ctx->timing = enable != 0;
  });
}

int cvs_context_kernel_time(cvs_context* ctx, const char* kernel, double* total_ms,
                            uint64_t* launches) {
  return guarded([&] {
    bind(ctx);
    if (!kernel || !total_ms || !launches) fail(CVS_ERR_INVALID_ARGUMENT, "null argument");
    CVS_HIP(hipStreamSynchronize(ctx->stream));
    double sum = 0.0;
    uint64_t cnt = 0;
    auto it = ctx->timers.find(kernel);
    if (it != ctx->timers.end()) {
      for (auto& p : it->second.pending) {
        float ms = 0.f;
        CVS_HIP(hipEventElapsedTime(&ms, p.first, p.second));
        sum += ms;
        ++cnt;
        it->second.pool.push_back(p.first);
        it->second.pool.push_back(p.second);
      }
      it->second.pending.clear();
    }
    *total_ms = sum;
    *launches = cnt;
  });
}

int cvs_calibrate_stream_read(cvs_context* ctx, size_t bytes, int workgroups, int reps, double* out_gbs) {
  return guarded([&] {
    bind(ctx);
    if (!out_gbs) fail(CVS_ERR_INVALID_ARGUMENT, "null out_gbs");
    if (workgroups < 1 || reps < 1) fail(CVS_ERR_INVALID_ARGUMENT, "workgroups and reps must be positive");
    const uint64_t step_bytes = kStreamStepVecs * 16;
    const uint64_t steps = uint64_t(bytes) / (step_bytes * uint64_t(workgroups));
    if (steps == 0) fail(CVS_ERR_INVALID_ARGUMENT, "fewer than 32 KiB per workgroup");
    if (steps * step_bytes >= (uint64_t(1) << 31))
      fail(CVS_ERR_UNSUPPORTED, "a workgroup's share must stay below 2 GiB (use more workgroups)");
    const size_t used = size_t(steps * step_bytes * uint64_t(workgroups));
    void* buf = nullptr;
    void* sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    auto cleanup = [&] {
      if (e0) (void)hipEventDestroy(e0);
      if (e1) (void)hipEventDestroy(e1);
      if (buf) (void)hipFree(buf);
      if (sink) (void)hipFree(sink);
    };
    try {
      CVS_HIP(hipMalloc(&buf, used));
      CVS_HIP(hipMalloc(&sink, size_t(workgroups) * 256 * sizeof(uint32_t)));
      CVS_HIP(hipMemsetAsync(buf, 0x5a, used, ctx->stream));
      CVS_HIP(hipEventCreate(&e0));
      CVS_HIP(hipEventCreate(&e1));
      auto launch = [&] {
        hipLaunchKernelGGL(stream_read_kernel, dim3(unsigned(workgroups)), dim3(256), 0, ctx->stream,
                           static_cast<const stream_vec*>(buf), steps, static_cast<uint32_t*>(sink));
        after_launch("stream_read_kernel");
      };
      for (int i = 0; i < 2; ++i) launch();  // warm-up
      CVS_HIP(hipEventRecord(e0, ctx->stream));
      for (int i = 0; i < reps; ++i) launch();
      CVS_HIP(hipEventRecord(e1, ctx->stream));
      CVS_HIP(hipEventSynchronize(e1));
      float ms = 0.f;
      CVS_HIP(hipEventElapsedTime(&ms, e0, e1));
      *out_gbs = double(used) * reps / (double(ms) * 1e-3) / 1e9;
    } catch (...) {
      cleanup();
      throw;
    }
    cleanup();
  });
}

int cvs_device_alloc(cvs_context* ctx, size_t bytes, void** out_ptr) {
  return guarded([&] {
    bind(ctx);
    if (!out_ptr) fail(CVS_ERR_INVALID_ARGUMENT, "null out_ptr");
    *out_ptr = nullptr;
    if (bytes == 0) fail(CVS_ERR_INVALID_ARGUMENT, "zero-byte allocation");
    CVS_HIP(hipMalloc(out_ptr, bytes));
  });
}

int cvs_device_free(cvs_context* ctx, void* ptr) {
  return guarded([&] {
    bind(ctx);
    if (ptr) CVS_HIP(hipFree(ptr));
  });
}

int cvs_copy_to_device(cvs_context* ctx, void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    bind(ctx);
    if (bytes == 0) return;
    if (!dst || !src) fail(CVS_ERR_INVALID_ARGUMENT, "null pointer");
    CVS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    CVS_HIP(hipStreamSynchronize(ctx->stream));
  });
}

int cvs_copy_to_host(cvs_context* ctx, void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    bind(ctx);
    if (bytes == 0) return;
    if (!dst || !src) fail(CVS_ERR_INVALID_ARGUMENT, "null pointer");
    CVS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    CVS_HIP(hipStreamSynchronize(ctx->stream));
  });
}

int cvs_dataset_create(cvs_context* ctx, const float* rows, int64_t n, int64_t d,
                       int rows_on_device, cvs_dataset** out_ds) {
  return guarded([&] {
    bind(ctx);
    if (!out_ds) fail(CVS_ERR_INVALID_ARGUMENT, "null out_ds");
    *out_ds = nullptr;
    if (!rows || n <= 0 || d <= 0)
      fail(CVS_ERR_INVALID_ARGUMENT, "dataset must be non-null and non-empty");
    if (n > int64_t(UINT32_MAX) - 1)
      fail(CVS_ERR_UNSUPPORTED, "dataset rows must fit uint32 ids");
    auto* ds = new cvs_dataset();
    ds->ctx = ctx;
    ds->n = n;
    ds->d = d;
    ds->dp = padded_dim(d);
    const int64_t tiles = (n + kTileRows - 1) / kTileRows;
    ds->n_tiles = (tiles + kTilePad - 1) / kTilePad * kTilePad;  // no ragged stage loads
    try {
      const size_t row_bytes = size_t(n) * size_t(d) * sizeof(float);
      CVS_HIP(hipMalloc(&ds->rows, row_bytes));
      CVS_HIP(hipMalloc(&ds->tiles, size_t(ds->n_tiles) * size_t(ds->dp / kStepCols) * kStepBytes));
      // + kNormSlack: stage copies read whole 64-float windows past the last tile.
      CVS_HIP(hipMalloc(&ds->norms, (size_t(ds->n_tiles) * kTileRows + kNormSlack) * sizeof(float)));
      CVS_HIP(hipMemsetAsync(ds->norms, 0, (size_t(ds->n_tiles) * kTileRows + kNormSlack) * sizeof(float),
                             ctx->stream));
      CVS_HIP(hipMemcpyAsync(ds->rows, rows, row_bytes,
                             rows_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                             ctx->stream));
      launch_to_tiles(ctx, ds->rows, n, d, ds->dp, ds->n_tiles, ds->tiles, ds->norms);
      CVS_HIP(hipStreamSynchronize(ctx->stream));
    } catch (...) {
      if (ds->rows) (void)hipFree(ds->rows);
      if (ds->tiles) (void)hipFree(ds->tiles);
      if (ds->norms) (void)hipFree(ds->norms);
      delete ds;
      throw;
    }
    ++ctx->live_children;
    *out_ds = ds;
  });
}

int cvs_dataset_destroy(cvs_dataset* ds) {
  return guarded([&] {
    if (!ds) return;
    bind(ds->ctx);
    (void)hipStreamSynchronize(ds->ctx->stream);
    (void)hipFree(ds->rows);
    (void)hipFree(ds->tiles);
    (void)hipFree(ds->norms);
    --ds->ctx->live_children;
    delete ds;
  });
}

int cvs_dataset_shape(const cvs_dataset* ds, int64_t* n, int64_t* d) {
  return guarded([&] {
    if (!ds) fail(CVS_ERR_INVALID_ARGUMENT, "null dataset");
    if (n) *n = ds->n;
    if (d) *d = ds->d;
  });
}

int cvs_dataset_rows(const cvs_dataset* ds, const float** out_rows) {
  return guarded([&] {
    if (!ds || !out_rows) fail(CVS_ERR_INVALID_ARGUMENT, "null argument");
    *out_rows = ds->rows;
  });
}

}  // extern "C"
