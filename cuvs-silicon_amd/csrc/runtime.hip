// Context, error, memory, timing and dataset-layout parts of the C ABI.
//
// Replaces the reference's MetalContext singleton and its buffer caches
// (src/metal_context.mm:22-117, :155-175): one explicit context per device
// with a single HIP stream, explicit dataset handles instead of a cache keyed
// by host pointer, and a device-side fp32 -> fp16 conversion in place of the
// host loop at src/metal_context.mm:161-167.
#include <algorithm>
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
// fp32 rows -> fp16 32-row tiles of scale * (row - mu) + squared norms of the
// fp16-rounded rows.  One 256-thread workgroup per tile; wave w converts
// k-steps w, w+4, ...  Lane l owns row 32t + l%32 and, in k-step s, the 8
// columns 16s + 8*(l/32) + [0,8).  Partial norms are combined across the two
// lanes of a row with one xor-shuffle and across the waves in a fixed order
// through LDS, so the result does not depend on scheduling.  Rows >= n and
// columns >= d are written as zeros; padding rows get norm +inf so that no
// distance involving them can pass a candidate filter.  With `stats`, the
// largest squared norm and the largest squared rounding error of a row are
// folded into stats[1] and stats[2] by atomicMax on their bit patterns
// (non-negative floats order as their bits; the maximum does not depend on
// the order of the updates).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void to_tiles_kernel(const float* __restrict__ rows,
                                                       int64_t n, int64_t d, int ksteps,
                                                       const float* __restrict__ mu, float scale,
                                                       uint4* __restrict__ tiles,
                                                       float* __restrict__ norms,
                                                       uint32_t* __restrict__ stats) {
  __shared__ float s_part[2][4][32];
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t r = t * kTileRows + (lane & 31);
  const int cgrp = lane >> 5;
  const bool row_ok = r < n;
  const float* src = rows + (row_ok ? r : 0) * d;
  const bool vec = (d & 3) == 0 && (reinterpret_cast<uintptr_t>(rows) & 15) == 0;
  float acc = 0.f, err = 0.f;
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
    if (mu) {
      // Means loaded unconditionally (column clamped) and the result masked
      // by an AND of its bits, which the compiler keeps out of branches: a
      // load used only under its lane condition is waited for before the
      // next one is issued.
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float mi = mu[c0 + i < d ? c0 + i : d - 1];
        const float r = (v[i] - mi) * scale;
        v[i] = __uint_as_float(__float_as_uint(r) & (c0 + i < d ? 0xffffffffu : 0u));
      }
    }
    _Float16 h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      h[i] = static_cast<_Float16>(v[i]);
      const float hv = static_cast<float>(h[i]);
      acc += hv * hv;
      const float e = hv - v[i];
      err += e * e;
    }
    uint4 packed;
    __builtin_memcpy(&packed, h, sizeof(packed));
    tiles[(t * ksteps + s) * 64 + lane] = packed;
  }
  acc += __shfl_xor(acc, 32);
  err += __shfl_xor(err, 32);
  if (cgrp == 0) {
    s_part[0][wave][lane] = acc;
    s_part[1][wave][lane] = err;
  }
  __syncthreads();
  if (threadIdx.x < 32) {
    const int i = threadIdx.x;
    const float sum = ((s_part[0][0][i] + s_part[0][1][i]) + s_part[0][2][i]) + s_part[0][3][i];
    const float esum = ((s_part[1][0][i] + s_part[1][1][i]) + s_part[1][2][i]) + s_part[1][3][i];
    const bool ok = t * kTileRows + i < n;
    norms[t * kTileRows + i] = ok ? sum : INFINITY;
    if (stats && ok) {
      // NaN maps above +inf, so a non-finite row shows up as a non-finite bound.
      atomicMax(&stats[1], __float_as_uint(sum));
      atomicMax(&stats[2], __float_as_uint(esum));
    }
  }
}

void launch_to_tiles(cvs_context* ctx, const float* rows, int64_t n, int64_t d, int64_t dp, int64_t n_tiles,
                     uint16_t* tiles, float* norms, const float* mu, float scale, uint32_t* stats) {
  if (n_tiles <= 0) return;
  hipLaunchKernelGGL(to_tiles_kernel, dim3(static_cast<unsigned>(n_tiles)), dim3(256), 0,
                     ctx->stream, rows, n, d, static_cast<int>(dp / kStepCols), mu, scale,
                     reinterpret_cast<uint4*>(tiles), norms, stats);
  after_launch("to_tiles_kernel");
}

// ---------------------------------------------------------------------------
// Column means for the centring of fp16 copies.  column_sum_kernel: block
// (chunk, column group) sums rows [chunk * rows_per_chunk, ...) of 256
// consecutive columns in fp64 (each row segment read as one coalesced
// 1 KiB access); column_mean_kernel adds the chunks in chunk order and
// divides by n, so the means do not depend on scheduling.  maxabs_kernel
// folds the largest |fl(x - mu)| into stats[0] by atomicMax on bit patterns.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void column_sum_kernel(const float* __restrict__ rows, int64_t n, int64_t d,
                                                         int64_t rows_per_chunk, double* __restrict__ partial) {
  const int64_t c = int64_t(blockIdx.y) * 256 + threadIdx.x;
  if (c >= d) return;
  const int64_t r0 = int64_t(blockIdx.x) * rows_per_chunk;
  const int64_t r1 = r0 + rows_per_chunk < n ? r0 + rows_per_chunk : n;
  double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
  int64_t r = r0;
  for (; r + 4 <= r1; r += 4) {
    s0 += rows[(r + 0) * d + c];
    s1 += rows[(r + 1) * d + c];
    s2 += rows[(r + 2) * d + c];
    s3 += rows[(r + 3) * d + c];
  }
  for (; r < r1; ++r) s0 += rows[r * d + c];
  partial[int64_t(blockIdx.x) * d + c] = (s0 + s1) + (s2 + s3);
}

__global__ __launch_bounds__(256) void column_mean_kernel(const double* __restrict__ partial, int chunks,
                                                          int64_t n, int64_t d, int64_t dp, float* __restrict__ mu) {
  const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (c >= dp) return;
  if (c >= d) {
    mu[c] = 0.f;
    return;
  }
  double s = 0.0;
  for (int i = 0; i < chunks; ++i) s += partial[int64_t(i) * d + c];
  mu[c] = float(s / double(n));
}

__global__ __launch_bounds__(256) void maxabs_kernel(const float* __restrict__ rows, int64_t n, int64_t d,
                                                     int64_t rows_per_chunk, const float* __restrict__ mu,
                                                     uint32_t* __restrict__ stats) {
  const int64_t c = int64_t(blockIdx.y) * 256 + threadIdx.x;
  float m = 0.f;
  if (c < d) {
    const float mc = mu[c];
    const int64_t r0 = int64_t(blockIdx.x) * rows_per_chunk;
    const int64_t r1 = r0 + rows_per_chunk < n ? r0 + rows_per_chunk : n;
    for (int64_t r = r0; r < r1; ++r) {
      const float v = fabsf(rows[r * d + c] - mc);
      m = (v > m || v != v) ? v : m;  // keeps a NaN
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float y = __shfl_xor(m, o);
    m = (y > m || y != y) ? y : m;
  }
  if ((threadIdx.x & 63) == 0) atomicMax(&stats[0], __float_as_uint(m));
}

float centre_rows(cvs_context* ctx, const float* rows, int64_t n, int64_t d, int64_t dp, float* mu) {
  const int64_t rows_per_chunk = std::max<int64_t>(64, (n + 255) / 256);
  const int chunks = int((n + rows_per_chunk - 1) / rows_per_chunk);
  double* partial = nullptr;
  uint32_t* stats = nullptr;
  CVS_HIP(hipMalloc(&partial, size_t(chunks) * size_t(d) * sizeof(double)));
  float scale = 1.f;
  try {
    CVS_HIP(hipMalloc(&stats, sizeof(uint32_t)));
    CVS_HIP(hipMemsetAsync(stats, 0, sizeof(uint32_t), ctx->stream));
    hipLaunchKernelGGL(column_sum_kernel, dim3(unsigned(chunks), unsigned((d + 255) / 256)), dim3(256), 0,
                       ctx->stream, rows, n, d, rows_per_chunk, partial);
    after_launch("column_sum_kernel");
    hipLaunchKernelGGL(column_mean_kernel, dim3(unsigned((dp + 255) / 256)), dim3(256), 0, ctx->stream,
                       static_cast<const double*>(partial), chunks, n, d, dp, mu);
    after_launch("column_mean_kernel");
    hipLaunchKernelGGL(maxabs_kernel, dim3(unsigned(chunks), unsigned((d + 255) / 256)), dim3(256), 0, ctx->stream,
                       rows, n, d, rows_per_chunk, static_cast<const float*>(mu), stats);
    after_launch("maxabs_kernel");
    uint32_t bits = 0;
    CVS_HIP(hipMemcpyAsync(&bits, stats, sizeof(bits), hipMemcpyDeviceToHost, ctx->stream));
    CVS_HIP(hipStreamSynchronize(ctx->stream));
    float m;
    std::memcpy(&m, &bits, sizeof(m));
    if (std::isfinite(m) && m > 0.f) {
      // m = f * 2^x with f in [0.5, 1), so m * 2^(8 - x) lies in [128, 256).
      int x = 0;
      (void)std::frexp(m, &x);
      scale = std::ldexp(1.f, std::max(-120, std::min(120, 8 - x)));
    }
  } catch (...) {
    (void)hipFree(partial);
    if (stats) (void)hipFree(stats);
    throw;
  }
  (void)hipFree(partial);
  (void)hipFree(stats);
  return scale;
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

// ---------------------------------------------------------------------------
// Device calibration for gather-bound kernels (the graph search): each
// 16-lane team of a workgroup reads whole rows of `row_bytes` at random,
// lane l taking the 16-byte pieces l, l + 16, ... of a row (so one load
// instruction of the team covers 256 contiguous bytes, as the search's row
// gathers do), two rows in flight per team.  Rows are picked by a
// multiplicative hash of (team, step) over n_rows rows, so the set of rows
// read is spread uniformly over the buffer.  The XOR of the data decides a
// store that never happens in practice but keeps every load.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gather_read_kernel(const stream_vec* __restrict__ buf, uint64_t n_rows,
                                                          uint32_t row_vecs, uint32_t rows_per_team, uint32_t seed,
                                                          uint32_t* __restrict__ sink) {
  const uint32_t team = blockIdx.x * 16u + (threadIdx.x >> 4);
  const uint32_t tp = threadIdx.x & 15u;
  uint32_t acc = 0;
  auto row_of = [&](uint32_t i) -> uint64_t {
    uint64_t h = (uint64_t(team) << 32 | i) * 0x9E3779B97F4A7C15ull + seed;
    h ^= h >> 29;
    h *= 0xBF58476D1CE4E5B9ull;
    h ^= h >> 32;
    return h % n_rows;
  };
  for (uint32_t i = 0; i < rows_per_team; i += 2) {
    const stream_vec* r0 = buf + row_of(i) * row_vecs + tp;
    const stream_vec* r1 = buf + row_of(i + 1) * row_vecs + tp;
    stream_vec v0[16], v1[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t c = tp + 16u * uint32_t(j);
      v0[j] = c < row_vecs ? r0[16 * j] : stream_vec{0, 0, 0, 0};
      v1[j] = c < row_vecs ? r1[16 * j] : stream_vec{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) acc ^= v0[j].x ^ v0[j].w ^ v1[j].y ^ v1[j].z;
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x * 256 + threadIdx.x] = acc;
}

}  // namespace cvs

using namespace cvs;

extern "C" {

int cvs_calibrate_gather_read(cvs_context* ctx, size_t row_bytes, int64_t n_rows, int workgroups, int rows_per_team,
                              int reps, double* out_gbs) {
  return guarded([&] {
    bind(ctx);
    if (!out_gbs) fail(CVS_ERR_INVALID_ARGUMENT, "null out_gbs");
    if (row_bytes == 0 || row_bytes % 16 != 0 || row_bytes > 4096)
      fail(CVS_ERR_INVALID_ARGUMENT, "row_bytes must be a multiple of 16 and at most 4096");
    if (n_rows < 1 || workgroups < 1 || rows_per_team < 2 || reps < 1)
      fail(CVS_ERR_INVALID_ARGUMENT, "n_rows, workgroups, reps positive; rows_per_team at least 2");
    const size_t bytes = size_t(n_rows) * row_bytes;
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
      CVS_HIP(hipMalloc(&buf, bytes));
      CVS_HIP(hipMalloc(&sink, size_t(workgroups) * 256 * sizeof(uint32_t)));
      CVS_HIP(hipMemsetAsync(buf, 0x5a, bytes, ctx->stream));
      CVS_HIP(hipEventCreate(&e0));
      CVS_HIP(hipEventCreate(&e1));
      const uint32_t rpt = uint32_t(rows_per_team + (rows_per_team & 1));
      auto launch = [&](uint32_t seed) {
        hipLaunchKernelGGL(gather_read_kernel, dim3(unsigned(workgroups)), dim3(256), 0, ctx->stream,
                           static_cast<const stream_vec*>(buf), uint64_t(n_rows), uint32_t(row_bytes / 16), rpt, seed,
                           static_cast<uint32_t*>(sink));
        after_launch("gather_read_kernel");
      };
      for (int i = 0; i < 2; ++i) launch(uint32_t(1000 + i));  // warm-up (fills the caches)
      CVS_HIP(hipEventRecord(e0, ctx->stream));
      for (int i = 0; i < reps; ++i) launch(uint32_t(i));
      CVS_HIP(hipEventRecord(e1, ctx->stream));
      CVS_HIP(hipEventSynchronize(e1));
      float ms = 0.f;
      CVS_HIP(hipEventElapsedTime(&ms, e0, e1));
      const double gathered = double(workgroups) * 16.0 * double(rpt) * double(row_bytes) * reps;
      *out_gbs = gathered / (double(ms) * 1e-3) / 1e9;
    } catch (...) {
      cleanup();
      throw;
    }
    cleanup();
  });
}


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
      CVS_HIP(hipMalloc(&ctx->bf_counters, 2 * sizeof(unsigned long long)));
      CVS_HIP(hipMemsetAsync(ctx->bf_counters, 0, 2 * sizeof(unsigned long long), ctx->stream));
      CVS_HIP(hipStreamSynchronize(ctx->stream));
    } catch (...) {
      if (ctx->bf_counters) (void)hipFree(ctx->bf_counters);
      if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
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
    if (ctx->bf_counters) (void)hipFree(ctx->bf_counters);
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
      // The pairs leave `pending` before any is read, so every event returns
      // to the pool exactly once.  A pair whose launch failed after it was
      // handed out was never recorded: its elapsed-time query fails, and the
      // pair is skipped instead of ending the loop.
      std::vector<std::pair<hipEvent_t, hipEvent_t>> pairs;
      pairs.swap(it->second.pending);
      for (auto& p : pairs) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, p.first, p.second) == hipSuccess) {
          sum += ms;
          ++cnt;
        }
        it->second.pool.push_back(p.first);
        it->second.pool.push_back(p.second);
      }
      (void)hipGetLastError();  // a skipped pair's error is not this call's
    }
    *total_ms = sum;
    *launches = cnt;
  });
}

int cvs_context_bf_escalations(cvs_context* ctx, uint64_t* escalated, uint64_t* rescanned, int reset) {
  return guarded([&] {
    bind(ctx);
    unsigned long long host[2] = {0, 0};
    CVS_HIP(hipMemcpyAsync(host, ctx->bf_counters, sizeof(host), hipMemcpyDeviceToHost, ctx->stream));
    if (reset) CVS_HIP(hipMemsetAsync(ctx->bf_counters, 0, sizeof(host), ctx->stream));
    CVS_HIP(hipStreamSynchronize(ctx->stream));
    if (escalated) *escalated = host[0];
    if (rescanned) *rescanned = host[1];
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
    uint32_t* stats = nullptr;
    try {
      const size_t row_bytes = size_t(n) * size_t(d) * sizeof(float);
      CVS_HIP(hipMalloc(&ds->rows, row_bytes));
      CVS_HIP(hipMalloc(&ds->tiles, size_t(ds->n_tiles) * size_t(ds->dp / kStepCols) * kStepBytes));
      // + kNormSlack: stage copies read whole 64-float windows past the last tile.
      CVS_HIP(hipMalloc(&ds->norms, (size_t(ds->n_tiles) * kTileRows + kNormSlack) * sizeof(float)));
      CVS_HIP(hipMalloc(&ds->mu, size_t(ds->dp) * sizeof(float)));
      CVS_HIP(hipMalloc(&stats, 4 * sizeof(uint32_t)));
      CVS_HIP(hipMemsetAsync(stats, 0, 4 * sizeof(uint32_t), ctx->stream));
      CVS_HIP(hipMemsetAsync(ds->norms, 0, (size_t(ds->n_tiles) * kTileRows + kNormSlack) * sizeof(float),
                             ctx->stream));
      CVS_HIP(hipMemcpyAsync(ds->rows, rows, row_bytes,
                             rows_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                             ctx->stream));
      ds->scale = centre_rows(ctx, ds->rows, n, d, ds->dp, ds->mu);
      launch_to_tiles(ctx, ds->rows, n, d, ds->dp, ds->n_tiles, ds->tiles, ds->norms, ds->mu, ds->scale, stats);
      uint32_t host[4] = {0, 0, 0, 0};
      CVS_HIP(hipMemcpyAsync(host, stats, sizeof(host), hipMemcpyDeviceToHost, ctx->stream));
      CVS_HIP(hipStreamSynchronize(ctx->stream));
      (void)hipFree(stats);
      stats = nullptr;
      float nmax, emax;
      std::memcpy(&nmax, &host[1], sizeof(float));
      std::memcpy(&emax, &host[2], sizeof(float));
      // Rounded up: the fp32 sums behind nmax and emax carry a relative error
      // below (d + 8) 2^-24; fl(x - mu) is within 2^-24 |x - mu| per element
      // of x - mu; an fp16 subnormal result is within 2^-25 absolute.
      const double rel = 1.0 + double(d + 8) * 0x1p-24;
      const double rmax = std::sqrt(double(nmax) * rel) * (1.0 + 0x1p-20);
      const double dx = std::sqrt(double(emax) * rel) * (1.0 + 0x1p-20) + rmax * 0x1p-23 +
                        std::sqrt(double(d)) * 0x1p-25;
      const bool finite = std::isfinite(nmax) && std::isfinite(emax);
      ds->cert_rmax = finite ? float(rmax * (1.0 + 0x1p-20)) : INFINITY;
      ds->cert_dx = finite ? float(dx * (1.0 + 0x1p-20)) : INFINITY;
    } catch (...) {
      if (stats) (void)hipFree(stats);
      if (ds->rows) (void)hipFree(ds->rows);
      if (ds->tiles) (void)hipFree(ds->tiles);
      if (ds->norms) (void)hipFree(ds->norms);
      if (ds->mu) (void)hipFree(ds->mu);
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
    (void)hipFree(ds->mu);
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
