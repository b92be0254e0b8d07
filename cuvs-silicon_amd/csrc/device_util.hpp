// Device helpers shared by the HIP kernels of libcvs_hip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cvs {

// Order-preserving map float -> uint32 (total order for non-NaN values;
// -0 and +0 map to the same key).
__device__ __forceinline__ uint32_t ord_f32(float f) {
  const uint32_t u = __float_as_uint(f + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float unord_f32(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

__device__ __forceinline__ int popc(uint64_t m) { return __builtin_popcountll(m); }

// Index of this lane among the set lanes of `mask` below it.
__device__ __forceinline__ int mbcnt(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(uint32_t(mask >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(mask), 0));
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t x, int mask) {
  const uint32_t lo = uint32_t(__shfl_xor(int(uint32_t(x)), mask));
  const uint32_t hi = uint32_t(__shfl_xor(int(uint32_t(x >> 32)), mask));
  return (uint64_t(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t shfl_u64(uint64_t x, int src_lane) {
  const uint32_t lo = uint32_t(__shfl(int(uint32_t(x)), src_lane));
  const uint32_t hi = uint32_t(__shfl(int(uint32_t(x >> 32)), src_lane));
  return (uint64_t(hi) << 32) | lo;
}

// Ascending wave-level bitonic sort of 64*E keys (position i = 64*slot + lane).
template <int E>
__device__ __forceinline__ void wave_sort_e(uint64_t (&v)[E]) {
  const int lane = __lane_id();
  constexpr int N = 64 * E;
#pragma unroll
  for (int size = 2; size <= N; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= 64) {
        const int s = stride / 64;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if ((e & s) == 0) {
            const bool asc = ((e * 64) & size) == 0;
            const uint64_t a = v[e], b = v[e + s];
            const bool sw = asc ? (b < a) : (a < b);
            v[e] = sw ? b : a;
            v[e + s] = sw ? a : b;
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const uint64_t y = shfl_xor_u64(v[e], stride);
          const bool lower = (lane & stride) == 0;
          const bool asc = ((e * 64 + lane) & size) == 0;
          v[e] = (lower == asc) ? (v[e] < y ? v[e] : y) : (v[e] < y ? y : v[e]);
        }
      }
    }
  }
}

// Merges 64 sorted keys (one per lane) into the sorted list v of 64*E keys.
template <int E>
__device__ __forceinline__ void wave_merge(uint64_t (&v)[E], uint64_t c) {
  const int lane = __lane_id();
  const uint64_t cr = shfl_u64(c, 63 - lane);
  v[E - 1] = v[E - 1] < cr ? v[E - 1] : cr;
#pragma unroll
  for (int s = E / 2; s >= 1; s >>= 1) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if ((e & s) == 0) {
        const uint64_t lo = v[e] < v[e + s] ? v[e] : v[e + s];
        const uint64_t hi = v[e] < v[e + s] ? v[e + s] : v[e];
        v[e] = lo;
        v[e + s] = hi;
      }
    }
  }
#pragma unroll
  for (int stride = 32; stride >= 1; stride >>= 1) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint64_t y = shfl_xor_u64(v[e], stride);
      const bool lower = (lane & stride) == 0;
      v[e] = lower ? (v[e] < y ? v[e] : y) : (v[e] < y ? y : v[e]);
    }
  }
}

}  // namespace cvs
