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

}  // namespace cvs
