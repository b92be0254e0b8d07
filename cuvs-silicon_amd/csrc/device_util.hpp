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

// Value of x held by lane (this lane ^ M) of the wave, without the LDS
// crossbar (ds_bpermute): lane ^ 1, 2, 3 within a quad are DPP quad
// permutes, lane ^ 15 and lane ^ 7 within a 16-lane row are the DPP row and
// half-row mirrors (so ^ 8 = row mirror then half-row mirror, ^ 4 = half-row
// mirror then quad permute ^ 3), and ^ 16 / ^ 32 are the gfx950 permlane
// swaps, which exchange the odd 16-lane rows (upper 32 lanes) of one operand
// with the even rows (lower 32 lanes) of the other: with both operands = x,
// a lane keeps the swapped copy that came from its partner.  Composite masks
// compose these steps.
namespace dpp {
constexpr int quad_xor(int v) { return (0 ^ v) | ((1 ^ v) << 2) | ((2 ^ v) << 4) | ((3 ^ v) << 6); }
constexpr int kRowMirror = 0x140;
constexpr int kHalfMirror = 0x141;
}  // namespace dpp

template <int M>
__device__ __forceinline__ uint32_t xor_lanes(uint32_t x) {
  static_assert(M > 0 && M < 64, "lane mask");
  typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
  const int lane = __lane_id();
  if constexpr ((M & 32) != 0) {
    const u32x2_t r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    x = (lane & 32) ? r.x : r.y;
  }
  if constexpr ((M & 16) != 0) {
    const u32x2_t r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    x = (lane & 16) ? r.x : r.y;
  }
  constexpr int L = M & 15;
  if constexpr (L == 15) {
    x = uint32_t(__builtin_amdgcn_mov_dpp(int(x), dpp::kRowMirror, 0xF, 0xF, false));
  } else if constexpr (L == 7) {
    x = uint32_t(__builtin_amdgcn_mov_dpp(int(x), dpp::kHalfMirror, 0xF, 0xF, false));
  } else {
    if constexpr ((L & 8) != 0) {
      x = uint32_t(__builtin_amdgcn_mov_dpp(int(x), dpp::kRowMirror, 0xF, 0xF, false));
      x = uint32_t(__builtin_amdgcn_mov_dpp(int(x), dpp::kHalfMirror, 0xF, 0xF, false));
    }
    if constexpr ((L & 4) != 0) {
      x = uint32_t(__builtin_amdgcn_mov_dpp(int(x), dpp::kHalfMirror, 0xF, 0xF, false));
      x = uint32_t(__builtin_amdgcn_mov_dpp(int(x), dpp::quad_xor(3), 0xF, 0xF, false));
    }
    if constexpr ((L & 3) != 0) x = uint32_t(__builtin_amdgcn_mov_dpp(int(x), dpp::quad_xor(L & 3), 0xF, 0xF, false));
  }
  return x;
}

// Runtime-mask form for the butterfly strides of unrolled loops (the switch
// folds to one case); other masks use ds_bpermute.
__device__ __forceinline__ uint32_t xor_lanes(uint32_t x, int mask) {
  switch (mask) {
    case 1: return xor_lanes<1>(x);
    case 2: return xor_lanes<2>(x);
    case 4: return xor_lanes<4>(x);
    case 8: return xor_lanes<8>(x);
    case 16: return xor_lanes<16>(x);
    case 32: return xor_lanes<32>(x);
    case 63: return xor_lanes<63>(x);
    default: return uint32_t(__shfl_xor(int(x), mask));
  }
}

__device__ __forceinline__ float xor_lanes_f(float x, int mask) {
  return __uint_as_float(xor_lanes(__float_as_uint(x), mask));
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t x, int mask) {
  const uint32_t lo = xor_lanes(uint32_t(x), mask);
  const uint32_t hi = xor_lanes(uint32_t(x >> 32), mask);
  return (uint64_t(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t shfl_u64(uint64_t x, int src_lane) {
  const uint32_t lo = uint32_t(__shfl(int(uint32_t(x)), src_lane));
  const uint32_t hi = uint32_t(__shfl(int(uint32_t(x >> 32)), src_lane));
  return (uint64_t(hi) << 32) | lo;
}

// Ascending bitonic sort of one 64-bit key per lane, within each group of S
// lanes (S = 64: the whole wave).
template <int S = 64>
__device__ __forceinline__ uint64_t wave_sort_lanes(uint64_t x) {
  const int lane = __lane_id();
#pragma unroll
  for (int size = 2; size <= S; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint64_t y = shfl_xor_u64(x, stride);
      const bool lower = (lane & stride) == 0;
      const bool asc = (lane & size) == 0;
      x = (lower == asc) ? (x < y ? x : y) : (x < y ? y : x);
    }
  }
  return x;
}

// Candidate keys (one per lane, `empty` for none) ahead of a merge into a
// sorted list whose last kept entry is `bound`: keys at or above it cannot
// enter the list (keys are unique) and become `empty`; the rest are sorted
// ascending into the first lanes, `empty` after them.  A few survivors are
// compacted through `scratch` (32 keys of LDS that only this wave uses here)
// and sorted over 16 or 32 lanes (10 or 15 steps instead of 21).  Returns
// the survivor count; with none the key is left unsorted and the merge can
// be skipped.
__device__ __forceinline__ int sort_below(uint64_t& key, uint64_t bound, uint64_t empty, uint64_t* scratch) {
  if (key >= bound) key = empty;
  const uint64_t m = __ballot(key != empty);
  const int cnt = popc(m);
  if (cnt == 0) return 0;
  if (cnt <= 32) {
    const int lane = __lane_id();
    if (key != empty) scratch[mbcnt(m)] = key;
    key = lane < cnt ? scratch[lane] : empty;
    key = cnt <= 16 ? wave_sort_lanes<16>(key) : wave_sort_lanes<32>(key);
  } else {
    key = wave_sort_lanes<64>(key);
  }
  return cnt;
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
  const uint64_t cr = shfl_xor_u64(c, 63);  // lane 63 - lane
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
