// Definitions shared by the brute-force kernels of bf_search.hip (the
// streaming scan, sample, select, merge) and bf_gemm.hip (the register-
// blocked scan of large query batches): operand types, the candidate-list
// geometry and the list compaction, and the large-batch launcher.
#pragma once

#include <cstdint>

#include "cvs_internal.hpp"
#include "device_util.hpp"

namespace cvs {
namespace bf {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define CVS_INLINE __attribute__((always_inline))

constexpr uint64_t kSentinel = ~0ull;
// Buffer resource word 3 for raw (untyped) buffer access on gfx9-family
// targets, and the non-temporal cache policy for the streamed dataset.
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kAuxNT = 2;

enum { kModeScan = 0, kModeSample = 1 };

// List geometry per kp.  Each (workgroup, query) list is split into two
// halves, one per lane holding that query (lanes l and l + 32 see different
// rows of every tile), so each lane appends to its own half with a counter
// in a register and no atomics.  A lane adds at most one key between two
// fill checks; a half that fills up (HALF keys) rebalances the query's list
// to its kp smallest keys, kp/2 per half, so the slack HALF - kp/2 sets how
// many appends one compaction is amortized over.  Lists of kp <= 64 live in
// LDS (bounded by the 160 KiB budget next to the stage buffers); kp = 128
// lists (large k) live in global memory, one per (query, workgroup), since
// 128 queries x 192 keys exceed the LDS budget and appends are rare once the
// sampled threshold is in place.
template <int KP, int MODE>
struct Lists {
  static constexpr bool GL = MODE == 0 && KP > 64;  // lists in global memory
  static constexpr int HALF = MODE != 0 ? 1 : (KP == 16 ? 40 : (KP <= 64 ? 44 : 96));
  static constexpr int CAP = 2 * HALF;
  static constexpr int NS = (CAP + 63) / 64;  // list entries per lane in a compaction
  static_assert(MODE != 0 || HALF >= KP / 2 + 8, "list slack");
};

// Rewrites the two-half list of one query (c0 keys at list[0..), c1 keys at
// list[half..)) as its kp smallest keys, the first kp/2 in half 0 and the
// rest in half 1, and returns the order image of the kp-th smallest distance
// (0xffffffff when c0 + c1 <= kp: every key is kept and the threshold stays).
// All 64 lanes take part (list, c0 and c1 are wave-uniform); entry e lives in
// lane e % 64, slot e / 64.  Every entry is read before any is written.
template <int NS>
__device__ __forceinline__ uint32_t compact_query(uint64_t* list, int half, uint32_t c0, uint32_t c1,
                                                  int kp) {
  const int lane = __lane_id();
  const uint32_t cnt = c0 + c1;
  bool v[NS];
  uint64_t k[NS];
  uint32_t h[NS], l[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint32_t e = uint32_t(lane + 64 * s);
    v[s] = e < uint32_t(half) ? e < c0 : (e - uint32_t(half)) < c1;
    k[s] = v[s] ? list[e] : kSentinel;
    h[s] = uint32_t(k[s] >> 32);
    l[s] = uint32_t(k[s]);
  }
  uint32_t kth_hi = 0xffffffffu, kth_lo = 0xffffffffu;
  if (cnt > uint32_t(kp)) {
    int need = kp;
    uint32_t pre = 0;
    for (int b = 31; b >= 0; --b) {
      int c = 0;
#pragma unroll
      for (int s = 0; s < NS; ++s) c += popc(__ballot(v[s] && ((h[s] ^ pre) >> b) == 0));
      if (c < need) {
        need -= c;
        pre |= 1u << b;
      }
    }
    kth_hi = pre;
    int lt = 0, eq = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      lt += popc(__ballot(v[s] && h[s] < kth_hi));
      eq += popc(__ballot(v[s] && h[s] == kth_hi));
    }
    if (eq > kp - lt) {  // ties on the distance word: select on the row id
      int need2 = kp - lt;
      uint32_t pre2 = 0;
      for (int b = 31; b >= 0; --b) {
        int c = 0;
#pragma unroll
        for (int s = 0; s < NS; ++s) c += popc(__ballot(v[s] && h[s] == kth_hi && ((l[s] ^ pre2) >> b) == 0));
        if (c < need2) {
          need2 -= c;
          pre2 |= 1u << b;
        }
      }
      kth_lo = pre2;
    }
  }
  const int kh = kp / 2;
  int base = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool keep = v[s] && (h[s] < kth_hi || (h[s] == kth_hi && l[s] <= kth_lo));
    const uint64_t m = __ballot(keep);
    const int p = base + mbcnt(m);
    if (keep) list[p < kh ? p : half + (p - kh)] = k[s];
    base += popc(m);
  }
  return cnt > uint32_t(kp) ? kth_hi : 0xffffffffu;
}

// Arguments of the register-blocked large-batch scan (bf_gemm.hip).  The
// candidate lists and their minima have the streaming scan's global-list
// layout: part[q][list][Lists<128, kModeScan>::CAP], first kp valid.
struct GemmArgs {
  const u32x4* tiles;   // dataset tiles (unit-padded; n_tiles a multiple of 64)
  const float* norms;   // dataset norms, 32 per tile
  int64_t n_rt;         // 128-row blocks of the dataset (n_tiles / 4)
  int ks;               // k-steps per tile (padded dimension / 16)
  const u32x4* qtiles;  // query tiles
  const float* qnorms;  // query norms, 32 per query tile
  int nq;
  int n_qtiles;         // number of 32-query tiles
  const float* thr0;    // per-query initial threshold
  uint64_t* part;       // [nq][n_lists][CAP] lists
  uint64_t* lmin;       // [nq][n_lists] smallest key of each list
  float* lcut;          // [nq][n_lists] final threshold of each list (rows it covers and does
                        // not hold have keys at or above it; +inf for an unused list)
  int n_lists;          // lists per query
};

// Launch shape of the register-blocked scan: n_wg workgroups (a multiple of
// 8) and n_lists candidate lists per query.  ok is false when the call is
// not one it handles (kp = 128 lists, 8 to 64 k-steps per tile, buffer and
// stage-count limits).
struct GemmPlan {
  bool ok = false;
  int n_wg = 0;
  int n_lists = 0;
};
GemmPlan plan_gemm_scan(int ks, int kp, int64_t n_rt, int n_qtiles, int compute_units);
// Launches it on the context stream; e0 / e1 (may be null) record the
// dispatch's start and end.
void launch_gemm_scan(cvs_context* ctx, const GemmArgs& args, int n_wg, hipEvent_t e0, hipEvent_t e1);

}  // namespace bf
}  // namespace cvs
