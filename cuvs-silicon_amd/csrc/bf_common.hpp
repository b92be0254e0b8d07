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

// ---------------------------------------------------------------------------
// Certificate of the fp16 selection.  A row's key is d~ = |q~|^2 + |x~|^2 -
// 2 q~.x~ in fp32, with q~, x~ the fp16 copies of s (q - mu), s (x - mu).  For
// the scaled exact distance D = s^2 |q - x|^2:
//   |d~ - |q~ - x~|^2| <= A = 2 (d + 16) 2^-24 (|q~| + rmax)^2
// (fp32 sums of d terms, including an MFMA accumulation that rounds twice
// per step, and the two final operations), and
//   | |q~ - x~| - sqrt(D) | <= E = |q~ - s(q - mu)| + dx
// (triangle inequality; dx bounds every row's rounding, measured when the
// dataset was made).  Hence D >= lb(d~) = (sqrt(d~ - A) - E)^2 when
// sqrt(d~ - A) > E, and 0 otherwise: a row whose key is at least T has an
// exact distance of at least lb(T) / s^2.
//
// The merge re-ranks the R smallest keys it holds exactly in fp32.  Every row
// not re-ranked has a key at or above T = min(key of the R-th candidate, the
// smallest final list threshold T*) (a list keeps every key of its range
// below its threshold).  If lb(T) exceeds s^2 d_k (1 + rho), with d_k the
// k-th exact distance and rho the relative error of the fp32 distances
// themselves, the result is the exact top k.  Otherwise the query
// escalates: every row with a key up to T_need = (sqrt(s^2 d_k (1 + rho)) +
// E)^2 + A (all of them are in the lists when T_need <= T*), or else every
// row of the dataset, is re-ranked exactly, and the top k of those is the
// answer.
// ---------------------------------------------------------------------------
struct Cert {
  float s2;              // scale^2: key units per squared distance unit
  float rmax;            // every row: |x~| <= rmax (scaled units)
  float dx;              // every row: |x~ - s (x - mu)| <= dx
  float a_coef;          // 2 (d + 16) 2^-24
  float rho;             // 2 (d + 8) 2^-24
  float qslack;          // sqrt(d) 2^-25 + fp32 error of a query's centring
  const float* qnorms;   // |q~|^2 per query
  const float* qerr;     // |q~ - s fl(q - mu)|^2 per query
  unsigned long long* counters;  // [0] escalated queries, [1] of them re-ranked over every row
};

enum { kCertPass = 0, kCertKeys = 1, kCertAll = 2 };

// Exact squared L2 distances of U rows to the query by the 64 lanes of the
// calling wave (ids >= n count as none and give 0).  The summation order is
// fixed: per lane, float4 partial sums over its 4-column pieces of 256-column
// chunks, then a butterfly, so a row always gets the same value.  All row
// loads of a 1024-column pass are issued before the first is used.
template <int U>
__device__ __forceinline__ void wave_exact(const uint32_t (&id)[U], const float* __restrict__ rows, int64_t n,
                                           int64_t d, const float* __restrict__ qv, bool vec, float (&out)[U]) {
  const int lane = threadIdx.x & 63;
  float acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) acc[u] = 0.f;
  if (vec) {
    for (int64_t i0 = int64_t(lane) * 4; i0 < d; i0 += 4 * 256) {
      float4 a4[4], b4[4][U];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int64_t i = i0 + c * 256;
        a4[c] = i < d ? *reinterpret_cast<const float4*>(qv + i) : float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < U; ++u)
          b4[c][u] = (i < d && int64_t(id[u]) < n) ? *reinterpret_cast<const float4*>(rows + int64_t(id[u]) * d + i)
                                                   : float4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float t0 = a4[c].x - b4[c][u].x, t1 = a4[c].y - b4[c][u].y;
          const float t2 = a4[c].z - b4[c][u].z, t3 = a4[c].w - b4[c][u].w;
          acc[u] += (t0 * t0 + t1 * t1) + (t2 * t2 + t3 * t3);
        }
    }
  } else {
    for (int64_t i = lane; i < d; i += 64) {
      const float a1 = qv[i];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (int64_t(id[u]) >= n) continue;
        const float t = a1 - rows[int64_t(id[u]) * d + i];
        acc[u] += t * t;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc[u] += xor_lanes_f(acc[u], o);
    out[u] = acc[u];
  }
}

constexpr int kExactU = 8;  // rows per wave and pass of the exact distances

// Exact keys ord(d) << 32 | id of the ids s_id[0..cnt) (a wave's own list),
// into s_key[0..cnt), by the calling wave.
__device__ __forceinline__ void wave_exact_keys(const uint32_t* s_id, int cnt, uint64_t* s_key, const float* rows,
                                                int64_t n, int64_t d, const float* qv, bool vec) {
  const int lane = threadIdx.x & 63;
  for (int c = 0; c < cnt; c += kExactU) {
    uint32_t id[kExactU];
#pragma unroll
    for (int u = 0; u < kExactU; ++u) id[u] = c + u < cnt ? s_id[c + u] : 0xffffffffu;
    float dd[kExactU];
    wave_exact<kExactU>(id, rows, n, d, qv, vec, dd);
#pragma unroll
    for (int u = 0; u < kExactU; ++u)
      if (lane == u && c + u < cnt) s_key[c + u] = (uint64_t(ord_f32(dd[u])) << 32) | id[u];
  }
}

// Certificate constants of a search over `ds` (defined in bf_search.hip).
Cert make_cert(cvs_context* ctx, const cvs_dataset* ds, const float* qnorms, const float* qerr);

// Converts q queries (device, q x d fp32) into q_rows / 32 query tiles of
// the dataset's layout and centring, their norms (q_rows, +inf past q) and
// squared rounding errors (q), on the context stream (bf_search.hip).
void launch_query_tiles(cvs_context* ctx, const cvs_dataset* ds, const float* queries, int64_t q, int64_t q_rows,
                        u32x4* qtiles, float* qnorms, float* qerr, hipEvent_t e0, hipEvent_t e1);

// Exact k-NN outside the fused scan's limits (d > 1024 or k > 112): fp16
// MFMA keys of a query chunk against every row, listed below a sampled
// per-query threshold (a radix select over the full key matrix where the list
// does not serve), and the certified exact re-rank (bf_wide.hip).  Device
// pointers, context stream.
void bf_wide_search(cvs_context* ctx, const cvs_dataset* ds, const float* queries, int64_t q, int64_t k,
                    uint32_t* nbr, float* dist);
constexpr int64_t kFusedMaxDim = 1024;  // the fused scan holds a query tile's operands for d <= 1024
constexpr int64_t kFusedMaxK = 112;     // and keeps up to 128 candidates per query

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
