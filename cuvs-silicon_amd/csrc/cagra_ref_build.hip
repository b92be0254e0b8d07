// The reference's own CAGRA graph build on gfx950 (cvs_cagra_build_reference).
//
// Restates MetalContext::build_knn_graph (src/metal_context.mm:289-914,
// called from src/cagra.cpp:47-59), so that a
// graph of the reference's algorithm can be built on the GPU and compared with
// this library's own build (cagra_build.hip):
//
//   N <= 50,000           exact all-pairs seeding (:324-349): the exact
//                         degree-G kNN graph, computed here with the fused
//                         brute-force search (queries = the rows).  The
//                         reference's 20 nn-descent iterations cannot change
//                         an exact graph and are not run.
//   50,000 < N <= 200,000 IVF k-means seeding (:351-435): K = clamp(sqrt N,
//                         G+1, 2000) centres from evenly strided rows, at most
//                         20 Lloyd iterations (stop when no row changes
//                         centre), each row's distance n_i - 2 x.c + n_c in
//                         fp32, the first centre winning ties, centres the
//                         row-order sum of their members times 1/count (an
//                         empty centre becomes zero);
//                         per-cluster exact seeding (:576-611, :712-792): each
//                         of the first (N/K)*4 + 64 members of a cluster takes
//                         its G nearest among the cluster's members and those
//                         of the 3 nearest centres' clusters (at most 8,192
//                         candidates), distance n_i - 2 x.y + n_y;
//                         random bucketing (:795-851): the reference's LCG
//                         permutation in buckets of 256, each row's
//                         min(G, 64) nearest bucket mates merged into its
//                         list;
//                         nn-descent (:853-911): 5 iterations over the
//                         2-hop neighbours (lists as at the start of the
//                         iteration), stopping early when no list changes.
//   N > 200,000           the same k-means and candidate lists, but the
//                         seeding ranks candidates by product-quantisation
//                         distance (:437-568, :614-681): 8 subspaces of 128
//                         dimensions, 256 centres each (k-means, at most 10
//                         iterations), distance = the sum over subspaces of
//                         the squared distance of the two rows' centres,
//                         computed here as the squared distance of the rows
//                         rebuilt from their codes; the kept entries then get
//                         exact distances (:683-709); random bucketing as
//                         above; no nn-descent (src/cagra.cpp:59).
//
// cvs_cagra_build_reference_ex takes the two size limits (50,000 and
// 200,000 in the reference) as arguments, so that the phases of a size
// class can also run at other sizes (tests).
//
// Differences, all deliberate: lists never hold an id twice (the reference's
// insert_neighbor does not check); an nn-descent iteration expands the
// node's neighbours as they were when the iteration began (the reference's
// kernel also follows neighbours its own loop inserted); fp32 sums run in
// this file's fixed orders (the reference's BLAS order is unspecified).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <numeric>
#include <vector>

#include "cvs_internal.hpp"
#include "device_util.hpp"

namespace cvs {
namespace {

constexpr uint32_t kNoId = 0xffffffffu;
constexpr uint64_t kNoKey = ~0ull;
constexpr int kTile = 64;      // rows x columns of a distance tile
constexpr int kChunk = 32;     // dimensions staged per step
constexpr int kMaxCand = 8192; // candidates per cluster (src/metal_context.mm:738-745)
constexpr int kMaxG = 64;      // graph degree supported (one key per lane)
constexpr int kHopHashBits = 13;

// Squared norms of the padded rows (one wave per row).
__global__ __launch_bounds__(256) void row_norms_kernel(const float* __restrict__ rows, int64_t n, int dp,
                                                        float* __restrict__ out) {
  const int64_t r = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= n) return;
  float acc = 0.f;
  for (int c = lane; c < dp; c += 64) {
    const float v = rows[r * dp + c];
    acc += v * v;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += xor_lanes_f(acc, o);
  if (lane == 0) out[r] = acc;
}

// Squared distance from two squared norms and a dot product, in one fixed
// rounding order (no contraction), so that every kernel whose keys meet in
// one list gives the same pair the same key and the lists' duplicate check
// (equal adjacent keys) sees it.
__device__ __forceinline__ float pair_dist(float na, float dot, float nb) {
  return __fadd_rn(__fsub_rn(na, __fmul_rn(2.f, dot)), nb);
}

// The fp32 dot products of a 64-row x 64-column tile: row i of A =
// a_rows[a_ids[i]] (i < na), column j = b_rows[b_ids[j]] (j < nb), staged 32
// dimensions at a time and transposed in LDS; thread (tr, tc) = (tid >> 4,
// tid & 15) accumulates rows 4 tr .. 4 tr + 3 by columns 4 tc .. 4 tc + 3,
// one fused multiply-add per product in dimension order.
__device__ __forceinline__ void dot_tile(const float* __restrict__ a_rows, const uint32_t* a_ids, int na,
                                         const float* __restrict__ b_rows, const uint32_t* b_ids, int nb, int dp,
                                         float (*sA)[kTile], float (*sB)[kTile], float (&acc)[4][4]) {
  const int tid = threadIdx.x;
  const int tr = tid >> 4, tc = tid & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
  // Loader: thread tid stages float4 number (tid & 7) of row (tid >> 3) and
  // of row (tid >> 3) + 32, for A and for B.
  const int lr = tid >> 3, lq = tid & 7;
  const float* ap0 = a_rows + int64_t(a_ids[lr < na ? lr : 0]) * dp + 4 * lq;
  const float* ap1 = a_rows + int64_t(a_ids[lr + 32 < na ? lr + 32 : 0]) * dp + 4 * lq;
  const float* bp0 = b_rows + int64_t(b_ids[lr < nb ? lr : 0]) * dp + 4 * lq;
  const float* bp1 = b_rows + int64_t(b_ids[lr + 32 < nb ? lr + 32 : 0]) * dp + 4 * lq;
  for (int c0 = 0; c0 < dp; c0 += kChunk) {
    const float4 a0 = *reinterpret_cast<const float4*>(ap0 + c0);
    const float4 a1 = *reinterpret_cast<const float4*>(ap1 + c0);
    const float4 b0 = *reinterpret_cast<const float4*>(bp0 + c0);
    const float4 b1 = *reinterpret_cast<const float4*>(bp1 + c0);
    __syncthreads();
    sA[4 * lq + 0][lr] = a0.x;
    sA[4 * lq + 1][lr] = a0.y;
    sA[4 * lq + 2][lr] = a0.z;
    sA[4 * lq + 3][lr] = a0.w;
    sA[4 * lq + 0][lr + 32] = a1.x;
    sA[4 * lq + 1][lr + 32] = a1.y;
    sA[4 * lq + 2][lr + 32] = a1.z;
    sA[4 * lq + 3][lr + 32] = a1.w;
    sB[4 * lq + 0][lr] = b0.x;
    sB[4 * lq + 1][lr] = b0.y;
    sB[4 * lq + 2][lr] = b0.z;
    sB[4 * lq + 3][lr] = b0.w;
    sB[4 * lq + 0][lr + 32] = b1.x;
    sB[4 * lq + 1][lr + 32] = b1.y;
    sB[4 * lq + 2][lr + 32] = b1.z;
    sB[4 * lq + 3][lr + 32] = b1.w;
    __syncthreads();
#pragma unroll 8
    for (int k = 0; k < kChunk; ++k) {
      const float4 av = *reinterpret_cast<const float4*>(&sA[k][4 * tr]);
      const float4 bv = *reinterpret_cast<const float4*>(&sB[k][4 * tc]);
      const float a4[4] = {av.x, av.y, av.z, av.w};
      const float b4[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a4[i], b4[j], acc[i][j]);
    }
  }
}

// Nearest centre per row (argmin over centres of n_i - 2 x.c + n_c, the
// lowest centre index winning ties) for 64 rows per workgroup; with
// all_out != null, instead every distance of the tile is written
// (all_out[i * n_cent + j], used for the centre-to-centre table).
__global__ __launch_bounds__(256) void nearest_centre_kernel(const float* __restrict__ rows,
                                                             const float* __restrict__ rnorm, int64_t n,
                                                             const float* __restrict__ cent,
                                                             const float* __restrict__ cnorm, int n_cent, int dp,
                                                             uint32_t* __restrict__ assign,
                                                             float* __restrict__ all_out) {
  __shared__ __attribute__((aligned(16))) float sA[kChunk][kTile];
  __shared__ __attribute__((aligned(16))) float sB[kChunk][kTile];
  __shared__ uint32_t s_aid[kTile], s_bid[kTile];
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const int64_t r0 = int64_t(blockIdx.x) * kTile;
  const int na = int(std::min<int64_t>(kTile, n - r0));
  if (tid < kTile) s_aid[tid] = uint32_t(r0 + (tid < na ? tid : 0));
  float best_d[4];
  uint32_t best_c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    best_d[i] = INFINITY;
    best_c[i] = kNoId;
  }
  for (int c0 = 0; c0 < n_cent; c0 += kTile) {
    const int nb = std::min(kTile, n_cent - c0);
    __syncthreads();
    if (tid < kTile) s_bid[tid] = uint32_t(c0 + (tid < nb ? tid : 0));
    __syncthreads();
    float acc[4][4];
    dot_tile(rows, s_aid, na, cent, s_bid, nb, dp, sA, sB, acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * tr + i;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = 4 * tc + j;
        if (r < na && c < nb) {
          const float dd = rnorm[r0 + r] - 2.f * acc[i][j] + cnorm[c0 + c];
          if (all_out) {
            all_out[(r0 + r) * n_cent + c0 + c] = dd;
          } else if (dd < best_d[i]) {  // columns ascend within the thread
            best_d[i] = dd;
            best_c[i] = uint32_t(c0 + c);
          }
        }
      }
    }
  }
  if (all_out) return;
  // Combine the 16 threads of each row group: smaller distance, then lower
  // centre index.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float dd = best_d[i];
    uint32_t cc = best_c[i];
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) {
      const float od = xor_lanes_f(dd, o);
      const uint32_t oc = xor_lanes(cc, o);
      if (od < dd || (od == dd && oc < cc)) {
        dd = od;
        cc = oc;
      }
    }
    const int r = 4 * tr + i;
    if (tc == 0 && r < na) assign[r0 + r] = cc;
  }
}

// Centre k = (row-order sum of its members) * (1 / count); zero when empty
// (src/metal_context.mm:421-434).
__global__ __launch_bounds__(256) void centre_sum_kernel(const float* __restrict__ rows, int dp,
                                                         const uint32_t* __restrict__ members,
                                                         const int64_t* __restrict__ starts,
                                                         float* __restrict__ cent) {
  const int k = blockIdx.x;
  const int64_t b = starts[k], e = starts[k + 1];
  for (int c = threadIdx.x; c < dp; c += blockDim.x) {
    float s = 0.f;
    for (int64_t i = b; i < e; ++i) s += rows[int64_t(members[i]) * dp + c];
    if (e > b) s *= 1.0f / float(e - b);
    cent[int64_t(k) * dp + c] = s;
  }
}

// The 3 (p) nearest other centres of each centre from the full table, by
// (distance, index) (src/metal_context.mm:583-611).  One thread per centre.
__global__ void nearest_other_kernel(const float* __restrict__ table, int n_cent, int p,
                                     uint32_t* __restrict__ out) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= n_cent) return;
  float bd[3] = {INFINITY, INFINITY, INFINITY};
  uint32_t bc[3] = {kNoId, kNoId, kNoId};
  for (int a = 0; a < n_cent; ++a) {
    if (a == k) continue;
    const float dd = table[int64_t(k) * n_cent + a];
    if (dd < bd[2]) {
      // Strict comparisons keep the lower index first among equal distances.
      if (dd < bd[0]) {
        bd[2] = bd[1]; bc[2] = bc[1];
        bd[1] = bd[0]; bc[1] = bc[0];
        bd[0] = dd; bc[0] = uint32_t(a);
      } else if (dd < bd[1]) {
        bd[2] = bd[1]; bc[2] = bc[1];
        bd[1] = dd; bc[1] = uint32_t(a);
      } else {
        bd[2] = dd; bc[2] = uint32_t(a);
      }
    }
  }
  for (int t = 0; t < p; ++t) out[int64_t(k) * p + t] = bc[t];
}

// Writes the sorted 64-key wave list v to dst[0..64) with adjacent copies of
// a key (the same id at the same distance) removed and only the first g kept,
// the rest kNoKey.
__device__ __forceinline__ void store_deduped(uint64_t v, int g, uint64_t* dst) {
  const int lane = __lane_id();
  const uint32_t lo = uint32_t(v), hi = uint32_t(v >> 32);
  const uint32_t plo = uint32_t(__shfl_up(int(lo), 1)), phi = uint32_t(__shfl_up(int(hi), 1));
  const uint64_t prev = (uint64_t(phi) << 32) | plo;
  const bool keep = v != kNoKey && (lane == 0 || v != prev);
  const uint64_t m = __ballot(keep);
  const int rank = mbcnt(m);
  const int kept = min(popc(m), g);
  if (keep && rank < g) dst[rank] = v;
  if (lane >= kept) dst[lane] = kNoKey;
}

// One group: rows own_ids[0..n_own) (n_own <= 64) against candidates
// cand[0..m): each row's list (keys ord(d) << 32 | id << 1, state[row * g
// ...], sorted, empty slots kNoKey) becomes the g nearest of (its list if
// merge_state, else nothing) and the candidates other than itself, distance
// n_i - 2 x.y + n_y.  Items: (offset of the group's candidates, m, offset of
// the rows within them, n_own).
struct GroupItem {
  int64_t cand_off;
  int m;
  int own_off;
  int n_own;
};

__global__ __launch_bounds__(256) void group_topk_kernel(const float* __restrict__ rows,
                                                         const float* __restrict__ rnorm, int dp,
                                                         const uint32_t* __restrict__ cand,
                                                         const GroupItem* __restrict__ items, int g,
                                                         int merge_state, uint64_t* __restrict__ state) {
  __shared__ __attribute__((aligned(16))) float sA[kChunk][kTile];
  __shared__ __attribute__((aligned(16))) float sB[kChunk][kTile];
  __shared__ uint32_t s_aid[kTile], s_bid[kTile];
  __shared__ uint64_t s_list[kTile][kTile];
  __shared__ float s_dist[kTile][kTile + 1];
  const GroupItem it = items[blockIdx.x];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tr = tid >> 4, tc = tid & 15;
  const uint32_t* cands = cand + it.cand_off;
  if (tid < kTile) s_aid[tid] = cands[it.own_off + (tid < it.n_own ? tid : 0)];
  __syncthreads();
  for (int r = wave; r < it.n_own; r += 4) {
    const uint64_t key = (merge_state && lane < g) ? state[int64_t(s_aid[r]) * g + lane] : kNoKey;
    s_list[r][lane] = key;
  }
  for (int c0 = 0; c0 < it.m; c0 += kTile) {
    const int nb = min(kTile, it.m - c0);
    __syncthreads();
    if (tid < kTile) s_bid[tid] = cands[c0 + (tid < nb ? tid : 0)];
    __syncthreads();
    float acc[4][4];
    dot_tile(rows, s_aid, it.n_own, rows, s_bid, nb, dp, sA, sB, acc);
    // Every (r, c) of the tile is written (ids past n_own or nb repeat a
    // valid one, and those entries are never read), so the norms' loads sit
    // under no branch and go out together: under the bounds test each pair
    // of loads was waited for before the next.
    float na[4], nbv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      na[i] = rnorm[s_aid[4 * tr + i]];
      nbv[i] = rnorm[s_bid[4 * tc + i]];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) s_dist[4 * tr + i][4 * tc + j] = pair_dist(na[i], acc[i][j], nbv[j]);
    __syncthreads();
    for (int r = wave; r < it.n_own; r += 4) {
      const uint64_t list = s_list[r][lane];
      const uint32_t cid = s_bid[lane];
      uint64_t key = kNoKey;
      if (lane < nb && cid != s_aid[r]) key = (uint64_t(ord_f32(s_dist[r][lane])) << 32) | (uint64_t(cid) << 1);
      // Only keys below the list's g-th entry can enter it.
      const uint64_t gth = shfl_u64(list, g - 1);
      if (__ballot(key < gth) == 0) continue;
      uint64_t v[1] = {key};
      wave_sort_e<1>(v);
      uint64_t l[1] = {list};
      wave_merge<1>(l, v[0]);
      store_deduped(l[0], g, &s_list[r][0]);
    }
  }
  __syncthreads();
  for (int r = wave; r < it.n_own; r += 4)
    if (lane < g) state[int64_t(s_aid[r]) * g + lane] = s_list[r][lane];
}

// One nn-descent iteration over 2-hop neighbours (src/metal_context.mm:
// 853-911, kernel shaders/cagra_kernels.metal:334-395): node u's list (state
// as at the start of the iteration, `prev`) takes the g nearest of itself
// and every neighbour of its neighbours other than u, distances summed over
// the padded row (float4 columns tp + 16 j per lane of each 16-lane team).
// One workgroup of 4 waves per node; wave 0 keeps the list; `changed`
// counts the nodes whose list changed.
__global__ __launch_bounds__(256) void two_hop_kernel(const float4* __restrict__ rows, int dq, int dv, uint32_t n,
                                                      int g, const uint64_t* __restrict__ prev,
                                                      uint64_t* __restrict__ next,
                                                      unsigned int* __restrict__ changed) {
  constexpr int H = 1 << kHopHashBits;
  constexpr int kMaxDv = 1024 / 64;
  __shared__ uint32_t s_hash[H];
  __shared__ uint32_t s_nbr[kMaxG];
  __shared__ uint32_t s_ids[64];
  __shared__ float s_dist[64];
  __shared__ uint64_t s_keys[32];
  __shared__ uint32_t s_ctl[2];
  const int tid = threadIdx.x, lane = tid & 63;
  const bool lead = __builtin_amdgcn_readfirstlane(tid >> 6) == 0;
  const int team = tid >> 4, tp = tid & 15;
  const uint32_t u = blockIdx.x;
  for (int i = tid; i < H; i += 256) s_hash[i] = kNoId;
  float4 qv[kMaxDv];
#pragma unroll
  for (int j = 0; j < kMaxDv; ++j)
    if (j < dv) qv[j] = rows[int64_t(u) * dq + tp + 16 * j];
  uint64_t list = kNoKey;
  __syncthreads();
  auto hash_insert = [&](uint32_t id) -> bool {
    uint32_t h = (id * 0x9E3779B1u) >> (32 - kHopHashBits);
    for (;;) {
      const uint32_t old = atomicCAS(&s_hash[h], kNoId, id);
      if (old == kNoId) return true;
      if (old == id) return false;
      h = (h + 1u) & uint32_t(H - 1);
    }
  };
  if (lead) {
    list = lane < g ? prev[int64_t(u) * g + lane] : kNoKey;
    const uint32_t id = list == kNoKey ? kNoId : uint32_t(list) >> 1;
    s_nbr[lane] = id;
    if (id != kNoId) hash_insert(id);
    if (lane == 0) hash_insert(u);
  }
  const uint64_t start_list = list;
  __syncthreads();
  int phase = 0;
  for (int j = 0; j < g; ++j) {
    const uint32_t nb = s_nbr[j];
    if (nb == kNoId) continue;
    uint32_t* const s_nf = s_ctl + phase;
    phase ^= 1;
    if (lead) {
      uint32_t id = kNoId;
      if (lane < g) {
        const uint64_t k2 = prev[int64_t(nb) * g + lane];
        if (k2 != kNoKey) id = uint32_t(k2) >> 1;
      }
      const bool fresh = id < n && hash_insert(id);
      const uint64_t m = __ballot(fresh);
      if (fresh) s_ids[mbcnt(m)] = id;
      if (lane == 0) *s_nf = uint32_t(popc(m));
    }
    __syncthreads();
    const int nf = int(*s_nf);
    if (nf == 0) continue;
    for (int r0 = 0; r0 < nf; r0 += 16) {
      const int r = r0 + team;
      const bool ok = r < nf;
      const float4* row = rows + int64_t(s_ids[ok ? r : 0]) * dq + tp;
      float4 x[kMaxDv];
#pragma unroll
      for (int jj = 0; jj < kMaxDv; ++jj)
        if (jj < dv) x[jj] = row[16 * jj];
      float acc = 0.f;
#pragma unroll
      for (int jj = 0; jj < kMaxDv; ++jj) {
        if (jj < dv) {
          const float dx = qv[jj].x - x[jj].x, dy = qv[jj].y - x[jj].y;
          const float dz = qv[jj].z - x[jj].z, dw = qv[jj].w - x[jj].w;
          acc += (dx * dx + dy * dy) + (dz * dz + dw * dw);
        }
      }
      acc += xor_lanes_f(acc, 8);
      acc += xor_lanes_f(acc, 4);
      acc += xor_lanes_f(acc, 2);
      acc += xor_lanes_f(acc, 1);
      if (ok && tp == 0) s_dist[r] = acc;
    }
    __syncthreads();
    if (lead) {
      // Candidates at or above the list's g-th key cannot enter it (ids
      // are unique here): no sort and merge when none is below it.
      uint64_t key = lane < nf ? (uint64_t(ord_f32(s_dist[lane])) << 32) | (uint64_t(s_ids[lane]) << 1) : kNoKey;
      const uint32_t glo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(list)), g - 1));
      const uint32_t ghi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(list >> 32)), g - 1));
      if (sort_below(key, (uint64_t(ghi) << 32) | glo, kNoKey, s_keys) > 0) {
        uint64_t l[1] = {list};
        wave_merge<1>(l, key);
        list = lane < g ? l[0] : kNoKey;
      }
    }
  }
  if (lead) {
    if (lane < g) next[int64_t(u) * g + lane] = list;
    const bool diff = __ballot(list != start_list) != 0;
    if (diff && lane == 0) atomicAdd(changed, 1u);
  }
}

// Product quantisation of the reference's N > 200,000 path
// (src/metal_context.mm:437-568): 8 subspaces of 128 dimensions, 256 centres
// each.  Rows rebuilt from their codes: dimensions 128 m .. 128 m + 127 of
// row i are centre codes[m][i] of subspace m, so the squared distance of two
// rebuilt rows is the reference's symmetric table sum
// sum_m |c_m(a) - c_m(b)|^2 (:552-566).  One workgroup per row.
constexpr int kPqM = 8, kPqDim = 128, kPqK = 256;

__global__ __launch_bounds__(256) void pq_decode_kernel(const uint32_t* __restrict__ codes,
                                                        const float* __restrict__ ctr, int64_t n,
                                                        float* __restrict__ out) {
  const int64_t i = blockIdx.x;
  const int t = threadIdx.x;  // float4 of the row
  const int m = t >> 5;       // 32 float4 per subspace
  const uint32_t c = codes[int64_t(m) * n + i];
  const float4 v = reinterpret_cast<const float4*>(ctr + (int64_t(m) * kPqK + c) * kPqDim)[t & 31];
  reinterpret_cast<float4*>(out + i * (kPqM * kPqDim))[t] = v;
}

// Exact squared L2 of every list entry (the reference's
// recompute_graph_distances after PQ seeding, src/metal_context.mm:683-709),
// then the list re-sorted by (distance, id).  One wave per row, lane e on
// entry e: the same arithmetic as group_topk_kernel (dimension-order fused
// multiply-adds, pair_dist), so a later bucketing merge that meets an entry
// again computes the same key and drops the copy.
__global__ __launch_bounds__(64) void rescore_keys_kernel(const float* __restrict__ rows,
                                                          const float* __restrict__ rnorm, int dp, int g,
                                                          uint64_t* __restrict__ keys) {
  const int64_t node = blockIdx.x;
  const int lane = threadIdx.x;
  uint64_t* lst = keys + node * g;
  const uint64_t key = lane < g ? lst[lane] : kNoKey;
  uint64_t nk = kNoKey;
  if (key != kNoKey) {
    const uint32_t j = uint32_t(key) >> 1;
    const float4* a = reinterpret_cast<const float4*>(rows + node * dp);
    const float4* b = reinterpret_cast<const float4*>(rows + int64_t(j) * dp);
    float acc = 0.f;
    for (int c = 0; c < dp / 4; ++c) {
      const float4 x = a[c], y = b[c];
      acc = __builtin_fmaf(x.x, y.x, acc);
      acc = __builtin_fmaf(x.y, y.y, acc);
      acc = __builtin_fmaf(x.z, y.z, acc);
      acc = __builtin_fmaf(x.w, y.w, acc);
    }
    nk = (uint64_t(ord_f32(pair_dist(rnorm[node], acc, rnorm[j]))) << 32) | uint32_t(key);
  }
  uint64_t v[1] = {nk};
  wave_sort_e<1>(v);
  if (lane < g) lst[lane] = v[0];
}

// keys -> ids (kNoId for empty slots).
__global__ void keys_to_ids_kernel(const uint64_t* __restrict__ keys, size_t count, uint32_t* __restrict__ ids) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < count) ids[i] = keys[i] == kNoKey ? kNoId : uint32_t(keys[i]) >> 1;
}

__global__ void gather_rows_kernel(const float* __restrict__ rows, int dp, const uint32_t* __restrict__ ids,
                                   int count, float* __restrict__ out) {
  const int r = blockIdx.x;
  if (r >= count) return;
  for (int c = threadIdx.x; c < dp; c += blockDim.x) out[int64_t(r) * dp + c] = rows[int64_t(ids[r]) * dp + c];
}

double seconds_since(std::chrono::steady_clock::time_point t) {
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t).count();
}

struct Mem {
  std::vector<void*> ptrs;
  template <typename T>
  T* alloc(size_t count) {
    void* p = nullptr;
    CVS_HIP(hipMalloc(&p, std::max<size_t>(count, 1) * sizeof(T)));
    ptrs.push_back(p);
    return static_cast<T*>(p);
  }
  ~Mem() {
    for (void* p : ptrs) (void)hipFree(p);
  }
};

void build_reference(cvs_context* ctx, const float* rows_in, int64_t n, int64_t d, int rows_on_device,
                     uint32_t graph_degree, int64_t exact_limit, int64_t pq_limit, uint32_t* out_graph,
                     int graph_on_device, cvs_ref_build_stats* stats) {
  const auto t_start = std::chrono::steady_clock::now();
  if (!rows_in || !out_graph) fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
  if (n <= 0 || d <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "dataset must be non-empty");
  if (d > 1024) fail(CVS_ERR_UNSUPPORTED, "dimension exceeds 1024");
  if (exact_limit < 0 || pq_limit < 0) fail(CVS_ERR_INVALID_ARGUMENT, "size limits must be non-negative");
  // Product-quantised seeding above pq_limit (the reference's N > 200,000
  // path) reads 8 subspaces of 128 dimensions of every row.
  const bool pq = n > exact_limit && n > pq_limit;
  if (pq && d != kPqM * kPqDim)
    fail(CVS_ERR_UNSUPPORTED, "product-quantised seeding (N above the PQ limit) needs d = 1024");
  const int g = int(std::min<int64_t>(graph_degree, n - 1));
  if (g > kMaxG) fail(CVS_ERR_UNSUPPORTED, "graph_degree exceeds 64 for the reference build");
  cvs_ref_build_stats st{};
  st.graph_degree = uint32_t(std::max(g, 0));
  hipStream_t s = ctx->stream;
  if (g == 0) {
    if (stats) *stats = st;
    return;
  }
  const int dp = int((d + 63) / 64 * 64);
  Mem mem;
  float* rows = mem.alloc<float>(size_t(n) * dp);
  float* rnorm = mem.alloc<float>(size_t(n));
  uint64_t* keys = mem.alloc<uint64_t>(size_t(n) * g);
  if (dp != d) CVS_HIP(hipMemsetAsync(rows, 0, size_t(n) * dp * sizeof(float), s));
  upload_rows(ctx, rows, dp, rows_in, n, d, rows_on_device);
  hipLaunchKernelGGL(row_norms_kernel, dim3(unsigned((n + 3) / 4)), dim3(256), 0, s, rows, n, dp, rnorm);
  after_launch("row_norms_kernel");
  CVS_HIP(hipMemsetAsync(keys, 0xff, size_t(n) * g * sizeof(uint64_t), s));

  if (n <= exact_limit) {
    // Exact seeding: the exact (g+1)-NN of every row by the fused brute-force
    // search, its own row dropped.
    const auto t_seed = std::chrono::steady_clock::now();
    cvs_dataset* ds = nullptr;
    if (cvs_dataset_create(ctx, rows_in, n, d, rows_on_device, &ds) != CVS_OK) fail(CVS_ERR_RUNTIME, cvs_last_error());
    const int k = g + 1;
    std::vector<uint32_t> nbr(static_cast<size_t>(n) * k);
    std::vector<float> dist(static_cast<size_t>(n) * k);
    const float* q_rows = rows_in;
    std::vector<float> host_rows;
    if (rows_on_device) {
      host_rows.resize(size_t(n) * d);
      CVS_HIP(hipMemcpy(host_rows.data(), rows_in, host_rows.size() * sizeof(float), hipMemcpyDeviceToHost));
      q_rows = host_rows.data();
    }
    const int rc = cvs_bf_search(ctx, ds, q_rows, n, k, nbr.data(), dist.data());
    (void)cvs_dataset_destroy(ds);
    if (rc != CVS_OK) fail(CVS_ERR_RUNTIME, cvs_last_error());
    std::vector<uint32_t> graph(static_cast<size_t>(n) * g, kNoId);
    for (int64_t i = 0; i < n; ++i) {
      int o = 0;
      for (int j = 0; j < k && o < g; ++j) {
        const uint32_t id = nbr[size_t(i) * k + j];
        if (id == uint32_t(i) || id == kNoId) continue;
        graph[size_t(i) * g + o++] = id;
      }
    }
    if (graph_on_device) {
      CVS_HIP(hipMemcpyAsync(out_graph, graph.data(), graph.size() * sizeof(uint32_t), hipMemcpyHostToDevice, s));
      CVS_HIP(hipStreamSynchronize(s));
    } else {
      std::copy(graph.begin(), graph.end(), out_graph);
    }
    st.seconds_seed = seconds_since(t_seed);
    st.seconds_total = seconds_since(t_start);
    if (stats) *stats = st;
    return;
  }

  // IVF k-means seeding.
  const auto t_km = std::chrono::steady_clock::now();
  int K = int(std::sqrt(double(n)));
  K = std::max(K, g + 1);
  K = std::min(K, 2000);
  st.clusters = uint32_t(K);
  float* cent = mem.alloc<float>(size_t(K) * dp);
  float* cnorm = mem.alloc<float>(size_t(K));
  uint32_t* assign_d = mem.alloc<uint32_t>(size_t(n));
  uint32_t* members_d = mem.alloc<uint32_t>(size_t(n));
  int64_t* starts_d = mem.alloc<int64_t>(size_t(K) + 1);
  {
    std::vector<uint32_t> init(static_cast<size_t>(K));
    const double stride = double(n) / double(K);
    for (int k = 0; k < K; ++k)
      init[size_t(k)] = uint32_t(std::min<int64_t>(int64_t(double(k) * stride + stride * 0.5), n - 1));
    uint32_t* init_d = mem.alloc<uint32_t>(size_t(K));
    CVS_HIP(hipMemcpyAsync(init_d, init.data(), size_t(K) * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(gather_rows_kernel, dim3(unsigned(K)), dim3(256), 0, s, rows, dp, init_d, K, cent);
    after_launch("gather_rows_kernel");
  }
  std::vector<uint32_t> assign(static_cast<size_t>(n), 0u), fresh(static_cast<size_t>(n));
  std::vector<uint32_t> members(static_cast<size_t>(n));
  std::vector<int64_t> starts(static_cast<size_t>(K) + 1);
  auto cluster_lists = [&](const std::vector<uint32_t>& a) {
    std::fill(starts.begin(), starts.end(), 0);
    for (int64_t i = 0; i < n; ++i) starts[size_t(a[size_t(i)]) + 1]++;
    for (int k = 0; k < K; ++k) starts[size_t(k) + 1] += starts[size_t(k)];
    std::vector<int64_t> fill(starts.begin(), starts.end() - 1);
    for (int64_t i = 0; i < n; ++i) members[size_t(fill[a[size_t(i)]]++)] = uint32_t(i);
  };
  int iters = 0;
  for (int iter = 0; iter < 20; ++iter) {
    hipLaunchKernelGGL(row_norms_kernel, dim3(unsigned((K + 3) / 4)), dim3(256), 0, s, cent, int64_t(K), dp, cnorm);
    after_launch("row_norms_kernel");
    hipLaunchKernelGGL(nearest_centre_kernel, dim3(unsigned((n + kTile - 1) / kTile)), dim3(256), 0, s, rows, rnorm,
                       n, cent, cnorm, K, dp, assign_d, static_cast<float*>(nullptr));
    after_launch("nearest_centre_kernel");
    CVS_HIP(hipMemcpyAsync(fresh.data(), assign_d, size_t(n) * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    CVS_HIP(hipStreamSynchronize(s));
    ++iters;
    const bool changed = iter == 0 || fresh != assign;
    assign.swap(fresh);
    if (!changed) break;
    cluster_lists(assign);
    CVS_HIP(hipMemcpyAsync(members_d, members.data(), size_t(n) * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    CVS_HIP(hipMemcpyAsync(starts_d, starts.data(), (size_t(K) + 1) * sizeof(int64_t), hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(centre_sum_kernel, dim3(unsigned(K)), dim3(256), 0, s, rows, dp, members_d, starts_d, cent);
    after_launch("centre_sum_kernel");
  }
  st.kmeans_iterations = uint32_t(iters);
  cluster_lists(assign);
  // Centre-to-centre table and the 3 nearest other centres.
  const int n_probe = std::min(K - 1, 3);
  std::vector<uint32_t> nearc(static_cast<size_t>(K) * std::max(n_probe, 1));
  {
    hipLaunchKernelGGL(row_norms_kernel, dim3(unsigned((K + 3) / 4)), dim3(256), 0, s, cent, int64_t(K), dp, cnorm);
    after_launch("row_norms_kernel");
    float* table = mem.alloc<float>(size_t(K) * K);
    hipLaunchKernelGGL(nearest_centre_kernel, dim3(unsigned((K + kTile - 1) / kTile)), dim3(256), 0, s, cent, cnorm,
                       int64_t(K), cent, cnorm, K, dp, static_cast<uint32_t*>(nullptr), table);
    after_launch("nearest_centre_kernel");
    uint32_t* nearc_d = mem.alloc<uint32_t>(nearc.size());
    if (n_probe > 0) {
      hipLaunchKernelGGL(nearest_other_kernel, dim3(unsigned((K + 255) / 256)), dim3(256), 0, s,
                         static_cast<const float*>(table), K, n_probe, nearc_d);
      after_launch("nearest_other_kernel");
      CVS_HIP(hipMemcpyAsync(nearc.data(), nearc_d, nearc.size() * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    }
    CVS_HIP(hipStreamSynchronize(s));
  }
  st.seconds_kmeans = seconds_since(t_km);

  // Product quantisation (N above the PQ limit, src/metal_context.mm:449-568):
  // per subspace m, k-means with 256 centres seeded by evenly strided rows,
  // at most 10 Lloyd iterations (stopping when no row changes centre), then
  // one more assignment pass as the codes; the rows rebuilt from their codes
  // then stand in for the rows in the per-cluster seeding, whose distances
  // are then the reference's symmetric PQ table sums.
  float* seed_rows = rows;
  float* seed_norm = rnorm;
  if (pq) {
    const auto t_pq = std::chrono::steady_clock::now();
    float* sub = mem.alloc<float>(size_t(n) * kPqDim);
    float* snorm = mem.alloc<float>(size_t(n));
    float* pq_ctr = mem.alloc<float>(size_t(kPqM) * kPqK * kPqDim);
    float* pcnorm = mem.alloc<float>(size_t(kPqK));
    uint32_t* codes = mem.alloc<uint32_t>(size_t(kPqM) * n);
    uint32_t* pinit_d = mem.alloc<uint32_t>(size_t(kPqK));
    uint32_t* pmembers_d = mem.alloc<uint32_t>(size_t(n));
    int64_t* pstarts_d = mem.alloc<int64_t>(size_t(kPqK) + 1);
    std::vector<uint32_t> pinit(static_cast<size_t>(kPqK));
    const double pstride = double(n) / double(kPqK);
    for (int c = 0; c < kPqK; ++c)
      pinit[size_t(c)] = uint32_t(std::min<int64_t>(int64_t(double(c) * pstride + pstride * 0.5), n - 1));
    CVS_HIP(hipMemcpyAsync(pinit_d, pinit.data(), size_t(kPqK) * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    std::vector<uint32_t> passign(static_cast<size_t>(n)), pfresh(static_cast<size_t>(n));
    std::vector<uint32_t> pmembers(static_cast<size_t>(n));
    std::vector<int64_t> pstarts(static_cast<size_t>(kPqK) + 1);
    auto assign_step = [&](float* ctr, uint32_t* out) {
      hipLaunchKernelGGL(row_norms_kernel, dim3(unsigned((kPqK + 3) / 4)), dim3(256), 0, s, ctr, int64_t(kPqK),
                         kPqDim, pcnorm);
      after_launch("row_norms_kernel");
      hipLaunchKernelGGL(nearest_centre_kernel, dim3(unsigned((n + kTile - 1) / kTile)), dim3(256), 0, s, sub, snorm,
                         n, ctr, pcnorm, kPqK, kPqDim, out, static_cast<float*>(nullptr));
      after_launch("nearest_centre_kernel");
    };
    for (int m = 0; m < kPqM; ++m) {
      float* ctr = pq_ctr + size_t(m) * kPqK * kPqDim;
      uint32_t* code_m = codes + size_t(m) * n;
      CVS_HIP(hipMemcpy2DAsync(sub, kPqDim * sizeof(float), rows + m * kPqDim, size_t(dp) * sizeof(float),
                               kPqDim * sizeof(float), size_t(n), hipMemcpyDeviceToDevice, s));
      hipLaunchKernelGGL(row_norms_kernel, dim3(unsigned((n + 3) / 4)), dim3(256), 0, s, sub, n, kPqDim, snorm);
      after_launch("row_norms_kernel");
      hipLaunchKernelGGL(gather_rows_kernel, dim3(unsigned(kPqK)), dim3(256), 0, s, sub, kPqDim, pinit_d, kPqK, ctr);
      after_launch("gather_rows_kernel");
      for (int iter = 0; iter < 10; ++iter) {
        assign_step(ctr, code_m);
        CVS_HIP(hipMemcpyAsync(pfresh.data(), code_m, size_t(n) * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
        CVS_HIP(hipStreamSynchronize(s));
        ++st.pq_iterations;
        const bool changed = iter == 0 || pfresh != passign;
        passign.swap(pfresh);
        if (!changed) break;
        // Centre sums in row order (src/metal_context.mm:507-517).
        std::fill(pstarts.begin(), pstarts.end(), 0);
        for (int64_t i = 0; i < n; ++i) pstarts[size_t(passign[size_t(i)]) + 1]++;
        for (int c = 0; c < kPqK; ++c) pstarts[size_t(c) + 1] += pstarts[size_t(c)];
        std::vector<int64_t> fill(pstarts.begin(), pstarts.end() - 1);
        for (int64_t i = 0; i < n; ++i) pmembers[size_t(fill[passign[size_t(i)]]++)] = uint32_t(i);
        CVS_HIP(hipMemcpyAsync(pmembers_d, pmembers.data(), size_t(n) * sizeof(uint32_t), hipMemcpyHostToDevice, s));
        CVS_HIP(hipMemcpyAsync(pstarts_d, pstarts.data(), (size_t(kPqK) + 1) * sizeof(int64_t),
                               hipMemcpyHostToDevice, s));
        hipLaunchKernelGGL(centre_sum_kernel, dim3(unsigned(kPqK)), dim3(256), 0, s, sub, kPqDim, pmembers_d,
                           pstarts_d, ctr);
        after_launch("centre_sum_kernel");
      }
      assign_step(ctr, code_m);  // the codes (:519-548)
    }
    seed_rows = mem.alloc<float>(size_t(n) * dp);
    seed_norm = mem.alloc<float>(size_t(n));
    hipLaunchKernelGGL(pq_decode_kernel, dim3(unsigned(n)), dim3(256), 0, s, static_cast<const uint32_t*>(codes),
                       static_cast<const float*>(pq_ctr), n, seed_rows);
    after_launch("pq_decode_kernel");
    hipLaunchKernelGGL(row_norms_kernel, dim3(unsigned((n + 3) / 4)), dim3(256), 0, s, seed_rows, n, dp, seed_norm);
    after_launch("row_norms_kernel");
    CVS_HIP(hipStreamSynchronize(s));
    st.seconds_pq = seconds_since(t_pq);
  }

  // Per-cluster seeding: groups of up to 64 own rows against the cluster's
  // candidate list; exact distances, or PQ distances (rebuilt rows) then
  // exact distances of the kept entries (src/metal_context.mm:683-709).
  const auto t_seed = std::chrono::steady_clock::now();
  {
    const int64_t max_own = (n / K) * 4 + 64;
    std::vector<uint32_t> cand;
    std::vector<GroupItem> items;
    cand.reserve(size_t(n) * 4);
    for (int k = 0; k < K; ++k) {
      const int64_t own_n = starts[size_t(k) + 1] - starts[size_t(k)];
      if (own_n == 0) continue;
      const int64_t nk = std::min(own_n, max_own);
      const int64_t off = int64_t(cand.size());
      int m = 0;
      for (int64_t i = 0; i < nk && m < kMaxCand; ++i, ++m) cand.push_back(members[size_t(starts[size_t(k)] + i)]);
      for (int t = 0; t < n_probe; ++t) {
        const uint32_t c = nearc[size_t(k) * n_probe + t];
        for (int64_t i = starts[c]; i < starts[size_t(c) + 1] && m < kMaxCand; ++i, ++m) cand.push_back(members[size_t(i)]);
      }
      if (m <= 1) continue;
      const int own_rows = int(std::min<int64_t>(nk, m));
      for (int b = 0; b < own_rows; b += kTile) items.push_back({off, m, b, std::min(kTile, own_rows - b)});
    }
    uint32_t* cand_d = mem.alloc<uint32_t>(cand.size());
    GroupItem* items_d = mem.alloc<GroupItem>(items.size());
    CVS_HIP(hipMemcpyAsync(cand_d, cand.data(), cand.size() * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    CVS_HIP(hipMemcpyAsync(items_d, items.data(), items.size() * sizeof(GroupItem), hipMemcpyHostToDevice, s));
    if (!items.empty()) {
      hipLaunchKernelGGL(group_topk_kernel, dim3(unsigned(items.size())), dim3(256), 0, s, seed_rows, seed_norm, dp,
                         static_cast<const uint32_t*>(cand_d), static_cast<const GroupItem*>(items_d), g, 0, keys);
      after_launch("group_topk_kernel");
    }
    if (pq) {
      hipLaunchKernelGGL(rescore_keys_kernel, dim3(unsigned(n)), dim3(64), 0, s, static_cast<const float*>(rows),
                         static_cast<const float*>(rnorm), dp, g, keys);
      after_launch("rescore_keys_kernel");
    }
    CVS_HIP(hipStreamSynchronize(s));
  }
  // Random bucketing: the reference's LCG permutation, buckets of 256, each
  // row's min(g, 64) nearest mates merged into its list.
  {
    std::vector<uint32_t> perm(static_cast<size_t>(n));
    std::iota(perm.begin(), perm.end(), 0u);
    uint64_t r = 0xFEDCBA9876543210ULL;
    for (int64_t i = n - 1; i > 0; --i) {
      r = r * 6364136223846793005ULL + 1442695040888963407ULL;
      const int64_t j = int64_t(r >> 33) % (i + 1);
      std::swap(perm[size_t(i)], perm[size_t(j)]);
    }
    std::vector<GroupItem> items;
    for (int64_t b = 0; b < n; b += 256) {
      const int m = int(std::min<int64_t>(256, n - b));
      for (int o = 0; o < m; o += kTile) items.push_back({b, m, o, std::min(kTile, m - o)});
    }
    uint32_t* perm_d = mem.alloc<uint32_t>(size_t(n));
    GroupItem* items_d = mem.alloc<GroupItem>(items.size());
    CVS_HIP(hipMemcpyAsync(perm_d, perm.data(), size_t(n) * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    CVS_HIP(hipMemcpyAsync(items_d, items.data(), items.size() * sizeof(GroupItem), hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(group_topk_kernel, dim3(unsigned(items.size())), dim3(256), 0, s, rows, rnorm, dp,
                       static_cast<const uint32_t*>(perm_d), static_cast<const GroupItem*>(items_d), g, 1, keys);
    after_launch("group_topk_kernel");
    CVS_HIP(hipStreamSynchronize(s));
  }
  st.seconds_seed = seconds_since(t_seed);

  // nn-descent over 2-hop neighbours: at most 5 iterations, none on the PQ
  // path (src/cagra.cpp:59).
  const auto t_nd = std::chrono::steady_clock::now();
  {
    uint64_t* other = mem.alloc<uint64_t>(size_t(n) * g);
    unsigned int* changed_d = mem.alloc<unsigned int>(1);
    uint64_t* cur = keys;
    const int nd_iters = pq ? 0 : 5;
    for (int iter = 0; iter < nd_iters; ++iter) {
      CVS_HIP(hipMemsetAsync(changed_d, 0, sizeof(unsigned int), s));
      hipLaunchKernelGGL(two_hop_kernel, dim3(unsigned(n)), dim3(256), 0, s, reinterpret_cast<const float4*>(rows),
                         dp / 4, dp / 64, uint32_t(n), g, static_cast<const uint64_t*>(cur), other, changed_d);
      after_launch("two_hop_kernel");
      unsigned int changed = 0;
      CVS_HIP(hipMemcpyAsync(&changed, changed_d, sizeof(unsigned int), hipMemcpyDeviceToHost, s));
      CVS_HIP(hipStreamSynchronize(s));
      std::swap(cur, other);
      ++st.descent_iterations;
      st.descent_changed_nodes = changed;
      if (changed == 0) break;
    }
    uint32_t* ids = graph_on_device ? out_graph : mem.alloc<uint32_t>(size_t(n) * g);
    const size_t count = size_t(n) * g;
    hipLaunchKernelGGL(keys_to_ids_kernel, dim3(unsigned((count + 255) / 256)), dim3(256), 0, s,
                       static_cast<const uint64_t*>(cur), count, ids);
    after_launch("keys_to_ids_kernel");
    if (!graph_on_device)
      CVS_HIP(hipMemcpyAsync(out_graph, ids, count * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    CVS_HIP(hipStreamSynchronize(s));
  }
  st.seconds_descent = seconds_since(t_nd);
  st.seconds_total = seconds_since(t_start);
  if (stats) *stats = st;
}

}  // namespace
}  // namespace cvs

using namespace cvs;

extern "C" int cvs_cagra_build_reference(cvs_context* ctx, const float* rows, int64_t n, int64_t d,
                                         int rows_on_device, uint32_t graph_degree, uint32_t* out_graph,
                                         int graph_on_device, cvs_ref_build_stats* stats) {
  return guarded([&] {
    bind(ctx);
    build_reference(ctx, rows, n, d, rows_on_device, graph_degree, 50000, 200000, out_graph, graph_on_device, stats);
  });
}

extern "C" int cvs_cagra_build_reference_ex(cvs_context* ctx, const float* rows, int64_t n, int64_t d,
                                            int rows_on_device, uint32_t graph_degree, int64_t exact_limit,
                                            int64_t pq_limit, uint32_t* out_graph, int graph_on_device,
                                            cvs_ref_build_stats* stats) {
  return guarded([&] {
    bind(ctx);
    build_reference(ctx, rows, n, d, rows_on_device, graph_degree, exact_limit, pq_limit, out_graph,
                    graph_on_device, stats);
  });
}
