// CAGRA graph build for gfx950: random bucketing -> nn-descent -> pruning.
//
// Replaces the reference's build_knn_graph (src/metal_context.mm:289-914):
// CPU IVF k-means + per-cluster BLAS seeding, a `random_bucketing` kernel
// (shaders/cagra_kernels.metal:403-462) and a racy `nn_descent` kernel
// (:334-395) that recomputes full 2-hop distance sets per node.  Here every
// phase runs on the GPU and no update is lost to a race:
//
//  1. convert   fp32 rows -> fp16 rows of scale * (row - mean) (row stride dp
//               = d rounded up to 128) + fp32 squared norms of the
//               fp16-rounded rows.
//  2. bucket    rows are split into buckets of 256 consecutive entries of a
//               random permutation (the reference's LCG Fisher-Yates,
//               src/metal_context.mm:802-810).  One workgroup per bucket forms
//               the 256 x 256 Gram matrix on v_mfma_f32_32x32x16_f16 (fp32
//               accumulate) over LDS-staged 64-dimension chunks and gives each
//               row the `kd` nearest of its 255 bucket mates: the initial
//               degree-kd ("intermediate degree") list.  Three more rounds with
//               fresh permutations merge each row's 32 nearest mates of another
//               bucket into its list, so that lists span several buckets
//               before the first local join.
//  3. nn-descent, per iteration:
//     sample    per node, up to 32 "new" (never joined) and 32 "old"
//               neighbours; new ones are marked old.  Each sampled edge
//               u -> v also appends u to v's reverse new/old list (32 each).
//     join      per node, its sampled forward + reverse neighbours (at most
//               128 rows) are gathered into LDS chunk by chunk and their
//               128 x 128 Gram matrix is formed on MFMA: the local join.  For
//               every member, the 8 best partners (at least one of the pair
//               new) that beat the member's current worst neighbour are
//               appended to the member's update bin (128 slots).
//     apply     per node, the bin is deduplicated, filtered against the
//               list, sorted and merged into the sorted list (wave bitonic
//               merge); inserted entries are marked new and counted.
//     The loop stops after max_iterations or when the number of insertions
//     falls below termination_threshold * n * kd.
//  4. graph     by default CAGRA's rank-based detour count (Ootomo et al.,
//               2023): an edge u -> v_j (rank j) is detourable via v_i if
//               rank max(i, rank of v_j in v_i's list) < j.  Each node keeps
//               the g edges of fewest detours (ties by rank), in rank order.
//               Options: the first g list entries (the plain k-NN graph), or
//               the kept edges merged with r reverse edges (the closest g - r
//               kept edges, then up to r reverse edges, then the remaining
//               kept edges; CAGRA's graph has r = g/2).  On clustered N=1M
//               D=1024 rows reverse edges cost recall at small search beams
//               (itopk 64: 0.705 with r = 32 against 0.806 without).
//
// Lists are sorted 64-bit keys ord(distance) << 32 | id << 1 | new, so the
// order is (distance, id) and the new flag never reorders a list.  Distances
// in the build are fp16-input expanded-form estimates of the centred, scaled
// rows (scale^2 times the squared distance, up to rounding); they only rank
// candidates (the search computes exact fp32 distances).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <numeric>
#include <type_traits>
#include <vector>

#include <hipcub/hipcub.hpp>

#include "cvs_internal.hpp"
#include "device_util.hpp"

namespace cvs {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint64_t kEmpty = ~0ull;
constexpr uint32_t kInvalid = 0xffffffffu;
constexpr uint32_t kBinTag = 0x80000000u;  // apply's hash: an id from the bin (ids < 2^31)
// Bytes of each member row staged per step (64 fp16 dimensions); a staged
// row is padded by 16 bytes against LDS bank conflicts.  Larger join chunks
// (256 and 512 bytes per row per step) measured slower at N=1M D=1024: their
// registers and LDS cost occupancy, which the join needs more.
constexpr int kBucketChunkBytes = 128;
constexpr int kBucketDepth = 1;    // bucket Gram: chunks gathered ahead
constexpr int kJoinChunkBytes = 128;
constexpr int kRowAlignDims = 128;  // fp16 row stride: d rounded up to this
constexpr int kSample = 32;       // sampled forward/reverse new/old neighbours
constexpr int kJoinM = 4 * kSample;
constexpr int kBin = 128;         // update bin capacity per node
constexpr int kStatGroups = 256;  // workgroups of the per-iteration statistics reduction
// Locality order of the local join (see label_round_kernel): labels spread
// over each node's first kLabelK list entries for kLabelRounds rounds, once
// the lists of iteration kOrderAfter are in place.
constexpr int kLabelK = 16;
constexpr int kLabelRounds = 3;
constexpr int kOrderAfter = 0;
constexpr int kEmit = 8;          // partners emitted per member and join
constexpr int kBucket = 256;
constexpr int kBucketRounds = 4;   // random bucketings merged into the initial lists
constexpr int kBucketEmit = 32;    // mates per row merged by the rounds after the first
constexpr int kMaxKd = 256;       // intermediate degree limit (4 keys per lane)

__device__ __forceinline__ uint32_t key_id(uint64_t k) { return uint32_t(k) >> 1; }

// ---------------------------------------------------------------------------
// Gram tiles of a set of fp16 rows.  The member rows s_ids[0..m) (m <= M)
// are staged 64 dimensions at a time (M x 128 B, rows 144 B apart) and each
// wave accumulates NT 32x32 tiles: tile t = rows 32*rt[t].., columns
// 32*ct[t]..  Loads run DEPTH chunks ahead of the multiply.
//
// The gathers have no per-row branches: staging rows >= m re-read member 0's
// row (a valid address, a cache hit; their products are never used) and the
// prefetch past the last chunk re-reads the last chunk.  A branch around a
// load makes the compiler wait for every outstanding load where the branch
// rejoins, which would leave one chunk in flight whatever DEPTH is.
// ---------------------------------------------------------------------------
template <int M, int NT, int DEPTH, int CB>
__device__ __forceinline__ void gram_tiles(const char* __restrict__ x16, int64_t row_bytes, int m,
                                           const uint32_t* s_ids, char* s_stage, const int (&rt)[NT],
                                           const int (&ct)[NT], f32x16 (&acc)[NT]) {
  constexpr int SEG = CB / 16;        // 16-byte segments per staged row
  constexpr int STRIDE = CB + 16;     // staged row pitch
  constexpr int LPT = M * SEG / 256;  // 16-byte loads per thread and chunk
  static_assert(LPT * 256 == M * SEG, "staging split");
  const int n_chunks = int(row_bytes / CB);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const char* src[LPT];
  int dst[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int idx = tid + 256 * i;
    const int r = idx / SEG, seg = idx % SEG;
    src[i] = x16 + int64_t(s_ids[r < m ? r : 0]) * row_bytes + seg * 16;
    dst[i] = r * STRIDE + seg * 16;
  }
  bool tile_live[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    tile_live[t] = 32 * rt[t] < m && 32 * ct[t] < m;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[t][e] = 0.f;
  }
  const int last = n_chunks - 1;
  // Prologue loads in chunk order (the scheduler may not interleave them), so
  // that the loop's first use of chunk c waits only for the loads up to it.
  u32x4 reg[DEPTH][LPT];
#pragma unroll
  for (int c = 0; c < DEPTH; ++c) {
#pragma unroll
    for (int i = 0; i < LPT; ++i)
      reg[c][i] = *reinterpret_cast<const u32x4*>(src[i] + int64_t(min(c, last)) * CB);
    __builtin_amdgcn_sched_barrier(0);
  }
  // One chunk: stage it, prefetch chunk c + DEPTH into the freed registers,
  // multiply.
  auto step = [&](int c, u32x4(&r)[LPT]) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < LPT; ++i) *reinterpret_cast<u32x4*>(s_stage + dst[i]) = r[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < LPT; ++i)
      r[i] = *reinterpret_cast<const u32x4*>(src[i] + int64_t(min(c + DEPTH, last)) * CB);
#pragma unroll
    for (int s = 0; s < CB / 32; ++s) {
      const int koff = s * 32 + 16 * (lane >> 5);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (!tile_live[t]) continue;
        const half8 a = *reinterpret_cast<const half8*>(s_stage + (32 * rt[t] + (lane & 31)) * STRIDE + koff);
        const half8 b = *reinterpret_cast<const half8*>(s_stage + (32 * ct[t] + (lane & 31)) * STRIDE + koff);
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[t], 0, 0, 0);
      }
    }
  };
  // Whole groups of DEPTH chunks first: a loop body without early exits
  // reaches its back edge with the loads in chunk order, so each stage waits
  // only for its own chunk.  Then the remaining n_chunks % DEPTH chunks.
  int c0 = 0;
  for (; c0 + DEPTH <= n_chunks; c0 += DEPTH) {
#pragma unroll
    for (int cc = 0; cc < DEPTH; ++cc) step(c0 + cc, reg[cc]);
  }
#pragma unroll
  for (int cc = 0; cc + 1 < DEPTH; ++cc)
    if (c0 + cc < n_chunks) step(c0 + cc, reg[cc]);
}

// Gram columns of the local join: rows s_ids[0..m), 32 < m <= 32*R (or
// m <= 32 with R = 1), staged CB bytes per row and step.  The calling wave
// computes column tile `wave` against row tiles (row0 + t) % R, t < T, into
// acc[0..T) (T = 0: it only stages).  Every wave of the workgroup runs the same chunk
// steps and barriers whatever its T, so waves may run different T.  All tile
// guards are resolved by the template, so each k-step's LDS operand reads
// (one B tile, T A tiles) sit in one basic block with its T MFMAs and can be
// issued ahead of them.
// after_issue() runs once the first NS chunks' gathers are issued: loads it
// makes and waits for overlap them, and registers it holds are free again
// before the Gram loop.
constexpr int kJoinAcc = 3;  // accumulator tiles of a join wave (the most row tiles a role multiplies)

template <int R, int T, int CB, class AfterIssue>
__device__ __forceinline__ void gram_join(const char* __restrict__ x16, int64_t row_bytes, int m,
                                          const uint32_t* s_ids, char* s_stage, int wave, int row0,
                                          f32x16 (&acc)[kJoinAcc], AfterIssue&& after_issue) {
  static_assert(T <= kJoinAcc, "accumulator tiles");
  static_assert(T >= 0 && T <= R, "row tiles");
  constexpr int M = 32 * R;
  constexpr int SEG = CB / 16;
  constexpr int STRIDE = CB + 16;
  constexpr int LPT = M * SEG / 256;
  static_assert(LPT * 256 == M * SEG, "staging split");
  const int n_chunks = int(row_bytes / CB);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const char* src[LPT];
  int dst[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int idx = tid + 256 * i;
    const int r = idx / SEG, seg = idx % SEG;
    src[i] = x16 + int64_t(s_ids[r < m ? r : 0]) * row_bytes + seg * 16;
    dst[i] = r * STRIDE + seg * 16;
  }
#pragma unroll
  for (int t = 0; t < kJoinAcc; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[t][e] = 0.f;
  const int last = n_chunks - 1;
  const char* a_base = s_stage + (lane & 31) * STRIDE + 16 * (lane >> 5);
  const char* b_base = a_base + 32 * wave * STRIDE;
  const char* a_tile[T > 0 ? T : 1];
#pragma unroll
  for (int t = 0; t < T; ++t) a_tile[t] = a_base + 32 * ((row0 + t) % R) * STRIDE;
  // NS register sets: chunk c + NS is gathered while chunk c is multiplied,
  // so each gather has NS chunks of work to arrive in (four for the small
  // neighbourhoods that dominate once the lists settle, three for the
  // largest, whose staging registers with the accumulators bound the
  // kernel's occupancy).
  constexpr int NS = R <= 2 ? 4 : 3;
  u32x4 reg[NS][LPT];
#pragma unroll
  for (int k = 0; k < NS; ++k)
#pragma unroll
    for (int i = 0; i < LPT; ++i) reg[k][i] = *reinterpret_cast<const u32x4*>(src[i] + int64_t(min(k, last)) * CB);
  __builtin_amdgcn_sched_barrier(0);
  after_issue();
  __builtin_amdgcn_sched_barrier(0);
  auto step = [&](u32x4 (&rg)[LPT], int c) __attribute__((always_inline)) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < LPT; ++i) *reinterpret_cast<u32x4*>(s_stage + dst[i]) = rg[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < LPT; ++i)
      rg[i] = *reinterpret_cast<const u32x4*>(src[i] + int64_t(min(c + NS, last)) * CB);
    if constexpr (T > 0) {
#pragma unroll
      for (int s = 0; s < CB / 32; ++s) {
        const half8 b = *reinterpret_cast<const half8*>(b_base + s * 32);
        half8 av[T];
#pragma unroll
        for (int t = 0; t < T; ++t) av[t] = *reinterpret_cast<const half8*>(a_tile[t] + s * 32);
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[t], b, acc[t], 0, 0, 0);
      }
    }
  };
  int c = 0;
  for (; c + NS <= n_chunks; c += NS) {
#pragma unroll
    for (int k = 0; k < NS; ++k) step(reg[k], c + k);
  }
#pragma unroll
  for (int k = 0; k < NS; ++k)
    if (c + k < n_chunks) step(reg[k], c + k);
}

// fp32 rows -> fp16 rows of scale * (row - mu) (stride dp) + squared norms of
// the fp16-rounded rows.  Centring (mu: the column means) keeps the fp16
// rounding proportional to the rows' spread instead of their offset from the
// origin; every distance the build compares is between rows, so the shift
// and the power-of-two scale change no ranking.  One wave per row.
__global__ __launch_bounds__(256) void to_half_rows_kernel(const float* __restrict__ rows, int64_t n, int64_t d,
                                                           int64_t dp, const float* __restrict__ mu, float scale,
                                                           _Float16* __restrict__ out, float* __restrict__ norms) {
  const int64_t r = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= n) return;
  const float* src = rows + r * d;
  _Float16* dst = out + r * dp;
  float acc = 0.f;
  for (int64_t c = lane; c < dp; c += 64) {
    const _Float16 h = static_cast<_Float16>(c < d ? (src[c] - mu[c]) * scale : 0.f);
    dst[c] = h;
    const float hv = static_cast<float>(h);
    acc += hv * hv;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += xor_lanes_f(acc, o);
  if (lane == 0) norms[r] = acc;
}

struct BuildArgs {
  const char* x16;       // n x dp fp16
  const float* norms;    // n
  int64_t row_bytes;     // dp * 2
  uint32_t n;
  int kd;                // list length (intermediate degree, <= n - 1)
  int kp;                // list stride (kd rounded up to 64)
  uint64_t* lists;       // n x kp keys
  uint32_t* fwd;         // n x 2*kSample: new ids, then old ids
  uint32_t* fwd_cnt;     // n x 2
  uint32_t* rev;         // n x 2*kSample
  uint32_t* rev_cnt;     // n x 2
  uint64_t* bins;        // n x kBin
  uint32_t* bin_cnt;     // n
  // Per-node work statistics of the current iteration, written with plain
  // stores (global atomics on a few shared counters, hit by every workgroup
  // from every XCD, cost the join 4%): [0] join members, [1] updates emitted
  // (join), [2] insertions, [3] bin entries kept (apply).
  uint4* stats;
  // Node of each join workgroup (workgroup i joins node order[i]), or null
  // for node i.
  const uint32_t* order;
};

// One workgroup per bucket of up to 256 permuted rows.  First round
// (to_bins = 0): each row's list becomes its kd nearest bucket mates.  Later
// rounds (to_bins = 1): each row's kBucketEmit nearest mates go to its
// update bin, for the apply kernel to merge into the list.  The Gram matrix
// is formed 64 rows at a time and its distances sorted 32 rows at a time, so
// that two workgroups fit a CU's LDS.
__global__ __launch_bounds__(256) void bucket_kernel(BuildArgs a, const uint32_t* __restrict__ perm, int to_bins) {
  __shared__ __attribute__((aligned(16))) char s_stage[kBucket * (kBucketChunkBytes + 16)];
  __shared__ float s_dist[32 * 257];  // one 32-row block of the bucket's distances
  __shared__ uint32_t s_ids[kBucket];
  __shared__ float s_norm[kBucket];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t start = int64_t(blockIdx.x) * kBucket;
  const int mb = int(std::min<int64_t>(kBucket, int64_t(a.n) - start));
  {
    const uint32_t id = perm[start + (tid < mb ? tid : 0)];
    s_ids[tid] = id;
    s_norm[tid] = a.norms[id];
  }
  __syncthreads();
  for (int rb = 0; rb < 4; ++rb) {
    if (64 * rb >= mb) break;
    const int rt[4] = {2 * rb, 2 * rb, 2 * rb + 1, 2 * rb + 1};
    const int ct[4] = {2 * wave, 2 * wave + 1, 2 * wave, 2 * wave + 1};
    f32x16 acc[4];
    gram_tiles<kBucket, 4, kBucketDepth, kBucketChunkBytes>(a.x16, a.row_bytes, mb, s_ids, s_stage, rt, ct, acc);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
    const int r0 = 64 * rb + 32 * h;  // first row of this half
    if (r0 >= mb) break;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (rt[t] != 2 * rb + h) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = 32 * rt[t] + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int col = 32 * ct[t] + (lane & 31);
        s_dist[(row - r0) * 257 + col] = s_norm[row] + s_norm[col] - 2.0f * acc[t][e];
      }
    }
    __syncthreads();
    for (int i = 0; i < 8; ++i) {
      const int row = r0 + 8 * wave + i;
      if (row >= mb) break;
      uint64_t v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = e * 64 + lane;
        v[e] = (c < mb && c != row)
                   ? (uint64_t(ord_f32(s_dist[(row - r0) * 257 + c])) << 32) | (uint64_t(s_ids[c]) << 1) | 1ull
                   : kEmpty;
      }
      wave_sort_e<4>(v);
      const int64_t u = s_ids[row];
      if (to_bins) {
        if (lane < kBucketEmit) a.bins[u * kBin + lane] = v[0];
        if (lane == 0) a.bin_cnt[u] = uint32_t(min(kBucketEmit, mb - 1));
      } else {
        uint64_t* dst = a.lists + u * a.kp;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int p = e * 64 + lane;
          if (p < a.kp) dst[p] = p < a.kd ? v[e] : kEmpty;
        }
      }
    }
    __syncthreads();
    }
  }
}

// Per node (one wave): sample new/old neighbours, mark sampled new ones old,
// append reverse edges.  The list keys are loaded together, then every
// reverse-slot atomic is issued, then the stores: three round trips in all
// (a load or atomic whose result a later branch waits for would make each
// step wait for everything issued before it).
template <int E>
__global__ __launch_bounds__(256) void sample_kernel(BuildArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t u = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (u >= a.n) return;
  uint64_t* lst = a.lists + u * a.kp;
  uint32_t* fw = a.fwd + u * 2 * kSample;
  uint64_t key[E];
#pragma unroll
  for (int e = 0; e < E; ++e) key[e] = lst[min(e * 64 + lane, a.kd - 1)];
  int n_new = 0, n_old = 0;
  bool take_new[E], take_old[E];
  int pos[E];  // position in the forward sample (new: 0.., old: kSample..)
#pragma unroll
  for (int e = 0; e < E; ++e) {
    if (e * 64 + lane >= a.kd) key[e] = kEmpty;
    const bool valid = key[e] != kEmpty;
    const bool is_new = valid && (key[e] & 1ull);
    const uint64_t mn = __ballot(is_new), mo = __ballot(valid && !is_new);
    const int rn = mbcnt(mn), ro = mbcnt(mo);
    take_new[e] = is_new && n_new + rn < kSample;
    take_old[e] = valid && !is_new && n_old + ro < kSample;
    pos[e] = take_new[e] ? n_new + rn : kSample + n_old + ro;
    n_new = std::min(kSample, n_new + popc(mn));
    n_old = std::min(kSample, n_old + popc(mo));
  }
  uint32_t slot[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    slot[e] = kInvalid;
    if (take_new[e] || take_old[e])
      slot[e] = atomicAdd(&a.rev_cnt[2 * int64_t(key_id(key[e])) + (take_new[e] ? 0 : 1)], 1u);
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    if (!(take_new[e] || take_old[e])) continue;
    const uint32_t id = key_id(key[e]);
    fw[pos[e]] = id;
    if (take_new[e]) lst[e * 64 + lane] = key[e] & ~1ull;
    if (slot[e] < uint32_t(kSample))
      a.rev[int64_t(id) * 2 * kSample + (take_new[e] ? 0 : kSample) + slot[e]] = uint32_t(u);
  }
  if (lane == 0) {
    a.fwd_cnt[2 * u] = uint32_t(n_new);
    a.fwd_cnt[2 * u + 1] = uint32_t(n_old);
  }
}

// Per node (one workgroup): local join of its sampled neighbourhood.  The
// members (forward + reverse samples, new ones first, at most 128) form a
// symmetric Gram matrix; wave w owns the 32 columns [32w, 32w+32) over all
// row tiles, so a lane holds 64 of its column's 128 entries and the partner
// lane (lane ^ 32) the other 64.  Each column member keeps its 8 best
// partners in registers (at least one of the pair new, below the member's
// current worst key), merges them with the partner lane's, and appends them
// to its update bin.
// Transposed Gram tiles of the join's emit: one per pair of row tiles
// (c, r), c < r <= 3, 32 x 32 distances with rows 33 floats apart.
constexpr int kTrPitch = 33;
constexpr int kTrBytes = 6 * 32 * kTrPitch * 4;
constexpr int kJoinStageBytes = kJoinM * (kJoinChunkBytes + 16);
__device__ __forceinline__ int tr_pair(int c, int r) { return r * (r - 1) / 2 + c; }

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8))) void join_kernel(BuildArgs a) {
  // Gram operand staging, then (after the Gram) the transposed tiles.
  __shared__ __attribute__((aligned(16))) char s_stage[kJoinStageBytes > kTrBytes ? kJoinStageBytes : kTrBytes];
  __shared__ uint32_t s_ids[kJoinM + 1];  // + a spare slot for unused list entries
  __shared__ float s_norm[kJoinM + 1];
  __shared__ uint64_t s_worst[kJoinM + 1];
  __shared__ int s_m[2];  // members, new members
  __shared__ unsigned int s_emit;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t u = a.order ? int64_t(a.order[blockIdx.x]) : int64_t(blockIdx.x);
  if (tid < 64) {
    // Lane-parallel member list: new forward, new reverse, old forward, old
    // reverse.  Lanes 0-31 take the new samples, lanes 32-63 the old.  Both
    // lists are loaded whole, in the same round trip as the counts, and
    // stored without branches: entries past a count (in bounds, stale) go to
    // the spare slot s_ids[kJoinM].  A load under a branch of its own would
    // be waited for before the next.
    const int t = tid & (kSample - 1);
    const uint32_t idf = a.fwd[u * 2 * kSample + tid];
    const uint32_t idr = a.rev[u * 2 * kSample + tid];
    const uint32_t fn = a.fwd_cnt[2 * u], fo = a.fwd_cnt[2 * u + 1];
    const uint32_t rn = min(a.rev_cnt[2 * u], uint32_t(kSample));
    const uint32_t ro = min(a.rev_cnt[2 * u + 1], uint32_t(kSample));
    const int o1 = int(fn), o2 = o1 + int(rn), o3 = o2 + int(fo);
    const bool old = tid >= kSample;
    s_ids[uint32_t(t) < (old ? fo : fn) ? (old ? o2 : 0) + t : kJoinM] = idf;
    s_ids[uint32_t(t) < (old ? ro : rn) ? (old ? o3 : o1) + t : kJoinM] = idr;
    if (tid == 0) {
      s_m[0] = o3 + int(ro);
      s_m[1] = o2;
      s_emit = 0;
    }
  }
  __syncthreads();
  // Wave-uniform in registers the compiler knows to be scalar, so that the
  // tile and row guards below are scalar branches.
  const int m = __builtin_amdgcn_readfirstlane(s_m[0]), mnew = __builtin_amdgcn_readfirstlane(s_m[1]);
  if (mnew == 0 || m < 2) {
    if (tid == 0) *reinterpret_cast<uint2*>(&a.stats[u]) = make_uint2(0u, 0u);
    return;
  }
  // Norm and current worst key of member tid, loaded once the first row
  // gathers are issued and stored to LDS for the emit: the wait for them
  // overlaps the gathers', and no register holds them through the Gram loop
  // (for the largest neighbourhoods that would spill, and the spill's store
  // would wait for these loads before any gather is issued).  Threads past
  // the last member store to the spare slot kJoinM.
  const uint32_t member_id = s_ids[tid < m ? tid : 0];
  const int member_slot = tid < m ? tid : kJoinM;
  auto member_side = [&]() __attribute__((always_inline)) {
    const float nrm = a.norms[member_id];
    const uint64_t worst = a.lists[int64_t(member_id) * a.kp + a.kd - 1];
    s_norm[member_slot] = nrm;
    s_worst[member_slot] = worst | 1ull;
  };
  // Tiles of the Gram matrix.  Row tiles in use: R = ceil(m / 32) (most
  // nodes hold at most 64 members once the lists settle, and stage only
  // those rows).  Wave `role` owns column tile `role` (roles rotate with the
  // workgroup, so that the heavier ones spread over the SIMDs).  The join
  // uses each pair of members once and no pair of two old members (members
  // are ordered new first, new_tiles tiles hold the new ones), so the role
  // multiplies only row tiles r <= role, or r < new_tiles when its own tile
  // holds no new member: a prefix of `tiles` row tiles.  Tile (r, c) with
  // r < c serves column c from the registers of role c and, transposed
  // through LDS, column r.
  // When every row tile holds new members and there are 3 or 4, all pairs
  // of tiles are needed, and the roles take circulant windows of row tiles
  // instead (role c: tiles c, c + 1, and c + 2 for c < 2 when there are 4),
  // which balances them at 3, 3, 2, 2 (2, 2, 2) tiles: no role multiplies 4,
  // so kJoinAcc = 3 accumulator tiles serve every case.  Accumulator k holds
  // row tile (row0 + k) % row_tiles.
  f32x16 acc[kJoinAcc];
  const int role = (wave + int(blockIdx.x)) & 3;
  const int new_tiles = (mnew + 31) / 32;
  const int row_tiles = (m + 31) / 32;
  const bool circulant = new_tiles == row_tiles && row_tiles >= 3;
  const int tiles = role >= row_tiles ? 0
                    : circulant       ? (row_tiles == 4 && role < 2 ? 3 : 2)
                    : role < new_tiles ? role + 1
                                       : new_tiles;
  const int row0 = circulant ? role : 0;
  auto gram = [&](auto r_c) __attribute__((always_inline)) {
    constexpr int R = decltype(r_c)::value;
    auto run = [&](auto t_c) __attribute__((always_inline)) {
      gram_join<R, decltype(t_c)::value, kJoinChunkBytes>(a.x16, a.row_bytes, m, s_ids, s_stage, role, row0, acc,
                                                          member_side);
    };
    if (tiles == 0) run(std::integral_constant<int, 0>());
    else if (tiles == 1 || R == 1) run(std::integral_constant<int, 1>());
    else if constexpr (R >= 2) {
      if (tiles == 2 || R == 2) run(std::integral_constant<int, 2>());
      else if constexpr (R >= 3) run(std::integral_constant<int, 3>());
    }
  };
  if (m <= 32) gram(std::integral_constant<int, 1>());
  else if (m <= 64) gram(std::integral_constant<int, 2>());
  else if (m <= 96) gram(std::integral_constant<int, 3>());
  else gram(std::integral_constant<int, 4>());
  __syncthreads();  // the Gram's operand reads are done: s_stage is free

  const int half = lane >> 5;
  float* s_tr = reinterpret_cast<float*>(s_stage);
  // This role's tiles (t, role), t != role, transposed for role t: distance
  // (i, j) of row i in tile t and column j in tile role at [i * kTrPitch + j]
  // of the pair's slot.
#pragma unroll
  for (int k = 0; k < kJoinAcc; ++k) {
    if (k >= tiles) continue;
    const int t = (row0 + k) % row_tiles;
    if (t == role) continue;
    float* tr = s_tr + tr_pair(min(t, role), max(t, role)) * 32 * kTrPitch;
    const float nj = s_norm[32 * role + (lane & 31)];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int i = 8 * (e >> 2) + 4 * half + (e & 3);
      tr[i * kTrPitch + (lane & 31)] = s_norm[32 * t + i] + nj - 2.0f * acc[k][e];
    }
  }
  __syncthreads();

  const int col = 32 * role + (lane & 31);
  unsigned int emitted = 0;
  if (32 * role < m) {
    const bool col_ok = col < m;
    const uint32_t cid = s_ids[col_ok ? col : 0];
    const float cn = s_norm[col_ok ? col : 0];
    const uint64_t worst = s_worst[col_ok ? col : 0];
    const bool col_new = col < mnew;
    uint64_t best[kEmit];
#pragma unroll
    for (int p = 0; p < kEmit; ++p) best[p] = kEmpty;
    // A candidate pair (row member, this lane's column member) at distance
    // dist: kept if it beats the column member's current worst neighbour.
    auto consider = [&](int row, float dist) __attribute__((always_inline)) {
      const uint32_t rid = s_ids[row];
      if (rid == cid) return;
      const uint64_t key = (uint64_t(ord_f32(dist)) << 32) | (uint64_t(rid) << 1) | 1ull;
      if (key < worst && key < best[kEmit - 1]) {
        best[kEmit - 1] = key;
#pragma unroll
        for (int p = kEmit - 1; p > 0; --p) {
          if (best[p] < best[p - 1]) {
            const uint64_t tmp = best[p];
            best[p] = best[p - 1];
            best[p - 1] = tmp;
          }
        }
      }
    };
    // Row tiles this role multiplied, from its accumulators.
#pragma unroll
    for (int k = 0; k < kJoinAcc; ++k) {
      if (k >= tiles) break;
      const int t = (row0 + k) % row_tiles;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = 32 * t + 8 * (e >> 2) + 4 * half + (e & 3);
        if (!col_ok || row >= m || !(col_new || row < mnew)) continue;
        consider(row, cn + s_norm[row] - 2.0f * acc[k][e]);
      }
    }
    // Row tiles another role multiplied, transposed through LDS; past them
    // only pairs of two old members remain (skipped by the test below).
    for (int t = 0; t < 4; ++t) {
      if (32 * t >= m) break;
      if (t == role || (t - row0 + row_tiles) % row_tiles < tiles) continue;
      const float* tr = s_tr + tr_pair(min(t, role), max(t, role)) * 32 * kTrPitch + (lane & 31) * kTrPitch;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = 32 * t + 8 * (e >> 2) + 4 * half + (e & 3);
        if (!col_ok || row >= m || !(col_new || row < mnew)) continue;
        consider(row, tr[row & 31]);
      }
    }
    // Merge with the partner lane's list (same column, the other 64 rows):
    // min against the reversed list gives the 8 smallest as a bitonic
    // sequence, three half-cleaner steps sort it.
    uint64_t mg[kEmit];
#pragma unroll
    for (int p = 0; p < kEmit; ++p) {
      const uint64_t o = shfl_xor_u64(best[kEmit - 1 - p], 32);
      mg[p] = best[p] < o ? best[p] : o;
    }
#pragma unroll
    for (int stride = kEmit / 2; stride >= 1; stride >>= 1) {
#pragma unroll
      for (int p = 0; p < kEmit; ++p) {
        if ((p & stride) == 0) {
          const uint64_t lo = mg[p] < mg[p + stride] ? mg[p] : mg[p + stride];
          const uint64_t hi = mg[p] < mg[p + stride] ? mg[p + stride] : mg[p];
          mg[p] = lo;
          mg[p + stride] = hi;
        }
      }
    }
    // Equal keys are the same partner seen twice (a member sampled both
    // forward and reverse): keep one.
    bool keep[kEmit];
    int cnt = 0;
#pragma unroll
    for (int p = 0; p < kEmit; ++p) {
      keep[p] = mg[p] != kEmpty && !(p > 0 && mg[p] == mg[p - 1]);
      cnt += keep[p] ? 1 : 0;
    }
    if (half == 0 && cnt > 0) {
      const uint32_t base = atomicAdd(&a.bin_cnt[cid], uint32_t(cnt));
      uint64_t* bin = a.bins + int64_t(cid) * kBin;
      // Slots first, without branches, so that the atomic is waited for once:
      // a count advanced inside the store branches below made the compiler
      // wait for every outstanding store (a full round trip) before each one.
      uint32_t q[kEmit];
      uint32_t next = base;
#pragma unroll
      for (int p = 0; p < kEmit; ++p) {
        q[p] = next;
        next += keep[p] ? 1u : 0u;
      }
#pragma unroll
      for (int p = 0; p < kEmit; ++p)
        if (keep[p] && q[p] < uint32_t(kBin)) bin[q[p]] = mg[p];
      emitted = unsigned(cnt);
    }
  }
  atomicAdd(&s_emit, emitted);
  __syncthreads();
  if (tid == 0) *reinterpret_cast<uint2*>(&a.stats[u]) = make_uint2(uint32_t(m), s_emit);
}

// Per node (one wave): merge the update bin into the list.
template <int E>
__global__ __launch_bounds__(256) void apply_kernel(BuildArgs a) {
  __shared__ uint32_t s_hash[4][512];
  __shared__ uint64_t s_keep[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t u = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (u >= a.n) return;
  uint32_t* stat = &a.stats[u].z;
  const uint32_t cnt = a.bin_cnt[u];
  if (cnt == 0) {
    if (lane == 0) *reinterpret_cast<uint2*>(stat) = make_uint2(0u, 0u);
    return;
  }
  const int c = int(min(cnt, uint32_t(kBin)));
  uint32_t* h = s_hash[wave];
  for (int i = lane; i < 512; i += 64) h[i] = kInvalid;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  uint64_t* lst = a.lists + u * a.kp;
  // The list and the whole bin are loaded together (bin entries past the
  // count are in bounds and dropped below), before the list's hash inserts
  // wait for the list: one round trip instead of two.
  uint64_t v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int p = e * 64 + lane;
    v[e] = lst[p < a.kd ? p : 0];
  }
  uint64_t bin_raw[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) bin_raw[e] = a.bins[u * kBin + e * 64 + lane];
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (e * 64 + lane >= a.kd) v[e] = kEmpty;
  auto insert = [&](uint32_t id) -> bool {  // true if newly inserted
    uint32_t s = (id * 0x9E3779B1u) >> 23;
    for (;;) {
      const uint32_t old = atomicCAS(&h[s], kInvalid, id);
      if (old == kInvalid) return true;
      if (old == id) return false;
      s = (s + 1u) & 511u;
    }
  };
  // Only the list's own ids (untagged) count as contained.
  auto contains = [&](uint32_t id) -> bool {
    uint32_t s = (id * 0x9E3779B1u) >> 23;
    for (;;) {
      const uint32_t cur = h[s];
      if (cur == kInvalid) return false;
      if (cur == id) return true;
      s = (s + 1u) & 511u;
    }
  };
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (v[e] != kEmpty) insert(key_id(v[e]));
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  // Bin (up to 128 keys, two per lane): keep one copy of each id that is
  // not in the list yet.  Copies of an id carry the same key (the distance
  // of the same pair of rows, formed in the same order), so any copy will
  // do: each bin id is inserted into the list's hash with the tag bit, and
  // the lane whose insertion lands first keeps it.  (A 128-key sort by id
  // did this before, at about twice the apply's VALU time.)
  uint64_t nk[2];
  int n_keep = 0;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int pos = e * 64 + lane;
    const uint64_t b = pos < c ? bin_raw[e] : kEmpty;
    bool keep = false;
    if (b != kEmpty) {
      const uint32_t id = key_id(b);
      uint32_t s = (id * 0x9E3779B1u) >> 23;
      for (;;) {
        const uint32_t old = atomicCAS(&h[s], kInvalid, id | kBinTag);
        if (old == kInvalid) {
          keep = true;
          break;
        }
        if ((old & ~kBinTag) == id) break;
        s = (s + 1u) & 511u;
      }
    }
    nk[e] = keep ? (b | 1ull) : kEmpty;
    n_keep += popc(__ballot(keep));
  }
  if (n_keep <= 64) {
    // Usually a few dozen kept: packed into one key per lane (through LDS,
    // in bin order), one 64-wide sort and one merge.
    uint64_t* kp = s_keep[wave];
    kp[lane] = kEmpty;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    int base = 0;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint64_t m = __ballot(nk[e] != kEmpty);
      if (nk[e] != kEmpty) kp[base + mbcnt(m)] = nk[e];
      base += popc(m);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    uint64_t c[1] = {kp[lane]};
    wave_sort_e<1>(c);
    wave_merge<E>(v, c[0]);
  } else {
    wave_sort_e<2>(nk);
    wave_merge<E>(v, nk[0]);
    wave_merge<E>(v, nk[1]);
  }
  int inserted = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int p = e * 64 + lane;
    if (p >= a.kd) v[e] = kEmpty;
    const bool ins = v[e] != kEmpty && !contains(key_id(v[e]));
    inserted += popc(__ballot(ins));
    if (p < a.kd) lst[p] = v[e];
  }
  if (lane == 0) {
    a.bin_cnt[u] = 0;
    *reinterpret_cast<uint2*>(stat) = make_uint2(uint32_t(inserted), uint32_t(n_keep));
  }
}

// Locality order of the local join.  A node's sampled neighbourhood is drawn
// from its list and its list's reverse edges, so nodes close in the graph
// gather overlapping member rows.  Workgroups are dispatched in order and
// round-robin over the XCDs, so joining such nodes one after another lets all
// XCDs share their rows in the last-level cache (on clustered data at N=1M,
// nodes ordered by cluster made the join 10% faster).  The order: every node
// starts with its own id as label; each round replaces a node's label by the
// smallest label among its own and its first kLabelK neighbours'.  After r
// rounds a node holds the smallest id within r hops, so equal labels form
// connected regions of the graph around local minima of the ids, and the
// nodes are sorted by label.  One 16-lane group per node.
__global__ __launch_bounds__(256) void label_round_kernel(const uint64_t* __restrict__ lists, int kp, int kd,
                                                          const uint32_t* __restrict__ in,
                                                          uint32_t* __restrict__ out, int64_t n) {
  static_assert(kLabelK == 16, "one 16-lane group per node");
  const int64_t u = (int64_t(blockIdx.x) * 256 + threadIdx.x) / kLabelK;
  const int j = threadIdx.x % kLabelK;
  if (u >= n) return;  // whole 16-lane groups
  const uint64_t key = lists[u * kp + min(j, kd - 1)];
  const uint32_t v = key == kEmpty ? uint32_t(u) : key_id(key);
  uint32_t m = in ? min(in[u], in[v]) : min(uint32_t(u), v);
  m = min(m, xor_lanes<8>(m));
  m = min(m, xor_lanes<4>(m));
  m = min(m, xor_lanes<2>(m));
  m = min(m, xor_lanes<1>(m));
  if (j == 0) out[u] = m;
}

__global__ __launch_bounds__(256) void iota_kernel(uint32_t* __restrict__ out, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = uint32_t(i);
}

// Sums of the per-node statistics: workgroup g writes its partial sums of the
// four fields to partial[4 g .. 4 g + 3].
__global__ __launch_bounds__(256) void stats_reduce_kernel(const uint4* __restrict__ stats, int64_t n,
                                                           unsigned long long* __restrict__ partial) {
  __shared__ unsigned long long s_sum[4][4];
  unsigned long long sum[4] = {0, 0, 0, 0};
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
    const uint4 v = stats[i];
    sum[0] += v.x;
    sum[1] += v.y;
    sum[2] += v.z;
    sum[3] += v.w;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum[k] += shfl_xor_u64(sum[k], o);
    if (lane == 0) s_sum[wave][k] = sum[k];
  }
  __syncthreads();
  if (threadIdx.x < 4)
    partial[4 * blockIdx.x + threadIdx.x] =
        s_sum[0][threadIdx.x] + s_sum[1][threadIdx.x] + s_sum[2][threadIdx.x] + s_sum[3][threadIdx.x];
}

// Per node (one workgroup): exact fp32 squared L2 distance to each entry of
// its list (a 16-lane team per entry, summing over the fp32 rows), then the
// list re-keyed with those distances and re-sorted by (distance, id), so
// that the pruning ranks neighbours by exact distances instead of the build's
// fp16-input expanded-form estimates.
template <int E>
__global__ __launch_bounds__(256) void rescore_kernel(const float* __restrict__ rows, int64_t d, BuildArgs a) {
  __shared__ float s_d[kMaxKd];
  const int tid = threadIdx.x, team = tid >> 4, tp = tid & 15, lane = tid & 63;
  // In the join's locality order when there is one (neighbour rows of
  // graph-close nodes then meet in the caches).
  const int64_t u = a.order ? int64_t(a.order[blockIdx.x]) : int64_t(blockIdx.x);
  uint64_t* lst = a.lists + u * a.kp;
  const float* x = rows + u * d;
  const bool vec = (d & 3) == 0 && (reinterpret_cast<uintptr_t>(rows) & 15) == 0;
  for (int e = team; e < a.kd; e += 16) {
    const uint64_t key = lst[e];
    float acc = INFINITY;
    if (key != kEmpty) {
      const float* y = rows + int64_t(key_id(key)) * d;
      float sum = 0.f;
      if (vec) {
#pragma unroll 4
        for (int64_t i = 4 * int64_t(tp); i < d; i += 64) {
          const float4 xa = *reinterpret_cast<const float4*>(x + i);
          const float4 ya = *reinterpret_cast<const float4*>(y + i);
          const float t0 = xa.x - ya.x, t1 = xa.y - ya.y, t2 = xa.z - ya.z, t3 = xa.w - ya.w;
          sum += (t0 * t0 + t1 * t1) + (t2 * t2 + t3 * t3);
        }
      } else {
        for (int64_t i = tp; i < d; i += 16) {
          const float t = x[i] - y[i];
          sum += t * t;
        }
      }
      sum += xor_lanes_f(sum, 8);
      sum += xor_lanes_f(sum, 4);
      sum += xor_lanes_f(sum, 2);
      sum += xor_lanes_f(sum, 1);
      acc = sum;
    }
    if (tp == 0) s_d[e] = acc;
  }
  __syncthreads();
  if (tid >= 64) return;
  uint64_t v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int p = e * 64 + lane;
    const uint64_t key = p < a.kd ? lst[p] : kEmpty;
    v[e] = key == kEmpty ? kEmpty : (uint64_t(ord_f32(s_d[p])) << 32) | (key & 0xffffffffull);
  }
  wave_sort_e<E>(v);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int p = e * 64 + lane;
    if (p < a.kd) lst[p] = v[e];
  }
}

// Lists -> id rows (n x kd) for pruning.
__global__ __launch_bounds__(256) void list_ids_kernel(const uint64_t* __restrict__ lists, int64_t n, int kd, int kp,
                                                       uint32_t* __restrict__ ids) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n * kd) return;
  const int64_t r = i / kd, j = i - r * kd;
  const uint64_t k = lists[r * kp + j];
  ids[i] = k == kEmpty ? kInvalid : key_id(k);
}

// Caller-supplied k-NN lists -> id rows for pruning, per row (one wave):
// ids >= n, the row's own id and repeats (all but the first occurrence) are
// dropped, the rest keep their order and the row ends in kInvalid.  The
// pruning below needs exactly that: valid ids first, each naming a row.
__global__ __launch_bounds__(256) void compact_lists_kernel(const uint32_t* __restrict__ knn, int64_t n, int kd,
                                                            uint32_t* __restrict__ ids) {
  constexpr int kHash = 512;  // at most kMaxKd = 256 ids: half full at most
  __shared__ uint32_t s_key[4][kHash];
  __shared__ uint32_t s_first[4][kHash];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t u = int64_t(blockIdx.x) * 4 + wave;
  if (u >= n) return;
  uint32_t* hk = s_key[wave];
  uint32_t* hf = s_first[wave];
  for (int i = lane; i < kHash; i += 64) {
    hk[i] = kInvalid;
    hf[i] = kInvalid;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  const uint32_t* row = knn + u * kd;
  uint32_t w[4], slot[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int j = e * 64 + lane;
    w[e] = j < kd ? row[j] : kInvalid;
    if (int64_t(w[e]) >= n || int64_t(w[e]) == u) w[e] = kInvalid;
    slot[e] = 0;
    if (w[e] != kInvalid) {
      uint32_t s = (w[e] * 0x9E3779B1u) >> 23;
      for (;;) {
        const uint32_t prev = atomicCAS(&hk[s], kInvalid, w[e]);
        if (prev == kInvalid || prev == w[e]) break;
        s = (s + 1u) & uint32_t(kHash - 1);
      }
      slot[e] = s;
      atomicMin(&hf[s], uint32_t(j));
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  uint32_t* dst = ids + u * kd;
  int m = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int j = e * 64 + lane;
    const bool keep = w[e] != kInvalid && hf[slot[e]] == uint32_t(j);
    const uint64_t mask = __ballot(keep);
    if (keep) dst[m + int(mbcnt(mask))] = w[e];
    m += int(popc(mask));
  }
  for (int j = m + lane; j < kd; j += 64) dst[j] = kInvalid;
}

// Per node (one wave): detour counts, keep g edges, append reverse edges.
template <int E>
__global__ __launch_bounds__(256) void prune_kernel(const uint32_t* __restrict__ ids, int64_t n, int kd, int g,
                                                    const uint32_t* __restrict__ order,
                                                    uint32_t* __restrict__ kept, uint32_t* __restrict__ rev,
                                                    uint32_t* __restrict__ rev_cnt) {
  __shared__ uint32_t s_hkey[4][512];
  __shared__ uint32_t s_hval[4][512];
  __shared__ uint32_t s_det[4][kMaxKd];
  __shared__ uint32_t s_nb[4][kMaxKd];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // Nodes in the join's locality order when there is one: graph-close nodes
  // read overlapping neighbour lists, which then meet in the caches.
  const int64_t i_node = int64_t(blockIdx.x) * 4 + wave;
  if (i_node >= n) return;
  const int64_t u = order ? int64_t(order[i_node]) : i_node;
  uint32_t* hk = s_hkey[wave];
  uint32_t* hv = s_hval[wave];
  for (int i = lane; i < 512; i += 64) hk[i] = kInvalid;
  for (int i = lane; i < kMaxKd; i += 64) s_det[wave][i] = 0;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  const uint32_t* row = ids + u * kd;
  int valid_n = 0;
  for (int j = lane; j < kd; j += 64) {
    const uint32_t w = row[j];
    s_nb[wave][j] = w;
    if (w != kInvalid) {
      uint32_t s = (w * 0x9E3779B1u) >> 23;
      while (atomicCAS(&hk[s], kInvalid, w) != kInvalid) s = (s + 1u) & 511u;
      hv[s] = uint32_t(j);
    }
  }
  for (int j = 0; j < kd; j += 64) valid_n += popc(__ballot(j + lane < kd && row[j + lane] != kInvalid));
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  // Edge u -> v_j is detourable via v_i when max(i, rank of v_j in v_i's list) < j.
  // The lists of U neighbours are loaded together, and the first hash slot
  // of every entry is read before any is resolved, so that memory and LDS
  // latencies overlap; the table is at most a quarter full, so a further
  // probe is rare.
  constexpr int U = 8;
  for (int i0 = 0; i0 < valid_n; i0 += U) {
    uint32_t wv[U][E];
#pragma unroll
    for (int uu = 0; uu < U; ++uu) {
      const uint32_t vi = s_nb[wave][i0 + uu < valid_n ? i0 + uu : i0];
      const uint32_t* li = ids + int64_t(vi) * kd;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int p = e * 64 + lane;
        wv[uu][e] = p < kd && i0 + uu < valid_n ? li[p] : kInvalid;
      }
    }
    uint32_t slot[U][E], cur[U][E];
#pragma unroll
    for (int uu = 0; uu < U; ++uu)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        slot[uu][e] = (wv[uu][e] * 0x9E3779B1u) >> 23;
        cur[uu][e] = hk[slot[uu][e]];
      }
#pragma unroll
    for (int uu = 0; uu < U; ++uu) {
      const int i = i0 + uu;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int p = e * 64 + lane;
        const uint32_t w = wv[uu][e];
        if (w == kInvalid) continue;
        uint32_t s = slot[uu][e], c = cur[uu][e];
        while (c != kInvalid && c != w) {
          s = (s + 1u) & 511u;
          c = hk[s];
        }
        if (c == w) {
          const int j = int(hv[s]);
          if (i < j && p < j) atomicAdd(&s_det[wave][j], 1u);
        }
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  // Keep the g edges of fewest detours (ties by rank), in rank order.
  uint64_t v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int j = e * 64 + lane;
    v[e] = j < valid_n ? (uint64_t(s_det[wave][j]) << 32) | uint32_t(j) : kEmpty;
  }
  wave_sort_e<E>(v);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int p = e * 64 + lane;
    v[e] = (p < g && v[e] != kEmpty) ? (v[e] & 0xffffffffull) : kEmpty;  // rank only
  }
  wave_sort_e<E>(v);
  uint32_t* out = kept + u * g;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int p = e * 64 + lane;
    if (p < g) {
      const uint32_t w = v[e] == kEmpty ? kInvalid : s_nb[wave][uint32_t(v[e])];
      out[p] = w;
      if (w != kInvalid && rev) {
        const uint32_t slot = atomicAdd(&rev_cnt[w], 1u);
        if (slot < uint32_t(g)) rev[int64_t(w) * g + slot] = uint32_t(u);
      }
    }
  }
}

// Per node (one wave): the closest g - r kept edges, then up to r reverse
// edges, then the remaining kept edges, then the remaining reverse edges,
// until g; no duplicates.  Each phase checks its candidates against a wave
// hash set of the ids placed so far and takes the new ones in order (ballot
// prefix ranks).  The candidates of one phase are distinct (kept edges come
// from a duplicate-free list, and a node appears at most once in another's
// reverse list), so a phase's checks need not see its own insertions.
__global__ __launch_bounds__(256) void merge_reverse_kernel(const uint32_t* __restrict__ kept,
                                                            const uint32_t* __restrict__ rev,
                                                            const uint32_t* __restrict__ rev_cnt, int64_t n, int g,
                                                            int r, uint32_t* __restrict__ out) {
  constexpr int kHash = 1024;  // at most g <= 256 ids are placed: a quarter full at most
  __shared__ uint32_t s_hash[4][kHash];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t u = int64_t(blockIdx.x) * 4 + wave;
  if (u >= n) return;
  uint32_t* hs = s_hash[wave];
  for (int i = lane; i < kHash; i += 64) hs[i] = kInvalid;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  auto has = [&](uint32_t w) {
    uint32_t s = (w * 0x9E3779B1u) >> 22;
    for (;;) {
      const uint32_t cur = hs[s];
      if (cur == w) return true;
      if (cur == kInvalid) return false;
      s = (s + 1u) & uint32_t(kHash - 1);
    }
  };
  auto insert = [&](uint32_t w) {
    uint32_t s = (w * 0x9E3779B1u) >> 22;
    while (atomicCAS(&hs[s], kInvalid, w) != kInvalid) s = (s + 1u) & uint32_t(kHash - 1);
  };
  const uint32_t* kr = kept + u * g;
  const uint32_t* rr = rev + u * g;
  const int rc = int(min(rev_cnt[u], uint32_t(g)));
  const int half = g - r;
  uint32_t* dst = out + u * g;
  int m = 0;
  // Takes, in index order, candidates src[i] for i in [lo, hi) that are valid
  // and new, until `quota` are taken or the list is full.
  auto phase = [&](const uint32_t* src, int lo, int hi, int quota) {
    int taken = 0;
    for (int c = lo; c < hi && taken < quota && m < g; c += 64) {
      const int i = c + lane;
      const uint32_t w = i < hi ? src[i] : kInvalid;
      const bool cand = w != kInvalid && !has(w);
      const uint64_t mask = __ballot(cand);
      const int rank = int(mbcnt(mask));
      const int room = min(quota - taken, g - m);
      const bool take = cand && rank < room;
      if (take) {
        dst[m + rank] = w;
        insert(w);
      }
      const int nt = min(int(popc(mask)), room);
      m += nt;
      taken += nt;
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    }
  };
  phase(kr, 0, half, g);
  phase(rr, 0, rc, g - half);
  phase(kr, half, g, g);
  phase(rr, 0, rc, g);
  for (int i = m + lane; i < g; i += 64) dst[i] = kInvalid;
}

template <typename K>
void launch_e(int e, dim3 grid, hipStream_t s, BuildArgs a) {
  switch (e) {
    case 1: hipLaunchKernelGGL(K::template fn<1>(), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL(K::template fn<2>(), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(K::template fn<4>(), grid, dim3(256), 0, s, a); break;
  }
}
struct SampleK {
  template <int E>
  static constexpr auto fn() { return sample_kernel<E>; }
};
struct ApplyK {
  template <int E>
  static constexpr auto fn() { return apply_kernel<E>; }
};

struct DevMem {
  std::vector<void*> ptrs;
  template <typename T>
  T* alloc(size_t count) {
    void* p = nullptr;
    check_hip(hipMalloc(&p, std::max<size_t>(count, 1) * sizeof(T)), "hipMalloc(build)");
    ptrs.push_back(p);
    return static_cast<T*>(p);
  }
  ~DevMem() {
    for (void* p : ptrs) (void)hipFree(p);
  }
};

// The join's locality order (see label_round_kernel), in device memory owned
// by mem.
uint32_t* join_order(DevMem& mem, hipStream_t st, const BuildArgs& a, int64_t n) {
  uint32_t* lab[2] = {mem.alloc<uint32_t>(size_t(n)), mem.alloc<uint32_t>(size_t(n))};
  const dim3 grid(unsigned((n * kLabelK + 255) / 256));
  for (int r = 0; r < kLabelRounds; ++r) {
    hipLaunchKernelGGL(label_round_kernel, grid, dim3(256), 0, st, static_cast<const uint64_t*>(a.lists), a.kp,
                       a.kd, r == 0 ? static_cast<const uint32_t*>(nullptr) : lab[(r + 1) & 1], lab[r & 1], n);
    after_launch("label_round_kernel");
  }
  const uint32_t* keys = lab[(kLabelRounds - 1) & 1];
  uint32_t* keys_out = lab[kLabelRounds & 1];
  uint32_t* ids = mem.alloc<uint32_t>(size_t(n));
  uint32_t* order = mem.alloc<uint32_t>(size_t(n));
  hipLaunchKernelGGL(iota_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, ids, n);
  after_launch("iota_kernel");
  int bits = 1;
  while (bits < 32 && (int64_t(1) << bits) < n) ++bits;
  size_t temp_bytes = 0;
  CVS_HIP(hipcub::DeviceRadixSort::SortPairs(nullptr, temp_bytes, keys, keys_out, ids, order, int(n), 0, bits, st));
  void* temp = mem.alloc<char>(temp_bytes);
  CVS_HIP(hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, keys, keys_out, ids, order, int(n), 0, bits, st));
  after_launch("radix_sort");
  return order;
}

double elapsed_s(std::chrono::steady_clock::time_point t0) {
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

// n x kd id rows (valid ids first) -> n x g graph rows in out_graph (device
// or host memory), then waits for the stream.  CVS_GRAPH_KNN: the first g ids
// of each row.  CVS_GRAPH_DETOUR: the g edges of fewest detours
// (prune_kernel), in rank order, of which the last r give way to reverse
// edges if there are any (merge_reverse_kernel).
void make_graph(DevMem& mem, hipStream_t st, const uint32_t* ids, int64_t n, int kd, int g, int mode, int r,
                const uint32_t* order, uint32_t* out_graph, int graph_on_device) {
  if (mode == CVS_GRAPH_KNN) {
    CVS_HIP(hipMemcpy2DAsync(out_graph, size_t(g) * sizeof(uint32_t), ids, size_t(kd) * sizeof(uint32_t),
                             size_t(g) * sizeof(uint32_t), size_t(n),
                             graph_on_device ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, st));
    CVS_HIP(hipStreamSynchronize(st));
    return;
  }
  const bool reverse = r > 0;
  const dim3 wave_grid(unsigned((n + 3) / 4));
  uint32_t* kept = (reverse || !graph_on_device) ? mem.alloc<uint32_t>(size_t(n) * g) : out_graph;
  uint32_t* rev = reverse ? mem.alloc<uint32_t>(size_t(n) * g) : nullptr;
  uint32_t* rev_cnt = reverse ? mem.alloc<uint32_t>(size_t(n)) : nullptr;
  if (reverse) CVS_HIP(hipMemsetAsync(rev_cnt, 0, size_t(n) * sizeof(uint32_t), st));
  switch (kd <= 64 ? 1 : kd <= 128 ? 2 : 4) {
    case 1: hipLaunchKernelGGL(prune_kernel<1>, wave_grid, dim3(256), 0, st, ids, n, kd, g, order, kept, rev, rev_cnt); break;
    case 2: hipLaunchKernelGGL(prune_kernel<2>, wave_grid, dim3(256), 0, st, ids, n, kd, g, order, kept, rev, rev_cnt); break;
    default: hipLaunchKernelGGL(prune_kernel<4>, wave_grid, dim3(256), 0, st, ids, n, kd, g, order, kept, rev, rev_cnt); break;
  }
  after_launch("prune_kernel");
  uint32_t* final_graph = kept;
  if (reverse) {
    final_graph = graph_on_device ? out_graph : mem.alloc<uint32_t>(size_t(n) * g);
    hipLaunchKernelGGL(merge_reverse_kernel, wave_grid, dim3(256), 0, st, static_cast<const uint32_t*>(kept),
                       static_cast<const uint32_t*>(rev), static_cast<const uint32_t*>(rev_cnt), n, g, r,
                       final_graph);
    after_launch("merge_reverse_kernel");
  }
  if (!graph_on_device)
    CVS_HIP(hipMemcpyAsync(out_graph, final_graph, size_t(n) * g * sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  CVS_HIP(hipStreamSynchronize(st));
}

void cagra_build_device(cvs_context* ctx, const float* rows, int64_t n, int64_t d, int rows_on_device,
                        uint32_t intermediate_degree, uint32_t graph_degree, uint32_t max_iterations,
                        float termination_threshold, uint64_t seed, uint32_t* out_graph, int graph_on_device,
                        const cvs_build_options* opts, cvs_build_stats* stats) {
  const bool rescore = opts && opts->rescore_fp32;
  const int graph_mode = opts ? opts->graph_mode : CVS_GRAPH_DETOUR;
  const uint32_t reverse_edges = opts ? opts->reverse_edges : 0u;
  if (graph_mode != CVS_GRAPH_KNN && graph_mode != CVS_GRAPH_DETOUR)
    fail(CVS_ERR_INVALID_ARGUMENT, "unknown graph_mode");
  if (reverse_edges && graph_mode != CVS_GRAPH_DETOUR)
    fail(CVS_ERR_INVALID_ARGUMENT, "reverse_edges needs graph_mode CVS_GRAPH_DETOUR");
  const auto t_start = std::chrono::steady_clock::now();
  if (!rows || n <= 0 || d <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "dataset must be non-null and non-empty");
  if (!out_graph) fail(CVS_ERR_INVALID_ARGUMENT, "null out_graph");
  if (n < 2) fail(CVS_ERR_INVALID_ARGUMENT, "a graph needs at least 2 rows");
  if (n > int64_t(INT32_MAX)) fail(CVS_ERR_UNSUPPORTED, "graph build needs n < 2^31");
  if (graph_degree == 0) fail(CVS_ERR_INVALID_ARGUMENT, "graph_degree must be positive");
  if (intermediate_degree > uint32_t(kMaxKd)) fail(CVS_ERR_UNSUPPORTED, "intermediate_graph_degree exceeds 256");
  const int kd = int(std::min<int64_t>(std::max<uint32_t>(intermediate_degree, graph_degree), n - 1));
  if (kd > kMaxKd) fail(CVS_ERR_UNSUPPORTED, "graph_degree exceeds 256");
  const int g = int(std::min<int64_t>(graph_degree, kd));
  const int kp = (kd + 63) / 64 * 64;
  const int e_slots = kp / 64 == 3 ? 4 : kp / 64;
  const int64_t dp = (d + kRowAlignDims - 1) / kRowAlignDims * kRowAlignDims;
  static_assert(kRowAlignDims * 2 % kJoinChunkBytes == 0 && kRowAlignDims * 2 % kBucketChunkBytes == 0,
                "row stride must hold whole chunks");
  hipStream_t st = ctx->stream;
  cvs_build_stats s{};

  DevMem mem;
  _Float16* x16 = mem.alloc<_Float16>(size_t(n) * dp);
  float* norms = mem.alloc<float>(size_t(n));
  // fp32 rows on the device (kept for the re-score).
  const float* rows32 = rows;
  if (!rows_on_device) {
    float* tmp = mem.alloc<float>(size_t(n) * d);
    CVS_HIP(hipMemcpyAsync(tmp, rows, size_t(n) * d * sizeof(float), hipMemcpyHostToDevice, st));
    rows32 = tmp;
  }
  float* mu = mem.alloc<float>(size_t(dp));
  const float scale = centre_rows(ctx, rows32, n, d, dp, mu);
  hipLaunchKernelGGL(to_half_rows_kernel, dim3(unsigned((n + 3) / 4)), dim3(256), 0, st, rows32, n, d, dp,
                     static_cast<const float*>(mu), scale, x16, norms);
  after_launch("to_half_rows_kernel");
  // Random permutations: the reference's LCG Fisher-Yates
  // (src/metal_context.mm:802-810); later rounds continue the sequence.
  std::vector<uint32_t> perm(static_cast<size_t>(n));
  uint64_t r = seed;
  auto next_perm = [&] {
    std::iota(perm.begin(), perm.end(), 0u);
    for (int64_t i = n - 1; i > 0; --i) {
      r = r * 6364136223846793005ULL + 1442695040888963407ULL;
      const int64_t j = int64_t(r >> 33) % (i + 1);
      std::swap(perm[size_t(i)], perm[size_t(j)]);
    }
  };
  uint32_t* d_perm = mem.alloc<uint32_t>(size_t(n));

  BuildArgs a{};
  a.x16 = reinterpret_cast<const char*>(x16);
  a.norms = norms;
  a.row_bytes = dp * 2;
  a.n = uint32_t(n);
  a.kd = kd;
  a.kp = kp;
  a.lists = mem.alloc<uint64_t>(size_t(n) * kp);
  a.fwd = mem.alloc<uint32_t>(size_t(n) * 2 * kSample);
  a.fwd_cnt = mem.alloc<uint32_t>(size_t(n) * 2);
  a.rev = mem.alloc<uint32_t>(size_t(n) * 2 * kSample);
  a.rev_cnt = mem.alloc<uint32_t>(size_t(n) * 2);
  a.bins = mem.alloc<uint64_t>(size_t(n) * kBin);
  a.bin_cnt = mem.alloc<uint32_t>(size_t(n));
  a.stats = mem.alloc<uint4>(size_t(n));
  a.order = nullptr;
  unsigned long long* d_partial = mem.alloc<unsigned long long>(4 * kStatGroups);
  CVS_HIP(hipMemsetAsync(a.bin_cnt, 0, size_t(n) * sizeof(uint32_t), st));

  const int64_t n_buckets = (n + kBucket - 1) / kBucket;
  const dim3 wave_grid(unsigned((n + 3) / 4));
  const int rounds = n <= kBucket ? 1 : kBucketRounds;
  for (int round = 0; round < rounds; ++round) {
    next_perm();
    CVS_HIP(hipMemcpyAsync(d_perm, perm.data(), size_t(n) * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    hipLaunchKernelGGL(bucket_kernel, dim3(unsigned(n_buckets)), dim3(256), 0, st, a,
                       static_cast<const uint32_t*>(d_perm), round > 0 ? 1 : 0);
    after_launch("bucket_kernel");
    if (round > 0) {
      launch_e<ApplyK>(e_slots, wave_grid, st, a);
      after_launch("apply_kernel");
    }
    // The host permutation buffer is reused: wait for its copy.
    CVS_HIP(hipStreamSynchronize(st));
  }
  CVS_HIP(hipStreamSynchronize(st));
  s.seconds_seed = elapsed_s(t_start);

  // nn-descent.
  const auto t_nd = std::chrono::steady_clock::now();
  hipEvent_t ev0, ev1;
  CVS_HIP(hipEventCreate(&ev0));
  CVS_HIP(hipEventCreate(&ev1));
  double join_ms = 0.0;
  uint32_t it = 0;
  double rate = 1.0;
  std::vector<unsigned long long> partial(4 * kStatGroups);
  for (; it < max_iterations; ++it) {
    CVS_HIP(hipMemsetAsync(a.rev_cnt, 0, size_t(n) * 2 * sizeof(uint32_t), st));
    launch_e<SampleK>(e_slots, wave_grid, st, a);
    after_launch("sample_kernel");
    CVS_HIP(hipEventRecord(ev0, st));
    hipLaunchKernelGGL(join_kernel, dim3(unsigned(n)), dim3(256), 0, st, a);
    after_launch("join_kernel");
    CVS_HIP(hipEventRecord(ev1, st));
    launch_e<ApplyK>(e_slots, wave_grid, st, a);
    after_launch("apply_kernel");
    hipLaunchKernelGGL(stats_reduce_kernel, dim3(kStatGroups), dim3(256), 0, st,
                       static_cast<const uint4*>(a.stats), n, d_partial);
    after_launch("stats_reduce_kernel");
    CVS_HIP(hipMemcpyAsync(partial.data(), d_partial, partial.size() * sizeof(unsigned long long),
                           hipMemcpyDeviceToHost, st));
    CVS_HIP(hipStreamSynchronize(st));
    unsigned long long cnt[4] = {0, 0, 0, 0};
    for (int g = 0; g < kStatGroups; ++g)
      for (int k = 0; k < 4; ++k) cnt[k] += partial[size_t(4 * g + k)];
    float ms = 0.f;
    CVS_HIP(hipEventElapsedTime(&ms, ev0, ev1));
    join_ms += ms;
    const unsigned long long ins = cnt[2];
    s.join_members += cnt[0];
    s.updates_emitted += cnt[1];
    s.updates_kept += cnt[3];
    s.insertions += ins;
    rate = double(ins) / (double(n) * double(kd));
    if (rate < double(termination_threshold)) {
      ++it;
      break;
    }
    if (it == kOrderAfter && !a.order) a.order = join_order(mem, st, a, n);
  }
  (void)hipEventDestroy(ev0);
  (void)hipEventDestroy(ev1);
  s.iterations = it;
  s.final_update_rate = it ? rate : 0.0;
  s.join_ms = join_ms;
  s.join_bytes = double(s.join_members) * double(dp) * 2.0;
  s.seconds_descent = elapsed_s(t_nd);

  // Optional exact fp32 re-score of the final lists.
  if (rescore) {
    const auto t_rs = std::chrono::steady_clock::now();
    switch (e_slots) {
      case 1: hipLaunchKernelGGL(rescore_kernel<1>, dim3(unsigned(n)), dim3(256), 0, st, rows32, d, a); break;
      case 2: hipLaunchKernelGGL(rescore_kernel<2>, dim3(unsigned(n)), dim3(256), 0, st, rows32, d, a); break;
      default: hipLaunchKernelGGL(rescore_kernel<4>, dim3(unsigned(n)), dim3(256), 0, st, rows32, d, a); break;
    }
    after_launch("rescore_kernel");
    CVS_HIP(hipStreamSynchronize(st));
    s.seconds_rescore = elapsed_s(t_rs);
  }

  // Prune + reverse edges.
  const auto t_pr = std::chrono::steady_clock::now();
  uint32_t* ids = mem.alloc<uint32_t>(size_t(n) * kd);
  hipLaunchKernelGGL(list_ids_kernel, dim3(unsigned((n * kd + 255) / 256)), dim3(256), 0, st,
                     static_cast<const uint64_t*>(a.lists), n, kd, kp, ids);
  after_launch("list_ids_kernel");
  if (opts && opts->intermediate_out)
    CVS_HIP(hipMemcpyAsync(opts->intermediate_out, ids, size_t(n) * kd * sizeof(uint32_t), hipMemcpyDeviceToDevice,
                           st));
  make_graph(mem, st, ids, n, kd, g, graph_mode, int(std::min<uint32_t>(reverse_edges, uint32_t(g))), a.order,
             out_graph, graph_on_device);
  s.seconds_prune = elapsed_s(t_pr);
  s.graph_degree = uint32_t(g);
  s.intermediate_degree = uint32_t(kd);
  s.seconds_total = elapsed_s(t_start);
  if (stats) *stats = s;
}

void cagra_optimize_device(cvs_context* ctx, const uint32_t* knn, int64_t n, uint32_t kd_in, int knn_on_device,
                           uint32_t graph_degree, uint32_t reverse_edges, uint32_t* out_graph,
                           int graph_on_device) {
  if (!knn || !out_graph) fail(CVS_ERR_INVALID_ARGUMENT, "null k-NN lists or out_graph");
  if (n < 2) fail(CVS_ERR_INVALID_ARGUMENT, "a graph needs at least 2 rows");
  if (n > int64_t(INT32_MAX)) fail(CVS_ERR_UNSUPPORTED, "graph optimize needs n < 2^31");
  if (kd_in == 0 || graph_degree == 0) fail(CVS_ERR_INVALID_ARGUMENT, "degrees must be positive");
  if (kd_in > uint32_t(kMaxKd)) fail(CVS_ERR_UNSUPPORTED, "k-NN list width exceeds 256");
  if (graph_degree > kd_in) fail(CVS_ERR_INVALID_ARGUMENT, "graph_degree exceeds the k-NN list width");
  if (reverse_edges > graph_degree) fail(CVS_ERR_INVALID_ARGUMENT, "reverse_edges exceeds graph_degree");
  const int kd = int(kd_in), g = int(graph_degree);
  hipStream_t st = ctx->stream;
  DevMem mem;
  const uint32_t* src = knn;
  if (!knn_on_device) {
    uint32_t* tmp = mem.alloc<uint32_t>(size_t(n) * kd);
    CVS_HIP(hipMemcpyAsync(tmp, knn, size_t(n) * kd * sizeof(uint32_t), hipMemcpyHostToDevice, st));
    src = tmp;
  }
  uint32_t* ids = mem.alloc<uint32_t>(size_t(n) * kd);
  hipLaunchKernelGGL(compact_lists_kernel, dim3(unsigned((n + 3) / 4)), dim3(256), 0, st, src, n, kd, ids);
  after_launch("compact_lists_kernel");
  make_graph(mem, st, ids, n, kd, g, CVS_GRAPH_DETOUR, int(reverse_edges), nullptr, out_graph, graph_on_device);
}

}  // namespace
}  // namespace cvs

using namespace cvs;

extern "C" {

int cvs_cagra_build(cvs_context* ctx, const float* rows, int64_t n, int64_t d, int rows_on_device,
                    uint32_t intermediate_degree, uint32_t graph_degree, uint32_t max_iterations,
                    float termination_threshold, uint64_t seed, uint32_t* out_graph, int graph_on_device,
                    cvs_build_stats* stats) {
  return guarded([&] {
    bind(ctx);
    cagra_build_device(ctx, rows, n, d, rows_on_device, intermediate_degree, graph_degree, max_iterations,
                       termination_threshold, seed, out_graph, graph_on_device, nullptr, stats);
  });
}

int cvs_cagra_build_ex(cvs_context* ctx, const float* rows, int64_t n, int64_t d, int rows_on_device,
                       uint32_t intermediate_degree, uint32_t graph_degree, uint32_t max_iterations,
                       float termination_threshold, uint64_t seed, const cvs_build_options* options,
                       uint32_t* out_graph, int graph_on_device, cvs_build_stats* stats) {
  return guarded([&] {
    bind(ctx);
    cagra_build_device(ctx, rows, n, d, rows_on_device, intermediate_degree, graph_degree, max_iterations,
                       termination_threshold, seed, out_graph, graph_on_device, options, stats);
  });
}

int cvs_cagra_optimize(cvs_context* ctx, const uint32_t* knn_graph, int64_t n, uint32_t knn_degree,
                       int knn_on_device, uint32_t graph_degree, uint32_t reverse_edges, uint32_t* out_graph,
                       int graph_on_device) {
  return guarded([&] {
    bind(ctx);
    cagra_optimize_device(ctx, knn_graph, n, knn_degree, knn_on_device, graph_degree, reverse_edges, out_graph,
                          graph_on_device);
  });
}

}  // extern "C"
