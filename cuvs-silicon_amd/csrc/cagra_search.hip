// CAGRA graph search for gfx950: one workgroup of 1-8 waves per query.
//
// Replaces the reference's `cagra_beam_search` kernel
// (shaders/cagra_kernels.metal:28-199, host src/metal_context.mm:918-1111)
// and its host-side entry-point selection (src/cagra.cpp:128-178).  The
// reference keeps an unsorted beam in device memory that thread 0 scans
// serially per neighbour, and a Q x N visited bitfield.  Here everything a
// query touches between iterations stays on chip:
//
//  - itopk list: sorted ascending 64-bit keys in registers, E = itopk/64 per
//    lane (position i = 64*slot + lane).  A key is
//        ord(distance) << 32 | id << 1 | expanded
//    so the order is (distance, id) and marking an entry expanded never
//    reorders the list.
//  - visited set: a bitmap of n bits in LDS when that is no larger than the
//    hash below (n <= 131,072 or 262,144); else an open-addressing hash of
//    2^hash_bits ids, filled to at most one half.  When the next iteration
//    could overflow the hash, it is cleared and the ids of the itopk list
//    re-inserted: an id that left the list can be evaluated again, but can
//    never re-enter it (its key is above the list's current worst), so the
//    list never holds duplicates and does not depend on which set is used.
//  - candidates: processed 64 at a time (one id per lane of the lead wave).
//    New ids pass the hash, are compacted into LDS, and their distances are
//    computed by the 16-lane teams of all waves (each lane reads 16 bytes at
//    a stride of 256 bytes, so a row is gathered in coalesced 256-byte
//    segments and one load instruction serves four rows).  The 64 keys are
//    sorted with a wave bitonic sort and merged into the itopk list with a
//    bitonic merge; candidates that cannot enter the list are dropped
//    before the sort.
//  - waves per query: 2 for large batches; 4 or 8 when the batch is small
//    and each query's chain of dependent gathers is the latency (Q = 1).
//
// Iteration: pick the first `width` unexpanded entries of the list as
// parents, mark them, evaluate their neighbours.  Stop when the list holds no
// unexpanded entry or after max_iterations.  The list is seeded with the
// index's seed nodes (the reference's navigation nodes, src/cagra.cpp:63-82:
// the reference starts from the single nearest one; here all of them enter
// the list, which contains that one); the free lanes of the last 64-id seed
// chunk (all 64 without seed nodes) take hashed ids led by the reference's
// fallback (q * 2654435761) mod n (shaders/cagra_kernels.metal:65-67).
//
// Distances are exact fp32 sums of squared differences (summation order of
// four 16-lane partial sums); outputs are sorted by (distance, id) and padded
// with UINT32_MAX / +inf (src/cagra.cpp:240-251).
#include <algorithm>
#include <cmath>

#include "cvs_internal.hpp"
#include "device_util.hpp"

namespace cvs {
namespace {

constexpr uint32_t kInvalidId = 0xffffffffu;
constexpr uint64_t kEmptyKey = ~0ull;
// Rows of up to kBigDim columns keep the query slice in registers; wider
// rows (up to CVS_CAGRA_MAX_DIM) keep it in LDS and are gathered in chunks
// of kBigDim columns.
constexpr int kBigDim = 1024;
constexpr int kMaxDv = kBigDim / 64;   // float4 per lane and row (fp32 traversal)
constexpr int kMaxDv8 = kBigDim / 128; // 8-column pieces per lane and row (fp16 traversal)

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

struct SearchArgs {
  const float4* rows;     // n rows of dq float4, zero-padded
  const uint4* rows16;    // n rows of dq8 x 8 fp16 of scale * (row - mu) (traversal copy), zero-padded
  const float* mu;        // dpad column means subtracted in the traversal copy (zero-padded)
  float scale;            // power of two applied after centring
  const uint32_t* graph;  // n x g
  const uint32_t* seeds;  // n_seeds seed ids, or null
  const float* queries;   // q x d fp32
  uint32_t* out_nbr;      // q x k
  float* out_dist;        // q x k
  uint32_t* stats;        // q x 2: distance evaluations, iterations (or null)
  int64_t d;
  uint32_t n;
  int g;
  int dq;  // float4 per padded row (16 * dv)
  int dq8; // 8-column pieces per padded row (16 * dv8)
  int dv8; // 8-column pieces per lane and row
  int dv;  // float4 per lane and row
  int n_seeds;
  int seed_lanes;  // seed candidates in all: n_seeds, then hashed ids
  int k;
  int itopk;
  int width;
  int max_iter;
  int hash_bits;
  int bitmap_words;     // > 0: the visited set is a bitmap of this many words (n bits, rounded up)
  int teams;            // workgroups per query (block b = query b / teams, team b % teams)
  uint64_t* team_keys;  // teams > 1: (q * teams) x itopk list keys, merged afterwards
  uint32_t* record;     // or null: the ids of each query's distance evaluations, in order,
  int record_cap;       // the first record_cap of them per query (q x record_cap)
};

// Merges 64 sorted keys `c` (one per lane) into the sorted list `top` of
// 64*E keys, keeping the 64*E smallest.  min(top[i], c'[N-1-i]) with c'
// = c padded by empty keys is bitonic; half-cleaners then sort it.
template <int E>
__device__ __forceinline__ void merge_into(uint64_t (&top)[E], uint64_t c) {
  const int lane = __lane_id();
  const uint64_t cr = shfl_xor_u64(c, 63);  // lane 63 - lane
  top[E - 1] = top[E - 1] < cr ? top[E - 1] : cr;
#pragma unroll
  for (int s = E / 2; s >= 1; s >>= 1) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if ((e & s) == 0) {
        const uint64_t lo = top[e] < top[e + s] ? top[e] : top[e + s];
        const uint64_t hi = top[e] < top[e + s] ? top[e + s] : top[e];
        top[e] = lo;
        top[e + s] = hi;
      }
    }
  }
#pragma unroll
  for (int stride = 32; stride >= 1; stride >>= 1) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint64_t y = shfl_xor_u64(top[e], stride);
      const bool lower = (lane & stride) == 0;
      top[e] = lower ? (top[e] < y ? top[e] : y) : (top[e] < y ? y : top[e]);
    }
  }
}

// One workgroup of W waves per query.  Wave 0 (the lead wave) owns the
// itopk list, the hash inserts, the sort and the merge; all 4W 16-lane teams
// gather candidate rows, so a chunk of 64 candidates costs ceil(64 / 4W)
// dependent gather rounds instead of 16.  The kernel also runs with W = 1 (no
// barriers between waves are needed then); the host launches W = 2 for large
// batches, where the other wave's gathers hide the lead wave's serial work,
// and W = 4 or 8 when few queries would leave most of the GPU idle.
// The large-batch fp16 instance (W = 2) runs four waves per SIMD (113 VGPRs):
// two queries per SIMD in flight instead of one and a half hide more of the
// lead wave's serial work.
template <int E, int W, bool F16, bool BIG>
__global__ __launch_bounds__(64 * W, (F16 && W == 2 && !BIG) ? 4 : 1) void cagra_search_kernel(SearchArgs a) {
  extern __shared__ uint32_t s_mem[];
  const bool bitmap = a.bitmap_words > 0;
  const int H = bitmap ? a.bitmap_words : 1 << a.hash_bits;  // visited-set words
  const uint32_t hmask = uint32_t(H) - 1u;
  const int hcap = bitmap ? (1 << 30) : H / 2;  // a bitmap is never cleared
  const uint32_t hempty = bitmap ? 0u : kInvalidId;
  uint32_t* s_hash = s_mem;
  uint32_t* s_ids = s_mem + H;                           // 64 fresh ids
  float* s_dist = reinterpret_cast<float*>(s_ids + 64);  // their distances
  uint32_t* s_par = s_ids + 128;                         // parents of this iteration
  // Control words written by the lead wave and read by all after a barrier:
  // [0, 1] fresh-id count (alternating per chunk), [2] hash fill after a
  // reset, [3, 4] parent count (alternating per iteration).  Alternating slots
  // keep a write for the next step from racing a slow wave's read.
  uint32_t* s_ctl = s_par + CVS_CAGRA_MAX_WIDTH;
  // d > 1024 (BIG): the query stays in LDS, as given (s_q) and, for fp16
  // traversal, centred and scaled (s_qc); dpad floats each, after the
  // control words.  fp16 traversal with d <= 1024: s_q receives the query as
  // given (kBigDim floats, zero past d) for the final exact re-rank.
  float* s_q = reinterpret_cast<float*>(s_ctl + 8);
  float* s_qc = s_q + (BIG ? a.dq * 4 : 0);

  constexpr int kThreads = 64 * W;
  constexpr int kTeams = 4 * W;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const bool lead = W == 1 || __builtin_amdgcn_readfirstlane(tid >> 6) == 0;
  const int64_t qi = blockIdx.x / a.teams;
  const int tm = int(blockIdx.x - qi * a.teams);
  const int team = tid >> 4, tp = lane & 15;

  for (int i = tid; i < H; i += kThreads) s_hash[i] = hempty;
  if constexpr (BIG) {
    const float* qg = a.queries + qi * a.d;
    for (int i = tid; i < 4 * a.dq; i += kThreads) {
      const float v = i < a.d ? qg[i] : 0.f;
      s_q[i] = v;
      if (F16) s_qc[i] = i < a.d ? (v - a.mu[i]) * a.scale : 0.f;
    }
  }

  // Query slice of this lane (d <= 1024).  fp32 traversal: float4 columns tp + 16 j of
  // the padded row.  fp16 traversal (and its fp32 re-rank): 8-column pieces
  // tp + 16 j, so that a 16-lane team reads 256 contiguous bytes of an fp16
  // row (512 of an fp32 row) per piece.  The fp16 traversal keeps its slice
  // of the centred, scaled query in fp16, as the rows are: a piece's
  // distance is four packed differences and four fp32-accumulating dot2s,
  // and the slice takes 32 VGPRs instead of 64.  The traversal's distances
  // only steer the search; the list is re-ranked against the fp32 query and
  // rows at the end.
  const float* qsrc = a.queries + qi * a.d;
  float4 qv[F16 || BIG ? 1 : kMaxDv];
  half8_t qh[F16 && !BIG ? kMaxDv8 : 1];
  if constexpr (BIG) {
  } else if constexpr (!F16) {
#pragma unroll
    for (int j = 0; j < kMaxDv; ++j) {
      float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
      if (j < a.dv) {
        const int64_t c = int64_t(tp + 16 * j) * 4;
        if (c + 0 < a.d) t.x = qsrc[c + 0];
        if (c + 1 < a.d) t.y = qsrc[c + 1];
        if (c + 2 < a.d) t.z = qsrc[c + 2];
        if (c + 3 < a.d) t.w = qsrc[c + 3];
      }
      qv[j] = t;
    }
  } else {
    // Centred and scaled as the traversal copy is (distances in the
    // traversal are scale^2 times the squared distance), rounded to fp16.
#pragma unroll
    for (int j = 0; j < kMaxDv8; ++j)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int64_t c = int64_t(tp + 16 * j) * 8 + t;
        qh[j][t] = _Float16((j < a.dv8 && c < a.d) ? (qsrc[c] - a.mu[c]) * a.scale : 0.f);
      }
  }

  // Squared distance of row rid to the query, summed over the 16 lanes of
  // this lane's team: from the traversal copy, or (exact) from the fp32 rows.
  auto team_dist = [&](uint32_t rid, bool exact) -> float {
    float acc = 0.f;
    if constexpr (BIG) {
      // Chunks of 1,024 columns: the row's pieces tp + 16 j of the chunk,
      // all loads of a chunk issued before the first is used; the query from
      // LDS.
      if (!F16 || exact) {
        // fp32 rows: float4 columns (F16: 8-column pieces as two float4).
        const float4* row = a.rows + int64_t(rid) * a.dq;
        const float4* qq = reinterpret_cast<const float4*>(s_q);
        for (int c0 = 0; c0 < a.dq; c0 += 256) {
          const int nj = (a.dq - c0) / 16 < 16 ? (a.dq - c0) / 16 : 16;
          float4 x[16];
#pragma unroll
          for (int j = 0; j < 16; ++j)
            if (j < nj) x[j] = row[c0 + tp + 16 * j];
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            if (j < nj) {
              const float4 qj = qq[c0 + tp + 16 * j];
              const float dx = qj.x - x[j].x, dy = qj.y - x[j].y;
              const float dz = qj.z - x[j].z, dw = qj.w - x[j].w;
              acc += (dx * dx + dy * dy) + (dz * dz + dw * dw);
            }
          }
        }
      } else {
        // fp16 traversal copy: 8-column pieces against the centred query.
        const uint4* row = a.rows16 + int64_t(rid) * a.dq8;
        for (int c0 = 0; c0 < a.dq8; c0 += 128) {
          const int nj = (a.dq8 - c0) / 16 < 8 ? (a.dq8 - c0) / 16 : 8;
          uint4 x[8];
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (j < nj) x[j] = row[c0 + tp + 16 * j];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (j < nj) {
              const half8_t h = __builtin_bit_cast(half8_t, x[j]);
              const float* qc = s_qc + 8 * (c0 + tp + 16 * j);
              float p[8];
#pragma unroll
              for (int t = 0; t < 8; ++t) {
                const float dt = qc[t] - float(h[t]);
                p[t] = dt * dt;
              }
              acc += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
            }
          }
        }
      }
    } else if constexpr (!F16) {
      const float4* row = a.rows + int64_t(rid) * a.dq + tp;
      float4 x[kMaxDv];
#pragma unroll
      for (int j = 0; j < kMaxDv; ++j)
        if (j < a.dv) x[j] = row[16 * j];
#pragma unroll
      for (int j = 0; j < kMaxDv; ++j) {
        if (j < a.dv) {
          const float dx = qv[j].x - x[j].x, dy = qv[j].y - x[j].y;
          const float dz = qv[j].z - x[j].z, dw = qv[j].w - x[j].w;
          acc += (dx * dx + dy * dy) + (dz * dz + dw * dw);
        }
      }
    } else if (!exact) {
      const uint4* row = a.rows16 + int64_t(rid) * a.dq8 + tp;
      uint4 x[kMaxDv8];
#pragma unroll
      for (int j = 0; j < kMaxDv8; ++j)
        if (j < a.dv8) x[j] = row[16 * j];
#pragma unroll
      for (int j = 0; j < kMaxDv8; ++j) {
        if (j < a.dv8) {
          const uint4 qw = __builtin_bit_cast(uint4, qh[j]);
          const uint32_t qa[4] = {qw.x, qw.y, qw.z, qw.w}, xa[4] = {x[j].x, x[j].y, x[j].z, x[j].w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const half2_t d2 = __builtin_bit_cast(half2_t, qa[t]) - __builtin_bit_cast(half2_t, xa[t]);
            acc = __builtin_amdgcn_fdot2(d2, d2, acc, false);
          }
        }
      }
    } else {
      // Exact: the fp32 rows against the query as given (staged in LDS, zero
      // past d as the rows are; this runs once per list entry at the end of
      // the search).
      const float4* row = a.rows + int64_t(rid) * a.dq + 2 * tp;
      const float4* qq = reinterpret_cast<const float4*>(s_q) + 2 * tp;
      float4 x[2 * kMaxDv8];
#pragma unroll
      for (int j = 0; j < kMaxDv8; ++j) {
        if (j < a.dv8) {
          x[2 * j] = row[32 * j];
          x[2 * j + 1] = row[32 * j + 1];
        }
      }
#pragma unroll
      for (int j = 0; j < kMaxDv8; ++j) {
        if (j < a.dv8) {
          const float4 ql = qq[32 * j], qh4 = qq[32 * j + 1];
          const float qr[8] = {ql.x, ql.y, ql.z, ql.w, qh4.x, qh4.y, qh4.z, qh4.w};
          const float4 lo = x[2 * j], hi = x[2 * j + 1];
          const float d0 = qr[0] - lo.x, d1 = qr[1] - lo.y, d2 = qr[2] - lo.z, d3 = qr[3] - lo.w;
          const float d4 = qr[4] - hi.x, d5 = qr[5] - hi.y, d6 = qr[6] - hi.z, d7 = qr[7] - hi.w;
          acc += ((d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3)) + ((d4 * d4 + d5 * d5) + (d6 * d6 + d7 * d7));
        }
      }
    }
    acc += xor_lanes_f(acc, 8);
    acc += xor_lanes_f(acc, 4);
    acc += xor_lanes_f(acc, 2);
    acc += xor_lanes_f(acc, 1);
    return acc;
  };

  uint64_t top[E];  // the list (lead wave)
#pragma unroll
  for (int e = 0; e < E; ++e) top[e] = kEmptyKey;
  int count = 0;       // ids in the hash table (workgroup-uniform)
  uint32_t evals = 0;  // distance evaluations (lead wave)
  int phase = 0;       // alternates the fresh-count slot
  __syncthreads();

  // Marks id (< n) visited; true if it was not.
  auto hash_insert = [&](uint32_t id) -> bool {
    if (bitmap) {
      const uint32_t bit = 1u << (id & 31u);
      return (atomicOr(&s_hash[id >> 5], bit) & bit) == 0u;
    }
    uint32_t h = (id * 0x9E3779B1u) >> (32 - a.hash_bits);
    for (;;) {
      const uint32_t old = atomicCAS(&s_hash[h], kInvalidId, id);
      if (old == kInvalidId) return true;
      if (old == id) return false;
      h = (h + 1u) & hmask;
    }
  };

  auto reset_hash = [&]() {
    __syncthreads();
    for (int i = tid; i < H; i += kThreads) s_hash[i] = hempty;
    __syncthreads();
    if (lead) {
      int c = 0;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const bool v = top[e] != kEmptyKey;
        if (v) hash_insert(uint32_t(top[e]) >> 1);
        c += popc(__ballot(v));
      }
      if (lane == 0) s_ctl[2] = uint32_t(c);
    }
    __syncthreads();
    count = int(s_ctl[2]);
  };

  // Evaluates the candidate ids held one per lane of the lead wave
  // (kInvalidId for none) and merges the new ones into the list.
  auto process = [&](uint32_t id) {
    uint32_t* const s_nf = s_ctl + phase;
    phase ^= 1;
    if (lead) {
      const bool fresh = id < a.n && hash_insert(id);
      const uint64_t m = __ballot(fresh);
      if (fresh) s_ids[mbcnt(m)] = id;
      if (lane == 0) *s_nf = uint32_t(popc(m));
      if (a.record && fresh) {
        const uint32_t pos = evals + uint32_t(mbcnt(m));
        if (pos < uint32_t(a.record_cap)) a.record[qi * a.record_cap + pos] = id;
      }
    }
    __syncthreads();
    const int nf = int(*s_nf);
    if (nf == 0) return;
    count += nf;
    evals += uint32_t(nf);
    for (int r0 = 0; r0 < nf; r0 += kTeams) {
      const int r = r0 + team;
      const bool ok = r < nf;
      const float acc = team_dist(s_ids[ok ? r : 0], false);
      if (ok && tp == 0) s_dist[r] = acc;
    }
    __syncthreads();
    if (lead) {
      uint64_t key =
          lane < nf ? (uint64_t(ord_f32(s_dist[lane])) << 32) | (uint64_t(s_ids[lane]) << 1) : kEmptyKey;
      // A key at or above the list's itopk-th key cannot enter the list
      // (keys are unique; an unfilled list holds the empty key there), so
      // such candidates are dropped first: no sort at all when none is
      // left, and a few are compacted into the first lanes (through the
      // id/distance slots, which every wave has finished reading) and
      // sorted over 16 or 32 lanes.  The merged list is the same.
      const int wpos = a.itopk - 1;
      uint64_t worst = kEmptyKey;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        if (e == (wpos >> 6)) {  // uniform: one slot is read
          const uint32_t wlo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(top[e])), wpos & 63));
          const uint32_t whi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(top[e] >> 32)), wpos & 63));
          worst = (uint64_t(whi) << 32) | wlo;
        }
      }
      if (sort_below(key, worst, kEmptyKey, reinterpret_cast<uint64_t*>(s_ids)) > 0) {
        merge_into<E>(top, key);
#pragma unroll
        for (int e = 0; e < E; ++e)
          if (e * 64 + lane >= a.itopk) top[e] = kEmptyKey;
      }
    }
    // With one wave, program order alone separates this chunk's LDS reads
    // from the next chunk's writes; with more, the lead wave writes the next
    // chunk's ids only after every wave has passed the barrier above.
    if (W == 1) __syncthreads();
  };

  // Seeds: seed_lanes candidates in chunks of 64, first the seed nodes, then
  // hashed ids led by the reference's fallback (q * 2654435761) mod n, so that
  // regions no seed node reaches (clusters the graph does not link) can still
  // be entered.  With several teams per query, team t takes the candidates
  // t, t + teams, t + 2 teams, ... of that sequence (the reference's teams
  // start from entry points rotated by n / teams,
  // shaders/cagra_kernels.metal:243-250).
  {
    const uint32_t h0 = uint32_t(qi) * 2654435761u;
    for (int c = 0; c < a.seed_lanes; c += 64) {
      if (count + 64 > hcap) reset_hash();
      const int i = (c + lane) * a.teams + tm;
      uint32_t id = kInvalidId;
      if (lead) {
        if (i < a.n_seeds)
          id = a.seeds[i];
        else if (uint32_t(i - a.n_seeds) < a.n)
          id = (h0 + uint32_t(i - a.n_seeds) * 0x9E3779B9u) % a.n;
      }
      process(id);
    }
  }

  // Iterations.
  int it = 0;
  for (; it < a.max_iter; ++it) {
    if (count + a.width * a.g > hcap) reset_hash();
    uint32_t* const s_np = s_ctl + 3 + (it & 1);
    if (lead) {
      int np = 0;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        uint64_t m = __ballot(top[e] != kEmptyKey && (top[e] & 1ull) == 0);
        while (m != 0 && np < a.width) {
          const int b = __builtin_ctzll(m);
          m &= m - 1;
          if (lane == b) {
            s_par[np] = uint32_t(top[e]) >> 1;
            top[e] |= 1ull;
          }
          ++np;
        }
      }
      if (lane == 0) *s_np = uint32_t(np);
    }
    __syncthreads();
    const int np = int(*s_np);
    if (np == 0) break;
    const int total = np * a.g;
    for (int c = 0; c < total; c += 64) {
      const int f = c + lane;
      uint32_t id = kInvalidId;
      if (lead && f < total) {
        const int p = f / a.g;
        const int j = f - p * a.g;
        id = a.graph[int64_t(s_par[p]) * a.g + j];
      }
      process(id);
    }
  }

  // fp16 traversal: the list's distances are recomputed exactly from the
  // fp32 rows (all teams, 64 entries per round) and the list re-sorted, so
  // the output is the exact top-k of the visited rows in the list.
  if constexpr (F16) {
    if constexpr (!BIG) {
      // The query as given into LDS for the exact distances (the loop's
      // first barrier publishes it): global loads issued together (column
      // clamped, value masked by an AND of its bits), where per-element
      // loads under the column test took one round trip per 8 columns.
      for (int i = tid; i < kBigDim; i += kThreads) {
        const float x = qsrc[i < a.d ? i : a.d - 1];
        s_q[i] = __uint_as_float(__float_as_uint(x) & (i < a.d ? 0xffffffffu : 0u));
      }
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (lead) s_ids[lane] = top[e] != kEmptyKey ? uint32_t(top[e]) >> 1 : 0u;
      __syncthreads();
      for (int r0 = 0; r0 < 64; r0 += kTeams) {
        const float acc = team_dist(s_ids[r0 + team], true);
        if (tp == 0) s_dist[r0 + team] = acc;
      }
      __syncthreads();
      if (lead && top[e] != kEmptyKey) top[e] = (uint64_t(ord_f32(s_dist[lane])) << 32) | (uint64_t(s_ids[lane]) << 1);
    }
    if (lead) wave_sort_e<E>(top);
  }

  if (lead && a.team_keys) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int pos = e * 64 + lane;
      if (pos < a.itopk) a.team_keys[int64_t(blockIdx.x) * a.itopk + pos] = top[e];
    }
  } else if (lead) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int pos = e * 64 + lane;
      if (pos < a.k) {
        const uint64_t key = top[e];
        a.out_nbr[qi * a.k + pos] = key == kEmptyKey ? kInvalidId : uint32_t(key) >> 1;
        a.out_dist[qi * a.k + pos] = key == kEmptyKey ? INFINITY : unord_f32(uint32_t(key >> 32));
      }
    }
    if (a.stats && lane == 0) {
      a.stats[2 * qi] = evals;
      a.stats[2 * qi + 1] = uint32_t(it);
    }
  }
}

// Waves per query (workgroups = queries x teams): 8 up to 128 workgroups, 4
// up to 512, else 2.  With 2 or more waves the lead wave's serial work (hash,
// sort, merge) overlaps other queries' gathers on the same SIMD without
// losing the gathering teams.  Wall time per batch at N=100K D=1024 itopk 64
// with the visited-hash sizes below (fp16 / fp32 traversal):
//   W=2: Q=1 0.28 / 0.33, Q=300 0.36 / 0.41, Q=1,000 0.42 / 0.63, Q=10,000 3.21 / 5.78 ms
//   W=4: Q=1 0.22 / 0.26, Q=300 0.28 / 0.36, Q=1,000 0.57 / 0.76, Q=10,000 3.96 / 5.69 ms
//   W=8: Q=1 0.23 / 0.26, Q=300 0.49 / 0.59, Q=1,000 1.00 / 1.20, Q=10,000 9.64 / 11.4 ms
// (one wave per query: Q=10,000 4.62 / 8.45 ms with the smallest table).
int waves_per_query(int64_t workgroups) {
  return workgroups <= 128 ? 8 : (workgroups <= 512 ? 4 : 2);
}

template <int E, bool F16>
void launch_search(int waves, bool big, dim3 grid, size_t lds, hipStream_t stream, const SearchArgs& a,
                   hipEvent_t e0, hipEvent_t e1) {
  if (big) {  // d > 1024: four waves per query at any batch size
    if (lds > 64 * 1024)
      CVS_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(cagra_search_kernel<E, 4, F16, true>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    hipExtLaunchKernelGGL((cagra_search_kernel<E, 4, F16, true>), grid, dim3(256), lds, stream, e0, e1, 0, a);
    return;
  }
  switch (waves) {
    case 2: hipExtLaunchKernelGGL((cagra_search_kernel<E, 2, F16, false>), grid, dim3(128), lds, stream, e0, e1, 0, a); break;
    case 4: hipExtLaunchKernelGGL((cagra_search_kernel<E, 4, F16, false>), grid, dim3(256), lds, stream, e0, e1, 0, a); break;
    default: hipExtLaunchKernelGGL((cagra_search_kernel<E, 8, F16, false>), grid, dim3(512), lds, stream, e0, e1, 0, a); break;
  }
}

template <int E>
void launch_search(bool f16, int waves, bool big, dim3 grid, size_t lds, hipStream_t stream, const SearchArgs& a,
                   hipEvent_t e0, hipEvent_t e1) {
  if (f16)
    launch_search<E, true>(waves, big, grid, lds, stream, a, e0, e1);
  else
    launch_search<E, false>(waves, big, grid, lds, stream, a, e0, e1);
}

// Merge of the teams' lists of one query (one wave per query): the teams x
// itopk keys are sorted, an id found by several teams is kept once (every
// team computes the same fp32 distance for it, so copies are adjacent once
// the expanded bit is ignored), and the k smallest are written, padded with
// UINT32_MAX / +inf.  The reference merges its teams' beams on the host with
// the same dedupe (src/metal_context.mm:1003-1035).
template <int E2>
__global__ __launch_bounds__(64) void team_merge_kernel(const uint64_t* __restrict__ keys, int total, int k,
                                                        uint32_t* __restrict__ out_nbr, float* __restrict__ out_dist) {
  const int64_t qi = blockIdx.x;
  const int lane = threadIdx.x;
  uint64_t v[E2];
#pragma unroll
  for (int e = 0; e < E2; ++e) {
    const int pos = e * 64 + lane;
    v[e] = pos < total ? (keys[qi * total + pos] | 1ull) : kEmptyKey;
  }
  wave_sort_e<E2>(v);
  int base = 0;
  uint32_t carry_lo = 0, carry_hi = 0;  // key at the previous slot's lane 63
#pragma unroll
  for (int e = 0; e < E2; ++e) {
    const uint32_t lo = uint32_t(v[e]), hi = uint32_t(v[e] >> 32);
    uint32_t plo = uint32_t(__shfl_up(int(lo), 1)), phi = uint32_t(__shfl_up(int(hi), 1));
    if (lane == 0) {
      plo = carry_lo;
      phi = carry_hi;
    }
    const uint64_t prev = (uint64_t(phi) << 32) | plo;
    const bool uniq = v[e] != kEmptyKey && ((e == 0 && lane == 0) || v[e] != prev);
    const uint64_t m = __ballot(uniq);
    const int rank = base + mbcnt(m);
    if (uniq && rank < k) {
      out_nbr[qi * k + rank] = uint32_t(v[e]) >> 1;
      out_dist[qi * k + rank] = unord_f32(uint32_t(v[e] >> 32));
    }
    base += popc(m);
    carry_lo = uint32_t(__builtin_amdgcn_readlane(int(lo), 63));
    carry_hi = uint32_t(__builtin_amdgcn_readlane(int(hi), 63));
  }
  for (int r = base + lane; r < k; r += 64) {
    out_nbr[qi * k + r] = kInvalidId;
    out_dist[qi * k + r] = INFINITY;
  }
}

// fp32 rows (n x dpad) -> the fp16 traversal copy of scale * (row - mu)
// (round to nearest even), 8 values per thread.  Centring keeps the fp16
// rounding proportional to the rows' spread, not their offset from the
// origin; the query is centred and scaled the same way in the search.
__global__ void rows_to_half_kernel(const float4* __restrict__ src, size_t pieces, int dpad8,
                                    const float4* __restrict__ mu, float scale, uint4* __restrict__ dst) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= pieces) return;
  const size_t c = (i % size_t(dpad8)) * 2;  // float4 column of the piece
  const float4 lo = src[2 * i], hi = src[2 * i + 1];
  const float4 ml = mu[c], mh = mu[c + 1];
  half8_t h;
  h[0] = _Float16((lo.x - ml.x) * scale);
  h[1] = _Float16((lo.y - ml.y) * scale);
  h[2] = _Float16((lo.z - ml.z) * scale);
  h[3] = _Float16((lo.w - ml.w) * scale);
  h[4] = _Float16((hi.x - mh.x) * scale);
  h[5] = _Float16((hi.y - mh.y) * scale);
  h[6] = _Float16((hi.z - mh.z) * scale);
  h[7] = _Float16((hi.w - mh.w) * scale);
  dst[i] = __builtin_bit_cast(uint4, h);
}

// Exact squared L2 length of every graph edge (the reference's
// recompute_graph_distances, shaders/cagra_kernels.metal:658-681).  One
// workgroup per node: the node's row stays in registers (float4 columns
// tp + 16 j per lane of each 16-lane team) and the 16 teams gather the
// neighbour rows, 256 contiguous bytes per load instruction and team.  Rows
// wider than 1,024 columns (BIG) go in chunks of 1,024, the node's piece of
// each chunk loaded again (from the caches).  Entries that are not row ids
// (UINT32_MAX, or >= n) get +inf.
template <bool BIG>
__global__ __launch_bounds__(256) void edge_distances_kernel(const float4* __restrict__ rows, int dq, int dv,
                                                             const uint32_t* __restrict__ graph, int g, uint32_t n,
                                                             float* __restrict__ out) {
  const int64_t node = blockIdx.x;
  const int tid = threadIdx.x, team = tid >> 4, tp = tid & 15;
  float4 xv[kMaxDv];
  const float4* self = rows + node * dq + tp;
  if constexpr (!BIG) {
#pragma unroll
    for (int j = 0; j < kMaxDv; ++j)
      if (j < dv) xv[j] = self[16 * j];
  }
  for (int e = team; e < g; e += 16) {
    const uint32_t nb = graph[node * g + e];
    const bool valid = nb < n;
    const float4* row = rows + int64_t(valid ? nb : uint32_t(node)) * dq + tp;
    float acc = 0.f;
    for (int c0 = 0; c0 < (BIG ? dq : 1); c0 += 256) {
      const int nj = BIG ? ((dq - c0) / 16 < kMaxDv ? (dq - c0) / 16 : kMaxDv) : dv;
      if constexpr (BIG) {
#pragma unroll
        for (int j = 0; j < kMaxDv; ++j)
          if (j < nj) xv[j] = self[c0 + 16 * j];
      }
      float4 x[kMaxDv];
#pragma unroll
      for (int j = 0; j < kMaxDv; ++j)
        if (j < nj) x[j] = row[c0 + 16 * j];
#pragma unroll
      for (int j = 0; j < kMaxDv; ++j) {
        if (j < nj) {
          const float dx = xv[j].x - x[j].x, dy = xv[j].y - x[j].y;
          const float dz = xv[j].z - x[j].z, dw = xv[j].w - x[j].w;
          acc += (dx * dx + dy * dy) + (dz * dz + dw * dw);
        }
      }
    }
    acc += xor_lanes_f(acc, 8);
    acc += xor_lanes_f(acc, 4);
    acc += xor_lanes_f(acc, 2);
    acc += xor_lanes_f(acc, 1);
    if (tp == 0) out[node * g + e] = valid ? acc : INFINITY;
  }
}

// Gathers, for every query, the rows its search evaluated (recorded by
// cvs_cagra_search_record_async), with the search's row shape and no search
// work: one workgroup per query, 16 teams of 16 lanes, lane l reading the
// 16-byte pieces l, l + 16, ... of a row (256 contiguous bytes per team and
// load), two rows in flight per team.  The time of this launch is the
// search's data movement alone.
__global__ __launch_bounds__(256) void gather_replay_kernel(const uint4* __restrict__ rows, int row_vecs,
                                                            const uint32_t* __restrict__ record, int cap,
                                                            const uint32_t* __restrict__ stats,
                                                            uint32_t* __restrict__ sink) {
  const int64_t qi = blockIdx.x;
  const int team = threadIdx.x >> 4, tp = threadIdx.x & 15;
  const uint32_t ev = stats[2 * qi];
  const int cnt = int(ev < uint32_t(cap) ? ev : uint32_t(cap));
  const uint32_t* ids = record + qi * cap;
  uint32_t acc = 0;
  for (int i = team; i < cnt; i += 32) {
    const uint4* r0 = rows + int64_t(ids[i]) * row_vecs + tp;
    const uint4* r1 = rows + int64_t(ids[i + 16 < cnt ? i + 16 : i]) * row_vecs + tp;
    for (int c0 = 0; c0 < row_vecs; c0 += 256) {
      uint4 v0[16], v1[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int c = c0 + tp + 16 * j;
        v0[j] = c < row_vecs ? r0[c0 + 16 * j] : uint4{0, 0, 0, 0};
        v1[j] = (c < row_vecs && i + 16 < cnt) ? r1[c0 + 16 * j] : uint4{0, 0, 0, 0};
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) acc ^= v0[j].x ^ v0[j].w ^ v1[j].y ^ v1[j].z;
    }
  }
  if (acc == 0x9E3779B9u) sink[qi * 256 + threadIdx.x] = acc;
}

int ceil_log2(int64_t v) {
  int b = 0;
  while ((int64_t(1) << b) < v) ++b;
  return b;
}

void cagra_search_device(cvs_context* ctx, const cvs_cagra_index* idx, const float* queries,
                         int64_t q, int64_t k, uint32_t itopk_size, uint32_t search_width,
                         uint32_t max_iterations, uint32_t* nbr, float* dist, uint32_t* stats, int teams = 1,
                         uint32_t* record = nullptr, int record_cap = 0) {
  if (!idx || idx->ctx != ctx) fail(CVS_ERR_INVALID_ARGUMENT, "index does not belong to context");
  if (!queries || !nbr || !dist) fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
  if (q <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "query count must be positive");
  if (k <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "k must be positive");
  if (q > int64_t(INT32_MAX)) fail(CVS_ERR_UNSUPPORTED, "too many queries in one call");
  const int64_t itopk = std::max<int64_t>(itopk_size ? itopk_size : 128, k);
  if (itopk > CVS_CAGRA_MAX_ITOPK)
    fail(CVS_ERR_UNSUPPORTED, "itopk_size (or k) exceeds CVS_CAGRA_MAX_ITOPK");
  if (teams < 1 || teams > CVS_CAGRA_MAX_TEAMS) fail(CVS_ERR_INVALID_ARGUMENT, "teams must be in [1, CVS_CAGRA_MAX_TEAMS]");
  if (teams > 1 && int64_t(teams) * itopk > CVS_CAGRA_MAX_ITOPK)
    fail(CVS_ERR_UNSUPPORTED, "teams * itopk_size exceeds CVS_CAGRA_MAX_ITOPK");
  if (q * teams > int64_t(INT32_MAX)) fail(CVS_ERR_UNSUPPORTED, "too many queries in one call");
  const int64_t width = search_width ? search_width : 1;
  if (width > CVS_CAGRA_MAX_WIDTH) fail(CVS_ERR_UNSUPPORTED, "search_width exceeds CVS_CAGRA_MAX_WIDTH");
  const int64_t per_iter = width * int64_t(idx->degree);
  if (per_iter > 2048) fail(CVS_ERR_UNSUPPORTED, "search_width * graph_degree exceeds 2048");
  const int e_slots = itopk <= 64 ? 1 : (itopk <= 128 ? 2 : (itopk <= 256 ? 4 : 8));
  int64_t iters = max_iterations;
  if (iters == 0) iters = std::max<int64_t>(200, 2 * itopk / width);
  const bool big = idx->d > kBigDim;
  const int waves = big ? 4 : waves_per_query(q * teams);
  // The visited hash at twice (W=2) or four times (W=4, 8) the size that
  // keeps it half empty, up to 2^13 entries (32 KiB): the lead wave's probe
  // chains stay short, and fewer mid-search clears mean fewer rows evaluated
  // twice.  W=2 serves the large batches, where a 2^13 table would cost
  // workgroups per CU (fp16 traversal, Q=10,000: 3.21 ms at 2^12, 3.70 ms at
  // 2^13, 4.43 ms at 2^11).
  int hash_bits = std::max(11, ceil_log2(2 * (64 * e_slots + std::max<int64_t>(64, per_iter))));
  hash_bits = std::max(hash_bits, std::min(hash_bits + (waves >= 4 ? 2 : 1), 13));
  // A bitmap of the n rows where it takes no more LDS than the hash: one
  // atomic per id, no probing, never cleared.  Whole 256-byte blocks keep the
  // words after it 8-byte aligned.
  const int64_t bitmap_words = (idx->n + 2047) / 2048 * 64;
  const bool use_bitmap = bitmap_words <= (int64_t(1) << hash_bits);
  const size_t visit_words = use_bitmap ? size_t(bitmap_words) : (size_t(1) << hash_bits);
  const size_t lds = visit_words * 4 + (64 + 64 + CVS_CAGRA_MAX_WIDTH + 8) * 4 +
                     (big ? size_t(idx->dpad) * 4 * (idx->traversal_bits == 16 ? 2 : 1)
                          : (idx->traversal_bits == 16 ? size_t(kBigDim) * 4 : 0));

  SearchArgs a{};
  a.rows = reinterpret_cast<const float4*>(idx->rows);
  a.graph = idx->graph;
  a.seeds = idx->seeds;
  a.queries = queries;
  a.out_nbr = nbr;
  a.out_dist = dist;
  a.stats = stats;
  a.d = idx->d;
  a.n = uint32_t(idx->n);
  a.g = int(idx->degree);
  a.rows16 = reinterpret_cast<const uint4*>(idx->rows16);
  a.mu = idx->mu;
  a.scale = idx->scale;
  a.dq = int(idx->dpad / 4);
  a.dv = int(idx->dpad / 64);
  a.dq8 = int(idx->dpad / 8);
  a.dv8 = int(idx->dpad / 128);
  a.n_seeds = int(idx->n_seeds);
  // At least itopk candidates (all seed nodes, then hashed ids; each team its
  // share of the seed nodes), in whole chunks of 64: a list of itopk entries
  // starts from as many distinct rows.
  const int64_t team_seeds = (int64_t(idx->n_seeds) + teams - 1) / teams;
  a.seed_lanes = int((std::max<int64_t>({team_seeds, itopk, 1}) + 63) / 64 * 64);
  a.k = int(k);
  a.itopk = int(itopk);
  a.width = int(width);
  a.max_iter = int(std::min<int64_t>(iters, INT32_MAX));
  a.hash_bits = hash_bits;
  a.bitmap_words = use_bitmap ? int(bitmap_words) : 0;
  a.teams = teams;
  a.record = teams == 1 ? record : nullptr;
  a.record_cap = record_cap;
  if (teams > 1) {
    ctx->ws_teams.reserve(size_t(q) * size_t(teams) * size_t(itopk) * sizeof(uint64_t));
    a.team_keys = ctx->ws_teams.as<uint64_t>();
    a.stats = nullptr;
  }

  const TimerSpan t0 = timer_span(ctx, "cagra_search");
  const dim3 grid(static_cast<unsigned>(q * teams));
  const bool f16 = idx->traversal_bits == 16;
  // The search kernel starts the span; the team merge (if any) ends it.
  hipEvent_t e1 = teams > 1 ? nullptr : t0.stop;
  switch (e_slots) {
    case 1: launch_search<1>(f16, waves, big, grid, lds, ctx->stream, a, t0.start, e1); break;
    case 2: launch_search<2>(f16, waves, big, grid, lds, ctx->stream, a, t0.start, e1); break;
    case 4: launch_search<4>(f16, waves, big, grid, lds, ctx->stream, a, t0.start, e1); break;
    default: launch_search<8>(f16, waves, big, grid, lds, ctx->stream, a, t0.start, e1); break;
  }
  after_launch("cagra_search_kernel");
  if (teams > 1) {
    const int total = int(teams * itopk);
    const uint64_t* keys = a.team_keys;
    const dim3 mg{unsigned(q)}, mb{64};
    if (total <= 64)
      hipExtLaunchKernelGGL(team_merge_kernel<1>, mg, mb, 0, ctx->stream, nullptr, t0.stop, 0, keys, total, int(k), nbr, dist);
    else if (total <= 128)
      hipExtLaunchKernelGGL(team_merge_kernel<2>, mg, mb, 0, ctx->stream, nullptr, t0.stop, 0, keys, total, int(k), nbr, dist);
    else if (total <= 256)
      hipExtLaunchKernelGGL(team_merge_kernel<4>, mg, mb, 0, ctx->stream, nullptr, t0.stop, 0, keys, total, int(k), nbr, dist);
    else
      hipExtLaunchKernelGGL(team_merge_kernel<8>, mg, mb, 0, ctx->stream, nullptr, t0.stop, 0, keys, total, int(k), nbr, dist);
    after_launch("team_merge_kernel");
  }
}

}  // namespace
}  // namespace cvs

using namespace cvs;

extern "C" {

int cvs_cagra_nav_nodes(int64_t n, uint32_t* out_ids, int64_t* out_count) {
  return guarded([&] {
    if (!out_count) fail(CVS_ERR_INVALID_ARGUMENT, "null out_count");
    if (n <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "row count must be positive");
    if (n > int64_t(UINT32_MAX)) fail(CVS_ERR_UNSUPPORTED, "row ids must fit in uint32");
    // min(200, floor(sqrt(n))) rows, row i at floor(i * (n / n_nav)) with the
    // spacing taken in double (src/cagra.cpp:65-72).
    int64_t n_nav = static_cast<int64_t>(std::sqrt(static_cast<double>(n)));
    if (n_nav > 200) n_nav = 200;
    *out_count = n_nav;
    if (out_ids) {
      const double step = static_cast<double>(n) / static_cast<double>(n_nav);
      for (int64_t i = 0; i < n_nav; ++i) out_ids[i] = static_cast<uint32_t>(static_cast<double>(i) * step);
    }
  });
}

int cvs_cagra_index_create(cvs_context* ctx, const float* rows, int64_t n, int64_t d,
                           int rows_on_device, const uint32_t* graph, uint32_t degree,
                           int graph_on_device, const uint32_t* seeds, uint32_t n_seeds,
                           cvs_cagra_index** out_index) {
  return guarded([&] {
    bind(ctx);
    if (!out_index) fail(CVS_ERR_INVALID_ARGUMENT, "null out_index");
    *out_index = nullptr;
    if (!rows || n <= 0 || d <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "dataset must be non-null and non-empty");
    if (!graph || degree == 0) fail(CVS_ERR_INVALID_ARGUMENT, "graph must be non-null with degree > 0");
    if (n_seeds > 0 && !seeds) fail(CVS_ERR_INVALID_ARGUMENT, "null seed ids");
    if (n > int64_t(INT32_MAX)) fail(CVS_ERR_UNSUPPORTED, "graph search needs n < 2^31");
    if (d > CVS_CAGRA_MAX_DIM) fail(CVS_ERR_UNSUPPORTED, "dimension exceeds CVS_CAGRA_MAX_DIM");
    if (degree > 1024) fail(CVS_ERR_UNSUPPORTED, "graph degree exceeds 1024");
    for (uint32_t i = 0; i < n_seeds; ++i)
      if (seeds[i] >= uint64_t(n)) fail(CVS_ERR_INVALID_ARGUMENT, "seed id out of range");
    auto* ix = new cvs_cagra_index();
    ix->ctx = ctx;
    ix->n = n;
    ix->d = d;
    ix->dpad = (d + 127) / 128 * 128;
    ix->degree = degree;
    ix->n_seeds = n_seeds;
    try {
      const size_t row_bytes = size_t(n) * size_t(ix->dpad) * sizeof(float);
      CVS_HIP(hipMalloc(&ix->rows, row_bytes));
      CVS_HIP(hipMalloc(&ix->graph, size_t(n) * degree * sizeof(uint32_t)));
      if (n_seeds) CVS_HIP(hipMalloc(&ix->seeds, size_t(n_seeds) * sizeof(uint32_t)));
      if (ix->dpad != d) CVS_HIP(hipMemsetAsync(ix->rows, 0, row_bytes, ctx->stream));
      upload_rows(ctx, ix->rows, ix->dpad, rows, n, d, rows_on_device);
      CVS_HIP(hipMalloc(&ix->rows16, size_t(n) * size_t(ix->dpad) * 2));
      CVS_HIP(hipMalloc(&ix->mu, size_t(ix->dpad) * sizeof(float)));
      ix->scale = centre_rows(ctx, ix->rows, n, ix->dpad, ix->dpad, ix->mu);
      hipLaunchKernelGGL(rows_to_half_kernel, dim3(unsigned((size_t(n) * size_t(ix->dpad) / 8 + 255) / 256)), dim3(256),
                         0, ctx->stream, reinterpret_cast<const float4*>(ix->rows), size_t(n) * size_t(ix->dpad) / 8,
                         int(ix->dpad / 8), reinterpret_cast<const float4*>(ix->mu), ix->scale,
                         reinterpret_cast<uint4*>(ix->rows16));
      after_launch("rows_to_half_kernel");
      CVS_HIP(hipMemcpyAsync(ix->graph, graph, size_t(n) * degree * sizeof(uint32_t),
                             graph_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, ctx->stream));
      if (n_seeds)
        CVS_HIP(hipMemcpyAsync(ix->seeds, seeds, size_t(n_seeds) * sizeof(uint32_t), hipMemcpyHostToDevice,
                               ctx->stream));
      CVS_HIP(hipStreamSynchronize(ctx->stream));
    } catch (...) {
      if (ix->rows) (void)hipFree(ix->rows);
      if (ix->rows16) (void)hipFree(ix->rows16);
      if (ix->mu) (void)hipFree(ix->mu);
      if (ix->graph) (void)hipFree(ix->graph);
      if (ix->seeds) (void)hipFree(ix->seeds);
      delete ix;
      throw;
    }
    ++ctx->live_children;
    *out_index = ix;
  });
}

int cvs_cagra_index_destroy(cvs_cagra_index* index) {
  return guarded([&] {
    if (!index) return;
    bind(index->ctx);
    (void)hipStreamSynchronize(index->ctx->stream);
    (void)hipFree(index->rows);
    (void)hipFree(index->rows16);
    (void)hipFree(index->mu);
    (void)hipFree(index->graph);
    if (index->seeds) (void)hipFree(index->seeds);
    --index->ctx->live_children;
    delete index;
  });
}

int cvs_cagra_index_edge_distances(cvs_context* ctx, const cvs_cagra_index* index, float* out_distances,
                                   int out_on_device) {
  return guarded([&] {
    bind(ctx);
    if (!index || index->ctx != ctx) fail(CVS_ERR_INVALID_ARGUMENT, "index does not belong to context");
    if (!out_distances) fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
    const size_t count = size_t(index->n) * index->degree;
    float* dst = out_distances;
    if (!out_on_device) {
      ctx->ws_io.reserve(count * sizeof(float));
      dst = ctx->ws_io.as<float>();
    }
    const TimerSpan t0 = timer_span(ctx, "cagra_edge_distances");
    auto kern = index->d > kBigDim ? edge_distances_kernel<true> : edge_distances_kernel<false>;
    hipExtLaunchKernelGGL(kern, dim3(unsigned(index->n)), dim3(256), 0, ctx->stream, t0.start,
                          t0.stop, 0, reinterpret_cast<const float4*>(index->rows), int(index->dpad / 4),
                          int(index->dpad / 64), static_cast<const uint32_t*>(index->graph), int(index->degree),
                          uint32_t(index->n), dst);
    after_launch("edge_distances_kernel");
    if (!out_on_device) {
      CVS_HIP(hipMemcpyAsync(out_distances, dst, count * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
      CVS_HIP(hipStreamSynchronize(ctx->stream));
    }
  });
}

int cvs_cagra_index_set_traversal(cvs_cagra_index* index, int bits) {
  return guarded([&] {
    if (!index) fail(CVS_ERR_INVALID_ARGUMENT, "null index");
    if (bits != 16 && bits != 32) fail(CVS_ERR_INVALID_ARGUMENT, "traversal precision must be 16 or 32 bits");
    index->traversal_bits = bits;
  });
}

int cvs_cagra_search_async(cvs_context* ctx, const cvs_cagra_index* index, const float* queries_dev,
                           int64_t q, int64_t k, uint32_t itopk_size, uint32_t search_width,
                           uint32_t max_iterations, uint32_t* out_neighbors_dev,
                           float* out_distances_dev, uint32_t* out_stats_dev) {
  return guarded([&] {
    bind(ctx);
    cagra_search_device(ctx, index, queries_dev, q, k, itopk_size, search_width, max_iterations,
                        out_neighbors_dev, out_distances_dev, out_stats_dev);
  });
}

int cvs_cagra_search_teams_async(cvs_context* ctx, const cvs_cagra_index* index, const float* queries_dev,
                                 int64_t q, int64_t k, uint32_t itopk_size, uint32_t search_width,
                                 uint32_t max_iterations, uint32_t teams, uint32_t* out_neighbors_dev,
                                 float* out_distances_dev) {
  return guarded([&] {
    bind(ctx);
    cagra_search_device(ctx, index, queries_dev, q, k, itopk_size, search_width, max_iterations,
                        out_neighbors_dev, out_distances_dev, nullptr, int(std::min<uint32_t>(teams, 1u << 20)));
  });
}

int cvs_cagra_search_record_async(cvs_context* ctx, const cvs_cagra_index* index, const float* queries_dev,
                                  int64_t q, int64_t k, uint32_t itopk_size, uint32_t search_width,
                                  uint32_t max_iterations, uint32_t* out_neighbors_dev, float* out_distances_dev,
                                  uint32_t* out_stats_dev, uint32_t* record_dev, uint32_t record_cap) {
  return guarded([&] {
    bind(ctx);
    if (!record_dev || record_cap == 0 || !out_stats_dev)
      fail(CVS_ERR_INVALID_ARGUMENT, "recording needs a record buffer, a positive capacity and stats");
    if (record_cap > (1u << 20)) fail(CVS_ERR_UNSUPPORTED, "record_cap above 2^20");
    cagra_search_device(ctx, index, queries_dev, q, k, itopk_size, search_width, max_iterations, out_neighbors_dev,
                        out_distances_dev, out_stats_dev, 1, record_dev, int(record_cap));
  });
}

int cvs_cagra_replay_gathers(cvs_context* ctx, const cvs_cagra_index* index, const uint32_t* record_dev,
                             uint32_t record_cap, const uint32_t* stats_dev, int64_t q, int bits, int reps,
                             double* out_ms) {
  return guarded([&] {
    bind(ctx);
    if (!index || index->ctx != ctx) fail(CVS_ERR_INVALID_ARGUMENT, "index does not belong to context");
    if (!record_dev || !stats_dev || !out_ms || record_cap == 0 || q <= 0 || reps < 1)
      fail(CVS_ERR_INVALID_ARGUMENT, "bad replay arguments");
    if (bits != 16 && bits != 32) fail(CVS_ERR_INVALID_ARGUMENT, "bits must be 16 or 32");
    if (q > int64_t(INT32_MAX)) fail(CVS_ERR_UNSUPPORTED, "too many queries");
    const int row_vecs = int(index->dpad * (bits / 8) / 16);
    const uint4* rows = bits == 16 ? static_cast<const uint4*>(index->rows16)
                                   : reinterpret_cast<const uint4*>(index->rows);
    void* sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    auto cleanup = [&] {
      if (e0) (void)hipEventDestroy(e0);
      if (e1) (void)hipEventDestroy(e1);
      if (sink) (void)hipFree(sink);
    };
    try {
      CVS_HIP(hipMalloc(&sink, size_t(q) * 256 * sizeof(uint32_t)));
      CVS_HIP(hipEventCreate(&e0));
      CVS_HIP(hipEventCreate(&e1));
      auto launch = [&] {
        hipLaunchKernelGGL(gather_replay_kernel, dim3(unsigned(q)), dim3(256), 0, ctx->stream, rows, row_vecs,
                           record_dev, int(record_cap), stats_dev, static_cast<uint32_t*>(sink));
        after_launch("gather_replay_kernel");
      };
      launch();  // warm-up
      CVS_HIP(hipEventRecord(e0, ctx->stream));
      for (int i = 0; i < reps; ++i) launch();
      CVS_HIP(hipEventRecord(e1, ctx->stream));
      CVS_HIP(hipEventSynchronize(e1));
      float ms = 0.f;
      CVS_HIP(hipEventElapsedTime(&ms, e0, e1));
      *out_ms = double(ms) / reps;
    } catch (...) {
      cleanup();
      throw;
    }
    cleanup();
  });
}

int cvs_cagra_search_teams(cvs_context* ctx, const cvs_cagra_index* index, const float* queries, int64_t q,
                           int64_t k, uint32_t itopk_size, uint32_t search_width, uint32_t max_iterations,
                           uint32_t teams, uint32_t* out_neighbors, float* out_distances) {
  return guarded([&] {
    bind(ctx);
    if (!index || !queries || !out_neighbors || !out_distances) fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
    if (index->ctx != ctx) fail(CVS_ERR_INVALID_ARGUMENT, "index does not belong to context");
    if (q <= 0 || k <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "query count and k must be positive");
    const size_t qbytes = size_t(q) * size_t(index->d) * sizeof(float);
    const size_t obytes = size_t(q) * size_t(k) * sizeof(float);
    ctx->ws_io.reserve(qbytes + 2 * obytes + 256);
    char* base = ctx->ws_io.as<char>();
    float* dq = reinterpret_cast<float*>(base);
    uint32_t* dn = reinterpret_cast<uint32_t*>(base + (qbytes + 127) / 128 * 128);
    float* dd = reinterpret_cast<float*>(reinterpret_cast<char*>(dn) + (obytes + 127) / 128 * 128);
    CVS_HIP(hipMemcpyAsync(dq, queries, qbytes, hipMemcpyHostToDevice, ctx->stream));
    cagra_search_device(ctx, index, dq, q, k, itopk_size, search_width, max_iterations, dn, dd, nullptr,
                        int(std::min<uint32_t>(teams, 1u << 20)));
    CVS_HIP(hipMemcpyAsync(out_neighbors, dn, obytes, hipMemcpyDeviceToHost, ctx->stream));
    CVS_HIP(hipMemcpyAsync(out_distances, dd, obytes, hipMemcpyDeviceToHost, ctx->stream));
    CVS_HIP(hipStreamSynchronize(ctx->stream));
  });
}

int cvs_cagra_search(cvs_context* ctx, const cvs_cagra_index* index, const float* queries, int64_t q,
                     int64_t k, uint32_t itopk_size, uint32_t search_width, uint32_t max_iterations,
                     uint32_t* out_neighbors, float* out_distances) {
  return guarded([&] {
    bind(ctx);
    if (!index || !queries || !out_neighbors || !out_distances) fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
    if (index->ctx != ctx) fail(CVS_ERR_INVALID_ARGUMENT, "index does not belong to context");
    if (q <= 0 || k <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "query count and k must be positive");
    const size_t qbytes = size_t(q) * size_t(index->d) * sizeof(float);
    const size_t obytes = size_t(q) * size_t(k) * sizeof(float);
    ctx->ws_io.reserve(qbytes + 2 * obytes + 256);
    char* base = ctx->ws_io.as<char>();
    float* dq = reinterpret_cast<float*>(base);
    uint32_t* dn = reinterpret_cast<uint32_t*>(base + (qbytes + 127) / 128 * 128);
    float* dd = reinterpret_cast<float*>(reinterpret_cast<char*>(dn) + (obytes + 127) / 128 * 128);
    CVS_HIP(hipMemcpyAsync(dq, queries, qbytes, hipMemcpyHostToDevice, ctx->stream));
    cagra_search_device(ctx, index, dq, q, k, itopk_size, search_width, max_iterations, dn, dd, nullptr);
    CVS_HIP(hipMemcpyAsync(out_neighbors, dn, obytes, hipMemcpyDeviceToHost, ctx->stream));
    CVS_HIP(hipMemcpyAsync(out_distances, dd, obytes, hipMemcpyDeviceToHost, ctx->stream));
    CVS_HIP(hipStreamSynchronize(ctx->stream));
  });
}

}  // extern "C"
