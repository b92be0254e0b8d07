// Exact brute-force k-NN beyond the fused scan's limits: d > 1024 (the scan
// keeps a query tile's fp16 operands for the whole dimension in registers)
// or k > 112 (the scan keeps at most 128 candidates per query).  The
// reference's CPU loop has neither limit (src/cagra.cpp:211-252); this path
// returns the same answers for d up to CVS_BF_MAX_DIM and k up to
// CVS_BF_MAX_K.
//
// Per chunk of up to 512 queries (a key matrix of the chunk within ~2 GiB):
//  sample     the fp16 MFMA keys d~ = |q~|^2 + |x~|^2 - 2 q~.x~ (centred,
//             scaled copies: the dataset's tiles and the queries converted
//             the same way) of up to 512 evenly strided dataset tiles, by the
//             keys kernel below with a strided tile index.
//  threshold  one workgroup per query: the r-th smallest sampled key, T0,
//             lies at or above the query's R-th smallest key
//             (R = max(2 k, k + 32)) with probability at least 1 - 1e-9 (r
//             from the Poisson rule of the fused path's sample).
//  keys       every (query, row) key, one wave per (32-row dataset tile, 4
//             query tiles), four v_mfma_f32_32x32x16_f16 per k-step; every key
//             at or below the query's T0 is appended with its row to the
//             query's list.  No key matrix is written on this pass.
//  select     one workgroup per query: when the list holds at least R keys
//             and fits, a radix select over it finds the R-th key exactly
//             (every key at or below T0 is listed).  Every row at or below it
//             is re-ranked exactly in fp32 into a running top k kept in LDS
//             (block bitonic sort of up to 2,048 keys).  The certificate of
//             the fused path (Cert, bf_common.hpp) then bounds the exact
//             distance of every row above the R-th key; if it does not clear
//             the k-th exact distance, every row with a key up to the bound
//             T_need is re-ranked too (from the list when T_need <= T0).  A
//             query the list does not serve is flagged and returns.
//  second     for flagged 128-query blocks only (the launches return at once
//  pass       otherwise): the keys kernel writes the block's chunk x N fp32
//             key matrix, and the select takes each flagged query through a
//             three-pass radix select (12 + 12 + 8 bits of the keys' order
//             image) over all its keys.  A query whose fp16 copy is not
//             finite re-ranks every row.
//
// Bytes per search: N * dp * 2 (tiles) + the sample tiles + the lists + the
// re-ranked rows; a flagged block adds its key matrix (128 * N * 4, written
// once and read three times) and another pass over the tiles.
#include <algorithm>
#include <cmath>

#include "bf_common.hpp"
#include "cvs_internal.hpp"
#include "device_util.hpp"

namespace cvs {
namespace bf {
namespace {

constexpr int kWT = 256;           // threads per workgroup (4 waves)
constexpr int kChunkQ = 512;       // queries per chunk at most
constexpr int kAccCap = 2048;      // exact keys held by the select's accumulator
constexpr int kIdsCap = 4096;      // candidate ids per streaming step (16 keys per thread)
constexpr int kSampleM = 64;       // sampled keys per thread (16,384 per query at most)
constexpr int kCandCap = 8192;     // (key, row) candidates collected below the sampled threshold
constexpr int kCandM = kCandCap / kWT;

struct KeysArgs {
  const u32x4* tiles;   // dataset tiles
  const float* norms;   // dataset norms (+inf past n)
  int ks;               // k-steps per tile
  const u32x4* qtiles;  // query tiles of the call (a multiple of 4 tiles)
  const float* qnorms;  // their norms (+inf past q)
  int qt0;              // first query tile of the chunk
  int nq;               // queries of the chunk
  float* keys;          // [nq][ldk]
  int64_t ldk;          // keys per query row (32 per tile index)
  int64_t n_idx;        // tile indices of this launch (indices past it repeat the last)
  int64_t tile_stride;  // tile index i multiplies dataset tile i * tile_stride
  int64_t n;            // dataset rows
  // Collection (t0 null: none): every key of query ql at or below the order
  // image t0[ql], with its row, is appended to cand[ql * cand_cap ...] at a
  // slot taken from cnt[ql] (slots past cand_cap are counted, not written).
  const uint32_t* t0;
  uint32_t* cnt;
  uint64_t* cand;
  int cand_cap;
  int write_keys;         // 0: the key matrix is not written
  const uint32_t* gflag;  // non-null: only query blocks with gflag[query block] set run
  int qgroups;            // 128-query blocks of the chunk (the grid is tile groups x qgroups)
};

// Workgroup (dataset tile group tg, 128-query block qg): wave w multiplies
// dataset tile 4 tg + w with the query tiles qt0 + 4 qg + j, j = 0..3.  Lane
// l holds, for query tile j, query 32 (qt0 + 4 qg + j) + l % 32 against rows
// 32 t + 8 (r / 4) + 4 (l / 32) + r % 4, r = 0..15.
//
// The k-steps run in blocks of KB (4; 2 for the 32-column padded
// dimension).  The four waves share the query tiles: each block's 4 KB
// fragments (k-step, query tile; 1 KiB each) are loaded once per workgroup
// (wave w loads query tile w) into one of two LDS buffers, and every wave
// reads them from there.  Each wave's own dataset fragments for the next
// block are loaded into the other of two register sets while the current
// block multiplies.  At 128 VGPRs and 32 KB of LDS four workgroups share a
// CU (16 waves, 4 KiB of dataset loads each in flight); blocks of 8 k-steps
// (180 VGPRs, 64 KB, two workgroups per CU) took 5% longer.
template <int kKB>
__global__ __launch_bounds__(256) void wide_keys_kernel(KeysArgs a) {
  __shared__ u32x4 s_b[2][kKB * 4 * 64];  // [buffer][k-step * 4 + query tile][lane]
  // One-dimensional grid of tile groups x query blocks.  Workgroup w runs on
  // XCD w % 8, so w is renumbered XCD-major: each XCD takes a contiguous run
  // of (tile group, query block) pairs, query block fastest, and the query
  // blocks of one tile group follow each other on one XCD, whose L2 then
  // serves their repeated reads of the tile group.
  const uint32_t wg = blockIdx.x, total = gridDim.x;
  const uint32_t L = total % 8 == 0 ? (wg % 8) * (total / 8) + wg / 8 : wg;
  const int qg = int(L % uint32_t(a.qgroups));
  const int64_t tg = L / uint32_t(a.qgroups);
  if (a.gflag && a.gflag[qg] == 0) return;  // uniform per workgroup, before any barrier
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t idx = tg * 4 + wave;                                      // tile index (key columns)
  const int64_t t = (idx < a.n_idx ? idx : a.n_idx - 1) * a.tile_stride;  // dataset tile
  const int qtb = a.qt0 + qg * 4;
  const int64_t tstep = int64_t(a.ks) * 64;  // u32x4 per tile
  const u32x4* A = a.tiles + t * tstep + lane;
  const u32x4* Bg = a.qtiles + int64_t(qtb + wave) * tstep + lane;
  const int nb = a.ks / kKB;
  f32x16 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;

  u32x4 aa[kKB], ab[kKB], bs[kKB];
  auto load_a = [&](u32x4 (&v)[kKB], int blk) {
#pragma unroll
    for (int s = 0; s < kKB; ++s) v[s] = A[int64_t(blk * kKB + s) * 64];
  };
  auto load_b = [&](int blk) {
#pragma unroll
    for (int s = 0; s < kKB; ++s) bs[s] = Bg[int64_t(blk * kKB + s) * 64];
  };
  auto store_b = [&](int buf) {
#pragma unroll
    for (int s = 0; s < kKB; ++s) s_b[buf][(s * 4 + wave) * 64 + lane] = bs[s];
  };
  auto mult = [&](const u32x4 (&v)[kKB], int buf) {
#pragma unroll
    for (int s = 0; s < kKB; ++s) {
      const half8 av = __builtin_bit_cast(half8, v[s]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            av, __builtin_bit_cast(half8, s_b[buf][(s * 4 + j) * 64 + lane]), acc[j], 0, 0, 0);
    }
  };
  // Blocks in pairs: register set aa and LDS buffer 0 for even blocks, ab
  // and buffer 1 for odd ones.  Loads are issued unconditionally (block
  // index clamped to the last block; the repeated loads of the last pair hit
  // the cache): a load under a branch, even a uniform one, makes the
  // compiler wait at the join for nearly every load in flight.  The
  // scheduling barriers keep a block's loads ahead of the previous block's
  // products; the workgroup barrier after a block both publishes the next
  // block's query fragments and retires the buffer just read before it is
  // written again.
  load_b(0);
  load_a(aa, 0);
  store_b(0);
  __syncthreads();
  for (int blk = 0; blk < nb; blk += 2) {
    const int b1 = blk + 1 < nb ? blk + 1 : nb - 1;
    const int b2 = blk + 2 < nb ? blk + 2 : nb - 1;
    load_b(b1);
    load_a(ab, b1);
    __builtin_amdgcn_sched_barrier(0);
    mult(aa, 0);
    store_b(1);
    __syncthreads();
    load_b(b2);
    load_a(aa, b2);
    __builtin_amdgcn_sched_barrier(0);
    if (blk + 1 < nb) mult(ab, 1);
    store_b(0);
    __syncthreads();
  }

  const int half = lane >> 5;
  const int64_t row0 = t * 32;
  f32x4 xn[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) xn[g] = *reinterpret_cast<const f32x4*>(a.norms + row0 + 8 * g + 4 * half);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int ql = (qtb + j) * 32 + (lane & 31) - a.qt0 * 32;  // query of the chunk
    if (ql >= a.nq) continue;
    const float qn = a.qnorms[a.qt0 * 32 + ql];
    float* dst = a.keys + int64_t(ql) * a.ldk + idx * 32 + 4 * half;
    f32x4 v[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[g][e] = qn + xn[g][e] - 2.0f * acc[j][4 * g + e];
      if (a.write_keys) *reinterpret_cast<f32x4*>(dst + 8 * g) = v[g];
    }
    if (a.t0) {
      // Row of v[g][e]: row0 + 8 g + 4 half + e (padding rows excluded).
      const uint32_t th = a.t0[ql];
      uint32_t hits = 0;
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          hits |= uint32_t((ord_f32(v[g][e]) <= th) & (row0 + 8 * g + 4 * half + e < a.n)) << (4 * g + e);
      if (hits) {
        uint32_t pos = atomicAdd(&a.cnt[ql], uint32_t(__builtin_popcount(hits)));
        uint64_t* out = a.cand + int64_t(ql) * a.cand_cap;
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if ((hits >> (4 * g + e)) & 1u) {
              if (pos < uint32_t(a.cand_cap))
                out[pos] = (uint64_t(ord_f32(v[g][e])) << 32) | uint32_t(row0 + 8 * g + 4 * half + e);
              ++pos;
            }
      }
    }
  }
}


// Ascending bitonic sort of s[0..p) (p a power of two, <= kAccCap) by the
// whole workgroup.
__device__ __forceinline__ void block_sort(uint64_t* s, int p) {
  for (int size = 2; size <= p; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < p / 2; i += kWT) {
        const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
        const bool asc = (lo & size) == 0;
        const uint64_t x = s[lo], y = s[hi];
        if (asc ? y < x : x < y) {
          s[lo] = y;
          s[hi] = x;
        }
      }
      __syncthreads();
    }
}

// Bin of the need-th smallest key counted in s_hist[0, nb) (1 <= need <= the
// count), for every thread of the workgroup: the bin, the keys in lower bins
// and the keys in the bin.  nb is a multiple of kWT.
__device__ __forceinline__ void hist_find(const uint32_t* s_hist, int nb, uint32_t need, uint32_t* s_wsum,
                                          uint32_t* s_sel, uint32_t& bin, uint32_t& lower, uint32_t& inbin) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = nb / kWT;
  uint32_t mine = 0;
  for (int b = 0; b < per; ++b) mine += s_hist[tid * per + b];
  uint32_t incl = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = uint32_t(__shfl_up(int(incl), o));
    if (lane >= o) incl += y;
  }
  if (lane == 63) s_wsum[wave] = incl;
  __syncthreads();
  uint32_t off = 0;
  for (int w2 = 0; w2 < wave; ++w2) off += s_wsum[w2];
  const uint32_t excl = off + incl - mine;
  if (excl < need && need <= excl + mine) {
    uint32_t c = excl;
    for (int b = 0; b < per; ++b) {
      const uint32_t h = s_hist[tid * per + b];
      if (need <= c + h) {
        s_sel[0] = uint32_t(tid * per + b);
        s_sel[1] = c;
        s_sel[2] = h;
        break;
      }
      c += h;
    }
  }
  __syncthreads();
  bin = s_sel[0];
  lower = s_sel[1];
  inbin = s_sel[2];
  __syncthreads();
}

// The need-th smallest (1 <= need <= the count) order image among keys the
// threads of the workgroup hold, M per thread (key(m) returns whether the
// m-th is one, and its order image): three radix passes of 12, 12 and 8 bits.
// With kAgg each wave counts a step's keys bin by bin (one atomic per distinct
// bin, for keys that crowd into few bins); without, one atomic per key (for
// few keys per thread, where the bin-by-bin loop's latency dominates).  tau is
// that key; below and eq count the keys under it and equal to it.
template <int M, bool kAgg, typename Key>
__device__ __forceinline__ void select_held(Key key, uint32_t need, uint32_t* s_hist, uint32_t* s_wsum,
                                            uint32_t* s_sel, uint32_t& tau, uint32_t& below, uint32_t& eq) {
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t prefix = 0;
  below = 0;
  eq = 0;
  const int shifts[3] = {20, 8, 0}, widths[3] = {12, 12, 8};
#pragma unroll 1
  for (int p = 0; p < 3; ++p) {
    const int sh = shifts[p], w = widths[p], nb = 1 << w, hs = sh + w;
    for (int i = tid; i < nb; i += kWT) s_hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; ++m) {
      bool in;
      uint32_t o;
      key(m, in, o);
      in = in && (hs >= 32 || (o >> hs) == prefix);
      const uint32_t bin = (o >> sh) & uint32_t(nb - 1);
      if (kAgg) {
        uint64_t todo = __ballot(in);
        while (todo) {
          const int leader = __builtin_ctzll(todo);
          const uint32_t lb = uint32_t(__builtin_amdgcn_readlane(int(bin), leader));
          const uint64_t same = __ballot(in && bin == lb);
          if (lane == leader) atomicAdd(&s_hist[lb], uint32_t(popc(same)));
          todo &= ~same;
        }
      } else if (in) {
        atomicAdd(&s_hist[bin], 1u);
      }
    }
    __syncthreads();
    uint32_t b, lower, inbin;
    hist_find(s_hist, nb, need, s_wsum, s_sel, b, lower, inbin);
    prefix = (prefix << w) | b;
    below += lower;
    need -= lower;
    eq = inbin;
  }
  tau = prefix;
}

// Ascending bitonic sort of the 32-bit values s[0..p) (p a power of two, at
// most 4096) by the whole workgroup.
__device__ __forceinline__ void block_sort32(uint32_t* s, int p) {
  for (int size = 2; size <= p; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < p / 2; i += kWT) {
        const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
        const bool asc = (lo & size) == 0;
        const uint32_t x = s[lo], y = s[hi];
        if (asc ? y < x : x < y) {
          s[lo] = y;
          s[hi] = x;
        }
      }
      __syncthreads();
    }
}

// Per query of a chunk: the s_rank-th smallest order image among its S
// sampled keys (skeys[ql * lds ...], S <= kSampleM * kWT), into t0[ql]; and
// cnt[ql] = 0 for the collection that follows, flag[ql] = 0 and, for the
// first query of each 128-query block, gflag[ql / 128] = 0.
//
// For s_rank <= kWT: each thread takes the minimum of its keys; the
// s_rank-th smallest of those kWT minima, U, is at least the s_rank-th
// smallest key (the minima are s_rank distinct keys at or below U).  Every
// key at or below U is then gathered and sorted, and the s_rank-th of them
// is the answer.  About s_rank keys lie at or below U, so the sorts are of
// a few hundred values.  A larger rank, or more than 4096 keys at or below
// U, takes the radix select over all S keys.
__global__ __launch_bounds__(256) void wide_threshold_kernel(const float* skeys, int64_t lds, int S, int s_rank,
                                                             uint32_t* t0, uint32_t* cnt, uint32_t* flag,
                                                             uint32_t* gflag) {
  __shared__ uint32_t s_hist[4096];
  __shared__ uint32_t s_wsum[4];
  __shared__ uint32_t s_sel[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* kr = skeys + int64_t(blockIdx.x) * lds;
  uint32_t sv[kSampleM];
#pragma unroll
  for (int m = 0; m < kSampleM; ++m) {
    const int j = m * kWT + tid;
    // Unconditional loads (index clamped, value masked after): a load under
    // a lane condition is waited for before the next is issued.
    const uint32_t o = ord_f32(kr[j < S ? j : S - 1]);
    sv[m] = j < S ? o : 0xffffffffu;
  }
  bool done = false;
  uint32_t tau = 0;
  if (s_rank <= kWT) {
    uint32_t mn = 0xffffffffu;
#pragma unroll
    for (int m = 0; m < kSampleM; ++m) mn = sv[m] < mn ? sv[m] : mn;
    s_hist[tid] = mn;
    __syncthreads();
    block_sort32(s_hist, kWT);
    const uint32_t U = s_hist[s_rank - 1];
    __syncthreads();
    // Gather every key at or below U (positions from a block scan).
    uint64_t bits = 0;
#pragma unroll
    for (int m = 0; m < kSampleM; ++m) bits |= uint64_t(sv[m] <= U) << m;
    const uint32_t mine = uint32_t(__builtin_popcountll(bits));
    uint32_t incl = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = uint32_t(__shfl_up(int(incl), o));
      if (lane >= o) incl += y;
    }
    if (lane == 63) s_wsum[wave] = incl;
    __syncthreads();
    uint32_t off = 0, total = 0;
    for (int w2 = 0; w2 < 4; ++w2) {
      if (w2 < wave) off += s_wsum[w2];
      total += s_wsum[w2];
    }
    if (total <= 4096u) {
      uint32_t pos = off + incl - mine;
#pragma unroll
      for (int m = 0; m < kSampleM; ++m)
        if ((bits >> m) & 1u) s_hist[pos++] = sv[m];
      int p = 1;
      while (p < int(total)) p <<= 1;
      for (int i = int(total) + tid; i < p; i += kWT) s_hist[i] = 0xffffffffu;
      __syncthreads();
      block_sort32(s_hist, p);
      tau = s_hist[s_rank - 1];
      done = true;
    }
    __syncthreads();
  }
  if (!done) {
    uint32_t below, eq;
    select_held<kSampleM, true>([&](int m, bool& in, uint32_t& o) { in = m * kWT + tid < S; o = sv[m]; },
                          uint32_t(s_rank), s_hist, s_wsum, s_sel, tau, below, eq);
  }
  if (tid == 0) {
    t0[blockIdx.x] = tau;
    cnt[blockIdx.x] = 0;
    flag[blockIdx.x] = 0;
    if (blockIdx.x % 128 == 0) gflag[blockIdx.x / 128] = 0;
  }
}

struct SelectArgs {
  const float* keys;     // [nq][ldk] of the chunk
  int64_t ldk;
  int64_t n;
  int64_t d;
  int q0;                // first query of the chunk
  int R;                 // rank of the radix select
  // Keys collected below a sampled threshold by the keys kernel (cand null:
  // none): t0, cnt and cand of KeysArgs, per query of the chunk.
  const uint32_t* t0;
  const uint32_t* cnt;
  const uint64_t* cand;
  int cand_cap;
  // Deferred keys: with `lazy` the key matrix has not been written; a query
  // that needs it sets flag[ql] and gflag[ql / 128] and returns without
  // output, for a second pass (`only_flagged`: other queries return at once)
  // after the matrix has been written for the flagged query blocks.
  uint32_t* flag;
  uint32_t* gflag;
  int lazy;
  int only_flagged;
  int64_t k;
  const float* rows;     // fp32 rows
  const float* queries;  // fp32 queries of the call
  uint32_t* out_nbr;
  float* out_dist;
};

__global__ __launch_bounds__(256) void wide_select_kernel(SelectArgs a, Cert cert) {
  extern __shared__ uint64_t s_cand[];  // kCandCap (key << 32 | row) candidates, dynamic LDS
  __shared__ uint32_t s_hist[4096];
  __shared__ uint64_t s_acc[kAccCap];
  __shared__ uint32_t s_ids[kIdsCap];
  __shared__ uint32_t s_wsum[4];
  __shared__ uint32_t s_sel[4];  // bin, keys below it
  __shared__ int s_mode;
  __shared__ float s_tneed;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t ql = blockIdx.x;          // query of the chunk
  if (a.only_flagged && a.flag[ql] == 0) return;
  const int64_t q = a.q0 + ql;            // query of the call
  const float* kr = a.keys + ql * a.ldk;
  const float* qv = a.queries + q * a.d;
  const bool vec = (a.d & 3) == 0 && (reinterpret_cast<uintptr_t>(qv) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(a.rows) & 15) == 0;
  const int64_t n = a.n, k = a.k;

  // The query's list size and threshold are loaded with its norm, so that
  // the three round trips overlap.
  const uint32_t nc = a.cand ? a.cnt[ql] : 0u;
  const uint32_t t0l = a.cand ? a.t0[ql] : 0u;
  // Finite inputs?  Otherwise no key means anything: every row is re-ranked.
  const float qn = cert.qnorms[q];
  const bool finite = qn <= 3.0e38f && cert.rmax <= 3.0e38f;

  // 1. The R-th smallest order image among the n keys, tau.
  uint32_t tau = 0xffffffffu, below = 0, eq = uint32_t(n);
  // 1a. From the collected keys: every (key, row) at or below the query's
  // sampled threshold t0, when there are at least R of them and all fit the
  // list, contains the R smallest keys and every key tied with the R-th.
  // They are copied to s_cand and the R-th is selected among them.
  bool use_cand = false;
  uint32_t t0 = 0;
  int ncand = 0;
  if (finite && a.cand) {
    t0 = t0l;
    if (nc >= uint32_t(a.R) && nc <= uint32_t(a.cand_cap) && nc <= uint32_t(kCandCap)) {
      ncand = int(nc);
      const uint64_t* src = a.cand + ql * a.cand_cap;
      // Eight loads per thread in flight (indices clamped, stores masked).
      for (int base = 0; base < ncand; base += 8 * kWT) {
        uint64_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int i = base + u * kWT + tid;
          v[u] = src[i < ncand ? i : ncand - 1];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int i = base + u * kWT + tid;
          if (i < ncand) s_cand[i] = v[u];
        }
      }
      __syncthreads();
      use_cand = true;
      select_held<kCandM, false>(
          [&](int m, bool& in, uint32_t& o) {
            const int i = m * kWT + tid;
            in = i < ncand;
            o = in ? uint32_t(s_cand[i] >> 32) : 0xffffffffu;
          },
          uint32_t(a.R), s_hist, s_wsum, s_sel, tau, below, eq);
    } else if (a.lazy) {
      // The list does not serve: the second pass takes this query.
      if (tid == 0) {
        a.flag[ql] = 1;
        a.gflag[ql / 128] = 1;
      }
      return;
    }
  }
  // 1b. Otherwise radix select over all n keys.
  if (finite && !use_cand) {
    uint32_t prefix = 0;
    int need = a.R;
    below = 0;
    const int shifts[3] = {20, 8, 0}, widths[3] = {12, 12, 8};
#pragma unroll 1
    for (int p = 0; p < 3; ++p) {
      const int sh = shifts[p], w = widths[p], nb = 1 << w;
      for (int i = tid; i < nb; i += kWT) s_hist[i] = 0;
      __syncthreads();
      const int hs = sh + w;  // bits above this pass must equal the prefix
      // 16 keys per thread and step as four 16-byte loads (the row starts
      // 128-byte aligned; indices clamped, keys past n masked).  Keys crowd
      // into few bins (distances of one query span few exponents), so each
      // wave counts its keys bin by bin: the lowest pending lane's bin, the
      // ballot of the lanes holding it, one atomic for all of them.
      const float4* kr4 = reinterpret_cast<const float4*>(kr);
      const int64_t n4 = (n + 3) / 4;
      for (int64_t b4 = 0; b4 < n4; b4 += int64_t(kWT) * 4) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int64_t i4 = b4 + int64_t(u) * kWT + tid;
          v[u] = kr4[i4 < n4 ? i4 : n4 - 1];  // clamped; keys past n are masked below
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int64_t i0 = (b4 + int64_t(u) * kWT + tid) * 4;
          const float c[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t o = ord_f32(c[e]);
            const bool in = i0 + e < n && (hs >= 32 || (o >> hs) == prefix);
            const uint32_t bin = (o >> sh) & uint32_t(nb - 1);
            uint64_t todo = __ballot(in);
            while (todo) {
              const int leader = __builtin_ctzll(todo);
              const uint32_t lb = uint32_t(__builtin_amdgcn_readlane(int(bin), leader));
              const uint64_t same = __ballot(in && bin == lb);
              if (lane == leader) atomicAdd(&s_hist[lb], uint32_t(popc(same)));
              todo &= ~same;
            }
          }
        }
      }
      __syncthreads();
      // Bin holding the need-th key: each thread sums nb / 256 bins, a block
      // scan of those sums, then the owning thread walks its bins.
      const int per = nb / kWT;
      uint32_t mine = 0;
      for (int b = 0; b < per; ++b) mine += s_hist[tid * per + b];
      uint32_t incl = mine;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = uint32_t(__shfl_up(int(incl), o));
        if (lane >= o) incl += y;
      }
      if (lane == 63) s_wsum[wave] = incl;
      __syncthreads();
      uint32_t off = 0;
      for (int w2 = 0; w2 < wave; ++w2) off += s_wsum[w2];
      const uint32_t excl = off + incl - mine;
      if (excl < uint32_t(need) && uint32_t(need) <= excl + mine) {
        uint32_t c = excl;
        for (int b = 0; b < per; ++b) {
          const uint32_t h = s_hist[tid * per + b];
          if (uint32_t(need) <= c + h) {
            s_sel[0] = uint32_t(tid * per + b);
            s_sel[1] = c;
            s_sel[2] = h;
            break;
          }
          c += h;
        }
      }
      __syncthreads();
      prefix = (prefix << w) | s_sel[0];
      below += s_sel[1];
      need -= int(s_sel[1]);
      eq = s_sel[2];
      __syncthreads();
    }
    tau = prefix;
  }

  // Running exact top k in s_acc[0..fill): after a flush, the first min(k,
  // fill) entries are the best so far, sorted.
  int fill = 0;
  auto flush = [&]() {
    int p = 1;
    while (p < fill) p <<= 1;
    for (int i = fill + tid; i < p; i += kWT) s_acc[i] = kSentinel;
    __syncthreads();
    block_sort(s_acc, p);
    fill = fill < int(k) ? fill : int(k);
  };
  // Streams every row whose key passes `take` (by its order image) into the
  // running top k: 16 keys per thread and step, compacted into s_ids, then
  // re-ranked exactly by the four waves (8 rows per wave and pass).
  auto stream = [&](auto take) {
    for (int64_t base = 0; base < n; base += int64_t(kWT) * 16) {
      uint32_t bits = 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int64_t i = base + int64_t(j) * kWT + tid;
        const uint32_t o = ord_f32(kr[i < n ? i : n - 1]);  // unconditional load
        if (i < n && take(o)) bits |= 1u << j;
      }
      const uint32_t mine = uint32_t(__builtin_popcount(bits));
      uint32_t incl = mine;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = uint32_t(__shfl_up(int(incl), o));
        if (lane >= o) incl += y;
      }
      if (lane == 63) s_wsum[wave] = incl;
      __syncthreads();
      uint32_t off = 0, total = 0;
      for (int w2 = 0; w2 < 4; ++w2) {
        if (w2 < wave) off += s_wsum[w2];
        total += s_wsum[w2];
      }
      uint32_t pos = off + incl - mine;
      while (bits) {
        const int j = __builtin_ctz(bits);
        bits &= bits - 1;
        s_ids[pos++] = uint32_t(base + int64_t(j) * kWT + tid);
      }
      __syncthreads();
      for (uint32_t done = 0; done < total;) {
        const int m = int(std::min<uint32_t>(total - done, uint32_t(kAccCap - fill)));
        for (int c = kExactU * wave; c < m; c += kExactU * 4) {
          uint32_t id[kExactU];
#pragma unroll
          for (int u = 0; u < kExactU; ++u) id[u] = c + u < m ? s_ids[done + c + u] : 0xffffffffu;
          float dd[kExactU];
          wave_exact<kExactU>(id, a.rows, n, a.d, qv, vec, dd);
#pragma unroll
          for (int u = 0; u < kExactU; ++u)
            if (lane == u && c + u < m) s_acc[fill + c + u] = (uint64_t(ord_f32(dd[u])) << 32) | id[u];
        }
        fill += m;
        done += uint32_t(m);
        __syncthreads();
        if (fill == kAccCap) flush();
      }
    }
  };

  // The same over the collected keys (every key at or below t0).
  auto stream_cand = [&](auto take) {
    for (int base = 0; base < ncand; base += kWT * 16) {
      uint32_t bits = 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int i = base + j * kWT + tid;
        if (i < ncand && take(uint32_t(s_cand[i] >> 32))) bits |= 1u << j;
      }
      const uint32_t mine = uint32_t(__builtin_popcount(bits));
      uint32_t incl = mine;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = uint32_t(__shfl_up(int(incl), o));
        if (lane >= o) incl += y;
      }
      if (lane == 63) s_wsum[wave] = incl;
      __syncthreads();
      uint32_t off = 0, total = 0;
      for (int w2 = 0; w2 < 4; ++w2) {
        if (w2 < wave) off += s_wsum[w2];
        total += s_wsum[w2];
      }
      uint32_t pos = off + incl - mine;
      while (bits) {
        const int j = __builtin_ctz(bits);
        bits &= bits - 1;
        s_ids[pos++] = uint32_t(s_cand[base + j * kWT + tid]);
      }
      __syncthreads();
      for (uint32_t done = 0; done < total;) {
        const int m = int(std::min<uint32_t>(total - done, uint32_t(kAccCap - fill)));
        for (int c = kExactU * wave; c < m; c += kExactU * 4) {
          uint32_t id[kExactU];
#pragma unroll
          for (int u = 0; u < kExactU; ++u) id[u] = c + u < m ? s_ids[done + c + u] : 0xffffffffu;
          float dd[kExactU];
          wave_exact<kExactU>(id, a.rows, n, a.d, qv, vec, dd);
#pragma unroll
          for (int u = 0; u < kExactU; ++u)
            if (lane == u && c + u < m) s_acc[fill + c + u] = (uint64_t(ord_f32(dd[u])) << 32) | id[u];
        }
        fill += m;
        done += uint32_t(m);
        __syncthreads();
        if (fill == kAccCap) flush();
      }
    }
  };

  if (use_cand) {
    stream_cand([&](uint32_t o) { return o <= tau; });
  } else if (finite) {
    stream([&](uint32_t o) { return o <= tau; });
  } else {
    stream([](uint32_t) { return true; });
  }
  flush();

  // 2. Certificate (see Cert): every row not re-ranked has a key of at least
  // unord(tau).
  constexpr int kDeferred = -1;
  if (tid == 0) {
    int mode = kCertPass;
    float tneed = INFINITY;
    const uint64_t kth = k <= fill ? s_acc[k - 1] : kSentinel;
    if (finite && uint64_t(below) + eq < uint64_t(n)) {
      const double dk = kth == kSentinel ? INFINITY : double(unord_f32(uint32_t(kth >> 32)));
      const double qt = std::sqrt(double(qn)) * (1.0 + 0x1p-20);
      const double qe = std::sqrt(double(cert.qerr[q]) * (1.0 + double(a.d + 8) * 0x1p-24)) * (1.0 + 0x1p-20);
      const double E_ = qe + qt * 0x1p-23 + double(cert.qslack) + double(cert.dx);
      const double A = double(cert.a_coef) * (qt + double(cert.rmax)) * (qt + double(cert.rmax));
      const double V = double(cert.s2) * dk * (1.0 + double(cert.rho));
      const double T = double(unord_f32(tau));
      const double r = T > A ? std::sqrt(T - A) : 0.0;
      const double lb = r > E_ ? (r - E_) * (r - E_) : 0.0;
      if (!(lb * (1.0 - 0x1p-40) > V)) {
        mode = kCertKeys;
        tneed = V > 3.0e38 ? INFINITY
                           : float(((std::sqrt(V) + E_) * (std::sqrt(V) + E_) + A) * (1.0 + 0x1p-20));
      }
    }
    // Rows with keys up to T_need are re-ranked from the list when it holds
    // them all; otherwise from the key matrix, which a lazy pass defers.
    if (mode == kCertKeys && a.lazy && !(use_cand && ord_f32(tneed) <= t0)) {
      a.flag[ql] = 1;
      a.gflag[ql / 128] = 1;
      mode = kDeferred;
    } else {
      if (mode == kCertKeys) atomicAdd(&cert.counters[0], 1ull);
      if (!finite) {
        atomicAdd(&cert.counters[0], 1ull);
        atomicAdd(&cert.counters[1], 1ull);
      }
    }
    s_mode = mode;
    s_tneed = tneed;
  }
  __syncthreads();
  if (s_mode == kDeferred) return;
  if (s_mode != kCertPass) {
    const uint32_t hi = ord_f32(s_tneed);
    if (use_cand && hi <= t0)
      stream_cand([&](uint32_t o) { return o > tau && o <= hi; });
    else
      stream([&](uint32_t o) { return o > tau && o <= hi; });
    flush();
  }

  // 3. Output: k results by (distance, id), padded with UINT32_MAX / +inf.
  for (int64_t i = tid; i < k; i += kWT) {
    const uint64_t key = i < fill ? s_acc[i] : kSentinel;
    a.out_nbr[q * k + i] = key == kSentinel ? 0xffffffffu : uint32_t(key);
    a.out_dist[q * k + i] = key == kSentinel ? INFINITY : unord_f32(uint32_t(key >> 32));
  }
}

}  // namespace

void bf_wide_search(cvs_context* ctx, const cvs_dataset* ds, const float* queries, int64_t q, int64_t k,
                    uint32_t* nbr, float* dist) {
  const int ks = int(ds->dp / kStepCols);
  // k-steps per block of the keys kernel: 4 (padded dimensions of 64 and
  // more are multiples of 64), else the whole of 2.
  const int kb = ks % 4 == 0 ? 4 : ks;
  if (kb != 4 && kb != 2) fail(CVS_ERR_RUNTIME, "bf_wide_search: unexpected padded dimension");
  const int64_t q_tiles4 = ((q + 31) / 32 + 3) / 4 * 4;
  const int64_t ldk = ds->n_tiles * kTileRows;
  // Queries per chunk: a multiple of 128, at most 512, keys within ~2 GiB.
  int64_t qc = kChunkQ;
  while (qc > 128 && qc * ldk * 4 > (int64_t(2) << 30)) qc -= 128;
  qc = std::min<int64_t>(qc, (q + 127) / 128 * 128);
  auto align = [](size_t b) { return (b + 255) / 256 * 256; };
  const size_t off_qn = align(size_t(q_tiles4) * size_t(ks) * kStepBytes);
  const size_t off_qe = off_qn + align(size_t(q_tiles4) * 32 * sizeof(float));
  const size_t off_keys = off_qe + align(size_t(q) * sizeof(float));
  const size_t total = off_keys + align(size_t(qc) * size_t(ldk) * sizeof(float));

  // Rows re-ranked before the certificate: twice k (at least k + 32), as
  // the fused path keeps, so that the rank gap between the k-th result and
  // the R-th key clears the fp16 error on dense neighbourhoods.
  const int R = int(std::min<int64_t>(ds->n, std::max<int64_t>(2 * k, k + 32)));
  // Sampled threshold: the keys of S_tiles evenly strided dataset tiles
  // (S = 32 S_tiles rows, at most 16,384); the r-th smallest lies below the
  // query's R-th smallest key only if r of the sampled rows fall among its R
  // nearest, a count close to Poisson with mean lambda = R * S / n, so r is
  // the smallest rank with P(Poisson(lambda) >= r) <= 1e-9 (r = R when every
  // tile is sampled).  About r * n / S keys then lie at or below it; the
  // sample is used only when that many, six standard deviations over, fit
  // the candidate list.
  const int64_t real_tiles = (ds->n + kTileRows - 1) / kTileRows;
  const int64_t s_tiles = std::min<int64_t>(real_tiles, int64_t(kSampleM) * kWT / kTileRows);
  const int64_t s_stride = real_tiles / s_tiles;
  const int64_t S = s_tiles * kTileRows;
  const int64_t s_ld = (s_tiles + 3) / 4 * 4 * kTileRows;  // sample keys per query row
  int s_rank = R;
  if (s_tiles < real_tiles) {
    const double lambda = double(R) * double(S) / double(ds->n);
    double term = std::exp(-lambda), cdf = term;
    int r = 1;
    while (1.0 - cdf > 1e-9 && r < S) {
      term *= lambda / double(r);
      cdf += term;
      ++r;
    }
    s_rank = r;
  }
  const double per = double(ds->n) / double(S);
  const bool sampled = (double(s_rank) + 6.0 * std::sqrt(double(s_rank))) * per + per <= double(kCandCap);

  const size_t off_skeys = total;
  const size_t off_t0 = off_skeys + (sampled ? align(size_t(qc) * size_t(s_ld) * sizeof(float)) : 0);
  const size_t off_cnt = off_t0 + (sampled ? align(size_t(qc) * sizeof(uint32_t)) : 0);
  const size_t off_flag = off_cnt + (sampled ? align(size_t(qc) * sizeof(uint32_t)) : 0);
  const size_t off_gflag = off_flag + (sampled ? align(size_t(qc) * sizeof(uint32_t)) : 0);
  const size_t off_cand = off_gflag + (sampled ? align(size_t(qc / 128 + 1) * sizeof(uint32_t)) : 0);
  const size_t total_all = off_cand + (sampled ? align(size_t(qc) * kCandCap * sizeof(uint64_t)) : 0);
  ctx->ws_search.reserve(total_all);
  char* ws = ctx->ws_search.as<char>();
  u32x4* qtiles = reinterpret_cast<u32x4*>(ws);
  float* qnorms = reinterpret_cast<float*>(ws + off_qn);
  float* qerr = reinterpret_cast<float*>(ws + off_qe);
  float* keys = reinterpret_cast<float*>(ws + off_keys);
  float* skeys = sampled ? reinterpret_cast<float*>(ws + off_skeys) : nullptr;
  uint32_t* t0s = sampled ? reinterpret_cast<uint32_t*>(ws + off_t0) : nullptr;
  uint32_t* cnt = sampled ? reinterpret_cast<uint32_t*>(ws + off_cnt) : nullptr;
  uint64_t* cand = sampled ? reinterpret_cast<uint64_t*>(ws + off_cand) : nullptr;
  uint32_t* flag = sampled ? reinterpret_cast<uint32_t*>(ws + off_flag) : nullptr;
  uint32_t* gflag = sampled ? reinterpret_cast<uint32_t*>(ws + off_gflag) : nullptr;

  const TimerSpan t0 = timer_span(ctx, "bf_prep");
  launch_query_tiles(ctx, ds, queries, q, q_tiles4 * 32, qtiles, qnorms, qerr, t0.start, t0.stop);
  const Cert cert = make_cert(ctx, ds, qnorms, qerr);

  const size_t cand_lds = size_t(kCandCap) * sizeof(uint64_t);
  CVS_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(wide_select_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, int(cand_lds)));
  auto launch_keys = [&](dim3 grid, const KeysArgs& ka, hipEvent_t e0, hipEvent_t e1) {
    if (kb == 4)
      hipExtLaunchKernelGGL(wide_keys_kernel<4>, grid, dim3(kWT), 0, ctx->stream, e0, e1, 0, ka);
    else
      hipExtLaunchKernelGGL(wide_keys_kernel<2>, grid, dim3(kWT), 0, ctx->stream, e0, e1, 0, ka);
    after_launch("wide_keys_kernel");
  };
  for (int64_t c0 = 0; c0 < q; c0 += qc) {
    const int64_t nq = std::min(qc, q - c0);
    const unsigned qgroups = unsigned((nq + 127) / 128);
    KeysArgs ka{};
    ka.tiles = reinterpret_cast<const u32x4*>(ds->tiles);
    ka.norms = ds->norms;
    ka.ks = ks;
    ka.qtiles = qtiles;
    ka.qnorms = qnorms;
    ka.qt0 = int(c0 / 32);
    ka.nq = int(nq);
    ka.qgroups = int(qgroups);
    ka.n = ds->n;
    ka.write_keys = 1;
    if (sampled) {
      // Keys of the sampled tiles, then each query's threshold.
      KeysArgs sk = ka;
      sk.keys = skeys;
      sk.ldk = s_ld;
      sk.n_idx = s_tiles;
      sk.tile_stride = s_stride;
      const TimerSpan ts = timer_span(ctx, "bf_sample");
      launch_keys(dim3(unsigned(s_ld / kTileRows / 4) * qgroups), sk, ts.start, nullptr);
      hipExtLaunchKernelGGL(wide_threshold_kernel, dim3(unsigned(nq)), dim3(kWT), 0, ctx->stream, nullptr, ts.stop,
                            0, skeys, int64_t(s_ld), int(S), s_rank, t0s, cnt, flag, gflag);
      after_launch("wide_threshold_kernel");
      ka.t0 = t0s;
      ka.cnt = cnt;
      ka.cand = cand;
      ka.cand_cap = kCandCap;
      ka.write_keys = 0;  // written later, for flagged query blocks only
    }
    ka.keys = keys;
    ka.ldk = ldk;
    ka.n_idx = ds->n_tiles;
    ka.tile_stride = 1;
    const TimerSpan t1 = timer_span(ctx, "bf_scan");
    launch_keys(dim3(unsigned(ds->n_tiles / 4) * qgroups), ka, t1.start, t1.stop);
    SelectArgs sa{};
    sa.keys = keys;
    sa.ldk = ldk;
    sa.n = ds->n;
    sa.d = ds->d;
    sa.q0 = int(c0);
    sa.R = R;
    sa.t0 = t0s;
    sa.cnt = cnt;
    sa.cand = cand;
    sa.cand_cap = kCandCap;
    sa.flag = flag;
    sa.gflag = gflag;
    sa.lazy = sampled ? 1 : 0;
    sa.k = k;
    sa.rows = ds->rows;
    sa.queries = queries;
    sa.out_nbr = nbr;
    sa.out_dist = dist;
    const TimerSpan t2 = timer_span(ctx, "bf_merge");
    hipExtLaunchKernelGGL(wide_select_kernel, dim3(unsigned(nq)), dim3(kWT), cand_lds, ctx->stream, t2.start,
                          sampled ? nullptr : t2.stop, 0, sa, cert);
    after_launch("wide_select_kernel");
    if (sampled) {
      // Second pass for the queries the list did not serve (none on most
      // batches: its launches then return at once): the key matrix of the
      // flagged query blocks, then the full radix select for those queries.
      KeysArgs fk = ka;
      fk.t0 = nullptr;
      fk.write_keys = 1;
      fk.gflag = gflag;
      launch_keys(dim3(unsigned(ds->n_tiles / 4) * qgroups), fk, nullptr, nullptr);
      SelectArgs fs = sa;
      fs.cand = nullptr;
      fs.lazy = 0;
      fs.only_flagged = 1;
      hipExtLaunchKernelGGL(wide_select_kernel, dim3(unsigned(nq)), dim3(kWT), cand_lds, ctx->stream, nullptr,
                            t2.stop, 0, fs, cert);
      after_launch("wide_select_kernel");
    }
  }
}

}  // namespace bf
}  // namespace cvs
