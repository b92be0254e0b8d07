// Fused exact brute-force k-NN for gfx950.
//
// Replaces the reference's two-pass GPU brute force
// (src/metal_context.mm:139-255): an MPS fp16 GEMM that writes the whole
// Q x N fp32 cross matrix to memory (:203-225) followed by
// `l2_topk_from_cross` (shaders/cagra_kernels.metal:604-653), which re-reads
// it and keeps a per-thread K-slot list merged serially by thread 0.
//
// Here the cross matrix never leaves registers:
//
//  bf_scan   one persistent workgroup per compute unit streams a contiguous
//            range of 16-row fp16 tiles HBM -> VGPRs -> LDS (double-buffered
//            LDS, two stages of loads in flight).  Each of the 4 waves keeps
//            the fp16 MFMA operands of its 32 queries for the full dimension
//            resident in VGPRs and computes query.row cross terms with
//            v_mfma_f32_16x16x32_f16 (fp32 accumulate).  The epilogue forms
//            d = |q|^2 + |x|^2 - 2 q.x and appends (d, row) to the query's LDS
//            candidate list only if d is below the query's running threshold.
//            When a list nears capacity the owning wave compacts it to the
//            kp smallest keys with a radix select and lowers the threshold.
//            Each workgroup finally writes its kp best keys per query.
//  bf_merge  one workgroup per query selects the kp smallest of all partial
//            lists, re-ranks them with exact fp32 distances from the fp32
//            rows, sorts by (distance, id) and writes k results, padding with
//            UINT32_MAX / +inf (src/cagra.cpp:240-251).
//
// The fp16 pass only *selects*; reported distances come from the fp32
// re-rank, so distances agree with the reference's fp32 loop
// (src/cagra.cpp:218-226) up to summation order.  kp > k candidates are kept
// because fp16 inputs perturb |q-x|^2 by up to ~1e-4 absolute at unit norm,
// which is far below the gap between rank k and rank kp.
#include <cmath>

#include "cvs_internal.hpp"

namespace cvs {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves
constexpr int kWaves = 4;
constexpr int kStageBytes = 32768;
constexpr int kStageVecs = kStageBytes / 16;           // 16-byte vectors per stage
constexpr int kLoadsPerThread = kStageVecs / kThreads;  // 8
constexpr uint64_t kSentinel = ~0ull;

#define CVS_INLINE __attribute__((always_inline))

// Order-preserving map float -> uint32 (total order for non-NaN values).
__device__ __forceinline__ uint32_t ord_f32(float f) {
  const uint32_t u = __float_as_uint(f + 0.0f);  // -0 -> +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float unord_f32(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

template <int KS, int QS>
struct Scan {
  static constexpr int TPS = KS >= 32 ? 1 : 32 / KS;  // 16-row tiles per stage
  static constexpr int QPW = 16 * QS;                  // queries per wave
  static constexpr int QB = kWaves * QPW;              // queries per workgroup
  static constexpr int CAP = QS == 2 ? 88 : 176;       // LDS candidate slots per query
  static constexpr int EPL = CAP / 4;                  // slots per lane in compaction
  static_assert(KS * TPS * 1024 == kStageBytes || KS > 32, "stage must be 32 KiB");
};

struct ScanArgs {
  const u32x4* tiles;   // dataset tiles (stage-padded)
  const f32x4* norms;   // dataset norms, 16 per tile
  int64_t n_stages;
  const u32x4* qtiles;  // query tiles
  const float* qnorms;  // query norms, 16 per query tile
  int nq;
  int n_qslices;        // number of 16-query tiles
  int kp;               // candidates kept per (workgroup, query)
  uint64_t* part;       // [nq][gridDim.x][kp]
};

// Selects the kp-th smallest 64-bit key of one query's list, held by 4
// consecutive lanes (entries g, g+4, g+8, ... of `cnt`), and compacts the
// list in place to exactly min(cnt, kp) keys.  Returns the new threshold
// (distance of the kp-th key) through *thr_out on lane g == 0.
template <int EPL>
__device__ __forceinline__ void compact_list(uint64_t* list, uint32_t* cnt_slot, float* thr_slot,
                                             int g, int kp, bool active) {
  const uint32_t cnt = active ? *cnt_slot : 0u;
  const bool work = active && cnt > uint32_t(kp);
  const int nv = (work && cnt > uint32_t(g)) ? int((cnt - g + 3) / 4) : 0;
  uint32_t hi[EPL], lo[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    if (i < nv) {
      const uint64_t key = list[g + 4 * i];
      hi[i] = uint32_t(key >> 32);
      lo[i] = uint32_t(key);
    } else {
      hi[i] = 0xffffffffu;
      lo[i] = 0xffffffffu;
    }
  }
  // Radix select on the distance word.
  int need = kp;
  uint32_t pre = 0;
  for (int b = 31; b >= 0; --b) {
    int c = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) c += (i < nv && ((hi[i] ^ pre) >> b) == 0) ? 1 : 0;
    c += __shfl_xor(c, 1);
    c += __shfl_xor(c, 2);
    if (c < need) {
      need -= c;
      pre |= 1u << b;
    }
  }
  const uint32_t kth_hi = pre;
  int lt = 0, eq = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    lt += (i < nv && hi[i] < kth_hi) ? 1 : 0;
    eq += (i < nv && hi[i] == kth_hi) ? 1 : 0;
  }
  lt += __shfl_xor(lt, 1);
  lt += __shfl_xor(lt, 2);
  eq += __shfl_xor(eq, 1);
  eq += __shfl_xor(eq, 2);
  const int need_eq = kp - lt;
  uint32_t kth_lo = 0xffffffffu;
  if (__ballot(work && eq > need_eq) != 0) {
    // Ties on the distance word: select on the row id among them.
    int need2 = need_eq;
    uint32_t pre2 = 0;
    for (int b = 31; b >= 0; --b) {
      int c = 0;
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        c += (i < nv && hi[i] == kth_hi && ((lo[i] ^ pre2) >> b) == 0) ? 1 : 0;
      c += __shfl_xor(c, 1);
      c += __shfl_xor(c, 2);
      if (c < need2) {
        need2 -= c;
        pre2 |= 1u << b;
      }
    }
    if (eq > need_eq) kth_lo = pre2;
  }
  // In-place compaction (all entries are already in registers).
  int kc = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    kc += (i < nv && (hi[i] < kth_hi || (hi[i] == kth_hi && lo[i] <= kth_lo))) ? 1 : 0;
  const int lane = __lane_id();
  const int base = lane & ~3;
  const int k0 = __shfl(kc, base + 0), k1 = __shfl(kc, base + 1), k2 = __shfl(kc, base + 2);
  int pos = (g > 0 ? k0 : 0) + (g > 1 ? k1 : 0) + (g > 2 ? k2 : 0);
  if (work) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      if (i < nv && (hi[i] < kth_hi || (hi[i] == kth_hi && lo[i] <= kth_lo))) {
        list[pos++] = (uint64_t(hi[i]) << 32) | lo[i];
      }
    }
    if (g == 0) {
      *cnt_slot = uint32_t(kp);
      *thr_slot = unord_f32(kth_hi);
    }
  }
}

template <int KS, int QS>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void bf_scan_kernel(ScanArgs a) {
  using C = Scan<KS, QS>;
  constexpr int TPS = C::TPS, QPW = C::QPW, QB = C::QB, CAP = C::CAP;

  __shared__ u32x4 s_stage[2][kStageVecs];
  __shared__ float s_dn[2][TPS * 16];
  __shared__ uint32_t s_cnt[QB];
  __shared__ float s_thr[QB];
  __shared__ uint64_t s_buf[QB * CAP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int G = gridDim.x;
  const int x = blockIdx.x;
  const int qbase = blockIdx.y * QB;  // first query of this workgroup
  const int kp = a.kp;

  // Stage range of this workgroup.
  const int64_t st0 = (a.n_stages * x) / G;
  const int64_t st1 = (a.n_stages * (x + 1)) / G;

  // ---- per-query LDS state ----
  for (int i = tid; i < QB; i += kThreads) {
    s_cnt[i] = 0;
    s_thr[i] = (qbase + i < a.nq) ? INFINITY : -INFINITY;
  }

  // ---- resident query operands: wave owns queries [qbase + wave*QPW, +QPW) ----
  half8 qa[QS][KS];
  float qn[QS][4];
  float thr[QS][4];
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) {
    const int sl = (qbase >> 4) + wave * QS + qs;
    const bool ok = sl < a.n_qslices;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4 v = ok ? a.qtiles[(int64_t(sl) * KS + s) * 64 + lane] : u32x4{0, 0, 0, 0};
      half8 h = __builtin_bit_cast(half8, v);
      // Pin the resident operand to an AGPR: MFMA reads A from AGPRs, and the
      // 256 arch VGPRs stay free for stage loads and B-fragment prefetch.
      asm volatile("" : "+a"(h));
      qa[qs][s] = h;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = qbase + wave * QPW + qs * 16 + 4 * (lane >> 4) + j;
      qn[qs][j] = (ok && q < a.nq) ? a.qnorms[int64_t(sl) * 16 + 4 * (lane >> 4) + j] : INFINITY;
      thr[qs][j] = q < a.nq ? INFINITY : -INFINITY;
    }
  }

  // ---- stage loads: HBM -> registers -> LDS ----
  u32x4 ra[kLoadsPerThread], rb[kLoadsPerThread];
  f32x4 na = {0, 0, 0, 0}, nb = {0, 0, 0, 0};
  const bool norm_loader = tid < TPS * 4;
  auto gload = [&](u32x4 (&r)[kLoadsPerThread], f32x4& nr, int64_t st) CVS_INLINE {
    const u32x4* src = a.tiles + st * kStageVecs + tid;
#pragma unroll
    for (int i = 0; i < kLoadsPerThread; ++i) r[i] = __builtin_nontemporal_load(src + i * kThreads);
    if (norm_loader) nr = a.norms[st * TPS * 4 + tid];
  };
  auto lstore = [&](int buf, const u32x4 (&r)[kLoadsPerThread], const f32x4& nr) CVS_INLINE {
#pragma unroll
    for (int i = 0; i < kLoadsPerThread; ++i) s_stage[buf][tid + i * kThreads] = r[i];
    if (norm_loader) *reinterpret_cast<f32x4*>(&s_dn[buf][tid * 4]) = nr;
  };

  auto refresh_thr = [&]() CVS_INLINE {
#pragma unroll
    for (int qs = 0; qs < QS; ++qs)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        thr[qs][j] = s_thr[wave * QPW + qs * 16 + 4 * (lane >> 4) + j];
  };

  // Compacts the lists of this wave's queries whose count exceeds `limit`.
  auto compact_wave = [&](uint32_t limit) CVS_INLINE {
#pragma unroll
    for (int r = 0; r < QS; ++r) {
      const int qw = r * 16 + (lane >> 2);
      const int m = wave * QPW + qw;
      const bool active = qbase + m < a.nq && s_cnt[m] > limit;
      compact_list<C::EPL>(s_buf + m * CAP, &s_cnt[m], &s_thr[m], lane & 3, kp, active);
    }
    refresh_thr();
  };

  auto compute = [&](int buf, int64_t st) CVS_INLINE {
    const u32x4* sb = s_stage[buf];
#pragma unroll 1
    for (int rt = 0; rt < TPS; ++rt) {
      f32x4 acc[QS];
#pragma unroll
      for (int qs = 0; qs < QS; ++qs) acc[qs] = f32x4{0, 0, 0, 0};
      const u32x4* tb = sb + rt * KS * 64 + lane;
      // B fragments (16 rows x 32 columns per k-step) through a PF-deep
      // register ring so LDS latency overlaps the MFMAs.
      constexpr int PF = KS < 4 ? KS : 4;
      half8 bring[PF];
#pragma unroll
      for (int j = 0; j < PF; ++j) bring[j] = __builtin_bit_cast(half8, tb[j * 64]);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const half8 b = bring[s % PF];
        if (s + PF < KS) bring[s % PF] = __builtin_bit_cast(half8, tb[(s + PF) * 64]);
#pragma unroll
        for (int qs = 0; qs < QS; ++qs)
          acc[qs] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[qs][s], b, acc[qs], 0, 0, 0);
      }
      // Schedule: PF reads up front, then (QS MFMAs, 1 read) pairs, then drain.
#pragma unroll
      for (int j = 0; j < PF; ++j) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
      for (int j = 0; j < KS - PF; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, QS, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, QS * PF, 0);
      // Epilogue: lane holds rows 4*(lane/16)+j of each query slice, row lane%16.
      const float dn = s_dn[buf][rt * 16 + (lane & 15)];
      const uint32_t row = uint32_t((st * TPS + rt) * 16 + (lane & 15));
#pragma unroll
      for (int qs = 0; qs < QS; ++qs) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float d = qn[qs][j] + dn - 2.0f * acc[qs][j];
          if (d < thr[qs][j]) {
            const int m = wave * QPW + qs * 16 + 4 * (lane >> 4) + j;
            const uint32_t slot = atomicAdd(&s_cnt[m], 1u);
            s_buf[m * CAP + slot] = (uint64_t(ord_f32(d)) << 32) | row;
          }
        }
      }
      // Keep room for the next tile (at most 16 new keys per query).
      const bool over = lane < QPW && s_cnt[wave * QPW + lane] > uint32_t(CAP - 16);
      if (__ballot(over) != 0) compact_wave(uint32_t(CAP - 16));
    }
  };

  // ---- software pipeline: LDS double buffer, two stages of loads in flight ----
  if (st0 < st1) gload(ra, na, st0);
  if (st0 + 1 < st1) gload(rb, nb, st0 + 1);
  if (st0 < st1) lstore(0, ra, na);
  if (st0 + 2 < st1) gload(ra, na, st0 + 2);
  __syncthreads();
  for (int64_t st = st0; st < st1; st += 2) {
    // stage st in LDS buffer 0; rb holds st+1, ra holds st+2
    compute(0, st);
    if (st + 1 < st1) lstore(1, rb, nb);
    if (st + 3 < st1) gload(rb, nb, st + 3);
    __syncthreads();
    if (st + 1 >= st1) break;
    compute(1, st + 1);
    if (st + 2 < st1) lstore(0, ra, na);
    if (st + 4 < st1) gload(ra, na, st + 4);
    __syncthreads();
  }

  // ---- final compaction to kp and write-out ----
  compact_wave(uint32_t(kp));
  const int64_t G64 = G;
  for (int i = lane; i < QPW * kp; i += 64) {
    const int qw = i / kp, e = i - qw * kp;
    const int m = wave * QPW + qw;
    const int q = qbase + m;
    if (q >= a.nq) continue;
    const uint32_t c = s_cnt[m];
    a.part[(int64_t(q) * G64 + x) * kp + e] = uint32_t(e) < c ? s_buf[m * CAP + e] : kSentinel;
  }
}

// ---------------------------------------------------------------------------
// Merge + exact re-rank: one workgroup per query.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int block_sum(int v, int* s_red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s_red[wave] = v;
  __syncthreads();
  return s_red[0] + s_red[1] + s_red[2] + s_red[3];
}

template <int EPT>
__global__ __launch_bounds__(256) void bf_merge_kernel(const uint64_t* __restrict__ part, int m_keys,
                                                       int kp, const float* __restrict__ rows,
                                                       int64_t d, const float* __restrict__ queries,
                                                       int64_t k, uint32_t* __restrict__ out_nbr,
                                                       float* __restrict__ out_dist) {
  __shared__ int s_red[kWaves];
  __shared__ int s_n;
  __shared__ uint64_t s_sel[64];
  __shared__ float s_ex[64];
  const int tid = threadIdx.x;
  const int64_t q = blockIdx.x;
  const uint64_t* src = part + q * int64_t(m_keys);

  uint32_t hi[EPT], lo[EPT];
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int e = tid + i * kThreads;
    const uint64_t key = e < m_keys ? src[e] : kSentinel;
    hi[i] = uint32_t(key >> 32);
    lo[i] = uint32_t(key);
  }
  if (tid == 0) s_n = 0;

  // kp-th smallest key: radix select on the distance word, then on the id.
  int need = kp;
  uint32_t pre = 0;
  for (int b = 31; b >= 0; --b) {
    int c = 0;
#pragma unroll
    for (int i = 0; i < EPT; ++i) c += ((hi[i] ^ pre) >> b) == 0 ? 1 : 0;
    c = block_sum(c, s_red);
    if (c < need) {
      need -= c;
      pre |= 1u << b;
    }
  }
  const uint32_t kth_hi = pre;
  uint32_t pre2 = 0;
  for (int b = 31; b >= 0; --b) {
    int c = 0;
#pragma unroll
    for (int i = 0; i < EPT; ++i) c += (hi[i] == kth_hi && ((lo[i] ^ pre2) >> b) == 0) ? 1 : 0;
    c = block_sum(c, s_red);
    if (c < need) {
      need -= c;
      pre2 |= 1u << b;
    }
  }
  const uint64_t kth = (uint64_t(kth_hi) << 32) | pre2;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const uint64_t key = (uint64_t(hi[i]) << 32) | lo[i];
    if (key <= kth && key != kSentinel) {
      const int p = atomicAdd(&s_n, 1);
      if (p < 64) s_sel[p] = key;
    }
  }
  __syncthreads();
  const int n_sel = s_n < kp ? s_n : kp;

  // Exact fp32 distances: one wave per candidate.
  const int wave = tid >> 6, lane = tid & 63;
  const float* qv = queries + q * d;
  for (int c = wave; c < n_sel; c += kWaves) {
    const uint32_t row = uint32_t(s_sel[c]);
    const float* xv = rows + int64_t(row) * d;
    float acc = 0.f;
    for (int64_t i = lane; i < d; i += 64) {
      const float t = qv[i] - xv[i];
      acc += t * t;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
    if (lane == 0) s_ex[c] = acc;
  }
  __syncthreads();

  // Rank sort by (distance, id); write k results with padding.
  if (tid < n_sel) {
    const float dv = s_ex[tid];
    const uint32_t iv = uint32_t(s_sel[tid]);
    int rank = 0;
    for (int j = 0; j < n_sel; ++j) {
      const float dj = s_ex[j];
      const uint32_t ij = uint32_t(s_sel[j]);
      rank += (dj < dv || (dj == dv && ij < iv)) ? 1 : 0;
    }
    if (rank < k) {
      out_nbr[q * k + rank] = iv;
      out_dist[q * k + rank] = dv;
    }
  }
  for (int64_t r = n_sel + tid; r < k; r += kThreads) {
    out_nbr[q * k + r] = 0xffffffffu;
    out_dist[q * k + r] = INFINITY;
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
int choose_kp(int64_t k) {
  if (k <= 10) return 16;
  if (k <= 24) return 32;
  return 64;
}

template <int KS>
void launch_scan(cvs_context* ctx, dim3 grid, const ScanArgs& args) {
  hipLaunchKernelGGL((bf_scan_kernel<KS, 2>), grid, dim3(kThreads), 0, ctx->stream, args);
}

template <int EPT>
void launch_merge(cvs_context* ctx, int64_t q, const uint64_t* part, int m_keys, int kp,
                  const cvs_dataset* ds, const float* queries, int64_t k, uint32_t* nbr,
                  float* dist) {
  hipLaunchKernelGGL((bf_merge_kernel<EPT>), dim3(unsigned(q)), dim3(kThreads), 0, ctx->stream,
                     part, m_keys, kp, ds->rows, ds->d, queries, k, nbr, dist);
}

void bf_search_device(cvs_context* ctx, const cvs_dataset* ds, const float* queries, int64_t q,
                      int64_t k, uint32_t* nbr, float* dist) {
  if (!ds || ds->ctx != ctx) fail(CVS_ERR_INVALID_ARGUMENT, "dataset does not belong to context");
  if (!queries || !nbr || !dist) fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
  if (q <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "query count must be positive");
  if (k <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "k must be positive");
  if (k > CVS_BF_MAX_K) fail(CVS_ERR_UNSUPPORTED, "k exceeds CVS_BF_MAX_K for the fused kernel");
  if (ds->d > CVS_BF_MAX_DIM)
    fail(CVS_ERR_UNSUPPORTED, "dimension exceeds CVS_BF_MAX_DIM for the fused kernel");
  if (q > (int64_t(1) << 24)) fail(CVS_ERR_UNSUPPORTED, "too many queries in one call");

  const int ks = int(ds->dp / kStepCols);
  const int tps = ks >= 32 ? 1 : 32 / ks;
  const int64_t n_stages = ds->n_tiles / tps;
  int G = ctx->compute_units;
  if (G > 256) G = 256;
  if (int64_t(G) > n_stages) G = int(n_stages);
  const int kp = choose_kp(k);
  const int qb = 128;
  const int64_t q_tiles = (q + 15) / 16;

  // Workspaces: query tiles + norms, partial lists.
  const size_t qtile_bytes = size_t(q_tiles) * size_t(ks) * kStepBytes;
  const size_t qnorm_bytes = size_t(q_tiles) * 16 * sizeof(float);
  ctx->ws_queries.reserve(qtile_bytes + qnorm_bytes);
  uint16_t* qtiles = ctx->ws_queries.as<uint16_t>();
  float* qnorms = reinterpret_cast<float*>(ctx->ws_queries.as<char>() + qtile_bytes);
  const int m_keys = G * kp;
  ctx->ws_partial.reserve(size_t(q) * size_t(m_keys) * sizeof(uint64_t));
  uint64_t* part = ctx->ws_partial.as<uint64_t>();

  hipEvent_t t0 = timer_begin(ctx, "bf_prep");
  launch_to_tiles(ctx, queries, q, ds->d, ds->dp, q_tiles, qtiles, qnorms);
  timer_end(ctx, "bf_prep", t0);

  ScanArgs args;
  args.tiles = reinterpret_cast<const u32x4*>(ds->tiles);
  args.norms = reinterpret_cast<const f32x4*>(ds->norms);
  args.n_stages = n_stages;
  args.qtiles = reinterpret_cast<const u32x4*>(qtiles);
  args.qnorms = qnorms;
  args.nq = int(q);
  args.n_qslices = int(q_tiles);
  args.kp = kp;
  args.part = part;
  const dim3 grid(unsigned(G), unsigned((q + qb - 1) / qb));
  hipEvent_t t1 = timer_begin(ctx, "bf_scan");
  switch (ks) {
    case 1: launch_scan<1>(ctx, grid, args); break;
    case 2: launch_scan<2>(ctx, grid, args); break;
    case 4: launch_scan<4>(ctx, grid, args); break;
    case 8: launch_scan<8>(ctx, grid, args); break;
    case 16: launch_scan<16>(ctx, grid, args); break;
    case 32: launch_scan<32>(ctx, grid, args); break;
    default: fail(CVS_ERR_UNSUPPORTED, "unsupported padded dimension");
  }
  after_launch("bf_scan_kernel");
  timer_end(ctx, "bf_scan", t1);

  hipEvent_t t2 = timer_begin(ctx, "bf_merge");
  const int ept = (m_keys + kThreads - 1) / kThreads;
  if (ept <= 16)
    launch_merge<16>(ctx, q, part, m_keys, kp, ds, queries, k, nbr, dist);
  else if (ept <= 32)
    launch_merge<32>(ctx, q, part, m_keys, kp, ds, queries, k, nbr, dist);
  else
    launch_merge<64>(ctx, q, part, m_keys, kp, ds, queries, k, nbr, dist);
  after_launch("bf_merge_kernel");
  timer_end(ctx, "bf_merge", t2);
}

}  // namespace
}  // namespace cvs

using namespace cvs;

extern "C" {

int cvs_bf_search_async(cvs_context* ctx, const cvs_dataset* ds, const float* queries_dev,
                        int64_t q, int64_t k, uint32_t* out_neighbors_dev,
                        float* out_distances_dev) {
  return guarded([&] {
    bind(ctx);
    bf_search_device(ctx, ds, queries_dev, q, k, out_neighbors_dev, out_distances_dev);
  });
}

int cvs_bf_search(cvs_context* ctx, const cvs_dataset* ds, const float* queries, int64_t q,
                  int64_t k, uint32_t* out_neighbors, float* out_distances) {
  return guarded([&] {
    bind(ctx);
    if (!ds || !queries || !out_neighbors || !out_distances)
      fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
    if (q <= 0 || k <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "query count and k must be positive");
    const size_t qbytes = size_t(q) * size_t(ds->d) * sizeof(float);
    const size_t obytes = size_t(q) * size_t(k) * sizeof(float);
    ctx->ws_io.reserve(qbytes + 2 * obytes + 256);
    char* base = ctx->ws_io.as<char>();
    float* dq = reinterpret_cast<float*>(base);
    uint32_t* dn = reinterpret_cast<uint32_t*>(base + (qbytes + 127) / 128 * 128);
    float* dd = reinterpret_cast<float*>(reinterpret_cast<char*>(dn) + (obytes + 127) / 128 * 128);
    CVS_HIP(hipMemcpyAsync(dq, queries, qbytes, hipMemcpyHostToDevice, ctx->stream));
    bf_search_device(ctx, ds, dq, q, k, dn, dd);
    CVS_HIP(hipMemcpyAsync(out_neighbors, dn, obytes, hipMemcpyDeviceToHost, ctx->stream));
    CVS_HIP(hipMemcpyAsync(out_distances, dd, obytes, hipMemcpyDeviceToHost, ctx->stream));
    CVS_HIP(hipStreamSynchronize(ctx->stream));
  });
}

}  // extern "C"
