// Fused exact brute-force k-NN for gfx950.
//
// Replaces the reference's two-pass GPU brute force
// (src/metal_context.mm:139-255): an MPS fp16 GEMM that writes the whole
// Q x N fp32 cross matrix to memory (:203-225) followed by
// `l2_topk_from_cross` (shaders/cagra_kernels.metal:604-653), which re-reads
// it and keeps a per-thread K-slot list merged serially by thread 0.
//
// Here the cross matrix never leaves registers.  Five launches per batch:
//
//  prep     queries fp32 -> fp16 32-row tiles + norms (the dataset layout),
//           one wave per query.
//  sample   the scan kernel over an evenly strided sample of 16,384 rows
//           (65,536 for other large batches, 32,768 when the register-blocked
//           scan of bf_gemm.hip follows); each lane keeps the minimum distance
//           of the rows it sees, so every (query, workgroup, half-wave)
//           yields one minimum.
//  select   per query (one wave), the r-th smallest of those minima, T0.
//           The r smallest minima are r distinct dataset rows, so at least r
//           rows lie at or below T0 and every row above it can be dropped by
//           the scan.  r is set on the host (plan_bf) so that T0 falls below
//           the merge's R candidates with probability at most 1e-9.
//  scan     one persistent workgroup per compute unit streams a contiguous
//           range of fp16 tiles HBM -> VGPRs -> LDS (double-buffered LDS, two
//           stages of loads in flight).  Each wave keeps the fp16 operands of
//           its 32 queries for the full dimension resident in AGPRs; the
//           dataset tile is the A operand of v_mfma_f32_32x32x16_f16 (fp32
//           accumulate, two accumulation chains), so each lane owns one query
//           and 16 rows of the 32x32 result.  The epilogue forms
//           d = |q|^2 + |x|^2 - 2 q.x and appends (d, row) to the query's list
//           only if d is below the query's threshold (T0 at start).  Each
//           list has two halves, one per lane of its query, with the count in
//           a register; a rare append visits only the rows some lane passes.
//           A half that fills up is compacted by its wave to the kp smallest
//           keys (ballot radix select), lowering the threshold.  Lists of
//           kp <= 64 live in LDS, kp = 128 lists in global memory.  Each list
//           ends with its smallest key published for the merge.
//  merge    one workgroup per query: the R-th smallest list minimum bounds
//           the R-th smallest key (R = 2 kp, at most 256).  For kp <= 64 every
//           key within it is gathered into LDS and one wave keeps the R
//           smallest; for kp = 128 each wave merges the 64-key rows holding a
//           key within the bound into its running top-R.  The R candidates
//           are re-ranked with exact fp32 distances from the fp32 rows,
//           sorted by (distance, id), certified against the fp16 error bound
//           (bf_common.hpp, Cert; a query that fails is re-ranked over more
//           rows), and k results written, padded with UINT32_MAX / +inf
//           (src/cagra.cpp:240-251).
//
// The fp16 pass only *selects*; reported distances come from the fp32
// re-rank, so distances agree with the reference's fp32 loop
// (src/cagra.cpp:218-226) up to summation order, and the certificate makes
// the selection exact on any finite input: rows and queries are centred and
// scaled by a power of two before the fp16 conversion (runtime.hip).
#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>
#include <type_traits>

#include "bf_common.hpp"
#include "cvs_internal.hpp"
#include "device_util.hpp"

namespace cvs {
namespace {

using namespace bf;

constexpr int kThreads = 256;  // 4 waves
constexpr int kWaves = 4;
constexpr int kQB = 128;                                // queries per workgroup (32 per wave)
constexpr int kStageBlocks = 32;                        // 1 KiB blocks per stage
constexpr int kStageVecs = kStageBlocks * 64;           // 16-byte vectors per stage
constexpr int kLoadsPerThread = kStageVecs / kThreads;  // 8 16-byte loads per thread and stage

template <int KS>
struct Cfg {
  static constexpr int TPS = KS >= 32 ? 1 : 32 / KS;      // tiles per stage
  static constexpr int SPT = KS >= 32 ? KS / 32 : 1;      // stages per tile
  static constexpr int RPU = 2 * kStageBlocks * 32 / KS;  // rows per 2-stage unit
  static constexpr int NF = TPS * 32;                     // norms per stage
  static_assert(KS >= 2 && KS <= 64, "k-steps per tile");
};

struct ScanArgs {
  const u32x4* tiles;   // dataset tiles (unit-padded)
  const f32x4* norms;   // dataset norms, 32 per tile
  int64_t n_units;      // 2-stage units in the dataset
  const u32x4* qtiles;  // query tiles
  const float* qnorms;  // query norms, 32 per query tile
  int nq;
  int n_qtiles;         // number of 32-query tiles
  int kp;               // candidates kept per (workgroup, query)
  const float* thr0;    // per-query initial threshold (scan mode)
  uint64_t* part;       // scan: [nq][n_ranges][kp] keys (LDS lists) or
                        // [nq][n_ranges][CAP] lists, first kp valid (global lists)
  int n_ranges;         // dataset ranges (workgroups along N)
  int n_qblocks;        // 128-query blocks
  int qb_fast;          // 1: linear block id = range * n_qblocks + qblock
  float* sgmin;         // sample: [nq][2 * n_ranges] minima of each lane's sampled rows
  uint64_t* lmin;       // scan: [nq][n_ranges] smallest key of each list (sentinel if empty)
  float* lcut;          // scan: [nq][n_ranges] final threshold of each list: every row of the
                        // range that is not in its list has a distance key at or above it
  int64_t s_units;      // sample: number of sampled units
  int64_t s_stride;     // sample: unit stride
};

template <int KS, int MODE, int KP>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void bf_scan_kernel(ScanArgs a) {
  using C = Cfg<KS>;
  using L = Lists<KP, MODE>;
  constexpr int TPS = C::TPS, SPT = C::SPT, NF = C::NF;
  constexpr int CAP = L::CAP;
  // Scans over 32 or 64 k-steps per tile run the software-pipelined loop.
  constexpr bool PIPE = MODE == kModeScan && KS >= 32;

  __shared__ u32x4 s_stage[2][kStageVecs];
  __shared__ float s_dn[2][NF];
  __shared__ float s_dnp[PIPE ? 4 : 1][32];  // pipelined scan: norms of tiles t & 3
  __shared__ uint64_t s_buf[L::GL ? 1 : kQB * CAP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in a scalar register
  const int G = a.n_ranges;
  const int x = a.qb_fast ? int(blockIdx.x) / a.n_qblocks : int(blockIdx.x);
  const int qbase = (a.qb_fast ? int(blockIdx.x) % a.n_qblocks : int(blockIdx.y)) * kQB;
  // List of this workgroup's query slot m (0..127).
  auto list_of = [&](int m) CVS_INLINE -> uint64_t* {
    if constexpr (L::GL)
      return a.part + (int64_t(qbase + m) * G + x) * CAP;
    else
      return s_buf + m * CAP;
  };

  // Units of this workgroup: contiguous (scan) or a strided sample (sample).
  const int64_t total = MODE == kModeScan ? a.n_units : a.s_units;
  const int64_t i0 = (total * x) / G;
  const int64_t i1 = (total * (x + 1)) / G;
  const int n_stages = int(2 * (i1 - i0));
  auto unit_of = [&](int64_t i) CVS_INLINE -> int64_t {
    return MODE == kModeScan ? i : i * a.s_stride;
  };
  auto stage_of = [&](int j) CVS_INLINE -> int64_t { return 2 * unit_of(i0 + (j >> 1)) + (j & 1); };

  // ---- stage loads: HBM -> registers (two stages in flight) -> LDS ----
  constexpr int NPT = (NF + kThreads - 1) / kThreads;  // norms per thread and stage
  u32x4 ra[kLoadsPerThread], rb[kLoadsPerThread];
  float na[NPT], nb[NPT];
  auto gload = [&](u32x4 (&r)[kLoadsPerThread], float (&nr)[NPT], int j) CVS_INLINE {
    if (j >= n_stages) return;
    const int64_t st = stage_of(j);
    const u32x4* src = a.tiles + st * kStageVecs + tid;
#pragma unroll
    for (int i = 0; i < kLoadsPerThread; ++i) r[i] = __builtin_nontemporal_load(src + i * kThreads);
    const int64_t tile0 = KS >= 32 ? st / SPT : st * TPS;
    const float* ns = reinterpret_cast<const float*>(a.norms) + tile0 * 32;
#pragma unroll
    for (int i = 0; i < NPT; ++i)
      if (tid + i * kThreads < NF) nr[i] = ns[tid + i * kThreads];
  };
  auto lstore = [&](int buf, const u32x4 (&r)[kLoadsPerThread], const float (&nr)[NPT]) CVS_INLINE {
#pragma unroll
    for (int i = 0; i < kLoadsPerThread; ++i) s_stage[buf][tid + i * kThreads] = r[i];
#pragma unroll
    for (int i = 0; i < NPT; ++i)
      if (tid + i * kThreads < NF) s_dn[buf][tid + i * kThreads] = nr[i];
  };
  // Pipelined loop: buffer loads over this workgroup's contiguous stage
  // range; an offset past the range returns zeros without a memory access,
  // so loads beyond the last stage need no branch.
  constexpr uint32_t kStageBytes = kStageVecs * 16;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(reinterpret_cast<const char*>(a.tiles) + stage_of(0) * int64_t(kStageBytes)), 0,
      int(uint32_t(n_stages) * kStageBytes), kRsrcWord3);
  auto gload_b = [&](u32x4 (&r)[kLoadsPerThread], int j) CVS_INLINE {
    const uint32_t off = uint32_t(j) * kStageBytes + uint32_t(tid) * 16;
#pragma unroll
    for (int i = 0; i < kLoadsPerThread; ++i)
      r[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           rsrc, off + uint32_t(i * kThreads * 16), 0, kAuxNT));
  };
  if constexpr (PIPE) {
    gload_b(ra, 0);
    gload_b(rb, 1);
  } else {
    gload(ra, na, 0);
    gload(rb, nb, 1);
  }

  // ---- resident query operands: wave owns queries [qbase + 32*wave, +32) ----
  const int qt = (qbase >> 5) + wave;
  const int my_q = qbase + wave * 32 + (lane & 31);
  const bool q_ok = my_q < a.nq;
  // All KS operand loads are issued at once as buffer loads (a query tile
  // past the last one reads as zeros without a memory access), landing in
  // AGPRs, from which MFMA reads its B operand; this leaves the arch VGPRs
  // for the A-fragment ring, the accumulators and the epilogue.  They are
  // pinned to AGPRs only after the last load is issued, so the prologue
  // waits for one round trip.
  half8 qb[KS];
  const bool qt_ok = qt < a.n_qtiles;
  const __amdgpu_buffer_rsrc_t qrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4*>(a.qtiles + int64_t(qt_ok ? qt : 0) * KS * 64), 0, qt_ok ? KS * kStepBytes : 0,
      kRsrcWord3);
#pragma unroll
  for (int i = 0; i < KS; ++i)
    qb[i] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(
                                          qrsrc, uint32_t(lane) * 16u + uint32_t(i * kStepBytes), 0, 0));
#pragma unroll
  for (int i = 0; i < KS; ++i) asm volatile("" : "+a"(qb[i]));
  const float qn = q_ok ? a.qnorms[my_q] : INFINITY;
  const int qw = wave * 32 + (lane & 31);  // this lane's query slot in the workgroup
  const int half = lane >> 5;              // which half of the query's list this lane fills
  float thr = -INFINITY;
  float smin = INFINITY;  // sample mode: minimum over this lane's rows
  uint32_t cnt = 0;       // keys in this lane's half of its query's list
  if (MODE == kModeScan && q_ok) thr = nextafterf(a.thr0[my_q], INFINITY);

  // Rebalances every list of this wave with a half holding more than `limit`
  // keys (or, with limit = KP / 2 - 1 at the end, more than KP keys in all)
  // to its KP smallest keys and lowers the query's threshold to the kp-th
  // distance when keys were dropped.
  auto compact_wave = [&](uint32_t limit, bool total_only) CVS_INLINE {
    const uint32_t both = cnt + xor_lanes<32>(cnt);
    const uint64_t over64 = __ballot(total_only ? both > uint32_t(KP) : cnt > limit);
    uint32_t over = uint32_t(over64) | uint32_t(over64 >> 32);
    if (over == 0) return;
    if constexpr (L::GL) __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    while (over) {
      const int i = __builtin_ctz(over);
      over &= over - 1;
      const uint32_t c0 = uint32_t(__builtin_amdgcn_readlane(int(cnt), i));
      const uint32_t c1 = uint32_t(__builtin_amdgcn_readlane(int(cnt), i + 32));
      const uint32_t kth = compact_query<L::NS>(list_of(wave * 32 + i), L::HALF, c0, c1, KP);
      const uint32_t kept = c0 + c1 < uint32_t(KP) ? c0 + c1 : uint32_t(KP);
      if ((lane & 31) == i) {
        cnt = half == 0 ? (kept < uint32_t(KP / 2) ? kept : uint32_t(KP / 2))
                        : (kept > uint32_t(KP / 2) ? kept - uint32_t(KP / 2) : 0u);
        if (kth != 0xffffffffu) thr = fminf(thr, unord_f32(kth));
      }
    }
    if constexpr (L::GL) __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  };

  // Accumulators live in arch VGPRs so that all 256 AGPRs hold query operands.
  f32x16 acc0, acc1;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc0[i] = acc1[i] = 0.f;
  asm volatile("" : "+v"(acc0), "+v"(acc1));

  // Appends the passing (distance, row) keys of one finished tile to this
  // lane's half of its query's list.  Appends are rare once the sampled
  // threshold is in place (typically one or two lanes of a wave pass a row
  // of a tile, most tiles none), so the wave first ORs the pass masks of the
  // passing lanes (scalar reads of those lanes only), then visits just the
  // rows some lane passes: the row index is wave-uniform, so its distance is
  // picked from the 16-element vector by a uniform index, and each passing
  // lane appends one key to its half (counter in a register).  A half that
  // fills up triggers a compaction, and keys above the lowered threshold are
  // dropped from the rows not yet visited.
  auto commit = [&](const f32x16& dv, uint32_t pass, int64_t row0) CVS_INLINE {
    uint64_t lanes = __ballot(pass != 0);
    if (lanes == 0) return;
    uint32_t rows_any = 0;
    while (lanes) {
      const int l = __builtin_ctzll(lanes);
      lanes &= lanes - 1;
      rows_any |= uint32_t(__builtin_amdgcn_readlane(int(pass), l));
    }
    uint64_t* const mine = list_of(qw) + half * L::HALF;
    const uint32_t rbase = uint32_t(row0) + 4u * uint32_t(half);
    while (rows_any) {
      const int r = __builtin_ctz(rows_any);
      rows_any &= rows_any - 1;
      if ((pass >> r) & 1u) {
        mine[cnt] = (uint64_t(ord_f32(dv[r])) << 32) | (rbase + uint32_t(8 * (r >> 2) + (r & 3)));
        ++cnt;
      }
      if (__ballot(cnt >= uint32_t(L::HALF)) != 0) {
        compact_wave(uint32_t(L::HALF - 1), false);
#pragma unroll
        for (int r2 = 0; r2 < 16; ++r2)
          if (!(dv[r2] < thr)) pass &= ~(1u << r2);
      }
    }
  };

  // Epilogue for one finished 32-row tile: this lane holds query `my_q`
  // against rows row0 + 8*(r/4) + 4*(lane/32) + (r%4), r = 0..15.
  auto epilogue = [&](const float* dn, int64_t row0, int j) CVS_INLINE {
    f32x4 dn4[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) dn4[g] = *reinterpret_cast<const f32x4*>(dn + 8 * g + 4 * (lane >> 5));
    if (MODE == kModeSample) {
      // Running minimum over this lane's sampled rows (padding rows are +inf).
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          smin = fminf(smin, qn + dn4[g][e] - 2.0f * (acc0[4 * g + e] + acc1[4 * g + e]));
      (void)row0;
      (void)j;
    } else {
      // Branch-free pass mask over the 16 rows, then the rare append.
      f32x16 dv;
      uint32_t pass = 0;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        dv[r] = qn + dn4[r >> 2][r & 3] - 2.0f * (acc0[r] + acc1[r]);
        pass |= (dv[r] < thr ? 1u : 0u) << r;
      }
      commit(dv, pass, row0);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) acc0[i] = acc1[i] = 0.f;
    asm volatile("" : "+v"(acc0), "+v"(acc1));
  };

  // MFMA over NB consecutive 1 KiB blocks at `sb` (k-steps KOFF .. KOFF+NB-1),
  // A fragments through a PF-deep register ring, alternating two chains.
  auto mfma_run = [&](const u32x4* sb, auto nb_c, auto koff_c) CVS_INLINE {
    constexpr int NBLK = decltype(nb_c)::value, KOFF = decltype(koff_c)::value;
    constexpr int PF = NBLK < 8 ? NBLK : 8;
    half8 ring[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) ring[p] = __builtin_bit_cast(half8, sb[p * 64]);
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk) {
      const half8 av = ring[blk % PF];
      if (blk + PF < NBLK) ring[blk % PF] = __builtin_bit_cast(half8, sb[(blk + PF) * 64]);
      if (blk & 1)
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, qb[KOFF + blk], acc1, 0, 0, 0);
      else
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, qb[KOFF + blk], acc0, 0, 0, 0);
    }
    // Schedule: PF LDS reads up front, then (MFMA, read) pairs, then drain.
#pragma unroll
    for (int p = 0; p < PF; ++p) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
    for (int p = 0; p < NBLK - PF; ++p) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, PF, 0);
  };

  // Stage j in LDS buffer `buf`; PAR = j & 1 (static) selects the k-offset.
  auto compute = [&](auto par_c, int buf, int j) CVS_INLINE {
    constexpr int PAR = decltype(par_c)::value;
    const int64_t st = stage_of(j);
    const u32x4* sb = s_stage[buf] + lane;
    const float* dn = s_dn[buf];
    (void)st;
    if constexpr (KS >= 32) {
      // One stage is 32 k-steps of a single tile.
      constexpr int KOFF = (PAR * kStageBlocks) % KS;
      mfma_run(sb, std::integral_constant<int, kStageBlocks>{}, std::integral_constant<int, KOFF>{});
      if constexpr (KOFF + kStageBlocks == KS) epilogue(dn, (st / SPT) * 32, j);
    } else {
      // One stage holds TPS whole tiles.
#pragma unroll 1
      for (int t = 0; t < TPS; ++t) {
        mfma_run(sb + t * KS * 64, std::integral_constant<int, KS>{}, std::integral_constant<int, 0>{});
        epilogue(dn + t * 32, (st * TPS + t) * 32, j);
      }
    }
  };

  // ---- pipeline: per stage, registers -> LDS, reload the registers two
  // stages ahead, one barrier, compute.  One barrier per stage suffices with
  // two LDS buffers: buffer j&1 was last read in stage j-2, and every wave
  // has passed stage j-1's barrier since.
  auto step = [&](auto par_c, u32x4 (&r)[kLoadsPerThread], float (&nr)[NPT], int j) CVS_INLINE {
    constexpr int PAR = decltype(par_c)::value;
    lstore(PAR, r, nr);
    gload(r, nr, j + 2);
    __syncthreads();
    compute(par_c, PAR, j);
  };
  if constexpr (!PIPE) {
    for (int j = 0; j < n_stages; j += 2) {
      step(std::integral_constant<int, 0>{}, ra, na, j);
      step(std::integral_constant<int, 1>{}, rb, nb, j + 1);
    }
  } else {
    // ---- software-pipelined scan (32 or 64 k-steps per tile) ----
    // Stage j sits in LDS buffer j&1 and, until it is stored there, in
    // register set j&1 (ra / rb).  Per stage, after one barrier, a single scheduling region
    // interleaves with the stage's 32 MFMAs: the previous tile's
    // distance/threshold test (VALU), the LDS store of stage j+1 (its buffer
    // was last read in stage j-1, which every wave finished before the
    // barrier) and the HBM load of stage j+3 into the registers just stored.
    // A tile's norms travel with its last stage: loaded with that stage's
    // register set (one float per lane, row lane%32), stored to LDS slot
    // (tile & 3) together with the stage, and read by the epilogue in the
    // next tile's first stage, two barriers later.  Only the rare list
    // append after the MFMAs branches.
    auto lstore_b = [&](int buf, const u32x4 (&r)[kLoadsPerThread]) CVS_INLINE {
#pragma unroll
      for (int i = 0; i < kLoadsPerThread; ++i) s_stage[buf][tid + i * kThreads] = r[i];
    };
    // Turns the dot products of a finished tile (in `dv`) into distances and
    // its pass mask.
    auto prepare = [&](f32x16& dv, const f32x4 (&dn)[4]) CVS_INLINE -> uint32_t {
      uint32_t pass = 0;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        dv[r] = qn + dn[r >> 2][r & 3] - 2.0f * dv[r];
        pass |= (dv[r] < thr ? 1u : 0u) << r;
      }
      return pass;
    };
    // Norms of this workgroup's tiles (local tile t at byte 128 t); loads
    // past the last tile return zeros without a memory access.
    const __amdgpu_buffer_rsrc_t nrsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(reinterpret_cast<const float*>(a.norms) + (stage_of(0) / SPT) * 32), 0,
        int(uint32_t(n_stages / SPT) * 128u), kRsrcWord3);
    auto nload = [&](int s) CVS_INLINE -> float {
      return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                           nrsrc, uint32_t(s / SPT) * 128u + uint32_t(lane & 31) * 4u, 0, 0));
    };
    auto dn_slot = [&](int t) CVS_INLINE -> float* { return s_dnp[t & 3]; };
    f32x16 dv;
#pragma unroll
    for (int r = 0; r < 16; ++r) dv[r] = 0.f;

    // One stage as 32 slots separated by scheduling fences, so that the
    // interleave is fixed: slot i issues MFMA i, the LDS read of block i+8
    // (8-deep A ring, two accumulation chains), and one piece of the side
    // work.  Slot 0 of a tile's first stage first sums the previous tile's
    // two chains and slots 8-11 read that tile's norms from LDS; slots 12-19
    // store stage j+1 to LDS and reuse each register for stage j+3; slot 20
    // stores a tile's norms, slot 21 loads them; slots 16-31 of a first stage
    // turn the previous tile's dot products into distances and pass bits.
    auto pstep = [&](auto par_c, u32x4 (&r)[kLoadsPerThread], float& rn, int j) CVS_INLINE {
      constexpr int PAR = decltype(par_c)::value;
      constexpr bool FIRST = SPT == 1 || PAR == 0;    // first stage of its tile
      constexpr bool STORE_N = SPT == 1 || PAR == 0;  // stage j+1 (stored here) ends a tile
      constexpr bool LOAD_N = SPT == 1 || PAR == 0;   // stage j+3 (loaded here) ends a tile
      constexpr int KOFF = (PAR * kStageBlocks) % KS;
      constexpr int PF = 8;
      const int64_t tile = (stage_of(0) + j) / SPT;
      const int tl = j / SPT;  // tile of stage j, counted in this workgroup
      const u32x4* sb = s_stage[PAR] + lane;
      const uint32_t off = uint32_t(j + 3) * kStageBytes + uint32_t(tid) * 16;
      __syncthreads();
      if constexpr (FIRST) {
#pragma unroll
        for (int q = 0; q < 16; ++q) dv[q] = acc0[q] + acc1[q];
      }
      half8 ring[PF];
#pragma unroll
      for (int p = 0; p < PF; ++p) ring[p] = __builtin_bit_cast(half8, sb[p * 64]);
      uint32_t pass = 0;
      f32x4 dn4[4];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < kStageBlocks; ++i) {
        const half8 av = ring[i % PF];
        if (i + PF < kStageBlocks) ring[i % PF] = __builtin_bit_cast(half8, sb[(i + PF) * 64]);
        const f32x16 zero = {};
        if (i & 1)
          acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, qb[KOFF + i], (FIRST && i < 2) ? zero : acc1, 0, 0, 0);
        else
          acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, qb[KOFF + i], (FIRST && i < 2) ? zero : acc0, 0, 0, 0);
        if constexpr (FIRST) {
          if (i >= 8 && i < 12) {
            const int g = i - 8;
            // Slot of tile tl-1 (for the first tile: never written, masked below).
            dn4[g] = *reinterpret_cast<const f32x4*>(dn_slot(tl + 3) + 8 * g + 4 * (lane >> 5));
          }
        }
        if (i >= 12 && i < 12 + kLoadsPerThread) {
          const int e = i - 12;
          s_stage[PAR ^ 1][tid + e * kThreads] = r[e];  // past the last stage: zeros, never read
          r[e] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rsrc, off + uint32_t(e * kThreads * 16), 0, kAuxNT));
        }
        if constexpr (STORE_N) {
          if (i == 20) dn_slot((j + 1) / SPT)[lane & 31] = rn;
        }
        if constexpr (LOAD_N) {
          if (i == 21) rn = nload(j + 3);
        }
        if constexpr (FIRST) {
          if (i >= 16) {
            const int q = i - 16;
            dv[q] = qn + dn4[q >> 2][q & 3] - 2.0f * dv[q];
            pass |= (dv[q] < thr ? 1u : 0u) << q;
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (FIRST) {
        // No previous tile before the first stage.
        pass &= 0u - uint32_t(j > 0);
        commit(dv, pass, (tile - 1) * 32);
      }
    };
    // Register sets: stage s in set s & 1; ra and rb hold stages 0 and 1.
    float na = 0.f, nb = nload(1);
    if constexpr (SPT == 1) na = nload(0);
    lstore_b(0, ra);
    if constexpr (SPT == 1) dn_slot(0)[lane & 31] = na;
    gload_b(ra, 2);
    if constexpr (SPT == 1) na = nload(2);
    for (int j = 0; j < n_stages; j += 2) {
      pstep(std::integral_constant<int, 0>{}, rb, nb, j);
      pstep(std::integral_constant<int, 1>{}, ra, na, j + 1);
    }
    // Last tile (its norms were stored with its last stage, before the
    // final barrier).
    f32x4 dn_last[4];
#pragma unroll
    for (int g = 0; g < 4; ++g)
      dn_last[g] = *reinterpret_cast<const f32x4*>(dn_slot(n_stages / SPT - 1) + 8 * g + 4 * (lane >> 5));
#pragma unroll
    for (int q = 0; q < 16; ++q) dv[q] = acc0[q] + acc1[q];
    const uint32_t pass = prepare(dv, dn_last);
    commit(dv, pass, ((stage_of(0) + n_stages) / SPT - 1) * 32);
  }

  if (MODE == kModeSample) {
    // One minimum per (query, workgroup, half-wave): 2 * n_ranges per query.
    if (q_ok) a.sgmin[int64_t(my_q) * (2 * G) + 2 * x + (lane >> 5)] = smin;
  }
  if (MODE == kModeScan) {
    compact_wave(0u, true);
    if constexpr (!L::GL) {
      // LDS lists, written by all lanes at once: lane l writes entries
      // [KP/2 * half, KP/2 * (half + 1)) of its query's output (half 0's
      // keys, then half 1's, then sentinels), and the two lanes of a query
      // combine their minima.
      const uint32_t other = xor_lanes<32>(cnt);
      const uint32_t c0 = half == 0 ? cnt : other, c1 = half == 0 ? other : cnt;
      const int q = qbase + qw;
      const uint64_t* src = list_of(qw);
      uint64_t mn = kSentinel;
      uint64_t* dst = a.part + (int64_t(q < a.nq ? q : 0) * G + x) * KP;
#pragma unroll
      for (int i = 0; i < KP / 2; ++i) {
        const uint32_t e = uint32_t(half * (KP / 2) + i);
        const uint64_t key = e < c0 ? src[e] : (e < c0 + c1 ? src[L::HALF + (e - c0)] : kSentinel);
        mn = key < mn ? key : mn;
        if (q < a.nq) dst[e] = key;
      }
      const uint64_t y = shfl_xor_u64(mn, 32);
      mn = y < mn ? y : mn;
      if (half == 0 && q < a.nq) {
        a.lmin[int64_t(q) * G + x] = mn;
        a.lcut[int64_t(q) * G + x] = thr;
      }
      return;
    }
    for (int i = 0; i < 32; ++i) {
      const int m = wave * 32 + i;
      const int q = qbase + m;
      if (q >= a.nq) break;
      const uint32_t c0 = uint32_t(__builtin_amdgcn_readlane(int(cnt), i));
      const uint32_t c1 = uint32_t(__builtin_amdgcn_readlane(int(cnt), i + 32));
      // Entry e of the output: half 0's keys, then half 1's, then sentinels.
      const uint64_t* src = list_of(m);
      constexpr int NE = (KP + 63) / 64;
      uint64_t key[NE];
      uint64_t mn = kSentinel;
#pragma unroll
      for (int t = 0; t < NE; ++t) {
        const uint32_t e = uint32_t(lane + 64 * t);
        key[t] = e < c0 ? src[e] : (e < c0 + c1 ? src[L::HALF + (e - c0)] : kSentinel);
        if (e >= uint32_t(KP)) key[t] = kSentinel;
        mn = key[t] < mn ? key[t] : mn;
      }
      if constexpr (L::GL) {
        // In place (first kp entries of the global list): every entry is
        // read before any is written.
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        uint64_t* lst = list_of(m);
#pragma unroll
        for (int t = 0; t < NE; ++t)
          if (lane + 64 * t < KP) lst[lane + 64 * t] = key[t];
      } else {
#pragma unroll
        for (int t = 0; t < NE; ++t)
          if (lane + 64 * t < KP) a.part[(int64_t(q) * G + x) * KP + lane + 64 * t] = key[t];
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const uint64_t y = shfl_xor_u64(mn, o);
        mn = y < mn ? y : mn;
      }
      const float cut = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(thr), i));
      if (lane == 0) {
        a.lmin[int64_t(q) * G + x] = mn;
        a.lcut[int64_t(q) * G + x] = cut;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Queries fp32 -> fp16 tiles of scale * (q - mu) (the dataset's tile layout
// and centring) + squared norms of the fp16-rounded rows, one wave per
// query: lane l converts columns [16*l', 16*l'+16) for l' = l, l+64, ...; the
// norm is a fixed-order wave reduction.  qerr receives the squared rounding
// error |q~ - scale fl(q - mu)|^2 of each query (for the certificate in the
// merge).  Rows of the last tile beyond q are zero with norm +inf.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void query_tiles_kernel(const float* __restrict__ queries, int64_t q,
                                                          int64_t d, int ksteps, int64_t q_rows,
                                                          const float* __restrict__ mu, float scale,
                                                          u32x4* __restrict__ qtiles, float* __restrict__ qnorms,
                                                          float* __restrict__ qerr) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (r >= q_rows) return;
  const bool ok = r < q;
  const float* src = queries + (ok ? r : 0) * d;
  const bool vec = (d & 3) == 0 && (reinterpret_cast<uintptr_t>(queries) & 15) == 0;
  const int64_t t = r >> 5;
  float acc = 0.f, err = 0.f;
  for (int s = lane; s < ksteps; s += 64) {
#pragma unroll
    for (int hpart = 0; hpart < 2; ++hpart) {
      const int64_t c0 = int64_t(s) * kStepCols + 8 * hpart;
      float v[8];
      if (ok && vec && c0 + 8 <= d) {
        const float4 x = *reinterpret_cast<const float4*>(src + c0);
        const float4 y = *reinterpret_cast<const float4*>(src + c0 + 4);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
        v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (ok && c0 + j < d) ? src[c0 + j] : 0.f;
      }
      // The means are loaded unconditionally (column clamped) and the result
      // masked by an AND of its bits, which the compiler cannot move into a
      // branch: a load used only under its lane condition is waited for
      // before the next one is issued.
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool in = ok && c0 + j < d;
        const float mj = mu[c0 + j < d ? c0 + j : d - 1];
        const float r = (v[j] - mj) * scale;
        v[j] = __uint_as_float(__float_as_uint(r) & (in ? 0xffffffffu : 0u));
      }
      _Float16 h[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        h[j] = static_cast<_Float16>(v[j]);
        const float hv = static_cast<float>(h[j]);
        acc += hv * hv;
        const float e = hv - v[j];
        err += e * e;
      }
      u32x4 packed;
      __builtin_memcpy(&packed, h, sizeof(packed));
      // tile t, k-step s, lane (row % 32) + 32 * hpart
      qtiles[(t * ksteps + s) * 64 + (r & 31) + 32 * hpart] = packed;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    acc += xor_lanes_f(acc, o);
    err += xor_lanes_f(err, o);
  }
  if (lane == 0) {
    qnorms[r] = ok ? acc : INFINITY;
    if (ok) qerr[r] = err;
  }
}

// ---------------------------------------------------------------------------
// Initial scan threshold per query: the kp-th smallest of the sample minima.
// Any kp minima belong to kp distinct dataset rows, so at least kp rows lie
// at or below it.  One wave per query (m <= 512 minima, 8 per lane) on the
// order-preserving integer image: for kp <= 32 a tournament (each lane sorts
// its 8 values; each round takes the wave minimum of the lanes' smallest
// remaining values and removes it from the lanes holding it, so kp rounds at
// most), otherwise a ballot radix select (32 rounds of 8 ballots).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void bf_select_kernel(const float* __restrict__ sgmin, int m, int kp, int nq,
                                                        float* __restrict__ thr0) {
  const int lane = threadIdx.x & 63;
  const int q = int(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (q >= nq) return;
  const float* src = sgmin + int64_t(q) * m;
  uint32_t v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // Unconditional loads (index clamped, value masked after by an OR, which
    // the compiler cannot move into a branch): a load under a lane condition
    // is waited for before the next one is issued.
    const int e = lane + 64 * i;
    const float x = src[e < m ? e : (m > 0 ? m - 1 : 0)];
    v[i] = ord_f32(x) | (e < m ? 0u : 0xffffffffu);
  }
  if (m < kp) {
    if (lane == 0) thr0[q] = INFINITY;
    return;
  }
  int need = kp;
  if (kp <= 32) {
    // Sorting network for 8 values (19 compare-exchanges).
    auto cx = [&](int i, int j) {
      const uint32_t lo = min(v[i], v[j]), hi = max(v[i], v[j]);
      v[i] = lo;
      v[j] = hi;
    };
    cx(0, 1); cx(2, 3); cx(4, 5); cx(6, 7);
    cx(0, 2); cx(1, 3); cx(4, 6); cx(5, 7);
    cx(1, 2); cx(5, 6); cx(0, 4); cx(3, 7);
    cx(1, 5); cx(2, 6);
    cx(1, 4); cx(3, 6);
    cx(2, 4); cx(3, 5);
    cx(3, 4);
    uint32_t ans = 0xffffffffu;
    for (int round = 0; round <= 32; ++round) {
      uint32_t mn = v[0];
      mn = min(mn, xor_lanes<1>(mn));
      mn = min(mn, xor_lanes<2>(mn));
      mn = min(mn, xor_lanes<4>(mn));
      mn = min(mn, xor_lanes<8>(mn));
      mn = min(mn, xor_lanes<16>(mn));
      mn = min(mn, xor_lanes<32>(mn));
      const bool mine = v[0] == mn;
      const int c = popc(__ballot(mine));
      if (c >= need || mn == 0xffffffffu) {
        ans = mn;
        break;
      }
      need -= c;
      if (mine) {
#pragma unroll
        for (int i = 0; i < 7; ++i) v[i] = v[i + 1];
        v[7] = 0xffffffffu;
      }
    }
    if (lane == 0) thr0[q] = ans == 0xffffffffu ? INFINITY : unord_f32(ans);
    return;
  }
  uint32_t pre = 0;
  for (int b = 31; b >= 0; --b) {
    int c = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) c += popc(__ballot(((v[i] ^ pre) >> b) == 0));
    if (c < need) {
      need -= c;
      pre |= 1u << b;
    }
  }
  if (lane == 0) thr0[q] = pre == 0xffffffffu ? INFINITY : unord_f32(pre);
}

// Writes k results from a sorted list of exact keys (wave 0), padded with
// UINT32_MAX / +inf (src/cagra.cpp:240-251).
template <int E>
__device__ __forceinline__ void write_results(const uint64_t (&fin)[E], int64_t q, int64_t k, uint32_t* out_nbr,
                                              float* out_dist) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int64_t pos = e * 64 + lane;
    if (pos < k) {
      out_nbr[q * k + pos] = fin[e] == kSentinel ? 0xffffffffu : uint32_t(fin[e]);
      out_dist[q * k + pos] = fin[e] == kSentinel ? INFINITY : unord_f32(uint32_t(fin[e] >> 32));
    }
  }
}

// Key at position p (uniform) of a sorted 64*E list held by a wave.
template <int E>
__device__ __forceinline__ uint64_t key_at(const uint64_t (&v)[E], int p) {
  uint64_t r = kSentinel;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (e == p / 64) r = shfl_u64(v[e], p % 64);
  return r;
}

// Finishes one query from its R candidates (ids in s_cid, sorted by key,
// 0xffffffff for none) by the four waves of a workgroup: exact re-rank,
// certificate, and if needed the escalation described above; writes k
// sorted results.  t_cert: the bound T above (key units); t_star: the
// smallest list threshold; part / kp / stride: the candidate lists (entry e
// of the query's lists at part[(e / kp) * stride + e % kp], G * kp entries);
// key_r: the largest fp16 key among the candidates, which are the R smallest
// keys of the lists, so an escalation from the lists continues with the keys
// above it; 0 when the candidates are not known to be those (the escalation
// then starts afresh).
template <int E>
__device__ void finish_query(const uint32_t* s_cid, int R, float t_cert, float t_star, uint64_t key_r,
                             const uint64_t* part, int G, int kp, int stride, const float* __restrict__ rows,
                             int64_t n, int64_t d, const float* __restrict__ qv, int64_t q, int64_t k,
                             const Cert& cert, uint32_t* out_nbr, float* out_dist) {
  __shared__ uint64_t s_key[64 * E > 256 ? 64 * E : 256];  // exact keys: candidates, then per-wave rounds
  __shared__ uint32_t s_wid[kWaves][64];
  __shared__ uint64_t s_scr[32];
  __shared__ int s_mode;
  __shared__ float s_tneed;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool vec = (d & 3) == 0 && (reinterpret_cast<uintptr_t>(qv) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(rows) & 15) == 0;

  // 1. Exact distances of the R candidates, kExactU per wave and pass.
  for (int c = kExactU * wave; c < R; c += kExactU * kWaves) {
    uint32_t id[kExactU];
#pragma unroll
    for (int u = 0; u < kExactU; ++u) id[u] = c + u < R ? s_cid[c + u] : 0xffffffffu;
    float dd[kExactU];
    wave_exact<kExactU>(id, rows, n, d, qv, vec, dd);
#pragma unroll
    for (int u = 0; u < kExactU; ++u)
      if (lane == u && c + u < R)
        s_key[c + u] = int64_t(id[u]) < n ? (uint64_t(ord_f32(dd[u])) << 32) | id[u] : kSentinel;
  }
  __syncthreads();

  // 2. Wave 0: sort, certify.
  uint64_t fin[E];
  if (wave == 0) {
#pragma unroll
    for (int e = 0; e < E; ++e) fin[e] = e * 64 + lane < R ? s_key[e * 64 + lane] : kSentinel;
    wave_sort_e<E>(fin);
    const uint64_t kth = key_at<E>(fin, int(k - 1));
    if (lane == 0) {
      const double dk = kth == kSentinel ? INFINITY : double(unord_f32(uint32_t(kth >> 32)));
      const double qn = double(cert.qnorms[q]);
      int mode = kCertPass;
      float tneed = INFINITY;
      if (!(qn <= 3.0e38) || !(double(cert.rmax) <= 3.0e38)) {
        mode = kCertAll;  // keys overflowed or rows are not finite: no bound holds
      } else {
        const double qt = std::sqrt(qn) * (1.0 + 0x1p-20);
        const double qe = std::sqrt(double(cert.qerr[q]) * (1.0 + double(d + 8) * 0x1p-24)) * (1.0 + 0x1p-20);
        const double E_ = qe + qt * 0x1p-23 + double(cert.qslack) + double(cert.dx);
        const double A = double(cert.a_coef) * (qt + double(cert.rmax)) * (qt + double(cert.rmax));
        const double V = double(cert.s2) * dk * (1.0 + double(cert.rho));
        const double T = double(t_cert);
        bool ok;
        if (T > 3.0e38) {
          ok = true;  // every row with a finite key was re-ranked
        } else {
          const double r = T > A ? std::sqrt(T - A) : 0.0;
          const double lb = r > E_ ? (r - E_) * (r - E_) : 0.0;
          ok = lb * (1.0 - 0x1p-40) > V;
        }
        if (!ok) {
          const double tn = V > 3.0e38 ? INFINITY : ((std::sqrt(V) + E_) * (std::sqrt(V) + E_) + A) * (1.0 + 0x1p-20);
          mode = tn <= double(t_star) ? kCertKeys : kCertAll;
          tneed = float(tn);
        }
      }
      s_mode = mode;
      s_tneed = tneed;
      if (mode != kCertPass) {
        atomicAdd(&cert.counters[0], 1ull);
        if (mode == kCertAll) atomicAdd(&cert.counters[1], 1ull);
      }
    }
  }
  __syncthreads();
  const int mode = s_mode;
  if (mode == kCertPass) {
    if (wave == 0) write_results<E>(fin, q, k, out_nbr, out_dist);
    return;
  }

  // 3. Escalation: exact keys of every row with a key up to T_need (from the
  // lists; those above key_r when the candidates were the lists' R smallest,
  // whose exact keys seed the running list) or of every row, 64 per wave and
  // round, merged by wave 0 into its running exact top-128 (k <= 112 here).
  const float tneed = s_tneed;
  const bool incremental = mode == kCertKeys && key_r != 0;
  const int64_t total = mode == kCertKeys ? int64_t(G) * kp : n;
  uint64_t run[2] = {kSentinel, kSentinel};
  if (incremental && wave == 0) {
    run[0] = fin[0];
    if constexpr (E > 1) run[1] = fin[1];
  }
  for (int64_t base = 0; base < total; base += 64 * kWaves) {
    const int64_t pos = base + 64 * wave + lane;
    uint32_t id = 0xffffffffu;
    bool ok = false;
    if (mode == kCertKeys) {
      const uint64_t key = pos < total ? part[(pos / kp) * stride + pos % kp] : kSentinel;
      ok = key != kSentinel && unord_f32(uint32_t(key >> 32)) <= tneed && (!incremental || key > key_r);
      id = uint32_t(key);
    } else {
      ok = pos < n;
      id = uint32_t(pos);
    }
    const uint64_t m = __ballot(ok);
    if (ok) s_wid[wave][mbcnt(m)] = id;
    const int cnt = popc(m);
    uint64_t* wk = s_key + 64 * wave;
    wave_exact_keys(s_wid[wave], cnt, wk, rows, n, d, qv, vec);
    if (lane >= cnt) wk[lane] = kSentinel;
    __syncthreads();
    if (wave == 0) {
#pragma unroll 1
      for (int w = 0; w < kWaves; ++w) {
        uint64_t ck = s_key[64 * w + lane];
        if (sort_below(ck, key_at<2>(run, int(k - 1)), kSentinel, s_scr) > 0) wave_merge<2>(run, ck);
      }
    }
    __syncthreads();
  }
  if (wave == 0) write_results<2>(run, q, k, out_nbr, out_dist);
}

// ---------------------------------------------------------------------------
// Merge for kp <= 64, one workgroup (4 waves) per query.
//  1. The R-th smallest list minimum (R = min(2 kp, 64 E)) bounds the R-th
//     smallest key (R list minima are R distinct keys): only keys at or
//     below it can be among the R smallest.  Wave 0 computes it (a 256-key
//     wave sort) and the smallest list threshold T* while every wave's first
//     batch of keys is already in flight.
//  2. A key within the bound comes from one of the R lists whose minimum is
//     within it, so at most R * kp keys pass.  The four waves stream all
//     G * kp keys and append the passing ones to an LDS buffer of that size
//     (one atomic per wave and batch).
//  3. Wave 0 sorts the passing keys 64 at a time and merges them into its
//     running sorted top-64 E; its first R ids are finished (re-ranked,
//     certified) by finish_query.
// ---------------------------------------------------------------------------
template <int E>
__global__ __launch_bounds__(256) void bf_merge_filter_kernel(const uint64_t* __restrict__ part,
                                                              const uint64_t* __restrict__ lmin,
                                                              const float* __restrict__ lcut, int G, int kp,
                                                              const float* __restrict__ rows, int64_t n, int64_t d,
                                                              const float* __restrict__ queries, int64_t k,
                                                              Cert cert, uint32_t* __restrict__ out_nbr,
                                                              float* __restrict__ out_dist) {
  constexpr int kBatch = 16;        // keys per thread and batch
  constexpr int kMaxPass = 64 * 64; // passing keys held in LDS
  __shared__ uint64_t s_pass[kMaxPass];
  __shared__ uint32_t s_npass;
  __shared__ uint64_t s_bound, s_keyr;
  __shared__ float s_tcert, s_tstar;
  __shared__ uint32_t s_cid[64 * E];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t q = blockIdx.x;
  const uint64_t* src = part + q * int64_t(G) * kp;
  const int total = G * kp;
  const int R = 2 * kp < 64 * E ? 2 * kp : 64 * E;
  if (tid == 0) s_npass = 0;

  // 1. Bound from the list minima and the smallest list threshold (G <= 256),
  // by wave 0, which requests them before its share of the keys, so that it
  // waits for them alone.  For R <= 32 the bound is the R-th smallest of the
  // lanes' minima of their four list minima: those are R distinct list
  // minima, so at least R keys lie at or below it (one 64-key sort instead
  // of a 256-key one; the bound is a little looser).
  // Loads unconditional (index clamped); the values past G are masked, by
  // bitwise operations the compiler keeps out of branches, after the key
  // batch has been requested, so that all of them are in flight together.
  uint64_t mins[4];
  uint32_t cuts[4];
  float cut = INFINITY;
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int x = lane + 64 * i;
      const int64_t xi = q * G + (x < G ? x : G - 1);
      mins[i] = lmin[xi];
      cuts[i] = __float_as_uint(lcut[xi]);
    }
  }
  // First batch of keys, requested before the bound is known.
  uint64_t key[kBatch];
#pragma unroll
  for (int r = 0; r < kBatch; ++r) {
    const int e = r * kThreads + tid;
    key[r] = e < total ? src[e] : kSentinel;
  }
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool in = lane + 64 * i < G;
      mins[i] |= in ? 0ull : kSentinel;
      cut = fminf(cut, __uint_as_float((cuts[i] & (in ? 0xffffffffu : 0u)) | (in ? 0u : 0x7f800000u)));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) cut = fminf(cut, xor_lanes_f(cut, o));
    uint64_t bound;
    if (R <= 32) {
      uint64_t lm[1] = {mins[0]};
#pragma unroll
      for (int i = 1; i < 4; ++i) lm[0] = mins[i] < lm[0] ? mins[i] : lm[0];
      wave_sort_e<1>(lm);
      bound = key_at<1>(lm, R - 1);
    } else {
      wave_sort_e<4>(mins);
      bound = key_at<4>(mins, R - 1);
    }
    if (lane == 0) {
      s_bound = bound;
      s_tstar = cut;
    }
  }
  __syncthreads();
  const uint64_t bound = s_bound;

  // 2. Filter every key; append the passing ones (the ballots of the whole
  // batch first, then one LDS atomic per wave for their slots).
  for (int b0 = 0; b0 < total; b0 += kBatch * kThreads) {
    if (b0 > 0) {
#pragma unroll
      for (int r = 0; r < kBatch; ++r) {
        const int e = b0 + r * kThreads + tid;
        key[r] = e < total ? src[e] : kSentinel;
      }
    }
    uint64_t m[kBatch];
    uint32_t tot = 0;
#pragma unroll
    for (int r = 0; r < kBatch; ++r) {
      m[r] = __ballot(key[r] <= bound && key[r] != kSentinel);
      tot += uint32_t(popc(m[r]));
    }
    if (tot == 0) continue;
    uint32_t base = 0;
    if (lane == 0) base = atomicAdd(&s_npass, tot);
    base = uint32_t(__shfl(int(base), 0));
#pragma unroll
    for (int r = 0; r < kBatch; ++r) {
      const uint32_t slot = base + uint32_t(mbcnt(m[r]));
      if (((m[r] >> lane) & 1ull) && slot < uint32_t(kMaxPass)) s_pass[slot] = key[r];
      base += uint32_t(popc(m[r]));
    }
  }
  __syncthreads();

  // 3. Wave 0: top-R of the passing keys.  Should more keys pass than LDS
  // holds (not seen in practice), the candidates are not known to be the R
  // smallest: the certificate is then made to fail, and the escalation
  // re-ranks from the lists afresh.
  if (wave == 0) {
    const bool overflow = s_npass > uint32_t(kMaxPass);
    const int np = overflow ? kMaxPass : int(s_npass);
    uint64_t run[E];
#pragma unroll
    for (int e = 0; e < E; ++e) run[e] = kSentinel;
    for (int r0 = 0; r0 < np; r0 += 64) {
      uint64_t ck[1] = {r0 + lane < np ? s_pass[r0 + lane] : kSentinel};
      wave_sort_e<1>(ck);
      wave_merge<E>(run, ck[0]);
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int pos = e * 64 + lane;
      s_cid[pos] = (pos < R && run[e] != kSentinel) ? uint32_t(run[e]) : 0xffffffffu;
    }
    const uint64_t kr = key_at<E>(run, R - 1);
    const float tr = kr == kSentinel ? INFINITY : unord_f32(uint32_t(kr >> 32));
    if (lane == 0) {
      s_tcert = overflow ? 0.f : fminf(tr, s_tstar);
      s_keyr = overflow ? 0ull : kr;
    }
  }
  __syncthreads();
  finish_query<E>(s_cid, R, s_tcert, s_tstar, s_keyr, src, G, kp, kp, rows, n, d, queries + q * d, q, k, cert,
                  out_nbr, out_dist);
}

// ---------------------------------------------------------------------------
// Merge for kp = 128 (global lists), one workgroup (4 waves) per query; the
// R = 64 E smallest keys are the candidates.
//  1. The R-th smallest list minimum bounds the R-th smallest key (R list
//     minima are R distinct keys): only keys at or below it can be among
//     the R smallest.  Each wave computes it (a 256-key wave sort).
//  2. Each wave streams a quarter of the lists, 64 keys per row, all rows of
//     a batch loaded at once; a row holding a key within the bound is sorted
//     (wave bitonic) and merged into the wave's running sorted top-64*E,
//     whose R-th key then tightens the wave's bound.
//  3. Wave 0 merges the four running lists; the R candidates are finished
//     (re-ranked, certified) by finish_query.
// ---------------------------------------------------------------------------
template <int E>
__global__ __launch_bounds__(256) void bf_merge_kernel(const uint64_t* __restrict__ part,
                                                       const uint64_t* __restrict__ lmin,
                                                       const float* __restrict__ lcut, int G, int kp, int stride,
                                                       const float* __restrict__ rows, int64_t n, int64_t d,
                                                       const float* __restrict__ queries, int64_t k, Cert cert,
                                                       uint32_t* __restrict__ out_nbr,
                                                       float* __restrict__ out_dist) {
  constexpr int kBatch = 16;
  __shared__ uint64_t s_run[kWaves][64 * E];
  __shared__ uint32_t s_cid[64 * E];
  __shared__ float s_tcert;
  __shared__ uint64_t s_keyr;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t q = blockIdx.x;
  constexpr int R = 64 * E;  // candidates re-ranked (>= kp)

  // 1. Bound from the list minima (G <= 256), and the smallest list threshold.
  // Loads unconditional (index clamped; values past G masked to the sentinel
  // and +inf by bitwise operations the compiler keeps out of branches): all
  // eight in flight together.
  uint64_t mins[4];
  float cut = INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int x = lane + 64 * i;
    const int64_t xi = q * G + (x < G ? x : G - 1);
    const uint64_t mv = lmin[xi];
    const uint32_t cb = __float_as_uint(lcut[xi]);
    mins[i] = mv | (x < G ? 0ull : kSentinel);
    cut = fminf(cut, __uint_as_float((cb & (x < G ? 0xffffffffu : 0u)) | (x < G ? 0u : 0x7f800000u)));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) cut = fminf(cut, xor_lanes_f(cut, o));
  wave_sort_e<4>(mins);
  uint64_t bound = key_at<4>(mins, R - 1);

  // 2. This wave's quarter of the 64-key rows.
  uint64_t run[E];
#pragma unroll
  for (int e = 0; e < E; ++e) run[e] = kSentinel;
  const uint64_t* src = part + q * int64_t(G) * stride;
  const int total = G * kp;
  const int n_rows = (total + 63) / 64;
  const int r0 = (n_rows * wave) / kWaves, r1 = (n_rows * (wave + 1)) / kWaves;
  for (int rb = r0; rb < r1; rb += kBatch) {
    uint64_t key[kBatch];
#pragma unroll
    for (int r = 0; r < kBatch; ++r) {
      const int e = (rb + r) * 64 + lane;
      key[r] = (rb + r < r1 && e < total) ? src[int64_t(e / kp) * stride + e % kp] : kSentinel;
    }
#pragma unroll
    for (int r = 0; r < kBatch; ++r) {
      const bool pass = key[r] != kSentinel && key[r] <= bound;
      if (__ballot(pass) == 0) continue;
      uint64_t ck[1] = {pass ? key[r] : kSentinel};
      wave_sort_e<1>(ck);
      wave_merge<E>(run, ck[0]);
      const uint64_t kth = key_at<E>(run, R - 1);
      bound = kth < bound ? kth : bound;
    }
  }
#pragma unroll
  for (int e = 0; e < E; ++e) s_run[wave][e * 64 + lane] = run[e];
  __syncthreads();

  // 3. Merge the four running lists; finish the kp candidates.
  if (wave == 0) {
#pragma unroll
    for (int w = 1; w < kWaves; ++w)
#pragma unroll
      for (int e = 0; e < E; ++e) wave_merge<E>(run, s_run[w][e * 64 + lane]);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int pos = e * 64 + lane;
      s_cid[pos] = run[e] != kSentinel ? uint32_t(run[e]) : 0xffffffffu;
    }
    const uint64_t kr = key_at<E>(run, R - 1);
    const float tr = kr == kSentinel ? INFINITY : unord_f32(uint32_t(kr >> 32));
    if (lane == 0) {
      s_tcert = fminf(tr, cut);
      s_keyr = kr;
    }
  }
  __syncthreads();
  finish_query<E>(s_cid, R, s_tcert, cut, s_keyr, src, G, kp, stride, rows, n, d, queries + q * d, q, k, cert,
                  out_nbr, out_dist);
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
int choose_kp(int64_t k) {
  if (k <= 10) return 16;
  if (k <= 24) return 32;
  if (k <= 48) return 64;
  return 128;
}

template <int KS, int KP>
void launch_scan_kp(cvs_context* ctx, dim3 grid, const ScanArgs& args, int mode, hipEvent_t e0, hipEvent_t e1) {
  if (mode == kModeScan)
    hipExtLaunchKernelGGL((bf_scan_kernel<KS, kModeScan, KP>), grid, dim3(kThreads), 0, ctx->stream, e0, e1, 0,
                          args);
  else
    hipExtLaunchKernelGGL((bf_scan_kernel<KS, kModeSample, KP>), grid, dim3(kThreads), 0, ctx->stream, e0, e1, 0,
                          args);
}

template <int KS>
void launch_scan_ks(cvs_context* ctx, dim3 grid, const ScanArgs& args, int mode, hipEvent_t e0, hipEvent_t e1) {
  if (mode == kModeSample) {
    launch_scan_kp<KS, 16>(ctx, grid, args, mode, e0, e1);  // list geometry unused when sampling
    return;
  }
  switch (args.kp) {
    case 16: launch_scan_kp<KS, 16>(ctx, grid, args, mode, e0, e1); break;
    case 32: launch_scan_kp<KS, 32>(ctx, grid, args, mode, e0, e1); break;
    case 64: launch_scan_kp<KS, 64>(ctx, grid, args, mode, e0, e1); break;
    case 128: launch_scan_kp<KS, 128>(ctx, grid, args, mode, e0, e1); break;
    default: fail(CVS_ERR_RUNTIME, "unsupported candidate count");
  }
}

// Launches the scan kernel in `mode`; e0 / e1 (may be null) record the
// dispatch's start / end for the timing facility.
void launch_scan(cvs_context* ctx, int ks, dim3 grid, const ScanArgs& args, int mode, hipEvent_t e0 = nullptr,
                 hipEvent_t e1 = nullptr) {
  switch (ks) {
    case 2: launch_scan_ks<2>(ctx, grid, args, mode, e0, e1); break;
    case 4: launch_scan_ks<4>(ctx, grid, args, mode, e0, e1); break;
    case 8: launch_scan_ks<8>(ctx, grid, args, mode, e0, e1); break;
    case 16: launch_scan_ks<16>(ctx, grid, args, mode, e0, e1); break;
    case 32: launch_scan_ks<32>(ctx, grid, args, mode, e0, e1); break;
    case 64: launch_scan_ks<64>(ctx, grid, args, mode, e0, e1); break;
    default: fail(CVS_ERR_UNSUPPORTED, "unsupported padded dimension");
  }
  after_launch(mode == kModeScan ? "bf_scan_kernel" : "bf_sample_kernel");
}

// Launch geometry and workspace layout of one brute-force call.
struct BfPlan {
  int ks = 0;              // k-steps per tile (padded dimension / 16)
  int64_t n_units = 0;     // 2-stage units in the dataset
  int kp = 0;              // candidates per (dataset range, query)
  unsigned qblocks = 0;    // 128-query blocks
  bool large_batch = false;
  bool gemm = false;       // large batch, kp = 128: the register-blocked scan (bf_gemm.hip)
  int gemm_wg = 0;         // its workgroups
  int G = 0;               // candidate lists per query: dataset ranges of the streaming scan
  int stride = 0;          // keys per (query, range) list in the workspace
  int64_t s_units = 0, s_stride = 0;  // threshold sample
  int sel_rank = 0;        // the initial threshold is this smallest sample minimum
  int Gs = 0;              // dataset ranges of the sample
  int m_min = 0;           // sample minima per query
  int64_t q_tiles = 0;     // 32-query tiles
  // Workspace: query tiles | query norms | thresholds | sample minima |
  // list minima | candidate lists, each 256-byte aligned.
  size_t off_qnorm = 0, off_qerr = 0, off_thr = 0, off_smin = 0, off_lmin = 0, off_lcut = 0, off_part = 0,
         total = 0;
};

void validate_bf(cvs_context* ctx, const cvs_dataset* ds, const float* queries, int64_t q, int64_t k,
                 const uint32_t* nbr, const float* dist) {
  if (!ds || ds->ctx != ctx) fail(CVS_ERR_INVALID_ARGUMENT, "dataset does not belong to context");
  if (!queries || !nbr || !dist) fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
  if (q <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "query count must be positive");
  if (k <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "k must be positive");
  if (k > CVS_BF_MAX_K) fail(CVS_ERR_UNSUPPORTED, "k exceeds CVS_BF_MAX_K");
  if (ds->d > CVS_BF_MAX_DIM) fail(CVS_ERR_UNSUPPORTED, "dimension exceeds CVS_BF_MAX_DIM");
  if (q > (int64_t(1) << 24)) fail(CVS_ERR_UNSUPPORTED, "too many queries in one call");
}

// True when the call runs the fused scan (else the wide path, bf_wide.hip).
bool fused_shape(const cvs_dataset* ds, int64_t k) { return ds->d <= kFusedMaxDim && k <= kFusedMaxK; }

BfPlan plan_bf(cvs_context* ctx, const cvs_dataset* ds, const float* queries, int64_t q, int64_t k,
               const uint32_t* nbr, const float* dist) {
  validate_bf(ctx, ds, queries, q, k, nbr, dist);
  if (!fused_shape(ds, k)) fail(CVS_ERR_UNSUPPORTED, "shape outside the fused scan (d <= 1024, k <= 112)");

  BfPlan p;
  p.ks = int(ds->dp / kStepCols);
  const int rpu = 2 * kStageBlocks * 32 / p.ks;  // rows per unit
  p.n_units = ds->n_tiles * p.ks / (2 * kStageBlocks);
  p.kp = choose_kp(k);
  p.qblocks = unsigned((q + kQB - 1) / kQB);
  const bool global_lists = p.kp > 64;
  // Dataset ranges (workgroups along N): one per compute unit, at most 128
  // with kp = 128, and 32 for large batches, whose 128-query blocks then run
  // range-major so that the blocks sharing a range stream it together
  // through L2 / MALL.
  p.large_batch = p.qblocks > 8;
  int G = ctx->compute_units;
  if (G > 256) G = 256;
  if (global_lists && G > 128) G = 128;
  if (p.large_batch && G > 32) G = 32;
  if (int64_t(G) > p.n_units) G = int(p.n_units);
  // Large batches with kp = 128 run the register-blocked scan: persistent
  // workgroups over (query block, row block) units, n_lists lists per query.
  if (p.large_batch) {
    const GemmPlan gp = plan_gemm_scan(p.ks, p.kp, ds->n_tiles / 4, int((q + 31) / 32), ctx->compute_units);
    if (gp.ok) {
      p.gemm = true;
      p.gemm_wg = gp.n_wg;
      G = gp.n_lists;
    }
  }
  p.G = G;
  p.stride = global_lists ? Lists<128, kModeScan>::CAP : p.kp;

  // Sample: 16,384 rows for small batches, 65,536 for other large ones and
  // 32,768 for the register-blocked scan, in whole units, evenly strided,
  // over Gs workgroups; 2 minima per (query, workgroup).  The initial
  // threshold (below) then sits near rank r * n / sample of each query's
  // distances, so a workgroup's lists see about r * n / (sample * G)
  // appends per query over its range.  Small batches are bound by the
  // scan's HBM stream, where a few more appends cost little and the
  // sample's own latency is what shows.  The register-blocked scan's appends
  // and compactions sit on its critical path, so its threshold rank matters
  // (about 2 ms per doubling at N=1M Q=10,000 K=100); with the rank rule
  // below a 32,768-row sample keeps it at ~977 for 1.15 ms of sampling.
  p.s_units = (p.gemm ? 32768 : p.large_batch ? 65536 : 16384) / rpu;
  if (p.s_units < 1) p.s_units = 1;
  if (p.s_units > p.n_units) p.s_units = p.n_units;
  p.s_stride = p.n_units / p.s_units;
  p.Gs = std::min(ctx->compute_units, 256);
  if (int64_t(p.Gs) > p.s_units) p.Gs = int(p.s_units);
  p.m_min = 2 * p.Gs;
  // The r-th smallest sample minimum bounds r distinct rows (the minima
  // are over disjoint row sets).  The merge certifies its R candidates
  // against the lists' final thresholds, so that threshold should lie at
  // rank R or beyond among the query's n keys.  It lies below rank R only if
  // r of the sampled rows fall among the query's R nearest, and that count
  // is close to Poisson with mean lambda = R * sampled / n: r is the
  // smallest rank with P(Poisson(lambda) >= r) <= 1e-9, at most R (where
  // the sample covers every row, rank r is certain).  A threshold set too
  // low is caught by the certificate, but its remedy re-ranks every row.
  // A lower threshold means fewer appends for the scan, which is what lets
  // the large-batch sample shrink: at N=1M D=1024 Q=10,000 K=100, 32,768
  // rows and r = 32 put it at expected rank 977 (as 131,072 rows and
  // r = kp = 128 did), for a third of the sample's time.
  {
    const int R = p.kp > 64 ? 2 * p.kp : std::min(2 * p.kp, 128);
    const double lambda = double(R) * double(p.s_units * rpu) / double(ds->n);
    double term = std::exp(-lambda), cdf = term;
    int r = 1;
    while (1.0 - cdf > 1e-9 && r < R) {
      term *= lambda / double(r);
      cdf += term;
      ++r;
    }
    p.sel_rank = std::max(1, std::min({r, R, p.m_min}));
  }

  p.q_tiles = (q + 31) / 32;
  auto align = [](size_t b) { return (b + 255) / 256 * 256; };
  p.off_qnorm = align(size_t(p.q_tiles) * size_t(p.ks) * kStepBytes);
  p.off_qerr = p.off_qnorm + align(size_t(p.q_tiles) * 32 * sizeof(float));
  p.off_thr = p.off_qerr + align(size_t(q) * sizeof(float));
  p.off_smin = p.off_thr + align(size_t(q) * sizeof(float));
  p.off_lmin = p.off_smin + align(size_t(q) * size_t(p.m_min) * sizeof(float));
  p.off_lcut = p.off_lmin + align(size_t(q) * size_t(G) * sizeof(uint64_t));
  p.off_part = p.off_lcut + align(size_t(q) * size_t(G) * sizeof(float));
  p.total = p.off_part + align(size_t(q) * size_t(G) * size_t(p.stride) * sizeof(uint64_t));
  return p;
}

// Enqueues the five launches of one search on the context stream, with the
// workspace at `ws` (p.total bytes; nothing in it needs to start at zero:
// every byte a launch reads was written by an earlier launch of the same
// call).  `timed` = false skips the timing facility (no events).
void bf_launch(cvs_context* ctx, const cvs_dataset* ds, const BfPlan& p, const float* queries, int64_t q,
               int64_t k, uint32_t* nbr, float* dist, char* ws, bool timed) {
  u32x4* qtiles = reinterpret_cast<u32x4*>(ws);
  float* qnorms = reinterpret_cast<float*>(ws + p.off_qnorm);
  float* qerr = reinterpret_cast<float*>(ws + p.off_qerr);
  float* thr0 = reinterpret_cast<float*>(ws + p.off_thr);
  float* sgmin = reinterpret_cast<float*>(ws + p.off_smin);
  uint64_t* lmin = reinterpret_cast<uint64_t*>(ws + p.off_lmin);
  float* lcut = reinterpret_cast<float*>(ws + p.off_lcut);
  uint64_t* part = reinterpret_cast<uint64_t*>(ws + p.off_part);
  const int G = p.G, kp = p.kp;

  ScanArgs args{};
  args.tiles = reinterpret_cast<const u32x4*>(ds->tiles);
  args.norms = reinterpret_cast<const f32x4*>(ds->norms);
  args.n_units = p.n_units;
  args.qtiles = qtiles;
  args.qnorms = qnorms;
  args.nq = int(q);
  args.n_qtiles = int(p.q_tiles);
  args.kp = kp;
  args.thr0 = thr0;
  args.part = part;
  args.sgmin = sgmin;
  args.lmin = lmin;
  args.lcut = lcut;
  args.s_units = p.s_units;
  args.s_stride = p.s_stride;
  args.n_qblocks = int(p.qblocks);
  const unsigned wave_blocks = unsigned((q + kWaves - 1) / kWaves);

  const TimerSpan t0 = timed ? timer_span(ctx, "bf_prep") : TimerSpan{};
  hipExtLaunchKernelGGL(query_tiles_kernel, dim3(unsigned((p.q_tiles * 32 + kWaves - 1) / kWaves)),
                        dim3(kThreads), 0, ctx->stream, t0.start, t0.stop, 0, queries, q, ds->d, p.ks,
                        p.q_tiles * 32, static_cast<const float*>(ds->mu), ds->scale, qtiles, qnorms, qerr);
  after_launch("query_tiles_kernel");

  const TimerSpan t1 = timed ? timer_span(ctx, "bf_sample") : TimerSpan{};
  // Large batches sample range-major (the workgroups of one sampled range
  // for every query block dispatched together), so that the sampled rows are
  // read from HBM about once and then from L2, not once per query block.
  args.n_ranges = p.Gs;
  args.qb_fast = p.large_batch ? 1 : 0;
  launch_scan(ctx, p.ks, p.large_batch ? dim3(unsigned(p.Gs) * p.qblocks, 1) : dim3(unsigned(p.Gs), p.qblocks), args,
              kModeSample, t1.start, nullptr);
  hipExtLaunchKernelGGL(bf_select_kernel, dim3(wave_blocks), dim3(kThreads), 0, ctx->stream, nullptr, t1.stop, 0,
                        static_cast<const float*>(sgmin), p.m_min, p.sel_rank, int(q), thr0);
  after_launch("bf_select_kernel");

  const TimerSpan t2 = timed ? timer_span(ctx, "bf_scan") : TimerSpan{};
  if (p.gemm) {
    GemmArgs ga{};
    ga.tiles = args.tiles;
    ga.norms = ds->norms;
    ga.n_rt = ds->n_tiles / 4;
    ga.ks = p.ks;
    ga.qtiles = qtiles;
    ga.qnorms = qnorms;
    ga.nq = int(q);
    ga.n_qtiles = int(p.q_tiles);
    ga.thr0 = thr0;
    ga.part = part;
    ga.lmin = lmin;
    ga.lcut = lcut;
    ga.n_lists = G;
    launch_gemm_scan(ctx, ga, p.gemm_wg, t2.start, t2.stop);
  } else {
    args.n_ranges = G;
    args.qb_fast = p.large_batch ? 1 : 0;
    launch_scan(ctx, p.ks, p.large_batch ? dim3(unsigned(G) * p.qblocks, 1) : dim3(unsigned(G), p.qblocks), args,
                kModeScan, t2.start, t2.stop);
  }

  const Cert cert = make_cert(ctx, ds, qnorms, qerr);
  const TimerSpan t3 = timed ? timer_span(ctx, "bf_merge") : TimerSpan{};
  // Candidates re-ranked per query: 2 kp up to 128 (32 for k <= 10, 64 for
  // k <= 24, 128 for k <= 48), 256 for kp = 128 (k <= 112).  The rank gap
  // between the k-th result and the last candidate is what lets the
  // certificate pass: on the benchmark's distribution at N = 1M, 16
  // candidates for k = 10 or 128 for k = 100 leave most queries uncertified.
  if (kp <= 32)
    hipExtLaunchKernelGGL(bf_merge_filter_kernel<1>, dim3(unsigned(q)), dim3(kThreads), 0, ctx->stream, t3.start,
                          t3.stop, 0, static_cast<const uint64_t*>(part), static_cast<const uint64_t*>(lmin),
                          static_cast<const float*>(lcut), G, kp, static_cast<const float*>(ds->rows), ds->n, ds->d,
                          queries, k, cert, nbr, dist);
  else if (kp <= 64)
    hipExtLaunchKernelGGL(bf_merge_filter_kernel<2>, dim3(unsigned(q)), dim3(kThreads), 0, ctx->stream, t3.start,
                          t3.stop, 0, static_cast<const uint64_t*>(part), static_cast<const uint64_t*>(lmin),
                          static_cast<const float*>(lcut), G, kp, static_cast<const float*>(ds->rows), ds->n, ds->d,
                          queries, k, cert, nbr, dist);
  else
    hipExtLaunchKernelGGL(bf_merge_kernel<4>, dim3(unsigned(q)), dim3(kThreads), 0, ctx->stream, t3.start, t3.stop,
                          0, static_cast<const uint64_t*>(part), static_cast<const uint64_t*>(lmin),
                          static_cast<const float*>(lcut), G, kp, p.stride, static_cast<const float*>(ds->rows), ds->n,
                          ds->d, queries, k, cert, nbr, dist);
  after_launch("bf_merge_kernel");
}

void bf_search_device(cvs_context* ctx, const cvs_dataset* ds, const float* queries, int64_t q,
                      int64_t k, uint32_t* nbr, float* dist) {
  validate_bf(ctx, ds, queries, q, k, nbr, dist);
  if (!fused_shape(ds, k)) {
    bf_wide_search(ctx, ds, queries, q, k, nbr, dist);
    return;
  }
  const BfPlan p = plan_bf(ctx, ds, queries, q, k, nbr, dist);
  ctx->ws_search.reserve(p.total);
  bf_launch(ctx, ds, p, queries, q, k, nbr, dist, ctx->ws_search.as<char>(), true);
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point cvs_bf_search_noalloc: one
// array per device, loaded with the code object and held until the process
// ends.  In host code `scratch` only names the symbol; its device address
// comes from hipGetSymbolAddress, once per device, with that device
// current.  Every call on a device shares its array.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

char* scratch_on(int device) {
  if (device < 0 || device >= kMaxDevices) fail(CVS_ERR_UNSUPPORTED, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    CVS_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) fail(CVS_ERR_RUNTIME, "scratch array has no device address");
    g_scratch_ptr[device] = ptr;
  }
  return static_cast<char*>(g_scratch_ptr[device]);
}

}  // namespace

namespace bf {
void launch_query_tiles(cvs_context* ctx, const cvs_dataset* ds, const float* queries, int64_t q, int64_t q_rows,
                        u32x4* qtiles, float* qnorms, float* qerr, hipEvent_t e0, hipEvent_t e1) {
  hipExtLaunchKernelGGL(query_tiles_kernel, dim3(unsigned((q_rows + kWaves - 1) / kWaves)), dim3(kThreads), 0,
                        ctx->stream, e0, e1, 0, queries, q, ds->d, int(ds->dp / kStepCols), q_rows,
                        static_cast<const float*>(ds->mu), ds->scale, qtiles, qnorms, qerr);
  after_launch("query_tiles_kernel");
}

// Certificate constants of a search over `ds` (see Cert).
Cert make_cert(cvs_context* ctx, const cvs_dataset* ds, const float* qnorms, const float* qerr) {
  Cert c{};
  const double d = double(ds->d);
  c.s2 = ds->scale * ds->scale;
  c.rmax = ds->cert_rmax;
  c.dx = ds->cert_dx;
  c.a_coef = float(2.0 * (d + 16.0) * 0x1p-24 * (1.0 + 0x1p-20));
  c.rho = float(2.0 * (d + 8.0) * 0x1p-24 * (1.0 + 0x1p-20));
  // fp16 subnormal rounding (2^-25 absolute per element) is inside the
  // measured error; this covers fl(q - mu) against q - mu, which the
  // measured error does not see: 2^-24 |s (q - mu)| <= 2^-24 (|q~| + err),
  // added by the merge as |q~| 2^-23, plus the fp32 sum behind err.
  c.qslack = float(std::sqrt(d) * 0x1p-25);
  c.qnorms = qnorms;
  c.qerr = qerr;
  c.counters = ctx->bf_counters;
  return c;
}

}  // namespace bf
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

int cvs_bf_search_noalloc(cvs_context* ctx, const cvs_dataset* ds, const float* queries_dev, int64_t q,
                          int64_t k, uint32_t* out_neighbors_dev, float* out_distances_dev) {
  return guarded([&] {
    bind(ctx);
    validate_bf(ctx, ds, queries_dev, q, k, out_neighbors_dev, out_distances_dev);
    if (!fused_shape(ds, k))
      fail(CVS_ERR_UNSUPPORTED, "cvs_bf_search_noalloc runs the fused scan only: d <= 1024 and k <= 112");
    const BfPlan p = plan_bf(ctx, ds, queries_dev, q, k, out_neighbors_dev, out_distances_dev);
    if (p.total > kScratchBytes)
      fail(CVS_ERR_UNSUPPORTED, "cvs_bf_search_noalloc: this call needs " + std::to_string(p.total) +
                                    " bytes of scratch, more than the " + std::to_string(kScratchBytes) +
                                    " the library holds per device (use fewer queries or a smaller k)");
    char* ws = scratch_on(ctx->device);
    bf_launch(ctx, ds, p, queries_dev, q, k, out_neighbors_dev, out_distances_dev, ws, false);
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
