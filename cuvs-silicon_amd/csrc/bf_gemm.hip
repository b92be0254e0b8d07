// Register-blocked brute-force scan for large query batches (gfx950).
//
// The streaming scan (bf_search.hip) keeps each wave's 32 queries resident
// for the whole dimension, so every MFMA reads a fresh 1 KiB dataset fragment
// from LDS.  For batches of thousands of queries this kernel tiles like a
// GEMM instead:
//
//  - A workgroup tile is 128 dataset rows x 512 queries.  Each of the 4 waves
//    owns 128 queries (4 query tiles) against the same 128 rows (4 row tiles):
//    a 4 x 4 block of v_mfma_f32_32x32x16_f16 accumulators (256 fp32 per
//    lane, in AGPRs).  Per k-step a wave reads 4 row and 4 query fragments
//    for 16 MFMAs.
//  - The dimension is streamed in stages of 32 columns (2 k-steps): 32 KiB of
//    query tiles + 8 KiB of row tiles + the row block's norms, loaded
//    straight into LDS (buffer_load ... lds, no VGPR staging).  Query tiles
//    (shared in L2) are loaded 3 stages ahead into 3 buffers, row tiles
//    (streamed from the MALL / HBM, ~2 us away under load) 6 stages ahead
//    into 6 buffers.  One barrier per stage, in its middle: the MFMAs of
//    the first k-step run while the second's fragments are read, those of
//    the second while the next stage's first fragments are read and the
//    loads are issued, one per MFMA.  Out-of-range buffer loads return zeros
//    without a memory access, so every pipelined load is unconditional.
//  - After the last stage of a 128-row block the accumulators become
//    distances |q|^2 + |x|^2 - 2 q.x and pass the same thresholded two-half
//    candidate lists as the streaming scan's kp = 128 path (global lists,
//    rare appends, ballot radix compaction), so the sample / select / merge
//    kernels are shared.
//  - Scheduling is persistent and balanced: the work is the (512-query
//    block, 128-row block) units, block-major, split evenly over the
//    workgroups taken in XCD-major order (workgroup i runs on XCD i % 8,
//    round-robin dispatch).  Each XCD thus covers a contiguous run of query
//    blocks that its workgroups share in L2, and no XCD waits on another's
//    extra block.  A query block's lists are indexed by the covering
//    workgroup's position among those covering it, so each list has one
//    writer; the workgroup that ends a block fills the unused list slots
//    with empty lists.
//
// The same file holds cvs_calibrate_mfma, this register block's matrix-core
// rate with no memory traffic, the reference point for the scan's own rate.
#include <algorithm>
#include <cmath>

#include "bf_common.hpp"

namespace cvs {
namespace bf {
namespace {

constexpr int kGThreads = 256;
constexpr int kGWaves = 4;
constexpr int kRT = 4;           // 32-row tiles per workgroup tile (128 rows)
constexpr int kQT = 16;          // 32-query tiles per workgroup (512 queries)
constexpr int kQTW = kQT / kGWaves;  // query tiles per wave
constexpr int kSeg = 2048;       // bytes of one tile's 2 k-steps (a stage of one tile)
constexpr int kStageVec = (kQT + kRT) * kSeg / 16;  // 16-byte vectors per stage (2560)
constexpr int kRowVec0 = kQT * kSeg / 16;           // first row vector in a stage (2048)
constexpr int kQLoads = kRowVec0 / kGThreads;       // 16-byte query loads per thread and stage (8)
constexpr int kRLoads = (kStageVec - kRowVec0) / kGThreads;  // 16-byte row loads (2); + 1 norm load
constexpr int kRowVec = kStageVec - kRowVec0;       // 16-byte vectors of a stage's rows (512)
// Row tiles stream from the MALL / HBM with ~2 us of latency under load, far
// more than the query tiles (shared in L2), so they are loaded further ahead.
constexpr int kQAhead = 3, kRAhead = 6;             // stages loaded ahead = LDS buffers
constexpr int kNSlots = 4;                          // norm slots (128-row blocks in flight)
constexpr int kKP = 128;
using GL = Lists<kKP, kModeScan>;

// s_waitcnt immediate (gfx9 encoding): vmcnt[3:0] in bits 3:0, vmcnt[5:4] in
// bits 15:14, expcnt in 6:4, lgkmcnt in 11:8; 7 and 15 mean "no wait".
constexpr int waitcnt_imm(int vm, int lgkm) { return (vm & 0xF) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8); }

using rsrc4 = int __attribute__((ext_vector_type(4)));

// Buffer load straight to LDS (buffer_load ... lds): lane l writes kBytes at
// LDS byte address m0 + kBytes * l (m0 the same for every lane).  Written as
// inline assembly so that the compiler does not wait for every outstanding
// load before each later LDS read (it cannot tell which LDS bytes the load
// writes); the kernel orders these loads and the reads of their data with
// explicit s_waitcnt vmcnt and barriers.  M0 is an input operand, so the
// compiler knows it changes; one wait state separates its write from the
// load that reads it.
template <int kBytes, bool kNT>
__device__ CVS_INLINE void lds_dma(rsrc4 rs, int m0, uint32_t voff, int soff) {
  if constexpr (kBytes == 16 && kNT)
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen nt lds"
                 :: "v"(voff), "s"(rs), "s"(soff), "{m0}"(m0) : "memory");
  else if constexpr (kBytes == 16)
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :: "v"(voff), "s"(rs), "s"(soff), "{m0}"(m0) : "memory");
  else
    asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, %2 offen lds"
                 :: "v"(voff), "s"(rs), "s"(soff), "{m0}"(m0) : "memory");
}

// Raw buffer descriptor: 48-bit base, stride 0, num_records bytes.
__device__ CVS_INLINE rsrc4 make_rsrc(const void* base, int bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  rsrc4 r;
  r.x = int(uint32_t(b));
  r.y = int(uint32_t(b >> 32) & 0xFFFFu);
  r.z = bytes;
  r.w = kRsrcWord3;
  return r;
}

__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void bf_gemm_scan_kernel(GemmArgs a) {
  // Stage buffers: 3 x 32 KiB of query tiles, 6 x 8 KiB of row tiles, and
  // the norms of the 128-row blocks in 4 slots by the block's sequence
  // number (floats 0..127 of a slot; 128..255 receive a second copy).
  __shared__ u32x4 s_q[kQAhead][kRowVec0];
  __shared__ u32x4 s_r[kRAhead][kRowVec];
  __shared__ float s_norm[kNSlots][2 * kRT * 32];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int G = a.n_lists;
  const int NWG = int(gridDim.x);  // a multiple of 8
  const int xcd = int(blockIdx.x) % 8;
  const int v = xcd * (NWG / 8) + int(blockIdx.x) / 8;  // position in XCD-major order
  const int KS = a.ks;
  const int SPT = KS / 2;  // stages per 128-row block
  const int64_t n_rt = a.n_rt;
  const int QB = (a.n_qtiles + kQT - 1) / kQT;
  // Work units: (512-query block, 128-row block) pairs, block-major; this
  // workgroup's are [u0, u1), in segments of one query block each.  The
  // host guarantees W >= NWG, so no range is empty.
  const int64_t W = int64_t(QB) * n_rt;
  const int64_t u0 = int64_t(v) * W / NWG, u1 = int64_t(v + 1) * W / NWG;
  if (u0 >= u1) return;
  const int total = int(u1 - u0) * SPT;  // stages of this workgroup (< 2^31: checked by the host)
  // The workgroup whose range holds unit u.
  auto wg_of = [&](int64_t u) CVS_INLINE { return int(((u + 1) * NWG - 1) / W); };

  // Buffer resources: the row tiles and norms of the current segment's
  // row blocks, and the current query block's tiles.  A stage past the last
  // has zero-length resources, so its loads return zeros without a memory
  // access.
  const uint32_t tile_bytes = uint32_t(KS) * 1024u;
  auto rows_rsrc = [&](int64_t rb0, int64_t len) CVS_INLINE {
    return make_rsrc(a.tiles + rb0 * kRT * KS * 64, int(uint32_t(len) * kRT * tile_bytes));
  };
  auto norms_rsrc = [&](int64_t rb0, int64_t len) CVS_INLINE {
    return make_rsrc(a.norms + rb0 * kRT * 32, int(uint32_t(len) * kRT * 128u));
  };

  // Per-thread load offsets within a stage (the stage's own offset goes in
  // soffset): query load i covers query tile 2 i + tid / 128, row load i row
  // tile 2 i + tid / 128, each at 16 (tid % 128) bytes into the tile's
  // 2 KiB stage segment.  A query tile past the block's last lies past the
  // resource's end, so its load returns zeros.  The norm load (4 bytes) is
  // norm tid % 128 of the row block.
  const uint32_t toff = uint32_t(tid >> 7) * tile_bytes + uint32_t(tid & 127) * 16u;
  const uint32_t noff = uint32_t(tid & 127) * 4u;

  // Load cursors of the next stage's query tiles and of the next stage's
  // row tiles, all scalars kept as running offsets so that a stage costs a
  // few scalar adds: the stage's soffset, the LDS address (M0) of this
  // wave's slot in the stage's buffer, the stages left, and a resource that
  // becomes zero-length past the last stage.  The loads go straight to LDS
  // (buffer_load ... lds: lane l of a wave writes at M0 + size * l): per
  // stage 8 query loads, 2 row loads and 1 norm load per thread.
  auto lds_addr = [](const void* p) CVS_INLINE {
    return __builtin_amdgcn_readfirstlane(
        int(uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p))));
  };
  const int q_lds0 = lds_addr(&s_q[0][wave * 64]);
  const int r_lds0 = lds_addr(&s_r[0][wave * 64]);
  const int n_lds0 = lds_addr(&s_norm[0][wave * 64]);
  constexpr int kQBufBytes = kRowVec0 * 16, kRBufBytes = kRowVec * 16, kNSlotBytes = 2 * kRT * 32 * 4;
  constexpr int kLoadBytes = kGThreads * 16;  // LDS bytes between loads i and i + 1 of a stage
  auto qrsrc_of = [&](int blk) CVS_INLINE {
    const int qt0 = blk * kQT;
    return make_rsrc(a.qtiles + int64_t(qt0) * KS * 64, int(uint32_t(std::min(kQT, a.n_qtiles - qt0)) * tile_bytes));
  };
  // End of the segment that starts at unit u.
  auto seg_end = [&](int64_t u) CVS_INLINE {
    const int64_t e = (u / n_rt + 1) * n_rt;
    return e < u1 ? e : u1;
  };
  struct {
    rsrc4 rs;
    int soff = 0, m0, buf = 0, seg_left;
    int64_t seg_e;
  } lq;
  lq.seg_e = seg_end(u0);
  lq.seg_left = int(lq.seg_e - u0);
  lq.rs = qrsrc_of(int(u0 / n_rt));
  lq.m0 = q_lds0;
  struct {
    rsrc4 rs, ns;
    int soff = 0, nsoff = 0, s = 0, seg_left, left, m0, buf = 0, nm0, slot = 0;
    int64_t seg_e;
  } lr;
  lr.seg_e = seg_end(u0);
  lr.seg_left = int(lr.seg_e - u0);
  lr.rs = rows_rsrc(u0 % n_rt, lr.seg_left);
  lr.ns = norms_rsrc(u0 % n_rt, lr.seg_left);
  lr.left = total;
  lr.m0 = r_lds0;
  lr.nm0 = n_lds0;
  auto issue_q = [&](int i) CVS_INLINE {
    lds_dma<16, false>(lq.rs, lq.m0 + i * kLoadBytes, toff + uint32_t(2 * i) * tile_bytes, lq.soff);
  };
  auto issue_r = [&](int i) CVS_INLINE {
    if (i < kRLoads)
      lds_dma<16, true>(lr.rs, lr.m0 + i * kLoadBytes, toff + uint32_t(2 * i) * tile_bytes, lr.soff);
    else
      lds_dma<4, false>(lr.ns, lr.nm0, noff, lr.nsoff);
  };
  // Query stages: the 32 stage segments of each query tile, once per row
  // block of the segment; the last segment's end is the end of the
  // workgroup's stages.
  auto advance_q = [&]() CVS_INLINE {
    lq.soff += kSeg;
    lq.m0 = lq.buf == kQAhead - 1 ? q_lds0 : lq.m0 + kQBufBytes;
    lq.buf = lq.buf == kQAhead - 1 ? 0 : lq.buf + 1;
    if (lq.soff == int(tile_bytes)) {
      lq.soff = 0;
      if (--lq.seg_left == 0) {
        if (lq.seg_e < u1) {
          const int64_t e = seg_end(lq.seg_e);
          lq.rs = qrsrc_of(int(lq.seg_e / n_rt));
          lq.seg_left = int(e - lq.seg_e);
          lq.seg_e = e;
        } else {
          lq.rs.z = 0;
        }
      }
    }
  };
  // Row stage s of the segment's row block r is at soffset
  // 4 r tile_bytes + 2 KiB s: the last stage of a row block steps
  // 2 KiB + 3 tile_bytes to the next one.  A new segment starts at row
  // block 0.
  auto advance_r = [&]() CVS_INLINE {
    lr.soff += kSeg;
    lr.m0 = lr.buf == kRAhead - 1 ? r_lds0 : lr.m0 + kRBufBytes;
    lr.buf = lr.buf == kRAhead - 1 ? 0 : lr.buf + 1;
    if (++lr.s == SPT) {
      lr.s = 0;
      lr.soff += 3 * int(tile_bytes);
      lr.nsoff += kRT * 128;
      lr.nm0 = lr.slot == kNSlots - 1 ? n_lds0 : lr.nm0 + kNSlotBytes;
      lr.slot = lr.slot == kNSlots - 1 ? 0 : lr.slot + 1;
      if (--lr.seg_left == 0 && lr.seg_e < u1) {
        const int64_t e = seg_end(lr.seg_e);
        lr.seg_left = int(e - lr.seg_e);
        lr.rs = rows_rsrc(0, lr.seg_left);
        lr.ns = norms_rsrc(0, lr.seg_left);
        lr.seg_e = e;
        lr.soff = 0;
        lr.nsoff = 0;
      }
    }
    if (--lr.left == 0) {
      lr.rs.z = 0;
      lr.ns.z = 0;
    }
  };
  auto gload_q = [&]() CVS_INLINE {
#pragma unroll
    for (int i = 0; i < kQLoads; ++i) issue_q(i);
    advance_q();
  };
  auto gload_r = [&]() CVS_INLINE {
#pragma unroll
    for (int i = 0; i <= kRLoads; ++i) issue_r(i);
    advance_r();
  };
  // Issue order: rows of stages 0..2, then (queries g, rows g + 3) for
  // g = 0..2 in the prologue, and (queries g + 3, rows g + 6) in stage g.
  // Loads complete in issue order, so once stage h's query loads have
  // landed, so have its row loads (issued earlier).  Before the barrier that
  // publishes stage g + 1, the loads issued after stage g + 1's queries are
  // rows g + 4, queries g + 2 and rows g + 5: 14.  List appends issued since
  // only lengthen the wait.  The wait also covers this thread's LDS reads.
  constexpr int kAfterQ = 2 * (kRLoads + 1) + kQLoads;
  auto wait_older_stage = [&]() CVS_INLINE { __builtin_amdgcn_s_waitcnt(waitcnt_imm(kAfterQ, 0)); };

  // Per-block query state: lane holds query qw + 32 jq (jq = 0..3) of this
  // wave's 128, in half `half` of its list.
  float qn[kQTW], thr[kQTW];
  uint32_t cnt[kQTW];
  int qw0 = 0;   // first query of this wave in the current block
  int slot = 0;  // list slot of this workgroup in the current block
  auto list_of = [&](int q) CVS_INLINE -> uint64_t* { return a.part + (int64_t(q) * G + slot) * GL::CAP; };
  auto begin_block = [&](int blk, int slot_) CVS_INLINE {
    slot = slot_;
    qw0 = blk * (kQT * 32) + wave * (kQTW * 32);
#pragma unroll
    for (int j = 0; j < kQTW; ++j) {
      const int q = qw0 + 32 * j + (lane & 31);
      const bool ok = q < a.nq;
      qn[j] = ok ? a.qnorms[q] : INFINITY;
      thr[j] = ok ? nextafterf(a.thr0[q], INFINITY) : -INFINITY;
      cnt[j] = 0;
    }
  };

  // The list state of query tile j (0..3, wave-uniform) as scalars.
  auto get_state = [&](int j, uint32_t& c, float& t) CVS_INLINE {
    c = j == 0 ? cnt[0] : j == 1 ? cnt[1] : j == 2 ? cnt[2] : cnt[3];
    t = j == 0 ? thr[0] : j == 1 ? thr[1] : j == 2 ? thr[2] : thr[3];
  };
  auto set_state = [&](int j, uint32_t c, float t) CVS_INLINE {
#pragma unroll
    for (int i = 0; i < kQTW; ++i)
      if (i == j) {
        cnt[i] = c;
        thr[i] = t;
      }
  };

  // Rebalances the lists of query tile j (count c, threshold t): halves over
  // `limit`, or totals over kp at the end (see the streaming scan's
  // compact_wave).
  auto compact_tile = [&](int j, uint32_t& c, float& t, uint32_t limit, bool total_only) CVS_INLINE {
    const uint32_t both = c + xor_lanes<32>(c);
    const uint64_t over64 = __ballot(total_only ? both > uint32_t(kKP) : c > limit);
    uint32_t over = uint32_t(over64) | uint32_t(over64 >> 32);
    if (over == 0) return;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    while (over) {
      const int i = __builtin_ctz(over);
      over &= over - 1;
      const uint32_t c0 = uint32_t(__builtin_amdgcn_readlane(int(c), i));
      const uint32_t c1 = uint32_t(__builtin_amdgcn_readlane(int(c), i + 32));
      const uint32_t kth = compact_query<GL::NS>(list_of(qw0 + 32 * j + i), GL::HALF, c0, c1, kKP);
      const uint32_t kept = c0 + c1 < uint32_t(kKP) ? c0 + c1 : uint32_t(kKP);
      if ((lane & 31) == i) {
        c = half == 0 ? (kept < uint32_t(kKP / 2) ? kept : uint32_t(kKP / 2))
                      : (kept > uint32_t(kKP / 2) ? kept - uint32_t(kKP / 2) : 0u);
        if (kth != 0xffffffffu) t = fminf(t, unord_f32(kth));
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  };

  // Appends the (distance, row) keys of one 32 x 32 block (query tile j,
  // rows row0 + 8 (r / 4) + 4 half + r % 4) below the query's threshold to
  // this lane's half list.
  auto commit = [&](int j, const f32x16& dv, uint32_t row0) CVS_INLINE {
    uint32_t c;
    float t;
    get_state(j, c, t);
    uint32_t pass = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) pass |= (dv[r] < t ? 1u : 0u) << r;
    uint64_t lanes = __ballot(pass != 0);
    uint32_t rows_any = 0;
    while (lanes) {
      const int l = __builtin_ctzll(lanes);
      lanes &= lanes - 1;
      rows_any |= uint32_t(__builtin_amdgcn_readlane(int(pass), l));
    }
    uint64_t* const mine = list_of(qw0 + 32 * j + (lane & 31)) + half * GL::HALF;
    const uint32_t rbase = row0 + 4u * uint32_t(half);
    while (rows_any) {
      const int r = __builtin_ctz(rows_any);
      rows_any &= rows_any - 1;
      if ((pass >> r) & 1u) {
        mine[c] = (uint64_t(ord_f32(dv[r])) << 32) | (rbase + uint32_t(8 * (r >> 2) + (r & 3)));
        ++c;
      }
      if (__ballot(c >= uint32_t(GL::HALF)) != 0) {
        compact_tile(j, c, t, uint32_t(GL::HALF - 1), false);
#pragma unroll
        for (int r2 = 0; r2 < 16; ++r2)
          if (!(dv[r2] < t)) pass &= ~(1u << r2);
      }
    }
    set_state(j, c, t);
  };

  // Writes this wave's lists of the finished block in place (first kp
  // entries: half 0's keys, then half 1's, then sentinels) and their minima.
  auto end_block = [&]() CVS_INLINE {
#pragma unroll 1
    for (int j = 0; j < kQTW; ++j) {
      uint32_t c;
      float t;
      get_state(j, c, t);
      compact_tile(j, c, t, 0u, true);
      set_state(j, c, t);
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    for (int i = 0; i < 32; ++i) {
      uint64_t key[kQTW][2];
      uint64_t mn[kQTW];
#pragma unroll
      for (int j = 0; j < kQTW; ++j) {
        const int q = qw0 + 32 * j + i;
        const uint32_t c0 = uint32_t(__builtin_amdgcn_readlane(int(cnt[j]), i));
        const uint32_t c1 = uint32_t(__builtin_amdgcn_readlane(int(cnt[j]), i + 32));
        const uint64_t* src = list_of(q < a.nq ? q : 0);
        mn[j] = kSentinel;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const uint32_t e = uint32_t(lane + 64 * t);
          key[j][t] = q >= a.nq ? kSentinel
                                : (e < c0 ? src[e] : (e < c0 + c1 ? src[GL::HALF + (e - c0)] : kSentinel));
          mn[j] = key[j][t] < mn[j] ? key[j][t] : mn[j];
        }
      }
#pragma unroll
      for (int j = 0; j < kQTW; ++j) {
        const int q = qw0 + 32 * j + i;
        if (q >= a.nq) continue;
        uint64_t* lst = list_of(q);
#pragma unroll
        for (int t = 0; t < 2; ++t) lst[lane + 64 * t] = key[j][t];
        uint64_t m = mn[j];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
          const uint64_t y = shfl_xor_u64(m, o);
          m = y < m ? y : m;
        }
        const float cut = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(thr[j]), i));
        if (lane == 0) {
          a.lmin[int64_t(q) * G + slot] = m;
          a.lcut[int64_t(q) * G + slot] = cut;
        }
      }
    }
  };

  // Empty lists (kp sentinels, sentinel minimum) in slots [from, G) of this
  // wave's queries of the current block.
  auto fill_unused = [&](int from) CVS_INLINE {
    for (int sl = from; sl < G; ++sl)
      for (int i = 0; i < kQTW * 32; ++i) {
        const int q = qw0 + i;
        if (q >= a.nq) break;
        uint64_t* lst = a.part + (int64_t(q) * G + sl) * GL::CAP;
#pragma unroll
        for (int t = 0; t < kKP / 64; ++t) lst[lane + 64 * t] = kSentinel;
        if (lane == 0) {
          a.lmin[int64_t(q) * G + sl] = kSentinel;
          a.lcut[int64_t(q) * G + sl] = INFINITY;  // covers no rows
        }
      }
  };

  f32x16 acc[kRT][kQTW];
#pragma unroll
  for (int r = 0; r < kRT; ++r)
#pragma unroll
    for (int j = 0; j < kQTW; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[r][j][e] = 0.f;

  // Fragments of one k-step: 4 row tiles and this wave's 4 query tiles.
  half8 fa0[kRT], fb0[kQTW], fa1[kRT], fb1[kQTW];
  auto read_k = [&](int qbuf, int rbuf, int t, half8 (&fa)[kRT], half8 (&fb)[kQTW]) CVS_INLINE {
    const u32x4* sq = s_q[qbuf];
    const u32x4* sr = s_r[rbuf];
#pragma unroll
    for (int r = 0; r < kRT; ++r) fa[r] = __builtin_bit_cast(half8, sr[(r * 2 + t) * 64 + lane]);
#pragma unroll
    for (int j = 0; j < kQTW; ++j) fb[j] = __builtin_bit_cast(half8, sq[((wave * kQTW + j) * 2 + t) * 64 + lane]);
  };

  // Pipeline: stage g is computed from query buffer g % 3 and row buffer
  // g % 6.  Its first k-step's fragments are read before it starts; its
  // second k-step's are read under the first k-step's 16 MFMAs.  Then the
  // barrier that publishes stage g + 1 (every wave has waited for its own
  // loads of it, and has finished reading stage g's buffers), the loads of
  // stage g + 3's queries and stage g + 6's rows into them, and the second
  // k-step's MFMAs, under which stage g + 1's first fragments are read.
  gload_r();
  gload_r();
  gload_r();
#pragma unroll
  for (int i = 0; i < kQAhead; ++i) {
    gload_q();
    gload_r();
  }
  // Stage 0 landed: after its queries came rows 3, queries 1, rows 4,
  // queries 2, rows 5.
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(kAfterQ + kQLoads + kRLoads + 1, 0));
  __syncthreads();
  int cq = 0, cr6 = 0, cseq = 0;
  read_k(0, 0, 0, fa0, fb0);

  for (int64_t u = u0; u < u1;) {
    // Segment: query block blk, row blocks [rb_lo, rb_hi) of it.
    const int blk = int(u / n_rt);
    const int64_t bstart = int64_t(blk) * n_rt;
    const int64_t ue = seg_end(u);
    const int first_wg = wg_of(bstart);
    begin_block(blk, v - first_wg);
    for (int64_t row_blk = u - bstart; row_blk < ue - bstart; ++row_blk) {
      for (int cs = 0; cs < SPT; ++cs) {
        // First k-step: MFMA i on (row tile i / 4, query tile i % 4), each
        // of the first 8 followed by one of the second k-step's fragment
        // reads.  The order is pinned (sched_barrier) so that every LDS read
        // and load issues under a running MFMA.
        {
          const u32x4* sq = s_q[cq];
          const u32x4* sr = s_r[cr6];
#pragma unroll
          for (int i = 0; i < kRT * kQTW; ++i) {
            acc[i / kQTW][i % kQTW] =
                __builtin_amdgcn_mfma_f32_32x32x16_f16(fa0[i / kQTW], fb0[i % kQTW], acc[i / kQTW][i % kQTW], 0, 0, 0);
            if (i < kRT) fa1[i] = __builtin_bit_cast(half8, sr[(i * 2 + 1) * 64 + lane]);
            else if (i < kRT + kQTW)
              fb1[i - kRT] = __builtin_bit_cast(half8, sq[((wave * kQTW + i - kRT) * 2 + 1) * 64 + lane]);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        wait_older_stage();
        __syncthreads();
        cq = cq == kQAhead - 1 ? 0 : cq + 1;
        cr6 = cr6 == kRAhead - 1 ? 0 : cr6 + 1;
        // Second k-step: MFMAs interleaved with the next stage's first
        // fragment reads and with the 11 loads of stage g + 3's queries and
        // stage g + 6's rows (into the buffers stage g used).
        {
          const u32x4* sq = s_q[cq];
          const u32x4* sr = s_r[cr6];
#pragma unroll
          for (int i = 0; i < kRT * kQTW; ++i) {
            acc[i / kQTW][i % kQTW] =
                __builtin_amdgcn_mfma_f32_32x32x16_f16(fa1[i / kQTW], fb1[i % kQTW], acc[i / kQTW][i % kQTW], 0, 0, 0);
            if (i < kRT) fa0[i] = __builtin_bit_cast(half8, sr[(i * 2) * 64 + lane]);
            else if (i < kRT + kQTW)
              fb0[i - kRT] = __builtin_bit_cast(half8, sq[((wave * kQTW + i - kRT) * 2) * 64 + lane]);
            if (i < kQLoads) issue_q(i);
            else if (i <= kQLoads + kRLoads) issue_r(i - kQLoads);
            __builtin_amdgcn_sched_barrier(0);
          }
          advance_q();
          advance_r();
        }
      }
      // Epilogue of the 128-row block: lane holds query (lane % 32) of each
      // of its 4 tiles against rows 8 (e / 4) + 4 half + e % 4 of each row
      // tile.  A block's norm slot is next written for the block 4 later,
      // whose first loads are issued at least 2 barriers after this.
      const float* nslot = s_norm[cseq & (kNSlots - 1)];
      ++cseq;
#pragma unroll
      for (int r = 0; r < kRT; ++r) {
        f32x4 dn4[4];
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) dn4[gq] = *reinterpret_cast<const f32x4*>(nslot + r * 32 + 8 * gq + 4 * half);
        const uint32_t row0 = uint32_t((row_blk * kRT + r) * 32);
#pragma unroll
        for (int j = 0; j < kQTW; ++j) {
          f32x16 dv;
          float m = INFINITY;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            dv[e] = qn[j] + dn4[e >> 2][e & 3] - 2.0f * acc[r][j][e];
            m = fminf(m, dv[e]);
          }
          // fminf skips NaN, which never passes a threshold either.
          if (__ballot(m < thr[j]) != 0) commit(j, dv, row0);
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[r][j][e] = 0.f;
        }
      }
      // Nothing of this block may stay outstanding into the next block's
      // stages.  The compiler reloads spilled values here, and it counts
      // none of the inline-assembly LDS loads, so the wait it would place
      // for such a reload inside the stage loop is vmcnt(0) at every
      // stage, which drains the whole prefetch each time.  Waiting once
      // here costs the reload's latency alone: the epilogue has let every
      // prefetched load land.
      __builtin_amdgcn_s_waitcnt(0);
    }
    end_block();
    // The workgroup that ends a block fills the block's unused list slots
    // (slots past the last covering workgroup's) with empty lists.
    if (ue == bstart + n_rt) fill_unused(v - first_wg + 1);
    u = ue;
  }
  // Drain the loads issued past the last stage before the workgroup ends.
  __builtin_amdgcn_s_waitcnt(0);
}

// ---------------------------------------------------------------------------
// Device calibration for matrix-core-bound kernels: the rate this device
// sustains on this scan's register block with no memory traffic (built,
// like the scan, with the accumulators in AGPRs).  A workgroup of 4 waves (one per SIMD, as the scan runs)
// repeats k-steps of 16 v_mfma_f32_32x32x16_f16 on a 4 x 4 block of
// accumulators (256 fp32 per lane, in AGPRs), from two sets of 4 row and
// 4 query fragments that alternate between k-steps.  With kLds the
// fragments of every k-step are read from LDS under the previous k-step's
// MFMAs, one read after each of the first 8 MFMAs, as the scan reads them
// (rows shared by the 4 waves, query tiles per wave).  The fragments come
// from the caller's fp16 data: the rate of fp16 MFMA depends on the operand
// bits it switches, so random data and the scan's own tiles can differ.
// The sum of the accumulators decides a store that never happens in
// practice but keeps every MFMA.
// ---------------------------------------------------------------------------
constexpr int kCalTiles = 4 + 16;  // fragments of one k-step: 4 row tiles + 16 query tiles (4 per wave)
constexpr uint32_t kCalVecs = 2u * kCalTiles * 64;  // 16-byte vectors of the two k-steps (40 KiB)

template <bool kLds>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void mfma_rate_kernel(const u32x4* __restrict__ src, uint32_t src_sets, int64_t ksteps, float* __restrict__ sink) {
  __shared__ u32x4 s_f[kLds ? kCalVecs : 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const u32x4* set = src + uint64_t(blockIdx.x % src_sets) * kCalVecs;
  // Vector index of fragment (k-step t, row tile r) and (t, this wave's query tile j).
  auto row_at = [&](int t, int r) { return uint32_t((t * kCalTiles + r) * 64 + lane); };
  auto qry_at = [&](int t, int j) { return uint32_t((t * kCalTiles + 4 + wave * 4 + j) * 64 + lane); };
  half8 fa[2][4], fb[2][4];
  if constexpr (kLds) {
    for (uint32_t i = threadIdx.x; i < kCalVecs; i += 256) s_f[i] = set[i];
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[t][i] = __builtin_bit_cast(half8, kLds ? s_f[row_at(t, i)] : set[row_at(t, i)]);
      fb[t][i] = __builtin_bit_cast(half8, kLds ? s_f[qry_at(t, i)] : set[qry_at(t, i)]);
    }
  f32x16 acc[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[r][j][e] = 0.f;
  for (int64_t s = 0; s < ksteps; s += 2) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        acc[i / 4][i % 4] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[t][i / 4], fb[t][i % 4], acc[i / 4][i % 4], 0, 0, 0);
        if constexpr (kLds) {
          // The other set's fragments, re-read for the k-step after next.
          if (i < 4) fa[t ^ 1][i] = __builtin_bit_cast(half8, s_f[row_at(t ^ 1, i)]);
          else if (i < 8) fb[t ^ 1][i - 4] = __builtin_bit_cast(half8, s_f[qry_at(t ^ 1, i - 4)]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) sum += acc[r][j][e];
  if (sum == 1.2345678e30f) sink[blockIdx.x * 256 + threadIdx.x] = sum;
}

}  // namespace

GemmPlan plan_gemm_scan(int ks, int kp, int64_t n_rt, int n_qtiles, int compute_units) {
  GemmPlan p;
  if (kp != kKP || ks < 8 || ks > 64 || n_rt < 1 || n_qtiles < 1) return p;
  const int64_t qb = (n_qtiles + kQT - 1) / kQT;
  // Workgroups: one per compute unit, in groups of 8 (one per XCD), fewer
  // for few query blocks so that a block is covered by at most 64.
  int64_t per_xcd = std::min<int64_t>(std::max(1, compute_units / 8), (63 * qb) / 8);
  const int64_t w = qb * n_rt;
  per_xcd = std::min<int64_t>(per_xcd, w / 8);
  if (per_xcd < 1) return p;
  const int64_t nwg = 8 * per_xcd;
  // Limits: a segment's row tiles within one buffer resource (2 GiB), the
  // stage count of a workgroup within an int.
  const int64_t units = (w + nwg - 1) / nwg;
  const int64_t seg = std::min(units, n_rt);
  if (seg * kRT * int64_t(ks) * 1024 >= (int64_t(1) << 31)) return p;
  if (units * (ks / 2) >= (int64_t(1) << 31)) return p;
  // Lists per query: the most workgroups whose unit ranges meet one block.
  auto wg_of = [&](int64_t u) { return (u + 1) * nwg - 1 >= 0 ? ((u + 1) * nwg - 1) / w : 0; };
  int64_t g = 1;
  for (int64_t b = 0; b < qb; ++b) g = std::max(g, wg_of((b + 1) * n_rt - 1) - wg_of(b * n_rt) + 1);
  p.ok = true;
  p.n_wg = int(nwg);
  p.n_lists = int(g);
  return p;
}

void launch_gemm_scan(cvs_context* ctx, const GemmArgs& args, int n_wg, hipEvent_t e0, hipEvent_t e1) {
  hipExtLaunchKernelGGL(bf_gemm_scan_kernel, dim3(unsigned(n_wg)), dim3(kGThreads), 0, ctx->stream, e0,
                        e1, 0, args);
  after_launch("bf_gemm_scan_kernel");
}

}  // namespace bf
}  // namespace cvs

using namespace cvs;
using namespace cvs::bf;

extern "C" {

int cvs_calibrate_mfma(cvs_context* ctx, const void* fp16_data, size_t data_bytes, int workgroups, int64_t ksteps,
                       int from_lds, int reps, double* out_tflops) {
  return guarded([&] {
    bind(ctx);
    if (!out_tflops) fail(CVS_ERR_INVALID_ARGUMENT, "null out_tflops");
    if (!fp16_data) fail(CVS_ERR_INVALID_ARGUMENT, "null fp16_data");
    if (workgroups < 1 || reps < 1 || ksteps < 2)
      fail(CVS_ERR_INVALID_ARGUMENT, "workgroups and reps must be positive, ksteps at least 2");
    if (reinterpret_cast<uintptr_t>(fp16_data) % 16 != 0) fail(CVS_ERR_INVALID_ARGUMENT, "fp16_data must be 16-byte aligned");
    const size_t set_bytes = size_t(kCalVecs) * 16;
    const size_t sets = data_bytes / set_bytes;
    if (sets == 0) fail(CVS_ERR_INVALID_ARGUMENT, "fp16_data must hold at least 40 KiB");
    const int64_t ks = ksteps + (ksteps & 1);
    void* sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    auto cleanup = [&] {
      if (e0) (void)hipEventDestroy(e0);
      if (e1) (void)hipEventDestroy(e1);
      if (sink) (void)hipFree(sink);
    };
    try {
      CVS_HIP(hipMalloc(&sink, size_t(workgroups) * 256 * sizeof(float)));
      CVS_HIP(hipEventCreate(&e0));
      CVS_HIP(hipEventCreate(&e1));
      const uint32_t n_sets = uint32_t(std::min<size_t>(sets, size_t(1) << 20));
      auto launch = [&] {
        if (from_lds)
          hipLaunchKernelGGL(mfma_rate_kernel<true>, dim3(unsigned(workgroups)), dim3(256), 0, ctx->stream,
                             static_cast<const u32x4*>(fp16_data), n_sets, ks, static_cast<float*>(sink));
        else
          hipLaunchKernelGGL(mfma_rate_kernel<false>, dim3(unsigned(workgroups)), dim3(256), 0, ctx->stream,
                             static_cast<const u32x4*>(fp16_data), n_sets, ks, static_cast<float*>(sink));
        after_launch("mfma_rate_kernel");
      };
      for (int i = 0; i < 2; ++i) launch();  // warm-up
      CVS_HIP(hipEventRecord(e0, ctx->stream));
      for (int i = 0; i < reps; ++i) launch();
      CVS_HIP(hipEventRecord(e1, ctx->stream));
      CVS_HIP(hipEventSynchronize(e1));
      float ms = 0.f;
      CVS_HIP(hipEventElapsedTime(&ms, e0, e1));
      const double flop = double(workgroups) * 4.0 * double(ks) * 16.0 * (2.0 * 32 * 32 * 16) * reps;
      *out_tflops = flop / (double(ms) * 1e-3) / 1e12;
    } catch (...) {
      cleanup();
      throw;
    }
    cleanup();
  });
}

}  // extern "C"
