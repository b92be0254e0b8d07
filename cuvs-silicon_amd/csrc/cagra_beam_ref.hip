// The reference's own CAGRA search route on the GPU, for query-by-query
// parity with it and for its MetalContext::search_cagra interface.
//
//  entry   the per-query entry node (src/cagra.cpp:128-178): the navigation
//          node (the index's seed nodes) minimising |q|^2 - 2 q.v + |v|^2 in
//          fp32, the first on ties.  One wave per query: lanes over the
//          dimension, one butterfly per navigation node for q.v and |v|^2.
//  beam    the reference's beam search (shaders/cagra_kernels.metal:28-199),
//          same state and rules: an unsorted beam of beam_size (distance,
//          node) entries; the seed is entry[q] if < n, else
//          (q * 2654435761) mod n; each iteration expands the first
//          unexpanded entry of smallest distance (marking it -d - 1), the
//          16 teams of the workgroup evaluate its neighbours in fp32, and the
//          lead wave offers them in graph order: an unvisited one replaces
//          the first entry of largest |d| (expanded entries counting -c - 1)
//          when strictly closer; a neighbour is marked visited when first
//          offered.  Output sorted by (|d|, node), padded with UINT32_MAX /
//          +inf.
//
// The lead wave holds the beam in registers (entry i at slot i / 64 of lane
// i % 64), so "first smallest" and "first largest" are wave reductions of
// (value, index) pairs instead of the reference's serial scans.  The visited
// set is a bitmap of the n rows, in LDS up to 2^19 rows, else in a global
// workspace (one slice per query of a launch, cleared by its workgroup).  The
// distances are fp32 sums in a different order than the reference's
// sequential loop, so results are equal to the reference's where every sum
// is exact (integer-valued data, for instance) and otherwise within fp32
// rounding.
#include <algorithm>
#include <cmath>

#include "cvs_internal.hpp"
#include "device_util.hpp"

namespace cvs {
namespace {

constexpr uint32_t kNone = 0xffffffffu;
constexpr uint64_t kEmpty = ~0ull;
constexpr int kRefThreads = 256;           // 4 waves: 16 teams of 16 lanes
constexpr int64_t kLdsBitmapWords = 16384;  // 64 KiB: up to 2^19 rows

#pragma clang fp contract(off)

// Entry node per query (one wave each, four per workgroup).
__global__ __launch_bounds__(256) void cagra_entry_kernel(const float* __restrict__ queries, int64_t q, int64_t d,
                                                          const float* __restrict__ rows, int64_t dpad,
                                                          const uint32_t* __restrict__ nav, int n_nav,
                                                          uint32_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t qi = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (qi >= q) return;
  const float* qv = queries + qi * d;
  float qn = 0.f;
  for (int64_t c = lane; c < d; c += 64) qn += qv[c] * qv[c];
  for (int o = 32; o >= 1; o >>= 1) qn += xor_lanes_f(qn, o);
  float best = INFINITY;
  uint32_t best_n = n_nav > 0 ? nav[0] : 0u;
  for (int i = 0; i < n_nav; ++i) {
    const float* v = rows + int64_t(nav[i]) * dpad;
    float cross = 0.f, vn = 0.f;
    for (int64_t c = lane; c < d; c += 64) {
      cross += qv[c] * v[c];
      vn += v[c] * v[c];
    }
    for (int o = 32; o >= 1; o >>= 1) {
      cross += xor_lanes_f(cross, o);
      vn += xor_lanes_f(vn, o);
    }
    const float dd = (qn - 2.f * cross) + vn;
    if (dd < best) {  // strict: the first minimum wins
      best = dd;
      best_n = nav[i];
    }
  }
  if (lane == 0) out[qi] = best_n;
}

struct BeamArgs {
  const float4* rows;     // n rows of dq float4 (dpad fp32, zero-padded)
  const uint32_t* graph;  // n x g
  const float* queries;   // q x d
  const uint32_t* entry;  // q entry nodes, or null
  uint32_t* out_nbr;      // q x k
  float* out_dist;
  uint32_t* vis_global;   // bitmap slices when not in LDS: [launch query][words]
  int64_t d;
  int64_t q0;             // first query of this launch
  uint32_t n;
  int dq;                 // float4 per padded row
  int g;
  int k;
  int beam;
  uint32_t max_iter;
  int words;              // bitmap words
  int lds_bitmap;         // 1: the bitmap is in LDS
};

// Lexicographic (value, index) reductions across the wave.
__device__ __forceinline__ void wave_min_first(float& v, int& i) {
  for (int o = 32; o >= 1; o >>= 1) {
    const float v2 = xor_lanes_f(v, o);
    const int i2 = int(xor_lanes(uint32_t(i), o));
    if (v2 < v || (v2 == v && i2 < i)) {
      v = v2;
      i = i2;
    }
  }
}
__device__ __forceinline__ void wave_max_first(float& v, int& i) {
  for (int o = 32; o >= 1; o >>= 1) {
    const float v2 = xor_lanes_f(v, o);
    const int i2 = int(xor_lanes(uint32_t(i), o));
    if (v2 > v || (v2 == v && i2 < i)) {
      v = v2;
      i = i2;
    }
  }
}

template <int E>
__global__ __launch_bounds__(kRefThreads) void cagra_beam_ref_kernel(BeamArgs a) {
  extern __shared__ uint32_t s_mem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int team = tid >> 4, tp = tid & 15;
  const int64_t ql = blockIdx.x;  // query of this launch
  const int64_t qi = a.q0 + ql;
  float* s_q = reinterpret_cast<float*>(s_mem);                 // 4 dq floats
  float* s_td = s_q + 4 * a.dq;                                 // g distances
  uint32_t* s_tn = reinterpret_cast<uint32_t*>(s_td + a.g);     // g nodes
  uint32_t* s_ctl = s_tn + a.g;                                 // [0] expanded node
  uint32_t* vis = a.lds_bitmap ? s_ctl + 4 : a.vis_global + ql * int64_t(a.words);

  const float* qg = a.queries + qi * a.d;
  for (int i = tid; i < 4 * a.dq; i += kRefThreads) s_q[i] = i < a.d ? qg[i] : 0.f;
  for (int i = tid; i < a.words; i += kRefThreads) vis[i] = 0u;
  __syncthreads();

  // Squared distance to row `rid` summed over this lane's 16-lane team.
  auto team_dist = [&](uint32_t rid) -> float {
    const float4* row = a.rows + int64_t(rid) * a.dq;
    const float4* qq = reinterpret_cast<const float4*>(s_q);
    float acc = 0.f;
    for (int c = tp; c < a.dq; c += 16) {
      const float4 x = row[c], y = qq[c];
      const float dx = y.x - x.x, dy = y.y - x.y, dz = y.z - x.z, dw = y.w - x.w;
      acc += (dx * dx + dy * dy) + (dz * dz + dw * dw);
    }
    acc += xor_lanes_f(acc, 8);
    acc += xor_lanes_f(acc, 4);
    acc += xor_lanes_f(acc, 2);
    acc += xor_lanes_f(acc, 1);
    return acc;
  };

  // The beam (lead wave): entry i = 64 e + lane.
  float cd[E];
  uint32_t cn[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    cd[e] = INFINITY;
    cn[e] = kNone;
  }
  if (wave == 0) {
    const uint32_t e0 = a.entry ? a.entry[qi] : kNone;
    const uint32_t seed = e0 < a.n ? e0 : (uint32_t(qi) * 2654435761u) % a.n;
    const float ds = team_dist(seed);  // every team of the wave computes it
    if (lane == 0) {
      cd[0] = ds;
      cn[0] = seed;
      vis[seed >> 5] |= 1u << (seed & 31u);
    }
  }
  __syncthreads();

  for (uint32_t it = 0; it < a.max_iter; ++it) {
    // Expand the first unexpanded entry of smallest distance.
    if (wave == 0) {
      float bv = INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int i = 64 * e + lane;
        if (i < a.beam && cd[e] >= 0.f && cd[e] < bv) {
          bv = cd[e];
          bi = i;
        }
      }
      wave_min_first(bv, bi);
      uint32_t bn = kNone;
      if (bi != 0x7fffffff) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if (64 * e + lane == bi) {
            bn = cn[e];
            cd[e] = -cd[e] - 1.f;
          }
        }
        bn = uint32_t(__builtin_amdgcn_readlane(int(bn), bi & 63));
      }
      if (lane == 0) s_ctl[0] = bn;
    }
    __syncthreads();
    const uint32_t bn = s_ctl[0];
    if (bn == kNone) break;

    // Neighbour distances, one neighbour per team and round.
    for (int j0 = 0; j0 < a.g; j0 += 16) {
      const int j = j0 + team;
      const uint32_t nb = j < a.g ? a.graph[int64_t(bn) * a.g + j] : kNone;
      const bool ok = nb < a.n;
      const float dd = team_dist(ok ? nb : 0u);
      if (j < a.g && tp == 0) {
        s_td[j] = ok ? dd : INFINITY;
        s_tn[j] = ok ? nb : kNone;
      }
    }
    __syncthreads();

    // Offer them in graph order (lead wave).
    if (wave == 0) {
      for (int j = 0; j < a.g; ++j) {
        const uint32_t nb = s_tn[j];
        if (nb == kNone) continue;
        uint32_t seen = 0;
        if (lane == 0) {
          const uint32_t w = vis[nb >> 5], bit = 1u << (nb & 31u);
          seen = w & bit;
          if (!seen) vis[nb >> 5] = w | bit;
        }
        if (__builtin_amdgcn_readlane(int(seen), 0) != 0) continue;
        const float dist = s_td[j];
        float wv = 0.f;
        int wi = 0x7fffffff;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int i = 64 * e + lane;
          if (i < a.beam) {
            const float ab = cd[e] < 0.f ? (-cd[e] - 1.f) : cd[e];
            if (ab > wv) {
              wv = ab;
              wi = i;
            }
          }
        }
        wave_max_first(wv, wi);
        if (wi != 0x7fffffff && dist < wv) {
#pragma unroll
          for (int e = 0; e < E; ++e) {
            if (64 * e + lane == wi) {
              cd[e] = dist;
              cn[e] = nb;
            }
          }
        }
      }
    }
    __syncthreads();
  }

  // Output: valid entries by (|d|, node), padded.
  if (wave == 0) {
    uint64_t key[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = 64 * e + lane;
      const float ab = cd[e] < 0.f ? (-cd[e] - 1.f) : cd[e];
      key[e] = (i < a.beam && cn[e] != kNone) ? (uint64_t(ord_f32(ab)) << 32) | cn[e] : kEmpty;
    }
    wave_sort_e<E>(key);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int pos = 64 * e + lane;
      if (pos < a.k) {
        a.out_nbr[qi * a.k + pos] = key[e] == kEmpty ? kNone : uint32_t(key[e]);
        a.out_dist[qi * a.k + pos] = key[e] == kEmpty ? INFINITY : unord_f32(uint32_t(key[e] >> 32));
      }
    }
    for (int pos = 64 * E + lane; pos < a.k; pos += 64) {
      a.out_nbr[qi * a.k + pos] = kNone;
      a.out_dist[qi * a.k + pos] = INFINITY;
    }
  }
}

void check_index(cvs_context* ctx, const cvs_cagra_index* idx, const void* queries, int64_t q) {
  if (!idx || idx->ctx != ctx) fail(CVS_ERR_INVALID_ARGUMENT, "index does not belong to context");
  if (!queries) fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
  if (q <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "query count must be positive");
  if (q > int64_t(INT32_MAX)) fail(CVS_ERR_UNSUPPORTED, "too many queries in one call");
}

void entry_points_device(cvs_context* ctx, const cvs_cagra_index* idx, const float* queries, int64_t q,
                         uint32_t* out) {
  check_index(ctx, idx, queries, q);
  if (!out) fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
  if (idx->n_seeds == 0) fail(CVS_ERR_INVALID_ARGUMENT, "the index has no seed (navigation) nodes");
  hipLaunchKernelGGL(cagra_entry_kernel, dim3(unsigned((q + 3) / 4)), dim3(256), 0, ctx->stream, queries, q, idx->d,
                     static_cast<const float*>(idx->rows), idx->dpad, static_cast<const uint32_t*>(idx->seeds),
                     int(idx->n_seeds), out);
  after_launch("cagra_entry_kernel");
}

void beam_ref_device(cvs_context* ctx, const cvs_cagra_index* idx, const float* queries, int64_t q, int64_t k,
                     uint32_t beam, uint32_t max_iter, const uint32_t* entry, uint32_t* nbr, float* dist) {
  check_index(ctx, idx, queries, q);
  if (!nbr || !dist) fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
  if (k <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "k must be positive");
  if (beam == 0 || beam > CVS_CAGRA_MAX_ITOPK) fail(CVS_ERR_UNSUPPORTED, "beam_size must be in [1, CVS_CAGRA_MAX_ITOPK]");
  const int E = beam <= 64 ? 1 : beam <= 128 ? 2 : beam <= 256 ? 4 : 8;
  BeamArgs a{};
  a.rows = reinterpret_cast<const float4*>(idx->rows);
  a.graph = idx->graph;
  a.queries = queries;
  a.entry = entry;
  a.out_nbr = nbr;
  a.out_dist = dist;
  a.d = idx->d;
  a.n = uint32_t(idx->n);
  a.dq = int(idx->dpad / 4);
  a.g = int(idx->degree);
  a.k = int(k);
  a.beam = int(beam);
  a.max_iter = max_iter;
  a.words = int((idx->n + 31) / 32);
  a.lds_bitmap = a.words <= kLdsBitmapWords ? 1 : 0;
  const size_t lds = (size_t(idx->dpad) + 2 * size_t(idx->degree) + 4 + (a.lds_bitmap ? size_t(a.words) : 0)) * 4;
  // Queries per launch: all of them with an LDS bitmap; with a global one,
  // as many as keep the bitmap slices within 512 MiB.
  int64_t per = q;
  if (!a.lds_bitmap) {
    per = std::max<int64_t>(1, (int64_t(512) << 20) / (int64_t(a.words) * 4));
    ctx->ws_teams.reserve(size_t(std::min(per, q)) * size_t(a.words) * 4);
    a.vis_global = ctx->ws_teams.as<uint32_t>();
  }
  auto launch = [&](auto kern) {
    if (lds > 64 * 1024) CVS_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    const TimerSpan t0 = timer_span(ctx, "cagra_search");
    for (int64_t q0 = 0; q0 < q; q0 += per) {
      a.q0 = q0;
      hipExtLaunchKernelGGL(kern, dim3(unsigned(std::min(per, q - q0))), dim3(kRefThreads), lds, ctx->stream,
                            q0 == 0 ? t0.start : nullptr, q0 + per >= q ? t0.stop : nullptr, 0, a);
      after_launch("cagra_beam_ref_kernel");
    }
  };
  switch (E) {
    case 1: launch(cagra_beam_ref_kernel<1>); break;
    case 2: launch(cagra_beam_ref_kernel<2>); break;
    case 4: launch(cagra_beam_ref_kernel<4>); break;
    default: launch(cagra_beam_ref_kernel<8>); break;
  }
}

}  // namespace
}  // namespace cvs

using namespace cvs;

extern "C" {

int cvs_cagra_entry_points_async(cvs_context* ctx, const cvs_cagra_index* index, const float* queries_dev,
                                 int64_t q, uint32_t* out_entry_dev) {
  return guarded([&] {
    bind(ctx);
    entry_points_device(ctx, index, queries_dev, q, out_entry_dev);
  });
}

int cvs_cagra_entry_points(cvs_context* ctx, const cvs_cagra_index* index, const float* queries, int64_t q,
                           uint32_t* out_entry) {
  return guarded([&] {
    bind(ctx);
    check_index(ctx, index, queries, q);
    if (!out_entry) fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
    const size_t qbytes = size_t(q) * size_t(index->d) * sizeof(float);
    ctx->ws_io.reserve(qbytes + size_t(q) * 4 + 256);
    char* base = ctx->ws_io.as<char>();
    float* dq = reinterpret_cast<float*>(base);
    uint32_t* de = reinterpret_cast<uint32_t*>(base + (qbytes + 127) / 128 * 128);
    CVS_HIP(hipMemcpyAsync(dq, queries, qbytes, hipMemcpyHostToDevice, ctx->stream));
    entry_points_device(ctx, index, dq, q, de);
    CVS_HIP(hipMemcpyAsync(out_entry, de, size_t(q) * 4, hipMemcpyDeviceToHost, ctx->stream));
    CVS_HIP(hipStreamSynchronize(ctx->stream));
  });
}

int cvs_cagra_search_reference_async(cvs_context* ctx, const cvs_cagra_index* index, const float* queries_dev,
                                     int64_t q, int64_t k, uint32_t beam_size, uint32_t max_iter,
                                     const uint32_t* entry_nodes_dev, uint32_t* out_neighbors_dev,
                                     float* out_distances_dev) {
  return guarded([&] {
    bind(ctx);
    beam_ref_device(ctx, index, queries_dev, q, k, beam_size, max_iter, entry_nodes_dev, out_neighbors_dev,
                    out_distances_dev);
  });
}

int cvs_cagra_search_reference(cvs_context* ctx, const cvs_cagra_index* index, const float* queries, int64_t q,
                               int64_t k, uint32_t beam_size, uint32_t max_iter, const uint32_t* entry_nodes,
                               uint32_t* out_neighbors, float* out_distances) {
  return guarded([&] {
    bind(ctx);
    check_index(ctx, index, queries, q);
    if (!out_neighbors || !out_distances) fail(CVS_ERR_INVALID_ARGUMENT, "null buffer");
    if (k <= 0) fail(CVS_ERR_INVALID_ARGUMENT, "k must be positive");
    const size_t qbytes = size_t(q) * size_t(index->d) * sizeof(float);
    const size_t obytes = size_t(q) * size_t(k) * sizeof(float);
    const size_t ebytes = size_t(q) * 4;
    auto up = [](size_t b) { return (b + 127) / 128 * 128; };
    ctx->ws_io.reserve(up(qbytes) + 2 * up(obytes) + up(ebytes) + 256);
    char* base = ctx->ws_io.as<char>();
    float* dq = reinterpret_cast<float*>(base);
    uint32_t* dn = reinterpret_cast<uint32_t*>(base + up(qbytes));
    float* dd = reinterpret_cast<float*>(reinterpret_cast<char*>(dn) + up(obytes));
    uint32_t* de = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(dd) + up(obytes));
    CVS_HIP(hipMemcpyAsync(dq, queries, qbytes, hipMemcpyHostToDevice, ctx->stream));
    if (entry_nodes) CVS_HIP(hipMemcpyAsync(de, entry_nodes, ebytes, hipMemcpyHostToDevice, ctx->stream));
    beam_ref_device(ctx, index, dq, q, k, beam_size, max_iter, entry_nodes ? de : nullptr, dn, dd);
    CVS_HIP(hipMemcpyAsync(out_neighbors, dn, obytes, hipMemcpyDeviceToHost, ctx->stream));
    CVS_HIP(hipMemcpyAsync(out_distances, dd, obytes, hipMemcpyDeviceToHost, ctx->stream));
    CVS_HIP(hipStreamSynchronize(ctx->stream));
  });
}

}  // extern "C"
