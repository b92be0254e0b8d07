/*
 * CPU restatement of the reference's CAGRA search path (TEST INFRASTRUCTURE
 * ONLY; see oracle.h).  Compiled with -ffp-contract=off: every fp32 product
 * and sum rounds separately.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define INVALID_ID 0xffffffffu

int64_t oracle_cagra_nav_nodes(int64_t n, uint32_t* out_ids) {
  /* src/cagra.cpp:65-72: n_nav = min(200, (int64)sqrt(N)), nav[i] = (u32)(i * (N / n_nav)) */
  int64_t n_nav = (int64_t)sqrt((double)n);
  if (n_nav > 200) n_nav = 200;
  if (out_ids) {
    const double step = (double)n / (double)n_nav;
    for (int64_t i = 0; i < n_nav; ++i) out_ids[i] = (uint32_t)((double)i * step);
  }
  return n_nav;
}

void oracle_cagra_entry_points(const float* queries, int64_t q, int64_t d, const uint32_t* nav_ids,
                               const float* nav_vectors, int64_t n_nav, uint32_t* out_entry) {
  /* src/cagra.cpp:133-177.  The reference forms the cross terms with
   * cblas_sgemm (accumulation order unspecified); here they are sequential
   * fp32 dot products. */
  float* nn = (float*)malloc(sizeof(float) * (size_t)(n_nav > 0 ? n_nav : 1));
  for (int64_t i = 0; i < n_nav; ++i) {
    float s = 0.f;
    const float* v = nav_vectors + i * d;
    for (int64_t j = 0; j < d; ++j) s += v[j] * v[j];
    nn[i] = s;
  }
  for (int64_t qi = 0; qi < q; ++qi) {
    const float* qv = queries + qi * d;
    float qn = 0.f;
    for (int64_t j = 0; j < d; ++j) qn += qv[j] * qv[j];
    float best_d = INFINITY;
    uint32_t best_n = n_nav > 0 ? nav_ids[0] : 0u;
    for (int64_t i = 0; i < n_nav; ++i) {
      const float* v = nav_vectors + i * d;
      float cross = 0.f;
      for (int64_t j = 0; j < d; ++j) cross += qv[j] * v[j];
      const float dd = qn - 2.f * cross + nn[i];
      if (dd < best_d) { /* strict: the first minimum wins */
        best_d = dd;
        best_n = nav_ids[i];
      }
    }
    out_entry[qi] = best_n;
  }
  free(nn);
}

void oracle_cagra_search_policy(uint64_t itopk_size, uint64_t max_iterations, int64_t q,
                                uint32_t* out_beam, uint32_t* out_iters) {
  /* src/cagra.cpp:182-189 */
  uint32_t beam = (uint32_t)(itopk_size > 0 ? itopk_size : 128);
  uint32_t iters = (uint32_t)(max_iterations > 0 ? max_iterations : 200);
  if (q <= 4) {
    if (beam > 32) beam = 32;
    if (iters > 200) iters = 200;
  }
  *out_beam = beam;
  *out_iters = iters;
}

static float l2_seq(const float* a, const float* b, int64_t d) {
  float acc = 0.f;
  for (int64_t i = 0; i < d; ++i) {
    const float t = a[i] - b[i];
    acc += t * t;
  }
  return acc;
}

void oracle_cagra_search(const float* base, int64_t n, int64_t d, const uint32_t* graph,
                         uint32_t g, const float* queries, int64_t q, const uint32_t* entry,
                         int64_t k, uint32_t beam, uint32_t max_iter, uint32_t* out_nbr,
                         float* out_dist, int threads) {
  /* shaders/cagra_kernels.metal:28-199, one query at a time.  Phase 1 of an
   * iteration writes distinct slots and phase 2 runs on one thread, so the
   * kernel is deterministic and this serial order reproduces it. */
  const int64_t vw = (n + 31) / 32;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
  for (int64_t qi = 0; qi < q; ++qi) {
    const float* qv = queries + qi * d;
    float* cd = (float*)malloc(sizeof(float) * (beam > 0 ? beam : 1));
    uint32_t* cn = (uint32_t*)malloc(sizeof(uint32_t) * (beam > 0 ? beam : 1));
    uint32_t* visited = (uint32_t*)calloc((size_t)vw, sizeof(uint32_t));
    float* tg_dist = (float*)malloc(sizeof(float) * (g > 0 ? g : 1));
    uint32_t* tg_node = (uint32_t*)malloc(sizeof(uint32_t) * (g > 0 ? g : 1));
    float* sd = (float*)malloc(sizeof(float) * (beam > 0 ? beam : 1));
    uint32_t* si = (uint32_t*)malloc(sizeof(uint32_t) * (beam > 0 ? beam : 1));

    /* :62-80 seed */
    const uint32_t e = entry ? entry[qi] : INVALID_ID;
    const uint32_t seed = (e < (uint32_t)n) ? e : (uint32_t)(((uint32_t)qi * 2654435761u) % (uint32_t)n);
    if (beam > 0) {
      cd[0] = l2_seq(qv, base + (int64_t)seed * d, d);
      cn[0] = seed;
      for (uint32_t i = 1; i < beam; ++i) {
        cd[i] = INFINITY;
        cn[i] = INVALID_ID;
      }
    }
    visited[seed >> 5] |= 1u << (seed & 31u);

    for (uint32_t iter = 0; iter < max_iter && beam > 0; ++iter) {
      /* :86-107 best unexpanded (d >= 0), mark expanded as -d - 1 */
      float bd = INFINITY;
      uint32_t bn = INVALID_ID;
      for (uint32_t i = 0; i < beam; ++i) {
        const float c = cd[i];
        if (c >= 0.f && c < bd) {
          bd = c;
          bn = cn[i];
        }
      }
      if (bn != INVALID_ID) {
        for (uint32_t i = 0; i < beam; ++i) {
          if (cn[i] == bn) {
            cd[i] = -cd[i] - 1.f;
            break;
          }
        }
      }
      if (bn == INVALID_ID) break; /* :110 */
      /* :117-132 neighbour distances */
      for (uint32_t j = 0; j < g; ++j) {
        const uint32_t nb = graph[(int64_t)bn * g + j];
        if (nb < (uint32_t)n) {
          tg_dist[j] = l2_seq(qv, base + (int64_t)nb * d, d);
          tg_node[j] = nb;
        } else {
          tg_dist[j] = INFINITY;
          tg_node[j] = INVALID_ID;
        }
      }
      /* :137-159 visited check, replace the first entry of largest |d| */
      for (uint32_t j = 0; j < g; ++j) {
        const uint32_t nb = tg_node[j];
        if (nb == INVALID_ID) continue;
        const uint32_t bit = 1u << (nb & 31u);
        if (visited[nb >> 5] & bit) continue;
        visited[nb >> 5] |= bit;
        const float dist = tg_dist[j];
        float worst = 0.f;
        uint32_t widx = beam;
        for (uint32_t i = 0; i < beam; ++i) {
          const float c = cd[i];
          const float a = c < 0.f ? (-c - 1.f) : c;
          if (a > worst) {
            worst = a;
            widx = i;
          }
        }
        if (widx < beam && dist < worst) {
          cd[widx] = dist;
          cn[widx] = nb;
        }
      }
    }

    /* :164-198 collect, insertion sort by (d, node), pad */
    uint32_t nv = 0;
    for (uint32_t i = 0; i < beam; ++i) {
      if (cn[i] == INVALID_ID) continue;
      const float c = cd[i];
      sd[nv] = c < 0.f ? (-c - 1.f) : c;
      si[nv] = cn[i];
      ++nv;
    }
    for (uint32_t i = 1; i < nv; ++i) {
      const float kd = sd[i];
      const uint32_t kn = si[i];
      int64_t j = (int64_t)i - 1;
      while (j >= 0 && (sd[j] > kd || (sd[j] == kd && si[j] > kn))) {
        sd[j + 1] = sd[j];
        si[j + 1] = si[j];
        --j;
      }
      sd[j + 1] = kd;
      si[j + 1] = kn;
    }
    for (int64_t j = 0; j < k; ++j) {
      out_nbr[qi * k + j] = j < (int64_t)nv ? si[j] : INVALID_ID;
      out_dist[qi * k + j] = j < (int64_t)nv ? sd[j] : INFINITY;
    }
    free(cd);
    free(cn);
    free(visited);
    free(tg_dist);
    free(tg_node);
    free(sd);
    free(si);
  }
}

void oracle_knn_graph(const float* base, int64_t n, int64_t d, uint32_t g, uint32_t* out_graph,
                      int threads) {
  /* Exact degree-g kNN graph without self edges, rows sorted by (d, id);
   * missing entries UINT32_MAX.  For N <= 50,000 the reference's build is
   * exact all-pairs seeding (src/metal_context.mm:324-349) followed by
   * nn-descent, which cannot improve an exact graph beyond rounding. */
  const int64_t take = (int64_t)g < n - 1 ? (int64_t)g : n - 1;
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads > 0 ? threads : 1)
  for (int64_t i = 0; i < n; ++i) {
    float* bd = (float*)malloc(sizeof(float) * (size_t)(take > 0 ? take : 1));
    uint32_t* bi = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(take > 0 ? take : 1));
    int64_t m = 0;
    for (int64_t r = 0; r < n && take > 0; ++r) {
      if (r == i) continue;
      const float dist = l2_seq(base + i * d, base + r * d, d);
      /* insertion into a sorted list of the `take` best by (d, id) */
      if (m == take && !(dist < bd[m - 1] || (dist == bd[m - 1] && (uint32_t)r < bi[m - 1]))) continue;
      int64_t p = m < take ? m : take - 1;
      if (m < take) ++m;
      while (p > 0 && (dist < bd[p - 1] || (dist == bd[p - 1] && (uint32_t)r < bi[p - 1]))) {
        bd[p] = bd[p - 1];
        bi[p] = bi[p - 1];
        --p;
      }
      bd[p] = dist;
      bi[p] = (uint32_t)r;
    }
    for (int64_t j = 0; j < (int64_t)g; ++j) out_graph[i * g + j] = j < m ? bi[j] : INVALID_ID;
    free(bd);
    free(bi);
  }
}

/* recompute_graph_distances (reference shaders/cagra_kernels.metal:658-681):
 * per edge, the squared L2 distance of the node's row to its neighbour's,
 * accumulated over float4 groups (dist += dot(delta, delta), the four
 * products summed left to right) over the first 4*floor(d/4) columns only, as
 * the reference's D >> 2 loop does; UINT32_MAX entries get +inf.  Ids >= n
 * (out of range for the reference, which would read past the dataset) also
 * get +inf here. */
void oracle_edge_distances(const float* rows, int64_t n, int64_t d, const uint32_t* graph, uint32_t g,
                           float* out, int threads) {
  const int64_t d4 = d / 4;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (int64_t i = 0; i < n; ++i) {
    const float* a = rows + i * d;
    for (uint32_t e = 0; e < g; ++e) {
      const uint32_t nb = graph[i * (int64_t)g + e];
      if (nb == INVALID_ID || (int64_t)nb >= n) {
        out[i * (int64_t)g + e] = INFINITY;
        continue;
      }
      const float* b = rows + (int64_t)nb * d;
      float dist = 0.f;
      for (int64_t c = 0; c < d4; ++c) {
        const float dx = a[4 * c] - b[4 * c], dy = a[4 * c + 1] - b[4 * c + 1];
        const float dz = a[4 * c + 2] - b[4 * c + 2], dw = a[4 * c + 3] - b[4 * c + 3];
        const float dot = ((dx * dx + dy * dy) + dz * dz) + dw * dw;
        dist += dot;
      }
      out[i * (int64_t)g + e] = dist;
    }
  }
}
