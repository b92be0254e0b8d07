/*
 * CPU restatement of the reference's CAGRA graph build (TEST INFRASTRUCTURE
 * ONLY; see oracle.h): cagra::build (src/cagra.cpp:47-59) ->
 * MetalContext::build_knn_graph (src/metal_context.mm:289-914), all three
 * size classes (exact seeding, IVF seeding with exact distances, IVF seeding
 * with product-quantisation distances).  Compiled with -ffp-contract=off.
 *
 * Where the reference's arithmetic order is unspecified (cblas_sgemm cross
 * products, Metal's float4 dot), a fixed order is chosen and stated.  The
 * reference's nn-descent kernel runs one threadgroup per node concurrently
 * and races on the lists (src/metal_context.mm:870-871); this restatement
 * runs the schedule in which each node's reads of other nodes' lists see the
 * lists as they were at the start of the iteration, which makes it
 * deterministic under any thread count.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define INVALID_ID 0xffffffffu

/* ORACLE_PLANT selects one deliberate mistake for the pinning tests, which
 * build such variants of this file into temporary libraries and check that
 * their known answers reject them (tests/test_oracle_build.py,
 * tests/test_oracle_build_stages.py).  0, the default, is the restatement
 * itself. */
#ifndef ORACLE_PLANT
#define ORACLE_PLANT 0
#endif

/* Cross product in place of cblas_sgemm: eight interleaved fp32 partial sums
 * combined pairwise (the BLAS order is unspecified). */
static float dot_blk(const float* a, const float* b, int64_t d) {
  float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t i = 0;
  for (; i + 8 <= d; i += 8)
    for (int j = 0; j < 8; ++j) s[j] += a[i + j] * b[i + j];
  for (; i < d; ++i) s[i & 7] += a[i] * b[i];
  return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

/* Metal kernels' distance (shaders/cagra_kernels.metal:369-375, :435-440):
 * dist += dot(delta4, delta4) over D/4 float4 steps (a remainder of D % 4
 * columns is ignored, as there); dot taken left to right. */
static float l2_f4(const float* a, const float* b, int64_t d) {
  float dist = 0.f;
  for (int64_t i = 0; i + 4 <= d; i += 4) {
    const float x = a[i] - b[i], y = a[i + 1] - b[i + 1];
    const float z = a[i + 2] - b[i + 2], w = a[i + 3] - b[i + 3];
    dist += ((x * x + y * y) + z * z) + w * w;
  }
  return dist;
}

/* Four independent l2_f4 distances (same values, interleaved for speed). */
static void l2_f4_x4(const float* a, const float* const* b, int64_t d, float* out) {
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  for (int64_t i = 0; i + 4 <= d; i += 4) {
    float t[4];
    for (int c = 0; c < 4; ++c) {
      const float* bc = b[c];
      const float x = a[i] - bc[i], y = a[i + 1] - bc[i + 1];
      const float z = a[i + 2] - bc[i + 2], w = a[i + 3] - bc[i + 3];
      t[c] = ((x * x + y * y) + z * z) + w * w;
    }
    s0 += t[0];
    s1 += t[1];
    s2 += t[2];
    s3 += t[3];
  }
  out[0] = s0;
  out[1] = s1;
  out[2] = s2;
  out[3] = s3;
}

static float sq_norm(const float* v, int64_t d) {
  float s = 0.f;
  for (int64_t i = 0; i < d; ++i) s += v[i] * v[i];
  return s;
}

/* insert_neighbor (src/metal_context.mm:315-322): replace the first slot of
 * largest distance if closer; no duplicate check. */
static void insert_neighbor(uint32_t* graph, float* gdist, uint32_t g, int64_t vi, uint32_t nbr, float dist) {
  const int64_t row = vi * g;
  float worst = gdist[row];
  uint32_t wg = 0;
  for (uint32_t j = 1; j < g; ++j)
    if (gdist[row + j] > worst) {
      worst = gdist[row + j];
      wg = j;
    }
  if (dist < worst) {
    graph[row + wg] = nbr;
    gdist[row + wg] = dist;
  }
}

/* Selection of the `take` smallest of idx[0..m) by key[idx] (ties by
 * position, where std::partial_sort's tie order is unspecified), sorted. */
static void select_smallest(uint32_t* idx, int64_t m, int64_t take, const float* key) {
  for (int64_t t = 0; t < take && t < m; ++t) {
    int64_t best = t;
    for (int64_t j = t + 1; j < m; ++j)
      if (key[idx[j]] < key[idx[best]]) best = j;
    const uint32_t tmp = idx[t];
    idx[t] = idx[best];
    idx[best] = tmp;
  }
}

/* Product quantisation of the rows (src/metal_context.mm:437-568): for each
 * of 8 subspaces of 128 dimensions, k-means with 256 centres from evenly
 * strided rows, at most 10 iterations (stop when no row changes centre),
 * then one more assignment pass as the codes; and the symmetric table
 * lut[m][a][b] = sum over the subspace of (c_a - c_b)^2 in dimension order
 * (:552-566). */
void oracle_pq_train(const float* data, int64_t n, int64_t d, int nt, uint8_t* codes, float* lut) {
  enum { M = 8, DS = 128, KC = 256 };
  float* ctr = (float*)malloc(sizeof(float) * KC * DS);
  float* cn = (float*)malloc(sizeof(float) * KC);
  float* vn = (float*)malloc(sizeof(float) * (size_t)n);
  int32_t* asg = (int32_t*)calloc((size_t)n, sizeof(int32_t));
  int64_t* counts = (int64_t*)malloc(sizeof(int64_t) * KC);
  for (int m = 0; m < M; ++m) {
    const int64_t off = (int64_t)m * DS;
    const double stride = (double)n / KC;
    for (int c = 0; c < KC; ++c) {
      int64_t ix = (int64_t)((double)c * stride + stride * 0.5);
      if (ix > n - 1) ix = n - 1;
      memcpy(ctr + c * DS, data + ix * d + off, sizeof(float) * DS);
    }
    for (int64_t i = 0; i < n; ++i) vn[i] = sq_norm(data + i * d + off, DS);
    for (int iter = 0; iter <= 10; ++iter) {
      /* iterations 0..9 are Lloyd steps; pass 10 (or the pass after the
       * loop stopped) is the encoding E-step with the final centres */
      for (int c = 0; c < KC; ++c) cn[c] = sq_norm(ctr + c * DS, DS);
      int changed = iter == 0;
#pragma omp parallel for schedule(static) num_threads(nt) reduction(| : changed)
      for (int64_t i = 0; i < n; ++i) {
        float best = INFINITY;
        int32_t bc = 0;
        for (int c = 0; c < KC; ++c) {
          const float dd = vn[i] - 2.f * dot_blk(data + i * d + off, ctr + c * DS, DS) + cn[c];
          if (dd < best) {
            best = dd;
            bc = c;
          }
        }
        if (asg[i] != bc) {
          changed = 1;
          asg[i] = bc;
        }
        codes[i * M + m] = (uint8_t)bc;
      }
      if (iter == 10 || !changed) break;
      memset(ctr, 0, sizeof(float) * KC * DS);
      memset(counts, 0, sizeof(int64_t) * KC);
      for (int64_t i = 0; i < n; ++i) {
        counts[asg[i]]++;
        float* c = ctr + asg[i] * DS;
        const float* x = data + i * d + off;
        for (int j = 0; j < DS; ++j) c[j] += x[j];
      }
      for (int c = 0; c < KC; ++c)
        if (counts[c] > 0) {
          const float inv = 1.0f / (float)counts[c];
          for (int j = 0; j < DS; ++j) ctr[c * DS + j] *= inv;
        }
    }
    for (int a = 0; a < KC; ++a)
      for (int b = a; b < KC; ++b) {
        float s2 = 0.f;
        for (int j = 0; j < DS; ++j) {
          const float df = ctr[a * DS + j] - ctr[b * DS + j];
          s2 += df * df;
        }
        lut[((int64_t)m * KC + a) * KC + b] = s2;
        lut[((int64_t)m * KC + b) * KC + a] = s2;
      }
  }
  free(ctr);
  free(cn);
  free(vn);
  free(asg);
  free(counts);
}

/* Initial k-means centres (src/metal_context.mm:366-375): centre k is row
 * min(floor(k * s + s / 2), n - 1) with s = n / K in double. */
void oracle_kmeans_init(const float* data, int64_t n, int64_t d, int64_t K, float* centres) {
  const double stride = (double)n / (double)K;
  for (int64_t k = 0; k < K; ++k) {
    int64_t ix = (int64_t)((double)k * stride + (ORACLE_PLANT == 4 ? 0.0 : stride * 0.5));
    if (ix > n - 1) ix = n - 1;
    memcpy(centres + k * d, data + ix * d, sizeof(float) * (size_t)d);
  }
}

/* Lloyd iterations of the IVF k-means (src/metal_context.mm:381-435), from
 * the centres given: each E-step assigns every row to the centre of least
 * |x|^2 - 2 x.c + |c|^2 (first minimum wins; assignments start at 0, and
 * the first E-step counts as a change); when no row changes centre the loop
 * stops, otherwise the M-step sums each centre's rows in row order and
 * scales by 1 / count, and a centre with no rows becomes the zero vector.
 * Returns the number of E-steps run (at most max_iter). */
int oracle_ivf_kmeans(const float* data, int64_t n, int64_t d, int64_t K, int max_iter, float* cent,
                      uint32_t* assign, int threads) {
  const int nt = threads > 0 ? threads : 1;
  float* norms = (float*)malloc(sizeof(float) * (size_t)n);
  float* cn = (float*)malloc(sizeof(float) * (size_t)K);
  int64_t* counts = (int64_t*)malloc(sizeof(int64_t) * (size_t)K);
  for (int64_t i = 0; i < n; ++i) {
    norms[i] = sq_norm(data + i * d, d);
    assign[i] = 0;
  }
  int iters = 0;
  for (int iter = 0; iter < max_iter; ++iter) {
    ++iters;
    for (int64_t k = 0; k < K; ++k) cn[k] = sq_norm(cent + k * d, d);
    int changed = iter == 0;
#pragma omp parallel for schedule(static) num_threads(nt) reduction(| : changed)
    for (int64_t i = 0; i < n; ++i) {
      const float ni = norms[i];
      float best_d = INFINITY;
      uint32_t best_k = 0;
      for (int64_t k = 0; k < K; ++k) {
        const float dd = ni - 2.f * dot_blk(data + i * d, cent + k * d, d) + cn[k];
        if (ORACLE_PLANT == 1 ? dd <= best_d : dd < best_d) {
          best_d = dd;
          best_k = (uint32_t)k;
        }
      }
      if (assign[i] != best_k) {
        changed = 1;
        assign[i] = best_k;
      }
    }
    if (!changed) break;
    memset(counts, 0, sizeof(int64_t) * (size_t)K);
    for (int64_t i = 0; i < n; ++i) counts[assign[i]]++;
    for (int64_t k = 0; k < K; ++k)
      if (ORACLE_PLANT != 2 || counts[k] > 0) memset(cent + k * d, 0, sizeof(float) * (size_t)d);
    for (int64_t i = 0; i < n; ++i) {
      float* c = cent + (int64_t)assign[i] * d;
      const float* x = data + i * d;
      for (int64_t j = 0; j < d; ++j) c[j] += x[j];
    }
    for (int64_t k = 0; k < K; ++k)
      if (counts[k] > 0) {
        const float inv = 1.0f / (float)(counts[k] + (ORACLE_PLANT == 3 ? 1 : 0));
        for (int64_t j = 0; j < d; ++j) cent[k * d + j] *= inv;
      }
  }
  free(norms);
  free(cn);
  free(counts);
  return iters;
}

/* The n_probe nearest other centres of every centre (src/metal_context.mm:
 * 583-611), by |c_k|^2 - 2 c_k.c_a + |c_a|^2, nearest first; the candidate
 * order is 0..K-2 with centre k's own slot holding K-1, and a tie keeps the
 * earlier candidate.  Writes K x n_probe ids. */
void oracle_ivf_near_clusters(const float* cent, int64_t K, int64_t d, int64_t n_probe, uint32_t* nearc,
                              int threads) {
  const int nt = threads > 0 ? threads : 1;
  float* cn = (float*)malloc(sizeof(float) * (size_t)K);
  for (int64_t k = 0; k < K; ++k) cn[k] = sq_norm(cent + k * d, d);
#pragma omp parallel num_threads(nt)
  {
    float* key = (float*)malloc(sizeof(float) * (size_t)K);
    uint32_t* kidx = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t k = 0; k < K; ++k) {
      for (int64_t a = 0; a < K; ++a) key[a] = cn[k] - 2.f * dot_blk(cent + k * d, cent + a * d, d) + cn[a];
      for (int64_t a = 0; a < K; ++a) kidx[a] = (uint32_t)a;
      if (ORACLE_PLANT != 5) kidx[k] = kidx[K - 1];
      select_smallest(kidx, K - 1, n_probe, key);
      for (int64_t t = 0; t < n_probe; ++t) nearc[k * n_probe + t] = kidx[t];
    }
    free(key);
    free(kidx);
  }
  free(cn);
}

/* Per-cluster seeding (src/metal_context.mm:576-582, :614-681, :712-792).
 * For each cluster k with members (in row order): candidates = its first
 * min(count, max_own) members, then all members of its n_probe near
 * clusters in order, cut at 8,192.  Each of those first min(count,
 * max_own) members takes the min(g, m - 1) candidates of least key (itself
 * excluded; ties keep the earlier candidate) and inserts them into its row
 * with insert_neighbor (src/metal_context.mm:315-322).  The key is the
 * expanded-form squared distance |x|^2 - 2 x.y + |y|^2, or, when `codes`
 * is given, the product-quantisation table sum over 8 subspaces
 * lut[m][code_m(x)][code_m(y)] (:649-655), after which every entry's
 * distance is replaced by its exact float4 squared L2 (recompute_graph_
 * distances, shaders/cagra_kernels.metal:658-681; ids that are not rows
 * get +inf).  Members past max_own seed nothing. */
void oracle_ivf_seed(const float* data, int64_t n, int64_t d, uint32_t g, const uint32_t* assign, int64_t K,
                     const uint32_t* nearc, int64_t n_probe, int64_t max_own, const uint8_t* codes,
                     const float* lut, uint32_t* graph, float* gdist, int threads) {
  const int nt = threads > 0 ? threads : 1;
  const int pq = codes != NULL && lut != NULL;
  float* norms = (float*)malloc(sizeof(float) * (size_t)n);
  for (int64_t i = 0; i < n; ++i) norms[i] = sq_norm(data + i * d, d);
  int64_t* cstart = (int64_t*)calloc((size_t)K + 1, sizeof(int64_t));
  uint32_t* members = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)n);
  for (int64_t i = 0; i < n; ++i) cstart[assign[i] + 1]++;
  for (int64_t k = 0; k < K; ++k) cstart[k + 1] += cstart[k];
  {
    int64_t* fill = (int64_t*)malloc(sizeof(int64_t) * (size_t)K);
    for (int64_t k = 0; k < K; ++k) fill[k] = cstart[k];
    for (int64_t i = 0; i < n; ++i) members[fill[assign[i]]++] = (uint32_t)i;
    free(fill);
  }
#pragma omp parallel num_threads(nt)
  {
    uint32_t* probe = (uint32_t*)malloc(sizeof(uint32_t) * 8192);
    float* key = (float*)malloc(sizeof(float) * 8192);
    uint32_t* midx = (uint32_t*)malloc(sizeof(uint32_t) * 8192);
#pragma omp for schedule(dynamic, 1)
    for (int64_t k = 0; k < K; ++k) {
      const int64_t own_n = cstart[k + 1] - cstart[k];
      if (own_n == 0) continue;
      const uint32_t* own = members + cstart[k];
      const int64_t nk = (ORACLE_PLANT == 7 || own_n < max_own) ? own_n : max_own;
      int64_t m = 0;
      for (int64_t i = 0; i < nk && m < 8192; ++i) probe[m++] = own[i];
      for (int64_t t = 0; t < (ORACLE_PLANT == 6 && n_probe > 2 ? 2 : n_probe); ++t) {
        const uint32_t c = nearc[k * n_probe + t];
        for (int64_t i = cstart[c]; i < cstart[c + 1] && m < 8192; ++i) probe[m++] = members[i];
      }
      if (m <= 1) continue;
      const int64_t take = (int64_t)g < m - 1 ? (int64_t)g : m - 1;
      for (int64_t i = 0; i < nk; ++i) {
        const uint32_t vi = own[i];
        const float ni = norms[vi];
        for (int64_t p = 0; p < m; ++p) {
          if (probe[p] == vi) {
            key[p] = INFINITY;
          } else if (pq) {
            const uint8_t* ca = codes + (int64_t)vi * 8;
            const uint8_t* cb = codes + (int64_t)probe[p] * 8;
            float s2 = 0.f;
            for (int sm = 0; sm < (ORACLE_PLANT == 8 ? 7 : 8); ++sm) s2 += lut[((int64_t)sm * 256 + ca[sm]) * 256 + cb[sm]];
            key[p] = s2;
          } else {
            key[p] = ni - 2.f * dot_blk(data + (int64_t)vi * d, data + (int64_t)probe[p] * d, d) + norms[probe[p]];
          }
          midx[p] = (uint32_t)p;
        }
        select_smallest(midx, m, take, key);
        for (int64_t t = 0; t < take; ++t) {
          const uint32_t nb = probe[midx[t]];
          if (nb == vi) continue;
          insert_neighbor(graph, gdist, g, vi, nb, key[midx[t]]);
        }
      }
    }
    free(probe);
    free(key);
    free(midx);
  }
  if (pq) {
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < n; ++i)
      for (uint32_t e = 0; e < g; ++e) {
        const uint32_t nb = graph[i * g + e];
        gdist[i * g + e] = nb < (uint32_t)n ? l2_f4(data + i * d, data + (int64_t)nb * d, d) : INFINITY;
      }
  }
  free(norms);
  free(cstart);
  free(members);
}

/* The bucketing permutation (src/metal_context.mm:802-810): identity, then
 * for i = n-1 down to 1, r = r * 6364136223846793005 + 1442695040888963407
 * (mod 2^64, r starting at 0xFEDCBA9876543210) and swap of positions i and
 * (r >> 33) mod (i + 1). */
void oracle_bucketing_perm(int64_t n, uint32_t* perm) {
  for (int64_t i = 0; i < n; ++i) perm[i] = (uint32_t)i;
  uint64_t r = 0xFEDCBA9876543210ULL;
#if ORACLE_PLANT == 13
  for (int64_t i = 1; i < n; ++i) {
#else
  for (int64_t i = n - 1; i > 0; --i) {
#endif
#if ORACLE_PLANT != 14
    r = r * 6364136223846793005ULL + 1442695040888963407ULL;
#endif
    const int64_t j = (int64_t)(r >> (ORACLE_PLANT == 12 ? 32 : 33)) % (i + 1);
    const uint32_t tmp = perm[i];
    perm[i] = perm[j];
    perm[j] = tmp;
#if ORACLE_PLANT == 14
    r = r * 6364136223846793005ULL + 1442695040888963407ULL;
#endif
  }
}

/* One random-bucketing pass (random_bucketing, shaders/cagra_kernels.metal:
 * 403-462): positions [b * bucket, (b + 1) * bucket) of `perm` form bucket b.
 * Each row keeps its take = min(g, 64) nearest bucket mates by float4
 * squared L2 (a mate replaces the first slot of largest distance when
 * strictly closer), then inserts them into its row with insert_neighbor in
 * slot order, unreached slots skipped.  No duplicate check, as there. */
void oracle_bucketing_merge(const float* data, int64_t n, int64_t d, uint32_t g, const uint32_t* perm,
                            int64_t bucket, uint32_t* graph, float* gdist, int threads) {
  const int nt = threads > 0 ? threads : 1;
  const uint32_t take = g < 64 ? g : 64;
#pragma omp parallel for schedule(dynamic, 64) num_threads(nt)
  for (int64_t v = 0; v < n; ++v) {
    const int64_t start = (v / bucket) * bucket;
    const int64_t end = start + bucket < n ? start + bucket : n;
    const int64_t t = v - start;
    const uint32_t vi = perm[v];
    float hd[64];
    uint32_t hn[64];
    for (uint32_t h = 0; h < take; ++h) {
      hd[h] = INFINITY;
      hn[h] = INVALID_ID;
    }
    for (int64_t b = 0; b < end - start; ++b) {
      if (b == t) continue;
      const uint32_t nb = perm[start + b];
      const float dist = l2_f4(data + (int64_t)vi * d, data + (int64_t)nb * d, d);
      float worst = hd[0];
      uint32_t wi = 0;
      for (uint32_t h = 1; h < take; ++h)
        if (hd[h] > worst) {
          worst = hd[h];
          wi = h;
        }
      if (dist < worst) {
        hd[wi] = dist;
        hn[wi] = nb;
      }
    }
    for (uint32_t h = 0; h < take; ++h) {
      if (hn[h] == INVALID_ID) continue;
      if (ORACLE_PLANT == 9) {
        int dup = 0;
        for (uint32_t j = 0; j < g; ++j) dup |= graph[(int64_t)vi * g + j] == hn[h];
        if (dup) continue;
      }
      insert_neighbor(graph, gdist, g, vi, hn[h], hd[h]);
    }
  }
}

/* nn-descent (nn_descent, shaders/cagra_kernels.metal:334-395; host loop
 * src/metal_context.mm:853-911), at most max_iter iterations.  Per node, in
 * slot order of its current row: for each valid neighbour, each entry of
 * that neighbour's row as it was when the iteration began (the schedule
 * chosen for the reference's racy kernel) that is a row id, not the node,
 * and not in the node's current row is a candidate; its float4 squared L2
 * replaces the node's entry of largest distance (first such slot; distances
 * above 0 only) when strictly smaller.  Stops after an iteration that
 * changed no row.  Returns the number of iterations run. */
int oracle_nn_descent(const float* data, int64_t n, int64_t d, uint32_t g, uint32_t* graph, float* gdist,
                      uint32_t max_iter, int threads) {
  const int nt = threads > 0 ? threads : 1;
  uint32_t* snap = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)n * g);
  int iters = 0;
  for (uint32_t iter = 0; iter < max_iter; ++iter) {
    ++iters;
    memcpy(snap, graph, sizeof(uint32_t) * (size_t)n * g);
    int any = 0;
#pragma omp parallel for schedule(dynamic, 32) num_threads(nt) reduction(| : any)
    for (int64_t node = 0; node < n; ++node) {
      uint32_t* row = graph + node * g;
      float* rowd = gdist + node * g;
      const float* xv = data + node * d;
      for (uint32_t gi = 0; gi < g; ++gi) {
        const uint32_t nbr = row[gi];
        if (nbr >= (uint32_t)n) continue;
        const uint32_t* hop = snap + (int64_t)nbr * g;
        for (uint32_t h0 = 0; h0 < g; h0 += 4) {
          /* distances of up to four candidates, then the serial checks */
          const float* bp[4];
          uint32_t cand[4];
          for (int c = 0; c < 4; ++c) {
            const uint32_t h = h0 + (uint32_t)c;
            cand[c] = h < g ? hop[h] : INVALID_ID;
            bp[c] = data + (cand[c] < (uint32_t)n ? (int64_t)cand[c] : 0) * d;
          }
          float dist4[4];
          l2_f4_x4(xv, bp, d, dist4);
          for (int c = 0; c < 4; ++c) {
            const uint32_t cd = cand[c];
            if (cd >= (uint32_t)n || cd == (uint32_t)node) continue;
            int present = 0;
            for (uint32_t i = 0; i < g; ++i)
              if (row[i] == cd) {
                present = 1;
                break;
              }
            if (present) continue;
            float worst_d = 0.f;
            uint32_t worst_g = g;
            for (uint32_t i = 0; i < g; ++i)
              if (rowd[i] > worst_d) {
                worst_d = rowd[i];
                worst_g = i;
              }
            if (ORACLE_PLANT == 10 && worst_g < g) worst_g = 0;
            if (worst_g < g && dist4[c] < worst_d) {
              row[worst_g] = cd;
              rowd[worst_g] = dist4[c];
              any = 1;
            }
          }
        }
      }
    }
    if (!any) {
      if (ORACLE_PLANT == 11) --iters;
      break;
    }
  }
  free(snap);
  return iters;
}

int oracle_cagra_build_ref(const float* data, int64_t n, int64_t d, uint32_t graph_degree,
                           uint32_t* out_graph, int threads) {
  return oracle_cagra_build_ref_ex(data, n, d, graph_degree, out_graph, threads, 50000, 200000);
}

int oracle_cagra_build_ref_ex(const float* data, int64_t n, int64_t d, uint32_t graph_degree,
                              uint32_t* out_graph, int threads, int64_t exact_limit, int64_t pq_limit) {
  if (!data || !out_graph || n <= 0 || d <= 0 || exact_limit < 0 || pq_limit < 0) return 1;
  /* N > pq_limit: product-quantised seeding over 8 x 128 dimensions */
  const int pq = n > exact_limit && n > pq_limit;
  if (pq && d < 1024) return 2;
  const int nt = threads > 0 ? threads : 1;
  /* src/cagra.cpp:47-59 */
  const uint32_t g = graph_degree < (uint32_t)(n - 1) ? graph_degree : (uint32_t)(n - 1);
  const uint32_t nd_iters = n <= exact_limit ? 20u : (n <= pq_limit ? 5u : 0u);
  if (g == 0) return 0;

  uint32_t* graph = out_graph;
  float* gdist = (float*)malloc(sizeof(float) * (size_t)n * g);
  for (int64_t i = 0; i < n * (int64_t)g; ++i) {
    graph[i] = INVALID_ID;
    gdist[i] = INFINITY;
  }

  if (n <= exact_limit) {
    /* Exact all-pairs seeding (:324-349), one row at a time. */
    float* norms = (float*)malloc(sizeof(float) * (size_t)n);
    for (int64_t i = 0; i < n; ++i) norms[i] = sq_norm(data + i * d, d);
#pragma omp parallel num_threads(nt)
    {
      float* key = (float*)malloc(sizeof(float) * (size_t)n);
      uint32_t* idx = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)n);
#pragma omp for schedule(dynamic, 8)
      for (int64_t i = 0; i < n; ++i) {
        const float ni = norms[i];
        for (int64_t a = 0; a < n; ++a) key[a] = ni - 2.f * dot_blk(data + i * d, data + a * d, d) + norms[a];
        for (int64_t a = 0; a < n; ++a) idx[a] = (uint32_t)a;
        idx[i] = idx[n - 1];
        const int64_t take = (int64_t)g < n - 1 ? (int64_t)g : n - 1;
        select_smallest(idx, n - 1, take, key);
        for (int64_t k = 0; k < take; ++k) insert_neighbor(graph, gdist, g, i, idx[k], key[idx[k]]);
      }
      free(key);
      free(idx);
    }
    free(norms);
  } else {
    /* IVF seeding (:351-435, :576-792): K = clamp(floor(sqrt n), G + 1,
     * 2000) centres, 20 Lloyd iterations, the 3 nearest clusters, at most
     * (n / K) * 4 + 64 own members per cluster. */
    int64_t K = (int64_t)sqrt((double)n);
    if (K < (int64_t)g + 1) K = (int64_t)g + 1;
    if (K > 2000) K = 2000;
    float* cent = (float*)malloc(sizeof(float) * (size_t)(K * d));
    uint32_t* assign = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)n);
    oracle_kmeans_init(data, n, d, K, cent);
    oracle_ivf_kmeans(data, n, d, K, 20, cent, assign, nt);
    const int64_t n_probe = K - 1 < 3 ? K - 1 : 3;
    uint32_t* nearc = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(K * (n_probe > 0 ? n_probe : 1)));
    oracle_ivf_near_clusters(cent, K, d, n_probe, nearc, nt);
    uint8_t* codes = NULL;
    float* lut = NULL;
    if (pq) {
      codes = (uint8_t*)malloc((size_t)n * 8);
      lut = (float*)malloc(sizeof(float) * 8 * 256 * 256);
      oracle_pq_train(data, n, d, nt, codes, lut);
    }
    oracle_ivf_seed(data, n, d, g, assign, K, nearc, n_probe, (n / K) * 4 + 64, codes, lut, graph, gdist, nt);
    free(codes);
    free(lut);
    free(cent);
    free(assign);
    free(nearc);

    /* One random-bucketing pass (:795-851), buckets of 256. */
    uint32_t* rperm = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)n);
    oracle_bucketing_perm(n, rperm);
    oracle_bucketing_merge(data, n, d, g, rperm, 256, graph, gdist, nt);
    free(rperm);
  }

  /* nn-descent (:853-911). */
  oracle_nn_descent(data, n, d, g, graph, gdist, nd_iters, nt);
  free(gdist);
  return 0;
}
