/*
 * CPU restatement of the reference's exact search path (test infrastructure
 * only; see oracle.h).  Compile with -ffp-contract=off so that
 * `acc += t * t` rounds the product and the sum separately, as the
 * reference's loop does on x86-64 (src/cagra.cpp:221-224).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>

float oracle_l2_128(const float* a, const float* b) {
  /* src/distance.cpp:8-20 */
  if (!a || !b) return NAN;
  float acc = 0.0f;
  for (int i = 0; i < 128; ++i) {
    const float t = a[i] - b[i];
    acc += t * t;
  }
  return acc;
}

/* (d, id) strict order used by the reference's partial_sort comparator
 * (src/cagra.cpp:233-238). */
static int less_f(float da, uint32_t ia, float db, uint32_t ib) {
  return da < db || (da == db && ia < ib);
}
static int less_d(double da, uint32_t ia, double db, uint32_t ib) {
  return da < db || (da == db && ia < ib);
}

/* Bounded max-heap of the kk best (d, id) pairs seen so far. */
#define HEAP_IMPL(NAME, T, LESS)                                                       \
  static void NAME##_sift_down(T* hd, uint32_t* hi, int64_t m, int64_t i) {            \
    for (;;) {                                                                         \
      int64_t l = 2 * i + 1, r = l + 1, w = i;                                         \
      if (l < m && LESS(hd[w], hi[w], hd[l], hi[l])) w = l;                            \
      if (r < m && LESS(hd[w], hi[w], hd[r], hi[r])) w = r;                            \
      if (w == i) return;                                                              \
      T td = hd[i]; hd[i] = hd[w]; hd[w] = td;                                         \
      uint32_t ti = hi[i]; hi[i] = hi[w]; hi[w] = ti;                                  \
      i = w;                                                                           \
    }                                                                                  \
  }                                                                                    \
  static void NAME##_sift_up(T* hd, uint32_t* hi, int64_t i) {                         \
    while (i > 0) {                                                                    \
      int64_t p = (i - 1) / 2;                                                         \
      if (!LESS(hd[p], hi[p], hd[i], hi[i])) return;                                   \
      T td = hd[i]; hd[i] = hd[p]; hd[p] = td;                                         \
      uint32_t ti = hi[i]; hi[i] = hi[p]; hi[p] = ti;                                  \
      i = p;                                                                           \
    }                                                                                  \
  }                                                                                    \
  /* offer (d, id); heap holds at most kk entries, root = worst */                     \
  static void NAME##_offer(T* hd, uint32_t* hi, int64_t* m, int64_t kk, T d, uint32_t id) { \
    if (*m < kk) {                                                                     \
      hd[*m] = d; hi[*m] = id; NAME##_sift_up(hd, hi, *m); ++*m;                       \
    } else if (LESS(d, id, hd[0], hi[0])) {                                            \
      hd[0] = d; hi[0] = id; NAME##_sift_down(hd, hi, *m, 0);                          \
    }                                                                                  \
  }                                                                                    \
  /* heap -> ascending order in place */                                               \
  static void NAME##_sort(T* hd, uint32_t* hi, int64_t m) {                            \
    for (int64_t e = m - 1; e > 0; --e) {                                              \
      T td = hd[0]; hd[0] = hd[e]; hd[e] = td;                                         \
      uint32_t ti = hi[0]; hi[0] = hi[e]; hi[e] = ti;                                  \
      NAME##_sift_down(hd, hi, e, 0);                                                  \
    }                                                                                  \
  }

HEAP_IMPL(hf, float, less_f)
HEAP_IMPL(hd, double, less_d)

void oracle_bf_exact(const float* base, int64_t n, int64_t d, const float* queries, int64_t q,
                     int64_t k, uint32_t* out_nbr, float* out_dist, int threads) {
  const int64_t kk = k < n ? k : n; /* result_count, src/cagra.cpp:228 */
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
  for (int64_t qi = 0; qi < q; ++qi) {
    float* hdist = (float*)malloc(sizeof(float) * (size_t)(kk > 0 ? kk : 1));
    uint32_t* hid = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(kk > 0 ? kk : 1));
    int64_t m = 0;
    const float* qv = queries + qi * d;
    for (int64_t r = 0; r < n; ++r) {
      const float* xv = base + r * d;
      float acc = 0.0f; /* src/cagra.cpp:220-224 */
      for (int64_t i = 0; i < d; ++i) {
        const float t = qv[i] - xv[i];
        acc += t * t;
      }
      if (kk > 0) hf_offer(hdist, hid, &m, kk, acc, (uint32_t)r);
    }
    hf_sort(hdist, hid, m);
    for (int64_t j = 0; j < k; ++j) { /* src/cagra.cpp:240-251 */
      out_nbr[qi * k + j] = j < m ? hid[j] : 0xffffffffu;
      out_dist[qi * k + j] = j < m ? hdist[j] : INFINITY;
    }
    free(hdist);
    free(hid);
  }
}

void oracle_bf_fp64(const float* base, int64_t n, int64_t d, const float* queries, int64_t q,
                    int64_t k, uint32_t* out_nbr, double* out_dist, int threads) {
  const int64_t kk = k < n ? k : n;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
  for (int64_t qi = 0; qi < q; ++qi) {
    double* hdist = (double*)malloc(sizeof(double) * (size_t)(kk > 0 ? kk : 1));
    uint32_t* hid = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(kk > 0 ? kk : 1));
    int64_t m = 0;
    const float* qv = queries + qi * d;
    for (int64_t r = 0; r < n; ++r) {
      const float* xv = base + r * d;
      double acc = 0.0;
      for (int64_t i = 0; i < d; ++i) {
        const double t = (double)qv[i] - (double)xv[i];
        acc += t * t;
      }
      if (kk > 0) hd_offer(hdist, hid, &m, kk, acc, (uint32_t)r);
    }
    hd_sort(hdist, hid, m);
    for (int64_t j = 0; j < k; ++j) {
      out_nbr[qi * k + j] = j < m ? hid[j] : 0xffffffffu;
      out_dist[qi * k + j] = j < m ? hdist[j] : INFINITY;
    }
    free(hdist);
    free(hid);
  }
}
