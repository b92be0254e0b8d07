/*
 * oracle.h - CPU restatement of the reference's search path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker; the product (libcvs_hip, libcuvs_silicon) never links it.
 *
 * Each function cites the reference lines it restates.  Pinning (how each
 * function is itself checked) is listed per function; see tests/test_oracle.py.
 */
#ifndef CVS_ORACLE_H
#define CVS_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* squared_l2_distance_128 (reference src/distance.cpp:8-20): sequential fp32
 * sum over 128 dims.  Returns NaN for a null input (the reference throws).
 * Pinned: the reference's known answers tests/test_l2_distance.cpp:19-49 and
 * the reference object built in oracle/_ref. */
float oracle_l2_128(const float* a, const float* b);

/* Exact k-NN, the reference's CPU search loop (src/cagra.cpp:211-252):
 * d = sum_i (q_i - x_i)^2 accumulated sequentially in fp32 (no FMA), the
 * min(k, n) smallest by (d, id) ascending, remaining slots UINT32_MAX / +inf.
 * Queries are independent; `threads` > 1 splits them across OpenMP threads
 * without changing any result.  Pinned: FAISS smoke and dispatch-test known
 * answers, fp64 brute force on small inputs, and bit-identity with the
 * reference object built in oracle/_ref. */
void oracle_bf_exact(const float* base, int64_t n, int64_t d, const float* queries, int64_t q,
                     int64_t k, uint32_t* out_nbr, float* out_dist, int threads);

/* Same selection with distances accumulated in double (ground truth for
 * recall).  Pinned: closed-form distances on integer inputs. */
void oracle_bf_fp64(const float* base, int64_t n, int64_t d, const float* queries, int64_t q,
                    int64_t k, uint32_t* out_nbr, double* out_dist, int threads);

#ifdef __cplusplus
}
#endif
#endif
