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


/* ---- CAGRA search (oracle/cagra_oracle.c) ------------------------------- */

/* recompute_graph_distances (reference shaders/cagra_kernels.metal:658-681):
 * squared L2 length of every graph edge over float4 groups of the first
 * 4*floor(d/4) columns; +inf for UINT32_MAX (and, here, ids >= n).  Pinned:
 * numpy fp64 on random graphs (multiple-of-4 d), the truncation to 4*floor(d/4)
 * columns on a d = 6 case, and the +inf entries. */
void oracle_edge_distances(const float* rows, int64_t n, int64_t d, const uint32_t* graph, uint32_t g,
                           float* out, int threads);

/* Navigation nodes of a built index (src/cagra.cpp:65-72): returns
 * n_nav = min(200, floor(sqrt(n))) and, if out_ids is non-null, writes
 * out_ids[i] = (uint32)(i * (n / n_nav)).  Pinned: closed form at n = 1, 10,
 * 40,000 and 100,000 (tests/test_oracle_cagra.py). */
int64_t oracle_cagra_nav_nodes(int64_t n, uint32_t* out_ids);

/* Per-query entry point (src/cagra.cpp:133-177): argmin over the navigation
 * vectors of |q|^2 - 2 q.v + |v|^2 in fp32 (first minimum wins; cross terms
 * as sequential dot products where the reference uses cblas_sgemm).
 * Pinned: equals the exact nearest navigation node on well-separated data,
 * and the first-minimum tie rule on duplicated vectors. */
void oracle_cagra_entry_points(const float* queries, int64_t q, int64_t d, const uint32_t* nav_ids,
                               const float* nav_vectors, int64_t n_nav, uint32_t* out_entry);

/* Beam size and iteration cap (src/cagra.cpp:182-189): itopk 0 -> 128,
 * max_iterations 0 -> 200, and for q <= 4 the beam is clamped to 32.
 * Pinned: every branch against its closed form. */
void oracle_cagra_search_policy(uint64_t itopk_size, uint64_t max_iterations, int64_t q,
                                uint32_t* out_beam, uint32_t* out_iters);

/* The reference's beam search (shaders/cagra_kernels.metal:28-199): seed =
 * entry[q] if < n else (q * 2654435761) mod n; per iteration expand the
 * unexpanded entry of smallest distance (expanded entries hold -d-1),
 * compute its g neighbours' distances, and for each unvisited one replace
 * the first entry of largest |d| if closer; output sorted by (d, id), padded
 * with UINT32_MAX / +inf.  `entry` may be null.  Pinned: on a complete graph
 * it returns the exact k-NN (FAISS smoke database with g = n - 1); a
 * hand-traced path graph; its invariants (sorted, unique, in range, distances
 * equal to the exact fp32 distances of the returned ids); and a planted
 * mistake (expanding the worst entry) fails them. */
void oracle_cagra_search(const float* base, int64_t n, int64_t d, const uint32_t* graph,
                         uint32_t g, const float* queries, int64_t q, const uint32_t* entry,
                         int64_t k, uint32_t beam, uint32_t max_iter, uint32_t* out_nbr,
                         float* out_dist, int threads);

/* Exact degree-g kNN graph without self edges, rows sorted by (d, id),
 * missing entries UINT32_MAX (the reference's build for n <= 50,000 is exact
 * all-pairs seeding, src/metal_context.mm:324-349).  Pinned: rows equal
 * oracle_bf_exact's k = g + 1 results with the row itself removed. */
void oracle_knn_graph(const float* base, int64_t n, int64_t d, uint32_t g, uint32_t* out_graph,
                      int threads);

/* ---- CAGRA build (oracle/cagra_build_oracle.c) -------------------------- */

/* The reference's graph build for n <= 200,000 (src/cagra.cpp:47-59 ->
 * src/metal_context.mm:289-914): G = min(graph_degree, n - 1); n <= 50,000:
 * exact all-pairs seeding; otherwise IVF k-means (K = clamp(sqrt n, G+1,
 * 2000), 20 iterations, stride initialisation), exact seeding of each
 * cluster's rows against their own and the 3 nearest clusters' rows (at most
 * 8,192), then one random bucketing pass (LCG Fisher-Yates, buckets of 256,
 * top-min(G, 64) merged per row); then nn-descent for 20 (n <= 50,000) or 5
 * iterations.  Writes n x G ids (UINT32_MAX for missing).  Cross products use
 * a fixed 8-way summation where the reference calls cblas_sgemm; nn-descent
 * reads other nodes' lists as of the start of each iteration (one legal
 * schedule of the reference's racy kernel).  For n > 200,000 the per-cluster
 * seeding ranks candidates by product-quantisation table sums
 * (src/metal_context.mm:437-568, :614-681; 8 subspaces of 128 dimensions,
 * 256 centres) and re-scores the kept entries exactly (:683-709), with no
 * nn-descent.  Returns 0, 1 on bad arguments, 2 when the PQ path meets
 * d < 1024.  Pinned: equals the exact
 * kNN graph on integer data through the exact-seeding path; on the IVF path,
 * rows are full, in range, free of self edges and hold most exact neighbours
 * (tests/test_oracle_build.py).  Bit-exact graphs are parity unpinned (the
 * reference's own result depends on a GPU race and on BLAS order). */
int oracle_cagra_build_ref(const float* data, int64_t n, int64_t d, uint32_t graph_degree,
                           uint32_t* out_graph, int threads);

/* oracle_cagra_build_ref with the size limits as arguments (exact seeding
 * for n <= exact_limit, PQ seeding for n > max(exact_limit, pq_limit); the
 * reference's limits are 50,000 and 200,000), so that tests can run the
 * large-N phases at small n.  The PQ seeding is pinned by its equivalence
 * with exact per-cluster seeding over the rows rebuilt from their codes
 * (tests/test_oracle_build.py). */
int oracle_cagra_build_ref_ex(const float* data, int64_t n, int64_t d, uint32_t graph_degree,
                              uint32_t* out_graph, int threads, int64_t exact_limit, int64_t pq_limit);

/* The product-quantisation training of the build's PQ path, exposed for its
 * pinning tests: codes n x 8 (uint8), lut 8 x 256 x 256. */
void oracle_pq_train(const float* data, int64_t n, int64_t d, int threads, uint8_t* codes, float* lut);

#ifdef __cplusplus
}
#endif
#endif
