/*
 * oracle.h - CPU restatement of the reference's search path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only to check
 * results against it; the product (libcvs_hip, libcuvs_silicon) never
 * links it.
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
 * exact all-pairs seeding; otherwise the IVF stages below in the
 * reference's order and settings (oracle_kmeans_init, oracle_ivf_kmeans
 * with K = clamp(floor(sqrt n), G+1, 2000) and 20 iterations,
 * oracle_ivf_near_clusters with 3 probes, oracle_ivf_seed with max_own =
 * (n / K) * 4 + 64, oracle_bucketing_perm + oracle_bucketing_merge with
 * buckets of 256); then oracle_nn_descent for 20 (n <= 50,000) or 5
 * iterations.  Writes n x G ids (UINT32_MAX for missing).  Cross products
 * use a fixed 8-way summation where the reference calls cblas_sgemm.  For
 * n > 200,000 the seeding ranks candidates by product-quantisation table
 * sums (oracle_pq_train; src/metal_context.mm:437-568, :614-681) and
 * re-scores the kept entries exactly (:683-709), with no nn-descent.
 * Returns 0, 1 on bad arguments, 2 when the PQ path meets d < 1024.
 * Pinned: the exact-seeding path equals the exact kNN graph on integer data;
 * the IVF path equals the composition of the stage functions with the
 * reference's constants, each of which changes the graph on the test data
 * (tests/test_oracle_build.py).  Bit-exact graphs of the reference itself
 * are parity unpinned (they depend on a GPU race and on BLAS order). */
int oracle_cagra_build_ref(const float* data, int64_t n, int64_t d, uint32_t graph_degree,
                           uint32_t* out_graph, int threads);

/* oracle_cagra_build_ref with the size limits as arguments (exact seeding
 * for n <= exact_limit, PQ seeding for n > max(exact_limit, pq_limit); the
 * reference's limits are 50,000 and 200,000), so that tests can run the
 * large-N phases at small n. */
int oracle_cagra_build_ref_ex(const float* data, int64_t n, int64_t d, uint32_t graph_degree,
                              uint32_t* out_graph, int threads, int64_t exact_limit, int64_t pq_limit);

/* ---- stages of the build (pinned one by one in tests/test_oracle_build.py) */

/* Initial IVF centres (src/metal_context.mm:366-375): centre k = row
 * min(floor(k * s + s / 2), n - 1), s = n / K in double.  Pinned: the row
 * indices at n = 1000, K = 7 written out. */
void oracle_kmeans_init(const float* data, int64_t n, int64_t d, int64_t K, float* centres);

/* Lloyd iterations from the given centres (src/metal_context.mm:381-435):
 * E-step argmin of |x|^2 - 2 x.c + |c|^2 (first minimum wins), stop when no
 * row changes; M-step sums in row order times 1 / count; an empty centre
 * becomes zero.  Updates `centres`, writes `assign`, returns the E-steps
 * run (<= max_iter).  Pinned: a hand-worked case in which duplicated
 * initial centres tie (the lower index takes every row), the empty centre
 * becomes zero and then captures the rows near the origin; planted mistakes
 * (higher index wins, empty centre kept, wrong divisor) fail it. */
int oracle_ivf_kmeans(const float* data, int64_t n, int64_t d, int64_t K, int max_iter, float* centres,
                      uint32_t* assign, int threads);

/* The n_probe nearest other centres of each centre, nearest first
 * (src/metal_context.mm:583-611).  Pinned: centres on a parabola, where the
 * answer is written out. */
void oracle_ivf_near_clusters(const float* centres, int64_t K, int64_t d, int64_t n_probe, uint32_t* nearc,
                              int threads);

/* Per-cluster seeding (src/metal_context.mm:576-582, :614-681, :712-792):
 * the first min(count, max_own) members of each cluster take their g
 * nearest among those members and all members of the cluster's n_probe near
 * clusters (at most 8,192 candidates), inserted with insert_neighbor;
 * members past max_own seed nothing.  Exact expanded-form keys, or with
 * `codes`/`lut` the product-quantisation table sums followed by exact float4
 * distances of the kept entries.  Pinned: integer clusters where a true
 * neighbour lies only in the third near cluster, and the cap leaves later
 * members empty (brute force over the candidate sets); the PQ form equals
 * the exact form on rows built from the quantisation prototypes. */
void oracle_ivf_seed(const float* data, int64_t n, int64_t d, uint32_t g, const uint32_t* assign, int64_t K,
                     const uint32_t* nearc, int64_t n_probe, int64_t max_own, const uint8_t* codes,
                     const float* lut, uint32_t* graph, float* gdist, int threads);

/* The bucketing permutation (src/metal_context.mm:802-810).  Pinned without
 * re-running the loop: the swap index of every step is recovered from the
 * output by inverting the Fisher-Yates shuffle and must equal
 * (x_k >> 33) mod (i + 1), where x_k, the generator's state after k = n - i
 * steps, is computed in closed form (LCG jump-ahead by repeated squaring);
 * a shift of 32, ascending i, and the generator advanced after the swap
 * each fail that check (tests/test_oracle_build_stages.py). */
void oracle_bucketing_perm(int64_t n, uint32_t* perm);

/* One random-bucketing pass (shaders/cagra_kernels.metal:403-462) over
 * buckets of `bucket` consecutive positions of perm.  Pinned: with the
 * identity permutation on integer data every row receives its min(g, 64)
 * nearest bucket mates (brute force), a mate already in the row is inserted
 * again (the reference's duplicates), and bucket edges are respected. */
void oracle_bucketing_merge(const float* data, int64_t n, int64_t d, uint32_t g, const uint32_t* perm,
                            int64_t bucket, uint32_t* graph, float* gdist, int threads);

/* nn-descent over 2-hop neighbours (shaders/cagra_kernels.metal:334-395,
 * src/metal_context.mm:853-911), at most max_iter iterations; neighbour rows
 * are read as they were when each iteration began.  Returns the iterations
 * run.  Pinned: a chain in which each iteration can only move one hop,
 * whose state after t iterations is written out, and the early stop. */
int oracle_nn_descent(const float* data, int64_t n, int64_t d, uint32_t g, uint32_t* graph, float* gdist,
                      uint32_t max_iter, int threads);

/* The product-quantisation training of the build's PQ path, exposed for its
 * pinning tests: codes n x 8 (uint8), lut 8 x 256 x 256. */
void oracle_pq_train(const float* data, int64_t n, int64_t d, int threads, uint8_t* codes, float* lut);

#ifdef __cplusplus
}
#endif
#endif
