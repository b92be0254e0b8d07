/*
 * cvs_hip.h - C ABI of the MI355X (gfx950) search backend.
 *
 * This is the device boundary of the library.  It replaces the reference's
 * Objective-C++ backend class `cuvs_silicon::MetalContext`
 * (include/cuvs_silicon/metal_context.hpp:12-81, src/metal_context.mm) with
 * plain `extern "C"` functions over pointers and sizes, so that any host
 * language (C++, Python ctypes, cgo, JNI) can bind it.
 *
 * Conventions
 *  - Every function returns CVS_OK (0) or a CVS_ERR_* code; the message of the
 *    last failure on the calling thread is returned by cvs_last_error().
 *  - Matrices are row-major.  Dataset/query rows are fp32.  Neighbour ids are
 *    uint32 row indices into the dataset; distances are *squared* L2.
 *  - Result rows are sorted by (distance, id) ascending; slots beyond the
 *    number of available results hold UINT32_MAX / +inf
 *    (src/cagra.cpp:240-251 in the reference).
 *  - Functions without the `_async` suffix take HOST pointers and block until
 *    results are in the caller's host buffers (reference semantics:
 *    src/metal_context.mm:224-225, :242-243, :1099-1100).  `_async` variants
 *    take DEVICE pointers, are enqueued on the context's stream and return
 *    immediately; call cvs_context_synchronize() before reading results.
 *  - A context is not thread-safe: use one context per host thread.
 *  - There is no CPU fallback: without a usable gfx950 device every compute
 *    entry point fails with CVS_ERR_NO_DEVICE.
 */
#ifndef CVS_HIP_H
#define CVS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum cvs_status {
  CVS_OK = 0,
  CVS_ERR_INVALID_ARGUMENT = 1, /* bad shape / null pointer -> std::invalid_argument */
  CVS_ERR_RUNTIME = 2,          /* HIP runtime failure       -> std::runtime_error */
  CVS_ERR_NO_DEVICE = 3,        /* no usable GPU             -> std::runtime_error */
  CVS_ERR_OUT_OF_MEMORY = 4,    /* device allocation failed  -> std::runtime_error */
  CVS_ERR_UNSUPPORTED = 5       /* shape outside kernel limits -> std::invalid_argument */
};

typedef struct cvs_context cvs_context; /* one device + one HIP stream */
typedef struct cvs_dataset cvs_dataset; /* device-resident dataset (fp32 rows, fp16 tiles, norms) */
typedef struct cvs_cagra_index cvs_cagra_index; /* device-resident graph index (rows, graph, seeds) */

/* Limits of the brute force (checked by cvs_bf_search*).  Calls with
 * d <= 1024 and k <= 112 run the fused streaming scan; larger d or k run a
 * keys-matrix path with the same exact results (the reference's CPU loop,
 * src/cagra.cpp:211-252, has no limit on either). */
#define CVS_BF_MAX_DIM 16384
#define CVS_BF_MAX_K 1024

/* Limits of the graph search kernel (checked by cvs_cagra_search*).  Rows
 * of up to 1024 columns keep the query in registers, wider ones in LDS. */
#define CVS_CAGRA_MAX_DIM 8192
#define CVS_CAGRA_MAX_ITOPK 512
#define CVS_CAGRA_MAX_WIDTH 16
#define CVS_CAGRA_MAX_TEAMS 64

/* ---- errors, counters ---------------------------------------------------- */

/* Message of the last failed call on this thread ("" if none). */
const char* cvs_last_error(void);

/* Number of kernel launches made by this process since the last reset.
 * Backs the reference's dispatch instrumentation
 * (include/cuvs/neighbors/cagra.hpp:119-122, src/cagra.cpp:255-266). */
uint64_t cvs_dispatch_count(void);
void cvs_reset_dispatch_count(void);

/* ---- context ------------------------------------------------------------- */

/* Number of visible HIP devices (0 when none; never fails). */
int cvs_device_count(int* out_count);

/* Create a context on `device` (replaces MetalContext::instance(),
 * metal_context.hpp:15, and is_available(), metal_context.hpp:19). */
int cvs_context_create(int device, cvs_context** out_ctx);
int cvs_context_destroy(cvs_context* ctx);
int cvs_context_synchronize(cvs_context* ctx);

/* Device name and compute-unit count, for run metadata
 * (replaces MetalContext::chip_model(), metal_context.hpp:23). */
int cvs_context_device_info(cvs_context* ctx, char* name, size_t name_len,
                            int* compute_units, int64_t* total_mem_bytes);

/* Kernel timing: while enabled, each call times its kernel families with HIP
 * events that the runtime fills from the dispatches' own start and end
 * timestamps (the family's first launch starts the span, its last launch
 * ends it), so timing inserts nothing between kernels on the stream.
 * cvs_context_kernel_time() synchronizes and returns the summed elapsed
 * milliseconds and the number of spans for `kernel` ("bf_prep", "bf_sample",
 * "bf_scan", "bf_merge", "cagra_search", "cagra_edge_distances"), then
 * clears them. */
int cvs_context_set_timing(cvs_context* ctx, int enable);
int cvs_context_kernel_time(cvs_context* ctx, const char* kernel,
                            double* total_ms, uint64_t* launches);

/* Brute-force escalations since the context was made (or last reset): the
 * number of queries whose fp16 candidate selection could not be certified
 * exact and that were re-ranked exactly over every row with a key up to
 * the bound (see cvs_bf_search), and how many of those over every row of
 * the dataset.  Synchronizes; reset = 1 clears them afterwards.  No
 * counterpart in the reference, whose GPU path does not check its fp16
 * selection (src/metal_context.mm:203-246). */
int cvs_context_bf_escalations(cvs_context* ctx, uint64_t* escalated, uint64_t* rescanned, int reset);

/* Device calibration; no counterpart in the reference (its roofline figures
 * are nominal).  Streams `bytes` of device memory, rounded down to whole
 * 32 KiB steps per workgroup, with `workgroups` workgroups of 256 threads,
 * each reading one contiguous share with 16-byte non-temporal loads, `reps`
 * times after two warm-up passes, and returns the read rate in GB/s: the
 * achievable bound next to the nominal HBM peak.  Allocates and frees its
 * own buffer; synchronizes. */
int cvs_calibrate_stream_read(cvs_context* ctx, size_t bytes, int workgroups, int reps,
                              double* out_gbs);

/* Device calibration for gather-bound kernels; no counterpart in the
 * reference.  Allocates n_rows rows of row_bytes (a multiple of 16, at most
 * 4096), then `workgroups` workgroups of 16 teams of 16 lanes each read
 * rows_per_team rows picked uniformly at random, one 256-byte segment per
 * team and load instruction, two rows in flight per team (the graph search's
 * gather shape), `reps` times after two warm-up passes; returns the rate of
 * gathered bytes in GB/s.  Frees its buffer; synchronizes. */
int cvs_calibrate_gather_read(cvs_context* ctx, size_t row_bytes, int64_t n_rows, int workgroups, int rows_per_team,
                              int reps, double* out_gbs);

/* Device calibration for matrix-core-bound kernels; no counterpart in the
 * reference.  `workgroups` workgroups of 4 waves (one per SIMD) each run
 * `ksteps` (rounded up to even) k-steps of 16 v_mfma_f32_32x32x16_f16 on the
 * large-batch scan's 4 x 4 block of 32 x 32 accumulators, with fragments
 * taken from `fp16_data` (device memory, 16-byte aligned, whole 40 KiB
 * sets, workgroup i using set i mod sets) and held in registers, or, with
 * from_lds, re-read from LDS every k-step as the scan reads them; `reps`
 * launches after two warm-up launches.  Returns fp16 dense TFLOP/s, next to
 * the nominal 2.5 PFLOP/s.  Synchronizes. */
int cvs_calibrate_mfma(cvs_context* ctx, const void* fp16_data, size_t data_bytes, int workgroups, int64_t ksteps,
                       int from_lds, int reps, double* out_tflops);

/* ---- device memory helpers (device-resident benchmarking and tests) ----- */

int cvs_device_alloc(cvs_context* ctx, size_t bytes, void** out_ptr);
int cvs_device_free(cvs_context* ctx, void* ptr);
int cvs_copy_to_device(cvs_context* ctx, void* dst, const void* src, size_t bytes);
int cvs_copy_to_host(cvs_context* ctx, void* dst, const void* src, size_t bytes);

/* ---- dataset ------------------------------------------------------------- */

/* Upload an n x d fp32 row-major dataset and build its search layouts: the
 * fp32 rows (exact re-rank, graph search), fp16 16-row MFMA tiles and fp32
 * squared norms of the fp16-rounded rows.  Replaces the reference's
 * per-pointer dataset cache and host fp16 conversion
 * (src/metal_context.mm:155-175, compute_row_norms :127-137).
 * `rows_on_device` = 0: `rows` is a host pointer; 1: a device pointer. */
int cvs_dataset_create(cvs_context* ctx, const float* rows, int64_t n,
                       int64_t d, int rows_on_device, cvs_dataset** out_ds);
int cvs_dataset_destroy(cvs_dataset* ds);
int cvs_dataset_shape(const cvs_dataset* ds, int64_t* n, int64_t* d);
/* Device pointer of the fp32 rows (n x d, row-major). */
int cvs_dataset_rows(const cvs_dataset* ds, const float** out_rows);

/* ---- exact brute-force k-NN --------------------------------------------- */

/* Exact squared-L2 k-NN of q queries against the dataset.  Replaces
 * MetalContext::search_brute_force (metal_context.hpp:35-40;
 * src/metal_context.mm:139-255: MPS fp16 GEMM + l2_topk_from_cross) and
 * returns what the reference's CPU loop returns (src/cagra.cpp:211-252).
 * Fused: fp16 MFMA cross terms of the centred, scaled rows and queries over
 * LDS-staged tiles select candidates, which are re-ranked in fp32.  Each
 * query is certified: with a bound on the fp16 arithmetic's error, no row
 * outside the re-ranked candidates can be nearer than the k-th result; a
 * query that fails is re-ranked exactly over every row that could be (in
 * the worst case every row), so results are exact on any finite input.
 * Requires 1 <= k <= CVS_BF_MAX_K and d <= CVS_BF_MAX_DIM; d > 1024 or
 * k > 112 run a second path (a per-query threshold from sampled rows, fp16
 * MFMA keys of every row listing those at or below it, a select over the
 * list, the same certificate and exact re-rank; a query the list does not
 * serve is answered from the full key matrix of its 128-query block).  Its
 * workspace, held by the context, is sized for chunks of up to 512 queries:
 * the key matrix of a chunk (at most ~2 GiB, written only for such blocks),
 * 64 KiB of list per query and the sampled keys.  Host pointers, blocking. */
int cvs_bf_search(cvs_context* ctx, const cvs_dataset* ds,
                  const float* queries, int64_t q, int64_t k,
                  uint32_t* out_neighbors, float* out_distances);

/* Same, with device pointers; enqueued on the context stream. */
int cvs_bf_search_async(cvs_context* ctx, const cvs_dataset* ds,
                        const float* queries_dev, int64_t q, int64_t k,
                        uint32_t* out_neighbors_dev, float* out_distances_dev);

/* cvs_bf_search_async without any allocation, for d <= 1024 and k <= 112
 * (the fused scan): no counterpart in the reference.  For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The workspace (query tiles,
 * thresholds, sample minima, candidate lists) lives in a 64 MiB array that
 * the library holds on each device it runs on until the process ends; a call
 * whose workspace would exceed it fails with CVS_ERR_UNSUPPORTED and a
 * message giving the bytes needed.  On 256 compute units at D = 1024 and at
 * least 8,192 rows, batches of up to 1,024 queries (256 candidate lists per
 * query) fit for k <= 10, up to 922 for k <= 24, 485 for k <= 48 and 331
 * for k <= 112; larger batches (32 lists per query) fit up to 7,808 queries
 * for k <= 10, 5,286 for k <= 24 and 3,212 for k <= 48.  Device pointers;
 * enqueued on the context stream; no events.  Calls that overlap on one GPU
 * (several contexts or threads on the same device) share that array and
 * race: serialise them. */
#define CVS_BF_NOALLOC_SCRATCH_BYTES (64u << 20)
int cvs_bf_search_noalloc(cvs_context* ctx, const cvs_dataset* ds,
                          const float* queries_dev, int64_t q, int64_t k,
                          uint32_t* out_neighbors_dev, float* out_distances_dev);

/* ---- CAGRA graph search -------------------------------------------------- */

/* Navigation (seed) nodes of an n-row graph index, as the reference's
 * cagra::build chooses them (src/cagra.cpp:63-72): n_nav = min(200,
 * floor(sqrt(n))) rows, row i at floor(i * (n / n_nav)) with the spacing in
 * double.  Writes *out_count = n_nav and, when out_ids is non-null, the n_nav
 * ids (the caller sizes it: at most 200).  Host only; no device is needed. */
int cvs_cagra_nav_nodes(int64_t n, uint32_t* out_ids, int64_t* out_count);

/* Upload a graph index: n x d fp32 rows, its n x degree uint32 neighbour
 * lists (entries >= n are ignored) and `n_seeds` seed node ids (the
 * reference's navigation nodes, src/cagra.cpp:63-82; may be 0).  Replaces the
 * per-call buffer wraps of MetalContext::search_cagra
 * (src/metal_context.mm:1045-1054).  `*_on_device` = 1: the pointer is a
 * device pointer; seeds are always host memory. */
int cvs_cagra_index_create(cvs_context* ctx, const float* rows, int64_t n, int64_t d,
                           int rows_on_device, const uint32_t* graph, uint32_t degree,
                           int graph_on_device, const uint32_t* seeds, uint32_t n_seeds,
                           cvs_cagra_index** out_index);
int cvs_cagra_index_destroy(cvs_cagra_index* index);

/* Precision of the graph traversal: 32 (the default) evaluates every
 * candidate on the fp32 rows, as the reference's beam search does
 * (shaders/cagra_kernels.metal:117-132); 16 evaluates candidates on an fp16
 * copy of the centred, scaled rows made at index creation, then recomputes
 * the distances of the final itopk list from the fp32 rows and re-sorts it,
 * so that output distances are exact fp32.  No counterpart in the
 * reference: the fp16 copy halves the bytes each distance evaluation reads. */
int cvs_cagra_index_set_traversal(cvs_cagra_index* index, int bits);

/* Exact squared L2 length of every edge of the index's graph: out[i*degree
 * + j] = |row i - row graph[i][j]|^2 in fp32, +inf where the entry is not a
 * row id (UINT32_MAX, or >= n).  Replaces the reference's
 * recompute_graph_distances pass (shaders/cagra_kernels.metal:658-681, host
 * src/metal_context.mm:683-709).  out_on_device = 0: n x degree host floats,
 * blocking; 1: a device buffer, enqueued on the context stream. */
int cvs_cagra_index_edge_distances(cvs_context* ctx, const cvs_cagra_index* index, float* out_distances,
                                   int out_on_device);

/* Approximate k-NN by graph search.  Replaces MetalContext::search_cagra
 * (metal_context.hpp:57-73; src/metal_context.mm:918-1111) and the host
 * entry-point selection (src/cagra.cpp:128-178).  Parameters keep the
 * reference's meaning (include/cuvs/neighbors/cagra.hpp:36-50):
 * itopk_size = internal list length (0 -> 128, raised to k if smaller,
 * at most CVS_CAGRA_MAX_ITOPK); search_width = parents expanded per
 * iteration (0 -> 1); max_iterations (0 -> max(200, 2*itopk/width)).
 * The list starts from max(n_seeds, itopk) candidates rounded up to 64: all
 * seed nodes, then hashed row ids led by the reference's (q * 2654435761)
 * mod n (shaders/cagra_kernels.metal:65-67).
 * Results sorted by (distance, id), padded with UINT32_MAX / +inf.  Host
 * pointers, blocking. */
int cvs_cagra_search(cvs_context* ctx, const cvs_cagra_index* index, const float* queries, int64_t q,
                     int64_t k, uint32_t itopk_size, uint32_t search_width, uint32_t max_iterations,
                     uint32_t* out_neighbors, float* out_distances);

/* Multi-team graph search, the reference's cagra_beam_search_multi_cta
 * (shaders/cagra_kernels.metal:200-327, host merge src/metal_context.mm:
 * 1003-1035): `teams` independent searches per query (1 to
 * CVS_CAGRA_MAX_TEAMS), each with its own itopk list (itopk_size as above,
 * teams * itopk at most CVS_CAGRA_MAX_ITOPK) and its own share of the start
 * candidates (team t takes candidates t, t + teams, ...); the teams' lists are
 * merged on the GPU, an id found by several teams counted once.  Smaller
 * per-team lists need fewer iterations, so a small batch (Q = 1) answers
 * sooner.  Host pointers, blocking; the _async form takes device pointers. */
int cvs_cagra_search_teams(cvs_context* ctx, const cvs_cagra_index* index, const float* queries, int64_t q,
                           int64_t k, uint32_t itopk_size, uint32_t search_width, uint32_t max_iterations,
                           uint32_t teams, uint32_t* out_neighbors, float* out_distances);
int cvs_cagra_search_teams_async(cvs_context* ctx, const cvs_cagra_index* index, const float* queries_dev,
                                 int64_t q, int64_t k, uint32_t itopk_size, uint32_t search_width,
                                 uint32_t max_iterations, uint32_t teams, uint32_t* out_neighbors_dev,
                                 float* out_distances_dev);

/* Same, with device pointers; enqueued on the context stream.
 * `out_stats_dev` (q x 2 uint32, may be null) receives per query the number
 * of distance evaluations and of iterations (for byte accounting). */
int cvs_cagra_search_async(cvs_context* ctx, const cvs_cagra_index* index, const float* queries_dev,
                           int64_t q, int64_t k, uint32_t itopk_size, uint32_t search_width,
                           uint32_t max_iterations, uint32_t* out_neighbors_dev,
                           float* out_distances_dev, uint32_t* out_stats_dev);

/* Per-query entry node of the reference's search route (src/cagra.cpp:
 * 128-178): among the index's seed nodes (the navigation nodes), the one
 * that minimises |q|^2 - 2 q.v + |v|^2 in fp32, the first on ties, computed
 * on the GPU.  The index must have seed nodes.  Host pointers, blocking; the
 * _async form takes device pointers. */
int cvs_cagra_entry_points(cvs_context* ctx, const cvs_cagra_index* index, const float* queries, int64_t q,
                           uint32_t* out_entry);
int cvs_cagra_entry_points_async(cvs_context* ctx, const cvs_cagra_index* index, const float* queries_dev,
                                 int64_t q, uint32_t* out_entry_dev);

/* The reference's own beam search (shaders/cagra_kernels.metal:28-199, host
 * src/metal_context.mm:1041-1110), for query-by-query parity with it:
 * query i starts from entry_nodes[i] when that is < n, else (or with
 * entry_nodes null) from (i * 2654435761) mod n; an unsorted beam of
 * beam_size entries (1 to CVS_CAGRA_MAX_ITOPK, used as given: the
 * reference's defaults and its q <= 4 clamp, src/cagra.cpp:182-189, are the
 * caller's); each iteration expands the first unexpanded entry of smallest
 * distance and offers its neighbours in graph order, an unvisited one
 * replacing the first entry of largest distance if strictly closer; at most
 * max_iter iterations; fp32 distances over the fp32 rows.  Results sorted by
 * (distance, id), padded with UINT32_MAX / +inf.  Replaces
 * MetalContext::search_cagra (metal_context.hpp:58-67).  Host pointers,
 * blocking (entry_nodes: q host ids or null); the _async form takes device
 * pointers (entry_nodes_dev: q device ids or null). */
int cvs_cagra_search_reference(cvs_context* ctx, const cvs_cagra_index* index, const float* queries, int64_t q,
                               int64_t k, uint32_t beam_size, uint32_t max_iter, const uint32_t* entry_nodes,
                               uint32_t* out_neighbors, float* out_distances);
int cvs_cagra_search_reference_async(cvs_context* ctx, const cvs_cagra_index* index, const float* queries_dev,
                                     int64_t q, int64_t k, uint32_t beam_size, uint32_t max_iter,
                                     const uint32_t* entry_nodes_dev, uint32_t* out_neighbors_dev,
                                     float* out_distances_dev);

/* Measurement support for the graph search's roofline; no counterpart in
 * the reference.  cvs_cagra_search_record_async is cvs_cagra_search_async
 * (stats required) that also writes the ids of each query's distance
 * evaluations, in order, the first record_cap of them per query, to
 * record_dev (q x record_cap uint32, device).  cvs_cagra_replay_gathers then
 * gathers exactly those rows (of the fp16 copy for bits = 16, the fp32 rows
 * for 32) with the search's row shape and no search work, one workgroup per
 * query, `reps` times after a warm-up, and returns the mean ms per replay:
 * the time the search's data movement takes on its own. */
int cvs_cagra_search_record_async(cvs_context* ctx, const cvs_cagra_index* index, const float* queries_dev,
                                  int64_t q, int64_t k, uint32_t itopk_size, uint32_t search_width,
                                  uint32_t max_iterations, uint32_t* out_neighbors_dev, float* out_distances_dev,
                                  uint32_t* out_stats_dev, uint32_t* record_dev, uint32_t record_cap);
int cvs_cagra_replay_gathers(cvs_context* ctx, const cvs_cagra_index* index, const uint32_t* record_dev,
                             uint32_t record_cap, const uint32_t* stats_dev, int64_t q, int bits, int reps,
                             double* out_ms);

/* ---- CAGRA graph build --------------------------------------------------- */

/* Phase timings and work counters of one cvs_cagra_build call. */
typedef struct cvs_build_stats {
  uint32_t iterations;          /* nn-descent iterations run */
  uint32_t intermediate_degree; /* list length used (<= n - 1) */
  uint32_t graph_degree;        /* output degree (<= intermediate_degree) */
  double final_update_rate;     /* insertions / (n * intermediate_degree), last iteration */
  double seconds_seed;          /* upload + fp16 conversion + random bucketing */
  double seconds_descent;       /* all nn-descent iterations */
  double seconds_prune;         /* detour pruning + reverse edges + copy-out */
  double seconds_total;
  double join_ms;               /* summed local-join kernel time (HIP events) */
  double join_bytes;            /* rows gathered by the local joins x 2*dp (fp16 row bytes) */
  uint64_t join_members;        /* rows gathered by the local joins */
  uint64_t updates_emitted;     /* candidate neighbours the joins appended to update bins */
  uint64_t updates_kept;        /* bin entries left after deduplication against the lists */
  uint64_t insertions;          /* entries that entered a list */
  double seconds_rescore;       /* exact fp32 re-score of the final lists (cvs_cagra_build_ex), else 0 */
} cvs_build_stats;

/* Builds a fixed-degree search graph of an n x d fp32 dataset on the GPU:
 * random bucketing seeds a degree-`intermediate_degree` kNN list per row,
 * nn-descent refines it (at most `max_iterations` iterations; stops early
 * when insertions / (n * intermediate_degree) < termination_threshold), and
 * rank-based detour pruning keeps `graph_degree` (clamped to n - 1) of its
 * entries, in list order (cvs_cagra_build_ex offers the plain k-NN graph and
 * pruning with reverse edges instead).  Writes n x min(graph_degree, n - 1) uint32 ids to
 * out_graph (host memory, or device memory if graph_on_device = 1); rows
 * with fewer neighbours end in UINT32_MAX.  `seed` drives the bucketing
 * permutation.  Replaces MetalContext::build_knn_graph
 * (metal_context.hpp:47-55; src/metal_context.mm:289-914). */
int cvs_cagra_build(cvs_context* ctx, const float* rows, int64_t n, int64_t d, int rows_on_device,
                    uint32_t intermediate_degree, uint32_t graph_degree, uint32_t max_iterations,
                    float termination_threshold, uint64_t seed, uint32_t* out_graph, int graph_on_device,
                    cvs_build_stats* stats);

/* How the build turns each node's intermediate list into its graph row
 * (cvs_build_options.graph_mode). */
#define CVS_GRAPH_DETOUR 0 /* CAGRA's rank-based detour pruning (the default of cvs_cagra_build) */
#define CVS_GRAPH_KNN 1    /* the first graph_degree entries: the k-NN graph, the reference's graph */

/* Options of cvs_cagra_build_ex. */
typedef struct cvs_build_options {
  /* 1: before pruning, re-score every node's intermediate list with exact
   * fp32 squared L2 distances from the fp32 rows and re-sort it, so that the
   * rank-based pruning orders neighbours as the reference's fp32 build does
   * (src/metal_context.mm:289-914 ranks by BLAS fp32 distances); 0: rank by
   * the build's fp16-input estimates, as cvs_cagra_build does.  Reads
   * n * intermediate_degree fp32 rows once more. */
  int rescore_fp32;
  /* Optional device memory of n x min(max(intermediate_degree, graph_degree),
   * n - 1) uint32: receives each node's final intermediate list (the one the
   * pruning reads), nearest first, UINT32_MAX-padded.  NULL: not written. */
  uint32_t* intermediate_out;
  /* CVS_GRAPH_DETOUR (0, as cvs_cagra_build) or CVS_GRAPH_KNN. */
  int graph_mode;
  /* CVS_GRAPH_DETOUR only: the last reverse_edges kept edges of each row
   * give way to reverse edges (nodes that kept this one), as in
   * cvs_cagra_optimize; 0 (as cvs_cagra_build): none.  CAGRA's graph uses
   * graph_degree / 2.  Measured recall@10 of the graph search at itopk 64:
   * on clustered N=1M D=1024 rows (degree 128 -> 64) 0.806 with 0, 0.799
   * with 4, 0.705 with 32; on 3,000 rows in 20 far-apart 4-dimensional
   * patches (degree 64 -> 32) the queries left at zero recall fell from 7-18
   * of 300 with 0 to 1-13 with 4.  Reverse edges help where nodes few
   * others point to are hard to reach; on high-dimensional rows they cost
   * recall at small search beams. */
  uint32_t reverse_edges;
} cvs_build_options;

/* cvs_cagra_build with options (NULL: those of cvs_cagra_build).  No
 * counterpart in the reference, whose build has no such knob; it serves
 * callers that want the exact-distance ranking at a known cost. */
int cvs_cagra_build_ex(cvs_context* ctx, const float* rows, int64_t n, int64_t d, int rows_on_device,
                       uint32_t intermediate_degree, uint32_t graph_degree, uint32_t max_iterations,
                       float termination_threshold, uint64_t seed, const cvs_build_options* options,
                       uint32_t* out_graph, int graph_on_device, cvs_build_stats* stats);

/* Prunes caller-supplied k-NN lists (n x knn_degree uint32 ids per row,
 * nearest first; host memory, or device memory if knn_on_device = 1) into a
 * search graph with the build's rank-based detour pruning (CAGRA, Ootomo et
 * al. 2023): each node keeps the graph_degree edges of fewest detours, in
 * rank order.  With reverse_edges = r > 0 (r <= graph_degree) the row is
 * then the closest graph_degree - r kept edges, up to r reverse edges (nodes
 * that kept this one), then the remaining kept edges (CAGRA's graph uses
 * r = graph_degree / 2).  Ids >= n, a row's own id and repeated ids are
 * ignored.  knn_degree <= 256, graph_degree <= knn_degree.  Writes n x
 * graph_degree ids to out_graph (host, or device if graph_on_device = 1);
 * rows with fewer neighbours end in UINT32_MAX.  The reference has no such
 * entry point (its build keeps its k-NN lists as the graph,
 * src/cagra.cpp:47-60, and include/cuvs/neighbors/cagra.hpp declares no
 * cagra::optimize); it serves callers that hold k-NN lists of their own,
 * exact ones from cvs_bf_search included. */
int cvs_cagra_optimize(cvs_context* ctx, const uint32_t* knn_graph, int64_t n, uint32_t knn_degree,
                       int knn_on_device, uint32_t graph_degree, uint32_t reverse_edges, uint32_t* out_graph,
                       int graph_on_device);

/* Phase timings and counters of one cvs_cagra_build_reference call. */
typedef struct cvs_ref_build_stats {
  uint32_t graph_degree;          /* output degree (<= n - 1) */
  uint32_t clusters;              /* k-means centres (0 on the exact path) */
  uint32_t kmeans_iterations;     /* Lloyd iterations run (<= 20) */
  uint32_t descent_iterations;    /* 2-hop nn-descent iterations run (<= 5) */
  uint32_t descent_changed_nodes; /* nodes whose list changed in the last iteration */
  double seconds_kmeans;
  double seconds_seed;            /* exact or per-cluster seeding + random bucketing */
  double seconds_descent;
  double seconds_total;
  uint32_t pq_iterations;         /* product-quantisation k-means iterations, all subspaces (PQ path) */
  double seconds_pq;              /* product-quantisation training and encoding (PQ path) */
} cvs_ref_build_stats;

/* The reference's own graph build on the GPU: for n <= 50,000 the exact
 * degree-G kNN graph (src/metal_context.mm:324-349); above, IVF k-means
 * seeding with per-cluster neighbours over the own and 3 nearest clusters
 * (:351-435, :576-611, :712-792), one random bucketing round (:795-851) and
 * at most 5 nn-descent iterations over 2-hop neighbours (:853-911); for
 * n > 200,000 the per-cluster neighbours are ranked by product-quantisation
 * distance (8 x 128-dimension subspaces, 256 centres; :437-568, :614-681)
 * and re-scored exactly (:683-709), with no nn-descent (src/cagra.cpp:59);
 * this needs d = 1024.  G = min(graph_degree, n - 1) <= 64.  Lists never
 * repeat an id (the reference's may).  For graph-quality comparison with
 * cvs_cagra_build.  Output as cvs_cagra_build.  Replaces
 * MetalContext::build_knn_graph (metal_context.hpp:47-55) as called by
 * cagra::build (src/cagra.cpp:47-62). */
int cvs_cagra_build_reference(cvs_context* ctx, const float* rows, int64_t n, int64_t d, int rows_on_device,
                              uint32_t graph_degree, uint32_t* out_graph, int graph_on_device,
                              cvs_ref_build_stats* stats);

/* cvs_cagra_build_reference with the size limits of its phases as
 * arguments: exact seeding for n <= exact_limit, product-quantised seeding
 * for n > max(exact_limit, pq_limit), IVF seeding with exact distances
 * between them (the reference's limits: 50,000 and 200,000,
 * src/metal_context.mm:297, :438; src/cagra.cpp:59).  Lets tests run the
 * reference's large-N phases at small n; cvs_cagra_build_reference is this
 * call with the reference's limits. */
int cvs_cagra_build_reference_ex(cvs_context* ctx, const float* rows, int64_t n, int64_t d, int rows_on_device,
                                 uint32_t graph_degree, int64_t exact_limit, int64_t pq_limit, uint32_t* out_graph,
                                 int graph_on_device, cvs_ref_build_stats* stats);

#ifdef __cplusplus
}
#endif

#endif /* CVS_HIP_H */
