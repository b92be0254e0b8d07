/* Synthetic clustered vectors for benchmarks and tests.
 *
 * Distribution: `n_centers` centres drawn i.i.d. N(0, I_d); each row is a
 * uniformly chosen centre plus N(0, sigma^2 I_d) noise, then L2-normalised.
 * Every value is a pure function of (seed, stream, row, column) through a
 * counter-based generator (splitmix64 finaliser + Box-Muller in double), so
 * any row range can be generated independently, in parallel, and identically
 * on every run.  Use distinct `stream` values for base vectors and queries;
 * the centres depend on the seed only. */
#ifndef CVS_SYNTH_H
#define CVS_SYNTH_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define CVS_SYNTH_STREAM_BASE 1u
#define CVS_SYNTH_STREAM_QUERIES 2u

/* Writes rows [row0, row0 + n) of the stream into out (n x d, row-major). */
void cvs_synth_clustered(uint64_t seed, uint32_t stream, int64_t row0, int64_t n, int64_t d,
                         int n_centers, double sigma, float* out);

/* Standard normal value for (seed, stream, row, col) (exposed for tests). */
double cvs_synth_normal(uint64_t seed, uint32_t stream, uint64_t row, uint64_t col);

#ifdef __cplusplus
}
#endif
#endif
