/* Counter-based synthetic clustered data (see synth.h). */
#include "synth.h"

#include <math.h>
#include <stdlib.h>

static uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ULL;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

static uint64_t key4(uint64_t seed, uint32_t stream, uint64_t a, uint64_t b) {
  uint64_t h = mix64(seed ^ (0xd1b54a32d192ed03ULL * ((uint64_t)stream + 1)));
  h = mix64(h ^ a);
  return mix64(h ^ (b * 0x8cb92ba72f3d8dd7ULL));
}

/* Uniform in (0, 1]. */
static double unit(uint64_t h) { return ((double)(h >> 11) + 1.0) * (1.0 / 9007199254740992.0); }

double cvs_synth_normal(uint64_t seed, uint32_t stream, uint64_t row, uint64_t col) {
  const uint64_t pair = col >> 1;
  const double u1 = unit(key4(seed, stream, row, 2 * pair));
  const double u2 = unit(key4(seed, stream, row, 2 * pair + 1));
  const double r = sqrt(-2.0 * log(u1));
  const double a = 6.283185307179586476925286766559 * u2;
  return (col & 1) ? r * sin(a) : r * cos(a);
}

#define STREAM_CENTRES 0u
#define CHOICE_COLUMN 0xffffffffffffffffULL

void cvs_synth_clustered(uint64_t seed, uint32_t stream, int64_t row0, int64_t n, int64_t d,
                         int n_centers, double sigma, float* out) {
  if (n <= 0 || d <= 0 || n_centers <= 0 || !out) return;
  double* centres = (double*)malloc(sizeof(double) * (size_t)n_centers * (size_t)d);
  if (!centres) return;
  for (int c = 0; c < n_centers; ++c)
    for (int64_t i = 0; i < d; ++i)
      centres[(size_t)c * d + i] = cvs_synth_normal(seed, STREAM_CENTRES, (uint64_t)c, (uint64_t)i);
#pragma omp parallel
  {
    double* v = (double*)malloc(sizeof(double) * (size_t)d);
#pragma omp for schedule(static)
    for (int64_t r = 0; r < n; ++r) {
      const uint64_t row = (uint64_t)(row0 + r);
      const int c = (int)(key4(seed, stream, row, CHOICE_COLUMN) % (uint64_t)n_centers);
      const double* ctr = centres + (size_t)c * d;
      double ss = 0.0;
      for (int64_t i = 0; i < d; ++i) {
        v[i] = ctr[i] + sigma * cvs_synth_normal(seed, stream, row, (uint64_t)i);
        ss += v[i] * v[i];
      }
      const double inv = ss > 0.0 ? 1.0 / sqrt(ss) : 0.0;
      float* dst = out + (size_t)r * d;
      for (int64_t i = 0; i < d; ++i) dst[i] = (float)(v[i] * inv);
    }
    free(v);
  }
  free(centres);
}
