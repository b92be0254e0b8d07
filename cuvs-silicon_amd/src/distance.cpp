// cuvs_silicon::squared_l2_distance_128 (reference src/distance.cpp:8-20):
// same summation order and the same exception for null input, so the
// reference's known answers (tests/test_l2_distance.cpp:19-49) hold.
#include <cuvs_silicon/distance.hpp>

#include <stdexcept>

namespace cuvs_silicon {

float squared_l2_distance_128(const float* lhs, const float* rhs) {
  if (!lhs || !rhs) throw std::invalid_argument("squared_l2_distance_128 needs two non-null vectors");
  float sum = 0.0f;
  for (int i = 0; i < 128; ++i) {
    const float diff = lhs[i] - rhs[i];
    sum += diff * diff;
  }
  return sum;
}

}  // namespace cuvs_silicon
