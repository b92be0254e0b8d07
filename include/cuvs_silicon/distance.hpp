// Scalar squared L2 distance of two 128-dimensional vectors, the reference's
// public helper (reference include/cuvs_silicon/distance.hpp:5,
// src/distance.cpp:8-20): the 128 squared differences summed in dimension
// order in fp32; throws std::invalid_argument for a null vector.  A host
// function of libcuvs_silicon (cuvs-silicon_amd/src/distance.cpp).
#pragma once

namespace cuvs_silicon {

float squared_l2_distance_128(const float* lhs, const float* rhs);

}  // namespace cuvs_silicon
