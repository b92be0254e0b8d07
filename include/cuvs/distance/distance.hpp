// Distance metric selector of the cuVS-style API
// (reference: include/cuvs/distance/distance.hpp:5-8).
#pragma once

namespace cuvs::distance {

enum class DistanceType {
  L2Expanded,
  InnerProduct,
};

}  // namespace cuvs::distance
