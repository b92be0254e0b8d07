// SIFT-style vector files (.fvecs / .ivecs): each row is an int32 count
// followed by that many float32 (fvecs) or int32 (ivecs) values, little-endian.
//
// Same declarations, argument meanings and error behaviour as the
// reference's include/cuvs_silicon/sift_loader.hpp:9-69 (implementation
// src/sift_loader.cpp:21-214): every mismatch throws SiftLoadError, whose
// message names the failed check.  The files are memory-mapped and the rows
// copied by several threads; a dataset loaded here is handed to
// cuvs::neighbors::cagra::build or brute_force::build as a host matrix.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace cuvs_silicon {

// SIFT-1M (ANN_SIFT1M: sift_base / sift_query / sift_groundtruth).
constexpr std::size_t kSift1MBaseVectorCount = 1'000'000;
constexpr std::size_t kSift1MQueryVectorCount = 10'000;
constexpr std::size_t kSift1MVectorDimension = 128;
constexpr std::size_t kSift1MGroundTruthNeighborCount = 100;

class SiftLoadError : public std::runtime_error {
 public:
  explicit SiftLoadError(const std::string& message);
};

// rows x cols float32 matrix, row-major and contiguous.
struct FloatVectorDataset {
  std::size_t rows = 0;
  std::size_t cols = 0;
  std::vector<float> values;
};

// query_count x neighbor_count row ids, row-major.
struct GroundTruthDataset {
  std::size_t query_count = 0;
  std::size_t neighbor_count = 0;
  std::vector<std::uint32_t> neighbors;
};

struct SiftDataset {
  FloatVectorDataset base;
  FloatVectorDataset queries;
  GroundTruthDataset groundtruth;
};

// Reads exactly expected_rows rows of expected_cols floats; a row header other
// than expected_cols, a short file or bytes after the last row are errors.
FloatVectorDataset load_fvecs(const std::string& path, std::size_t expected_rows,
                              std::size_t expected_cols);

// Checks the row headers and the file length of an fvecs file without
// reading its payload.
void validate_fvecs_shape(const std::string& path, std::size_t expected_rows,
                          std::size_t expected_cols);

// As load_fvecs for int32 rows; a negative id is an error.
GroundTruthDataset load_ivecs(const std::string& path, std::size_t expected_rows,
                              std::size_t expected_cols);

// Loads base, queries and ground truth and checks that they fit together
// (ground-truth ids below the base row count).
SiftDataset load_sift_dataset(const std::string& base_path, const std::string& query_path,
                              const std::string& groundtruth_path, std::size_t expected_base_rows,
                              std::size_t expected_query_rows, std::size_t expected_cols,
                              std::size_t expected_groundtruth_cols);

FloatVectorDataset load_sift1m_base(const std::string& path);
void validate_sift1m_base_shape(const std::string& path);
FloatVectorDataset load_sift1m_queries(const std::string& path);
GroundTruthDataset load_sift1m_groundtruth(const std::string& path);
SiftDataset load_sift1m_dataset(const std::string& base_path, const std::string& query_path,
                                const std::string& groundtruth_path);

}  // namespace cuvs_silicon
