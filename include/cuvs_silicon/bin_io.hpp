// Row-matrix ".bin" files of the Cohere Wikipedia benchmark data: an int32
// row count, an int32 column count, then rows*cols values row-major
// (float32 for base vectors and queries, int32 for ground-truth ids),
// little-endian, nothing after the payload.
//
// The writer side is the reference's scripts/download_cohere_wiki.py:57-71
// (save_float32_bin / save_int32_bin); the reader is the static load_bin<T>
// of its harness tests/test_cohere_wiki_validation.cpp:40-52.  Those are not
// part of the reference's library, so this header is an addition: the same
// format and the same errors ("Cannot open: <path>", "Truncated file:
// <path>", both std::runtime_error), plus a rejection of negative shapes,
// which the harness's reader would turn into an allocation failure.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace cuvs_silicon {

// Reads a whole .bin file; rows and cols receive its header.  T is float,
// std::int32_t or std::uint32_t (the payload bytes are taken as they are).
template <typename T>
std::vector<T> load_bin(const std::string& path, std::int32_t& rows, std::int32_t& cols);

// Writes rows x cols values in the same format; throws std::runtime_error
// ("Cannot open: <path>", "Write failed: <path>").
template <typename T>
void save_bin(const std::string& path, const T* values, std::int32_t rows, std::int32_t cols);

}  // namespace cuvs_silicon
