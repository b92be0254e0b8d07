// fvecs / ivecs loaders with the interface and error behaviour of the
// reference's src/sift_loader.cpp:21-214.
//
// The reference streams a row at a time through an ifstream.  Here the file
// is mapped once; threads take contiguous row ranges, check each row's header
// (and, for ivecs, its ids) and copy its payload into the output.  Each thread
// stops at its first bad row, and the error reported is that of the lowest
// bad row, which is the one the reference's sequential reader meets first, so
// every file gets the same error as from the reference.  The exception is
// validate_fvecs_shape, which also requires the last row's payload to be
// present (the reference's reader seeks past it without checking).
#include <cuvs_silicon/sift_loader.hpp>

#include <algorithm>
#include <limits>

#include "file_map.hpp"

namespace cuvs_silicon {

SiftLoadError::SiftLoadError(const std::string& message) : std::runtime_error(message) {}

namespace {

using detail::MappedFile;

std::size_t checked_product(std::size_t a, std::size_t b) {
  if (b != 0 && a > std::numeric_limits<std::size_t>::max() / b)
    throw SiftLoadError("SIFT dataset shape overflows size_t");
  return a * b;
}

enum class RowFault { kNone, kHeaderMissing, kWrongWidth, kPayloadMissing, kNegative, kTrailing };

struct Fault {
  std::size_t row = std::numeric_limits<std::size_t>::max();
  RowFault what = RowFault::kNone;
};

// Walks `rows` records of (int32 count, cols x 4-byte values).  kIds: the
// values are ids that must be non-negative.  dst (may be null) receives the
// payloads, row-major.  Returns the first bad row.
template <bool kIds>
Fault scan_records(const MappedFile& file, std::size_t rows, std::size_t cols, void* dst) {
  const std::size_t payload = checked_product(cols, 4);
  if (payload > std::numeric_limits<std::size_t>::max() - 4) throw SiftLoadError("SIFT dataset shape overflows size_t");
  const std::size_t stride = payload + 4;
  const std::size_t size = file.size();
  const unsigned char* base = file.data();
  const unsigned threads = detail::copy_threads(rows, stride);
  std::vector<Fault> faults(threads);
  detail::parallel_ranges(rows, threads, [&](std::size_t b, std::size_t e, unsigned t) {
    for (std::size_t r = b; r < e; ++r) {
      Fault f;
      f.row = r;
      // Record r starts at r * stride when every earlier record is whole.
      if (r > size / stride || size - r * stride < 4) {
        f.what = RowFault::kHeaderMissing;
      } else {
        const std::size_t off = r * stride;
        const std::int32_t count = detail::read_i32(base + off);
        const std::size_t avail = size - off - 4;
        if (count < 0 || static_cast<std::size_t>(count) != cols) {
          f.what = RowFault::kWrongWidth;
        } else {
          if constexpr (kIds) {
            const std::size_t present = std::min(cols, avail / 4);
            for (std::size_t j = 0; j < present; ++j) {
              if (detail::read_i32(base + off + 4 + 4 * j) < 0) {
                f.what = RowFault::kNegative;
                break;
              }
            }
          }
          if (f.what == RowFault::kNone && avail < payload) f.what = RowFault::kPayloadMissing;
          if (f.what == RowFault::kNone && dst != nullptr && payload != 0)
            std::memcpy(static_cast<unsigned char*>(dst) + r * payload, base + off + 4, payload);
        }
      }
      if (f.what != RowFault::kNone) {
        faults[t] = f;
        return;
      }
    }
  });
  Fault first;
  for (const Fault& f : faults)
    if (f.what != RowFault::kNone && f.row < first.row) first = f;
  if (first.what == RowFault::kNone && size > rows * stride) {
    first.row = rows;
    first.what = RowFault::kTrailing;
  }
  return first;
}

void raise_fvecs(const Fault& f) {
  switch (f.what) {
    case RowFault::kNone: return;
    case RowFault::kTrailing: throw SiftLoadError("fvecs file has extra trailing bytes");
    case RowFault::kHeaderMissing: throw SiftLoadError("fvecs file ended before row dimension header");
    case RowFault::kWrongWidth: throw SiftLoadError("fvecs row dimension does not match expected width");
    default: throw SiftLoadError("fvecs file ended before row vector payload");
  }
}

void raise_ivecs(const Fault& f) {
  switch (f.what) {
    case RowFault::kNone: return;
    case RowFault::kTrailing: throw SiftLoadError("ivecs file has extra trailing bytes");
    case RowFault::kHeaderMissing: throw SiftLoadError("ivecs file ended before row neighbor-count header");
    case RowFault::kWrongWidth: throw SiftLoadError("ivecs row neighbor count does not match expected width");
    case RowFault::kNegative: throw SiftLoadError("ivecs neighbor index must be non-negative");
    default: throw SiftLoadError("ivecs file ended before row neighbor payload");
  }
}

void map_or_throw(MappedFile& file, const std::string& path, const char* kind) {
  if (!file.open(path)) throw SiftLoadError(std::string("failed to open ") + kind + " file: " + path);
}

}  // namespace

FloatVectorDataset load_fvecs(const std::string& path, std::size_t expected_rows, std::size_t expected_cols) {
  MappedFile file;
  map_or_throw(file, path, "fvecs");
  const std::size_t count = checked_product(expected_rows, expected_cols);
  // The headers are checked before the output is allocated, so that a file
  // with far fewer rows than expected fails without a large allocation.
  raise_fvecs(scan_records<false>(file, expected_rows, expected_cols, nullptr));
  FloatVectorDataset out;
  out.rows = expected_rows;
  out.cols = expected_cols;
  out.values.resize(count);
  raise_fvecs(scan_records<false>(file, expected_rows, expected_cols, out.values.data()));
  return out;
}

void validate_fvecs_shape(const std::string& path, std::size_t expected_rows, std::size_t expected_cols) {
  MappedFile file;
  map_or_throw(file, path, "fvecs");
  (void)checked_product(expected_rows, expected_cols);
  raise_fvecs(scan_records<false>(file, expected_rows, expected_cols, nullptr));
}

GroundTruthDataset load_ivecs(const std::string& path, std::size_t expected_rows, std::size_t expected_cols) {
  MappedFile file;
  map_or_throw(file, path, "ivecs");
  const std::size_t count = checked_product(expected_rows, expected_cols);
  raise_ivecs(scan_records<true>(file, expected_rows, expected_cols, nullptr));
  GroundTruthDataset out;
  out.query_count = expected_rows;
  out.neighbor_count = expected_cols;
  out.neighbors.resize(count);
  raise_ivecs(scan_records<true>(file, expected_rows, expected_cols, out.neighbors.data()));
  return out;
}

SiftDataset load_sift_dataset(const std::string& base_path, const std::string& query_path,
                              const std::string& groundtruth_path, std::size_t expected_base_rows,
                              std::size_t expected_query_rows, std::size_t expected_cols,
                              std::size_t expected_groundtruth_cols) {
  SiftDataset ds;
  ds.base = load_fvecs(base_path, expected_base_rows, expected_cols);
  ds.queries = load_fvecs(query_path, expected_query_rows, expected_cols);
  ds.groundtruth = load_ivecs(groundtruth_path, expected_query_rows, expected_groundtruth_cols);
  if (ds.base.cols != ds.queries.cols) throw SiftLoadError("SIFT base and query dimensions are incompatible");
  if (ds.groundtruth.query_count != ds.queries.rows)
    throw SiftLoadError("SIFT ground-truth query count is incompatible with queries");
  const auto bad = std::find_if(ds.groundtruth.neighbors.begin(), ds.groundtruth.neighbors.end(),
                                [&](std::uint32_t id) { return id >= ds.base.rows; });
  if (bad != ds.groundtruth.neighbors.end())
    throw SiftLoadError("SIFT ground-truth neighbor is outside base rows");
  return ds;
}

FloatVectorDataset load_sift1m_base(const std::string& path) {
  return load_fvecs(path, kSift1MBaseVectorCount, kSift1MVectorDimension);
}

void validate_sift1m_base_shape(const std::string& path) {
  validate_fvecs_shape(path, kSift1MBaseVectorCount, kSift1MVectorDimension);
}

FloatVectorDataset load_sift1m_queries(const std::string& path) {
  return load_fvecs(path, kSift1MQueryVectorCount, kSift1MVectorDimension);
}

GroundTruthDataset load_sift1m_groundtruth(const std::string& path) {
  return load_ivecs(path, kSift1MQueryVectorCount, kSift1MGroundTruthNeighborCount);
}

SiftDataset load_sift1m_dataset(const std::string& base_path, const std::string& query_path,
                                const std::string& groundtruth_path) {
  return load_sift_dataset(base_path, query_path, groundtruth_path, kSift1MBaseVectorCount,
                           kSift1MQueryVectorCount, kSift1MVectorDimension, kSift1MGroundTruthNeighborCount);
}

}  // namespace cuvs_silicon
