// Minimal RAFT surface used by the cuVS-style API
// (reference: include/raft/core/resources.hpp:8-45).
//
// `resources` carries no stream: every search/build call is synchronous.
// `device_matrix_view` is a non-owning (pointer, rows, cols) row-major view.
// As in the reference, the pointers handed to build()/search() are HOST
// pointers; the library copies them to the GPU itself.
#pragma once

#include <cstddef>
#include <cstdint>

namespace raft {

class resources {
 public:
  resources() = default;
  void sync_stream() const {}
};

template <typename ElementType, typename IndexType = std::int64_t>
class device_matrix_view {
 public:
  using element_type = ElementType;
  using index_type = IndexType;

  constexpr device_matrix_view(ElementType* data, IndexType rows, IndexType cols) noexcept
      : ptr_(data), extents_{rows, cols} {}

  constexpr ElementType* data_handle() const noexcept { return ptr_; }
  constexpr ElementType* data() const noexcept { return ptr_; }
  constexpr IndexType extent(std::size_t axis) const noexcept {
    return axis == 0 ? extents_[0] : extents_[1];
  }
  constexpr IndexType size() const noexcept { return extents_[0] * extents_[1]; }

 private:
  ElementType* ptr_;
  IndexType extents_[2];
};

template <typename ElementType, typename IndexType>
constexpr device_matrix_view<ElementType, IndexType> make_device_matrix_view(
    ElementType* data, IndexType rows, IndexType cols) noexcept {
  return device_matrix_view<ElementType, IndexType>(data, rows, cols);
}

}  // namespace raft
