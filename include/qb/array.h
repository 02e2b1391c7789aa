// qb::array: the array type of the C++ adapters. A dense, row-major array in HIP device memory, reference-counted
// like the reference's mx::array (copies share the buffer) and never written by the functions that take it.
// Unlike mx::array it is not lazy: operations are queued on qb::stream() at once and results are ready when that
// stream reaches them.
#pragma once
#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

namespace qb {

enum class Dtype : int { float32 = 0, bfloat16 = 1 };  // the values of qb_dtype
constexpr Dtype float32 = Dtype::float32;
constexpr Dtype bfloat16 = Dtype::bfloat16;
size_t size_of(Dtype dtype);

using Shape = std::vector<int>;

class array {
 public:
  array() = default;
  // An uninitialised device buffer of this shape.
  array(Shape shape, Dtype dtype);
  // A copy of host data (element type as dtype; bfloat16 as its 16-bit pattern). Waits until the copy is done.
  static array from_host(const void* data, Shape shape, Dtype dtype);
  static array zeros(Shape shape, Dtype dtype);

  // Copies the contents to host memory, after the work queued on qb::stream() before this call.
  void to_host(void* dst) const;

  const Shape& shape() const { return shape_; }
  int shape(int dim) const;  // a negative dim counts from the end, as in mx::array::shape
  int ndim() const { return int(shape_.size()); }
  size_t size() const;
  size_t nbytes() const { return size() * size_of(dtype_); }
  Dtype dtype() const { return dtype_; }
  bool empty() const { return !buf_; }
  void* data() { return buf_.get(); }
  const void* data() const { return buf_.get(); }

 private:
  std::shared_ptr<void> buf_;
  Shape shape_;
  Dtype dtype_ = Dtype::float32;
};

// x in another dtype (float32 <-> bfloat16, round to nearest even); x itself when it already has it.
array astype(const array& x, Dtype dtype);

// The hipStream_t every adapter call queues its work on; nullptr (the default) is the null stream.
void set_stream(void* stream);
void* stream();

}  // namespace qb
