// tensor.hpp — the minimal tensor type the C++ host layer needs.
//
// The reference's API takes candle_core::Tensor; this build's C++ host layer
// uses this small stand-in: a dtype, dims, strides and an element offset over a
// reference-counted buffer that lives in host memory or in HIP device memory
// (allocated through the C ABI, include/cmk_iq2.h).  Only what the IQ2 ops and
// their tests use is provided: construction from host data, zeros/empty,
// reshape, squeeze, narrow (offset views), transpose views, contiguous(), and
// copies between host and device.
#pragma once
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace candelora {

// candle_core::Error stand-in: every failure carries the reference's message.
class Error : public std::runtime_error {
 public:
  explicit Error(const std::string& msg) : std::runtime_error(msg) {}
};

enum class DType { U8, F16, BF16, F32, I64 };
size_t dtype_size(DType d);
const char* dtype_name(DType d);  // candle's Debug names: "U8", "F16", ...

struct Device {
  enum class Kind { Cpu, Hip };
  Kind kind = Kind::Cpu;
  int ordinal = 0;
  static Device cpu() { return Device{Kind::Cpu, 0}; }
  static Device hip(int ordinal = 0) { return Device{Kind::Hip, ordinal}; }
  bool is_hip() const { return kind == Kind::Hip; }
  bool same_device(const Device& o) const { return kind == o.kind && ordinal == o.ordinal; }
  std::string to_string() const;
};

class Tensor {
 public:
  Tensor() = default;

  // Copies `bytes` of host data into a new contiguous tensor on `dev`.
  static Tensor from_host(const void* data, size_t bytes, DType dt, std::vector<size_t> dims,
                          const Device& dev);
  template <class T>
  static Tensor from_vec(const std::vector<T>& v, std::vector<size_t> dims, DType dt,
                         const Device& dev) {
    return from_host(v.data(), v.size() * sizeof(T), dt, std::move(dims), dev);
  }
  static Tensor empty(std::vector<size_t> dims, DType dt, const Device& dev);
  static Tensor zeros(std::vector<size_t> dims, DType dt, const Device& dev);

  const std::vector<size_t>& dims() const { return dims_; }
  size_t rank() const { return dims_.size(); }
  size_t elem_count() const;
  DType dtype() const { return dtype_; }
  const Device& device() const { return device_; }
  size_t start_offset() const { return offset_; }  // in elements
  bool is_contiguous() const;

  // Views (share storage).
  Tensor reshape(std::vector<size_t> dims) const;  // needs a contiguous tensor
  Tensor squeeze(size_t dim) const;
  Tensor narrow(size_t dim, size_t start, size_t len) const;
  Tensor t() const;  // rank-2 transpose view (non-contiguous)

  Tensor contiguous() const;              // copy when not contiguous
  Tensor to_device(const Device& dev) const;
  std::vector<uint8_t> to_bytes() const;  // contiguous host image of the elements
  template <class T>
  std::vector<T> to_vec() const {
    std::vector<uint8_t> b = to_bytes();
    std::vector<T> out(b.size() / sizeof(T));
    if (!b.empty()) std::memcpy(out.data(), b.data(), b.size());
    return out;
  }

  // Address of element 0 (storage base + start_offset).
  const void* data_ptr() const;
  void* data_ptr_mut();

 private:
  struct Storage;
  std::shared_ptr<Storage> st_;
  DType dtype_ = DType::U8;
  std::vector<size_t> dims_, strides_;
  size_t offset_ = 0;
  Device device_;
};

}  // namespace candelora
