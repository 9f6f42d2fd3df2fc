// iq2_matmul.cpp — C++ host layer over the C ABI (libcmk_iq2.so).
//
// Mirrors the reference's host dispatch for the IQ2 ops: argument checks in the
// order and with the texts of iq2_matmul_metal / iq2_dequantize_to_f16_metal
// (src/iq2_matmul.rs:197-505) and parse_x_shape (:170-195), the activation-mode
// dispatch of iq2_matmul_with_activation_quant (:559-591), then one call into
// cmk_iq2_matmul / cmk_iq2_dequantize.  The C ABI repeats the size checks on
// the raw buffers, with the same texts, for callers that bind it directly.
#include "candelora/iq2_matmul.hpp"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <sstream>

#include "cmk_iq2.h"

namespace candelora {

// ---------------------------------------------------------------- dtype / device

size_t dtype_size(DType d) {
  switch (d) {
    case DType::U8: return 1;
    case DType::F16:
    case DType::BF16: return 2;
    case DType::F32: return 4;
    default: return 8;
  }
}

const char* dtype_name(DType d) {
  switch (d) {
    case DType::U8: return "U8";
    case DType::F16: return "F16";
    case DType::BF16: return "BF16";
    case DType::F32: return "F32";
    default: return "I64";
  }
}

std::string Device::to_string() const {
  return is_hip() ? "Hip(" + std::to_string(ordinal) + ")" : std::string("Cpu");
}

namespace {

[[noreturn]] void bail(const std::string& msg) { throw Error(msg); }

void check_abi(int rc) {
  if (rc != CMK_OK) bail(cmk_last_error());
}

}  // namespace

// ---------------------------------------------------------------- storage

struct Tensor::Storage {
  void* ptr = nullptr;
  size_t bytes = 0;
  Device dev;
  ~Storage() {
    if (!ptr) return;
    if (dev.is_hip())
      cmk_free(ptr);
    else
      std::free(ptr);
  }
};

static std::vector<size_t> row_major_strides(const std::vector<size_t>& dims) {
  std::vector<size_t> s(dims.size(), 1);
  for (size_t i = dims.size(); i-- > 1;) s[i - 1] = s[i] * dims[i];
  return s;
}

Tensor Tensor::empty(std::vector<size_t> dims, DType dt, const Device& dev) {
  Tensor t;
  t.dtype_ = dt;
  t.dims_ = std::move(dims);
  t.strides_ = row_major_strides(t.dims_);
  t.device_ = dev;
  t.st_ = std::make_shared<Storage>();
  t.st_->dev = dev;
  t.st_->bytes = t.elem_count() * dtype_size(dt);
  const size_t alloc = t.st_->bytes ? t.st_->bytes : 1;
  if (dev.is_hip()) {
    check_abi(cmk_set_device(dev.ordinal));
    check_abi(cmk_malloc(&t.st_->ptr, alloc));
  } else {
    t.st_->ptr = std::malloc(alloc);
    if (!t.st_->ptr) bail("host allocation failed");
  }
  return t;
}

Tensor Tensor::zeros(std::vector<size_t> dims, DType dt, const Device& dev) {
  Tensor t = empty(std::move(dims), dt, dev);
  if (t.st_->bytes) {
    if (dev.is_hip()) {
      check_abi(cmk_memset(t.st_->ptr, 0, t.st_->bytes, nullptr));
      check_abi(cmk_stream_synchronize(nullptr));
    } else {
      std::memset(t.st_->ptr, 0, t.st_->bytes);
    }
  }
  return t;
}

Tensor Tensor::from_host(const void* data, size_t bytes, DType dt, std::vector<size_t> dims,
                         const Device& dev) {
  Tensor t = empty(std::move(dims), dt, dev);
  if (bytes != t.st_->bytes)
    bail("shape mismatch: " + std::to_string(bytes) + " bytes for " +
         std::to_string(t.elem_count()) + " elements of " + dtype_name(dt));
  if (bytes) {
    if (dev.is_hip()) {
      check_abi(cmk_memcpy_htod(t.st_->ptr, data, bytes, nullptr));
      check_abi(cmk_stream_synchronize(nullptr));
    } else {
      std::memcpy(t.st_->ptr, data, bytes);
    }
  }
  return t;
}

size_t Tensor::elem_count() const {
  size_t n = 1;
  for (size_t d : dims_) n *= d;
  return n;
}

bool Tensor::is_contiguous() const {
  size_t expect = 1;
  for (size_t i = dims_.size(); i-- > 0;) {
    if (dims_[i] != 1 && strides_[i] != expect) return false;
    expect *= dims_[i];
  }
  return true;
}

const void* Tensor::data_ptr() const {
  return static_cast<const char*>(st_->ptr) + offset_ * dtype_size(dtype_);
}

void* Tensor::data_ptr_mut() { return static_cast<char*>(st_->ptr) + offset_ * dtype_size(dtype_); }

Tensor Tensor::reshape(std::vector<size_t> dims) const {
  size_t n = 1;
  for (size_t d : dims) n *= d;
  if (n != elem_count()) bail("reshape: element count mismatch");
  if (!is_contiguous()) return contiguous().reshape(std::move(dims));
  Tensor t = *this;
  t.dims_ = std::move(dims);
  t.strides_ = row_major_strides(t.dims_);
  return t;
}

Tensor Tensor::squeeze(size_t dim) const {
  if (dim >= dims_.size() || dims_[dim] != 1) return *this;
  Tensor t = *this;
  t.dims_.erase(t.dims_.begin() + dim);
  t.strides_.erase(t.strides_.begin() + dim);
  return t;
}

Tensor Tensor::narrow(size_t dim, size_t start, size_t len) const {
  if (dim >= dims_.size() || start + len > dims_[dim]) bail("narrow: out of range");
  Tensor t = *this;
  t.offset_ += start * strides_[dim];
  t.dims_[dim] = len;
  return t;
}

Tensor Tensor::t() const {
  if (rank() != 2) bail("t() needs a rank-2 tensor");
  Tensor r = *this;
  std::swap(r.dims_[0], r.dims_[1]);
  std::swap(r.strides_[0], r.strides_[1]);
  return r;
}

std::vector<uint8_t> Tensor::to_bytes() const {
  const size_t es = dtype_size(dtype_);
  // Host image of the whole storage span this view touches.
  size_t span = 0;
  if (elem_count()) {
    span = 1;
    for (size_t i = 0; i < dims_.size(); ++i) span += (dims_[i] - 1) * strides_[i];
  }
  std::vector<uint8_t> raw(span * es);
  if (span) {
    if (device_.is_hip()) {
      check_abi(cmk_stream_synchronize(nullptr));
      check_abi(cmk_memcpy_dtoh(raw.data(), data_ptr(), raw.size(), nullptr));
      check_abi(cmk_stream_synchronize(nullptr));
    } else {
      std::memcpy(raw.data(), data_ptr(), raw.size());
    }
  }
  if (is_contiguous()) {
    raw.resize(elem_count() * es);
    return raw;
  }
  std::vector<uint8_t> out(elem_count() * es);
  std::vector<size_t> idx(dims_.size(), 0);
  for (size_t e = 0; e < elem_count(); ++e) {
    size_t off = 0;
    for (size_t i = 0; i < dims_.size(); ++i) off += idx[i] * strides_[i];
    std::memcpy(&out[e * es], &raw[off * es], es);
    for (size_t i = dims_.size(); i-- > 0;) {
      if (++idx[i] < dims_[i]) break;
      idx[i] = 0;
    }
  }
  return out;
}

Tensor Tensor::contiguous() const {
  if (is_contiguous()) return *this;
  std::vector<uint8_t> b = to_bytes();
  return from_host(b.data(), b.size(), dtype_, dims_, device_);
}

Tensor Tensor::to_device(const Device& dev) const {
  std::vector<uint8_t> b = to_bytes();
  return from_host(b.data(), b.size(), dtype_, dims_, dev);
}

void synchronize() { check_abi(cmk_stream_synchronize(nullptr)); }

// ---------------------------------------------------------------- ops

namespace {

cmk_iq2_variant to_abi(Iq2MatmulVariant v) {
  switch (v) {
    case Iq2MatmulVariant::Iq2Xxs: return CMK_IQ2_XXS;
    case Iq2MatmulVariant::Iq2Xs: return CMK_IQ2_XS;
    case Iq2MatmulVariant::Iq2S: return CMK_IQ2_S;
    default: return CMK_IQ3_S;
  }
}

std::string shape_str(const std::vector<size_t>& d) {
  std::ostringstream o;
  o << "[";
  for (size_t i = 0; i < d.size(); ++i) o << (i ? ", " : "") << d[i];
  o << "]";
  return o.str();
}

// parse_x_shape, src/iq2_matmul.rs:170-195.
Tensor parse_x_shape(const Tensor& x, size_t in_dim, size_t* m, bool* squeeze) {
  const auto& d = x.dims();
  if (d.size() == 1) {
    if (d[0] != in_dim)
      bail("iq2_matmul input mismatch: x dim=" + std::to_string(d[0]) +
           " expected in_dim=" + std::to_string(in_dim));
    *m = 1;
    *squeeze = true;
    return x.reshape({1, in_dim});
  }
  if (d.size() == 2) {
    if (d[1] != in_dim)
      bail("iq2_matmul input mismatch: x last dim=" + std::to_string(d[1]) +
           " expected in_dim=" + std::to_string(in_dim));
    *m = d[0];
    *squeeze = false;
    return x;
  }
  bail("iq2_matmul expects x rank 1 or 2, got shape " + shape_str(d));
}

// Bytes / scale bytes per 256-weight block of each format (src/iq2_matmul.rs:12-29).
size_t bytes_per_block(Iq2MatmulVariant v) {
  switch (v) {
    case Iq2MatmulVariant::Iq2Xxs:
    case Iq2MatmulVariant::Iq2Xs: return 64;
    case Iq2MatmulVariant::Iq2S: return 72;
    default: return 104;
  }
}

size_t scales_per_block(Iq2MatmulVariant v) {
  switch (v) {
    case Iq2MatmulVariant::Iq2Xxs: return 2;
    case Iq2MatmulVariant::Iq2Xs:
    case Iq2MatmulVariant::Iq2S: return 10;
    default: return 6;
  }
}

bool checked_mul(size_t a, size_t b, size_t* out) {
  if (a != 0 && b > SIZE_MAX / a) return false;
  *out = a * b;
  return true;
}

// Size checks of src/iq2_matmul.rs:237-259 (and :403-421 with prefix `op`).
void check_sizes(const char* op, const Tensor& weight_bytes, const Tensor& weight_scales,
                 size_t out_dim, size_t in_dim, Iq2MatmulVariant variant) {
  const size_t bpr = (in_dim + 255) / 256;
  size_t blocks, expected_bytes, expected_scales;
  if (!checked_mul(out_dim, bpr, &blocks) ||
      !checked_mul(blocks, bytes_per_block(variant), &expected_bytes))
    bail(std::string(op) + " bytes size overflow");
  if (!checked_mul(blocks, scales_per_block(variant), &expected_scales))
    bail(std::string(op) + " scales size overflow");
  if (weight_bytes.elem_count() < expected_bytes)
    bail(std::string(op) + " weight_bytes too small: got " +
         std::to_string(weight_bytes.elem_count()) + " expected at least " +
         std::to_string(expected_bytes));
  if (weight_scales.elem_count() < expected_scales)
    bail(std::string(op) + " weight_scales too small: got " +
         std::to_string(weight_scales.elem_count()) + " expected at least " +
         std::to_string(expected_scales));
}

// Device scratch of cmk_iq2_matmul, one buffer per device, kept between calls
// and replaced by a larger one only when a call needs more (freeing the old one
// waits for the device).  Every launch of this layer goes to the device's
// default stream, which runs them in order, so calls never overlap on the
// buffer; the mutex is held from the lookup until the launch is enqueued, so
// no thread replaces a buffer another thread is about to pass.  A steady
// stream of calls therefore neither allocates nor synchronises.
class WorkspaceCache {
 public:
  static constexpr int kMaxDevices = 64;
  std::mutex mu;

  // Caller holds mu.
  void* get(int ordinal, size_t bytes) {
    if (ordinal < 0 || ordinal >= kMaxDevices) bail("device ordinal out of range");
    Slot& s = slots_[ordinal];
    if (s.bytes < bytes) {
      check_abi(cmk_set_device(ordinal));
      if (s.ptr) check_abi(cmk_free(s.ptr));
      s.ptr = nullptr;
      s.bytes = 0;
      check_abi(cmk_malloc(&s.ptr, bytes));
      s.bytes = bytes;
    }
    return s.ptr;
  }

 private:
  struct Slot {
    void* ptr = nullptr;
    size_t bytes = 0;
  };
  Slot slots_[kMaxDevices];
};

WorkspaceCache& workspace_cache() {
  static WorkspaceCache* cache = new WorkspaceCache();  // lives until the process ends
  return *cache;
}

// The ROCm body of iq2_matmul_metal (src/iq2_matmul.rs:197-365), checks in the
// reference's order.
Tensor iq2_matmul_hip(const Tensor& x, const Tensor& weight_bytes, const Tensor& weight_scales,
                      size_t out_dim, size_t in_dim, Iq2MatmulVariant variant,
                      ActivationQuantMode mode) {
  if (out_dim == 0 || in_dim == 0) bail("iq2_matmul expects non-zero dimensions");
  if (!x.device().is_hip()) bail("iq2_matmul requires a HIP device");
  if (!x.device().same_device(weight_bytes.device()) ||
      !x.device().same_device(weight_scales.device()))
    bail("iq2_matmul device mismatch: x=" + x.device().to_string() +
         ", bytes=" + weight_bytes.device().to_string() +
         ", scales=" + weight_scales.device().to_string());
  if (weight_bytes.dtype() != DType::U8 || weight_scales.dtype() != DType::U8)
    bail(std::string("iq2_matmul expects U8 weight bytes/scales, got bytes=") +
         dtype_name(weight_bytes.dtype()) + ", scales=" + dtype_name(weight_scales.dtype()));
  size_t m = 0;
  bool squeeze = false;
  Tensor x2 = parse_x_shape(x, in_dim, &m, &squeeze).contiguous();
  check_sizes("iq2_matmul", weight_bytes, weight_scales, out_dim, in_dim, variant);
  Tensor out = Tensor::empty({m, out_dim}, DType::F32, x.device());
  size_t total;
  if (!checked_mul(m, out_dim, &total)) bail("iq2_matmul output size overflow");
  if (total == 0) return squeeze ? out.squeeze(0) : out;
  if (!weight_bytes.is_contiguous() || !weight_scales.is_contiguous())
    bail("iq2_matmul expects contiguous layouts");

  // kernel selection (src/iq2_matmul.rs:297-303): dtype, then the format
  cmk_dtype xd;
  switch (x2.dtype()) {
    case DType::F32: xd = CMK_F32; break;
    case DType::F16: xd = CMK_F16; break;
    case DType::BF16: xd = CMK_BF16; break;
    default:
      bail(std::string(mode == ActivationQuantMode::W8A8 ? "iq2_matmul_w8a8" : "iq2_matmul") +
           " unsupported x dtype: " + dtype_name(x2.dtype()));
  }
  const cmk_act_quant_mode am =
      mode == ActivationQuantMode::W8A8 ? CMK_ACT_QUANT_W8A8 : CMK_ACT_QUANT_OFF;
  size_t ws_bytes = 0;
  check_abi(cmk_iq2_matmul_workspace_size(xd, m, out_dim, in_dim, to_abi(variant), am, &ws_bytes));
  WorkspaceCache& cache = workspace_cache();
  std::lock_guard<std::mutex> lk(cache.mu);
  void* work = ws_bytes ? cache.get(x.device().ordinal, ws_bytes) : nullptr;
  check_abi(cmk_set_device(x.device().ordinal));
  check_abi(cmk_iq2_matmul(x2.data_ptr(), xd, x2.elem_count(), m,
                           static_cast<const uint8_t*>(weight_bytes.data_ptr()),
                           weight_bytes.elem_count(),
                           static_cast<const uint8_t*>(weight_scales.data_ptr()),
                           weight_scales.elem_count(), out_dim, in_dim, to_abi(variant), am, 0,
                           static_cast<float*>(out.data_ptr_mut()), work, ws_bytes, nullptr));
  return squeeze ? out.squeeze(0) : out;
}

}  // namespace

Tensor iq2_matmul(const Tensor& x, const Tensor& weight_bytes, const Tensor& weight_scales,
                  size_t out_dim, size_t in_dim, Iq2MatmulVariant variant) {
  return iq2_matmul_hip(x, weight_bytes, weight_scales, out_dim, in_dim, variant,
                        ActivationQuantMode::Off);
}

Tensor iq2_matmul_with_activation_quant(const Tensor& x, const Tensor& weight_bytes,
                                        const Tensor& weight_scales, size_t out_dim,
                                        size_t in_dim, Iq2MatmulVariant variant,
                                        const ActivationQuantConfig& activation_quant) {
  switch (activation_quant.mode) {
    case ActivationQuantMode::Off:
      return iq2_matmul(x, weight_bytes, weight_scales, out_dim, in_dim, variant);
    case ActivationQuantMode::W8A8:
      return iq2_matmul_hip(x, weight_bytes, weight_scales, out_dim, in_dim, variant,
                            ActivationQuantMode::W8A8);
    default:
      if (activation_quant.strict)
        bail("activation quant mode W4A8 requested in strict mode, but W4A8 kernel path is not "
             "implemented yet");
      return iq2_matmul(x, weight_bytes, weight_scales, out_dim, in_dim, variant);
  }
}

Tensor iq2_dequantize_to_f16(const Tensor& weight_bytes, const Tensor& weight_scales,
                             size_t out_dim, size_t in_dim, Iq2MatmulVariant variant) {
  // iq2_dequantize_to_f16_metal guards (src/iq2_matmul.rs:367-433)
  if (out_dim == 0 || in_dim == 0) bail("iq2_dequantize_to_f16 expects non-zero dimensions");
  if (!weight_bytes.device().is_hip()) bail("iq2_dequantize_to_f16 requires a HIP device");
  if (!weight_bytes.device().same_device(weight_scales.device()))
    bail("iq2_dequantize_to_f16 device mismatch: bytes=" + weight_bytes.device().to_string() +
         ", scales=" + weight_scales.device().to_string());
  if (weight_bytes.dtype() != DType::U8 || weight_scales.dtype() != DType::U8)
    bail(std::string("iq2_dequantize_to_f16 expects U8 weight bytes/scales, got bytes=") +
         dtype_name(weight_bytes.dtype()) + ", scales=" + dtype_name(weight_scales.dtype()));
  check_sizes("iq2_dequantize_to_f16", weight_bytes, weight_scales, out_dim, in_dim, variant);
  Tensor out = Tensor::empty({out_dim, in_dim}, DType::F16, weight_bytes.device());
  if (!weight_bytes.is_contiguous() || !weight_scales.is_contiguous())
    bail("iq2_dequantize_to_f16 expects contiguous layouts");
  check_abi(cmk_iq2_dequantize(static_cast<const uint8_t*>(weight_bytes.data_ptr()),
                               weight_bytes.elem_count(),
                               static_cast<const uint8_t*>(weight_scales.data_ptr()),
                               weight_scales.elem_count(), out_dim, in_dim, to_abi(variant),
                               CMK_F16, out.data_ptr_mut(), nullptr));
  return out;
}

Tensor iq2_xxs_matmul(const Tensor& x, const Tensor& weight_bytes, const Tensor& weight_scales,
                      size_t out_dim, size_t in_dim) {
  return iq2_matmul(x, weight_bytes, weight_scales, out_dim, in_dim, Iq2MatmulVariant::Iq2Xxs);
}

Tensor iq2_xs_matmul(const Tensor& x, const Tensor& weight_bytes, const Tensor& weight_scales,
                     size_t out_dim, size_t in_dim) {
  return iq2_matmul(x, weight_bytes, weight_scales, out_dim, in_dim, Iq2MatmulVariant::Iq2Xs);
}

Tensor iq2_s_matmul(const Tensor& x, const Tensor& weight_bytes, const Tensor& weight_scales,
                    size_t out_dim, size_t in_dim) {
  return iq2_matmul(x, weight_bytes, weight_scales, out_dim, in_dim, Iq2MatmulVariant::Iq2S);
}

Tensor iq3_s_matmul(const Tensor& x, const Tensor& weight_bytes, const Tensor& weight_scales,
                    size_t out_dim, size_t in_dim) {
  return iq2_matmul(x, weight_bytes, weight_scales, out_dim, in_dim, Iq2MatmulVariant::Iq3S);
}

}  // namespace candelora
