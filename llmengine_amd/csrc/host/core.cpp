// core.cpp -- Status, DType, Device, Shape and Tensor (see include/minillm_hip/core.h).
#include "minillm_hip/core.h"

#include <hip/hip_runtime.h>

#include <limits>
#include <stdexcept>

namespace minillm {

// ---------------------------------------------------------------- Status
Status::Status(ErrorCode code, std::string message)
    : code_(code), message_(std::move(message)) {}

Status Status::make_ok() { return Status(); }
Status Status::invalid_argument(std::string m) { return {ErrorCode::InvalidArgument, std::move(m)}; }
Status Status::out_of_range(std::string m) { return {ErrorCode::OutOfRange, std::move(m)}; }
Status Status::shape_mismatch(std::string m) { return {ErrorCode::ShapeMismatch, std::move(m)}; }
Status Status::unsupported(std::string m) { return {ErrorCode::Unsupported, std::move(m)}; }
Status Status::not_implemented(std::string m) { return {ErrorCode::NotImplemented, std::move(m)}; }
Status Status::runtime_error(std::string m) { return {ErrorCode::RuntimeError, std::move(m)}; }
Status Status::internal_error(std::string m) { return {ErrorCode::InternalError, std::move(m)}; }
Status Status::io_error(std::string m) { return {ErrorCode::IOError, std::move(m)}; }
Status Status::not_found(std::string m) { return {ErrorCode::NotFound, std::move(m)}; }
Status Status::type_error(std::string m) { return {ErrorCode::TypeError, std::move(m)}; }

bool Status::ok() const { return code_ == ErrorCode::Ok; }
ErrorCode Status::code() const { return code_; }
std::string_view Status::message() const { return message_; }

std::string_view error_code_name(ErrorCode code) {
  switch (code) {
    case ErrorCode::Ok: return "Ok";
    case ErrorCode::InvalidArgument: return "InvalidArgument";
    case ErrorCode::OutOfRange: return "OutOfRange";
    case ErrorCode::ShapeMismatch: return "ShapeMismatch";
    case ErrorCode::Unsupported: return "Unsupported";
    case ErrorCode::NotImplemented: return "NotImplemented";
    case ErrorCode::RuntimeError: return "RuntimeError";
    case ErrorCode::InternalError: return "InternalError";
    case ErrorCode::IOError: return "IOError";
    case ErrorCode::NotFound: return "NotFound";
    case ErrorCode::TypeError: return "TypeError";
  }
  return "Unknown";
}

std::string Status::to_string() const {
  std::string s(error_code_name(code_));
  if (!message_.empty()) s += ": " + message_;
  return s;
}

// ---------------------------------------------------------------- DType
std::string_view dtype_name(DType type) {
  switch (type) {
    case DType::Float32: return "Float32";
    case DType::Float16: return "Float16";
    case DType::BFloat16: return "BFloat16";
    case DType::Q8_0: return "Q8_0";
    case DType::Int32: return "Int32";
    case DType::Int64: return "Int64";
    case DType::UInt8: return "UInt8";
    case DType::Int8: return "Int8";
    case DType::Bool: return "Bool";
    case DType::Unknown: return "Unknown";
  }
  return "Unknown";
}

expected<size_t, Status> dtype_size(DType type) {
  switch (type) {
    case DType::Float32: return size_t{4};
    case DType::Float16: return size_t{2};
    case DType::BFloat16: return size_t{2};
    case DType::Int32: return size_t{4};
    case DType::Int64: return size_t{8};
    case DType::UInt8: return size_t{1};
    case DType::Int8: return size_t{1};
    case DType::Bool: return size_t{1};
    case DType::Q8_0:
      return unexpected(
          Status::unsupported("Q8_0 is block-quantized and has no per-element byte size"));
    case DType::Unknown: break;
  }
  return unexpected(Status::unsupported("Unknown dtype has no size"));
}

bool is_floating_point(DType type) {
  return type == DType::Float32 || type == DType::Float16 || type == DType::BFloat16;
}

size_t q8_0_bytes(size_t numel) {
  return (numel + kQ8_0BlockElems - 1) / kQ8_0BlockElems * kQ8_0BlockBytes;
}

// ---------------------------------------------------------------- Device
std::string Device::to_string() const {
  switch (type) {
    case DeviceType::CPU: return "cpu:" + std::to_string(index);
    case DeviceType::CUDA: return "cuda:" + std::to_string(index);
    case DeviceType::HIP: return "hip:" + std::to_string(index);
    case DeviceType::Unknown: break;
  }
  return "unknown:" + std::to_string(index);
}

// ---------------------------------------------------------------- Shape
Shape::Shape(std::vector<int64_t> dims) : dims_(std::move(dims)) {
  for (int64_t d : dims_) {
    if (d == 0 || d < -1)
      throw std::invalid_argument("Shape dimension must be >= 1 or -1 (dynamic), got: " +
                                  std::to_string(d));
  }
}

int64_t Shape::dim(size_t i) const { return dims_.at(i); }
const std::vector<int64_t>& Shape::dims() const { return dims_; }

bool Shape::has_dynamic_dim() const {
  for (int64_t d : dims_)
    if (d < 0) return true;
  return false;
}

expected<size_t, Status> Shape::numel() const {
  if (has_dynamic_dim())
    return unexpected(Status::invalid_argument(
        "cannot compute numel of shape with dynamic dims: " + to_string()));
  size_t n = 1;
  for (int64_t d : dims_) {
    if (n > std::numeric_limits<size_t>::max() / static_cast<size_t>(d))
      return unexpected(Status::invalid_argument("numel overflow for shape: " + to_string()));
    n *= static_cast<size_t>(d);
  }
  return n;
}

std::string Shape::to_string() const {
  std::string s = "[";
  for (size_t i = 0; i < dims_.size(); ++i) {
    if (i) s += ", ";
    s += std::to_string(dims_[i]);
  }
  return s + "]";
}

// ---------------------------------------------------------------- Tensor
namespace {
Status hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return Status::make_ok();
  return Status::runtime_error(std::string(what) + ": " + hipGetErrorString(err));
}
}  // namespace

Tensor::Tensor(std::string name, Shape shape, DType dtype, Device device)
    : name_(std::move(name)), shape_(std::move(shape)), dtype_(dtype), device_(device) {}

Tensor::~Tensor() { (void)release(); }

Tensor::Tensor(Tensor&& o) noexcept
    : name_(std::move(o.name_)), shape_(std::move(o.shape_)), dtype_(o.dtype_),
      device_(o.device_), host_(std::move(o.host_)), external_(o.external_),
      external_bytes_(o.external_bytes_), hip_(o.hip_), hip_bytes_(o.hip_bytes_),
      layout_(o.layout_) {
  o.external_ = nullptr;
  o.external_bytes_ = 0;
  o.hip_ = nullptr;
  o.hip_bytes_ = 0;
  o.layout_ = StorageLayout::Raw;
}

Tensor& Tensor::operator=(Tensor&& o) noexcept {
  if (this == &o) return *this;
  (void)release();
  name_ = std::move(o.name_);
  shape_ = std::move(o.shape_);
  dtype_ = o.dtype_;
  device_ = o.device_;
  host_ = std::move(o.host_);
  external_ = o.external_;
  external_bytes_ = o.external_bytes_;
  hip_ = o.hip_;
  hip_bytes_ = o.hip_bytes_;
  layout_ = o.layout_;
  o.external_ = nullptr;
  o.external_bytes_ = 0;
  o.hip_ = nullptr;
  o.hip_bytes_ = 0;
  o.layout_ = StorageLayout::Raw;
  return *this;
}

const std::string& Tensor::name() const { return name_; }
const Shape& Tensor::shape() const { return shape_; }
DType Tensor::dtype() const { return dtype_; }
const Device& Tensor::device() const { return device_; }
expected<size_t, Status> Tensor::numel() const { return shape_.numel(); }

expected<size_t, Status> Tensor::nbytes() const {
  auto n = shape_.numel();
  if (!n) return unexpected(n.error());
  auto s = dtype_size(dtype_);
  if (!s) return unexpected(s.error());
  return *n * *s;
}

size_t Tensor::allocated_bytes() const {
  if (external_) return external_bytes_;
  if (hip_) return hip_bytes_;
  return host_.size();
}

bool Tensor::is_allocated() const { return external_ || hip_ || !host_.empty(); }

void* Tensor::data() {
  if (external_) return external_;
  if (hip_) return hip_;
  return host_.empty() ? nullptr : host_.data();
}

const void* Tensor::data() const {
  if (external_) return external_;
  if (hip_) return hip_;
  return host_.empty() ? nullptr : host_.data();
}

Status Tensor::allocate_cpu() {
  if (shape_.has_dynamic_dim())
    return Status::invalid_argument("cannot allocate tensor with dynamic shape: " +
                                    shape_.to_string());
  auto nb = nbytes();
  if (!nb) return nb.error();
  std::vector<std::byte> storage(*nb);
  TRY(release());
  host_ = std::move(storage);
  device_ = Device::cpu();
  return Status::make_ok();
}

Status Tensor::allocate_cpu_bytes(size_t bytes) {
  TRY(release());
  host_.resize(bytes);
  device_ = Device::cpu();
  return Status::make_ok();
}

// Bytes a buffer must hold for this tensor: ceil(numel/32)*34 for Q8_0,
// numel * element size otherwise.
static expected<size_t, Status> required_bytes(const Shape& shape, DType dtype) {
  auto n = shape.numel();
  if (!n) return unexpected(n.error());
  if (dtype == DType::Q8_0) return q8_0_bytes(*n);
  auto s = dtype_size(dtype);
  if (!s) return unexpected(s.error());
  return *n * *s;
}

Status Tensor::bind_cpu_data(void* data, size_t bytes) {
  TRY(release());
  if (!data) return Status::invalid_argument("cannot bind null CPU storage to tensor: " + name_);
  if (shape_.has_dynamic_dim())
    return Status::invalid_argument("cannot bind tensor with dynamic shape: " +
                                    shape_.to_string());
  auto need = required_bytes(shape_, dtype_);
  if (!need) return need.error();
  if (bytes < *need)
    return Status::out_of_range("external CPU storage is too small for tensor " + name_);
  external_ = data;
  external_bytes_ = bytes;
  device_ = Device::cpu();
  return Status::make_ok();
}

Status Tensor::allocate_hip() {
  if (shape_.has_dynamic_dim())
    return Status::invalid_argument("cannot allocate tensor with dynamic shape: " +
                                    shape_.to_string());
  auto need = required_bytes(shape_, dtype_);
  if (!need) return need.error();
  return allocate_hip_bytes(*need);
}

Status Tensor::allocate_hip_bytes(size_t bytes) {
  const int index = device_.index;
  TRY(release());
  TRY(hip_status(hipSetDevice(index), "hipSetDevice failed"));
  void* p = nullptr;
  const hipError_t err = hipMalloc(&p, bytes == 0 ? 1 : bytes);
  if (err != hipSuccess) return hip_status(err, "hipMalloc failed");
  hip_ = p;
  hip_bytes_ = bytes;
  device_ = Device::hip(index);
  return Status::make_ok();
}

Status Tensor::bind_hip_data(void* data, size_t bytes) {
  const int index = device_.index;
  TRY(release());
  if (!data) return Status::invalid_argument("cannot bind null HIP storage to tensor: " + name_);
  if (shape_.has_dynamic_dim())
    return Status::invalid_argument("cannot bind tensor with dynamic shape: " +
                                    shape_.to_string());
  auto need = required_bytes(shape_, dtype_);
  if (!need) return need.error();
  if (bytes < *need)
    return Status::out_of_range("external HIP storage is too small for tensor " + name_);
  external_ = data;
  external_bytes_ = bytes;
  device_ = Device::hip(index);
  return Status::make_ok();
}

Status Tensor::adopt_hip_bytes(void* data, size_t bytes, StorageLayout layout) {
  if (data == nullptr || hip_ == nullptr || device_.type != DeviceType::HIP)
    return Status::invalid_argument("adopt_hip_bytes needs a tensor that owns HIP storage: " +
                                    name_);
  const hipError_t err = hipFree(hip_);
  if (err != hipSuccess) return hip_status(err, "hipFree failed");
  hip_ = data;
  hip_bytes_ = bytes;
  layout_ = layout;
  return Status::make_ok();
}

Status Tensor::release() {
  Status st;
  if (hip_) {
    const hipError_t err = hipFree(hip_);
    if (err != hipSuccess) st = hip_status(err, "hipFree failed");
  }
  hip_ = nullptr;
  hip_bytes_ = 0;
  external_ = nullptr;
  external_bytes_ = 0;
  host_.clear();
  host_.shrink_to_fit();
  layout_ = StorageLayout::Raw;
  return st;
}

}  // namespace minillm
