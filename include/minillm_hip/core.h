// core.h -- Status, DType, Device, Shape and Tensor of the MiniLLMEngine host API,
// restated for the HIP (MI355X) backend.
//
// Same names, enumerator order and semantics as the reference core layer
// (include/minillm/core/status.h:20-59, dtype.h:12-61, device.h:7-22,
// shape.h:13-35, tensor.h:19-61), so code written against the reference's
// Tensor/Status compiles against this header.  Differences:
//   * DeviceType gains HIP (enumerator between CUDA and Unknown) and Device::hip();
//   * Tensor owns HIP device storage: allocate_hip()/allocate_hip_bytes()/
//     bind_hip_data() stand where the reference has allocate_cuda*/bind_cuda_data;
//   * expected<> is minillm::expected (see expected.h).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <string_view>
#include <vector>

#include "minillm_hip/expected.h"

#define TRY(expr)                       \
  do {                                  \
    auto _st_ = (expr);                 \
    if (!_st_.ok()) return _st_;        \
  } while (0)

namespace minillm {

// ---------------------------------------------------------------- Status
enum class ErrorCode {
  Ok,
  InvalidArgument,
  OutOfRange,
  ShapeMismatch,
  Unsupported,
  NotImplemented,
  RuntimeError,
  InternalError,
  IOError,
  NotFound,
  TypeError,
};

class Status {
 public:
  Status() = default;
  Status(ErrorCode code, std::string message);

  static Status make_ok();
  static Status invalid_argument(std::string message);
  static Status out_of_range(std::string message);
  static Status shape_mismatch(std::string message);
  static Status unsupported(std::string message);
  static Status not_implemented(std::string message);
  static Status runtime_error(std::string message);
  static Status internal_error(std::string message);
  static Status io_error(std::string message);
  static Status not_found(std::string message);
  static Status type_error(std::string message);

  bool ok() const;
  ErrorCode code() const;
  std::string_view message() const;
  std::string to_string() const;

 private:
  ErrorCode code_{ErrorCode::Ok};
  std::string message_;
};

std::string_view error_code_name(ErrorCode code);

// ---------------------------------------------------------------- DType
enum class DType {
  Float32,
  Float16,
  BFloat16,
  Q8_0,
  Int32,
  Int64,
  UInt8,
  Int8,
  Bool,
  Unknown,
};

std::string_view dtype_name(DType type);
// Per-element byte size; Q8_0 is block-quantised and has none (Unsupported).
expected<size_t, Status> dtype_size(DType type);
bool is_floating_point(DType type);

// Raw byte size of a Q8_0 tensor with `numel` elements: ceil(numel/32)*34.
constexpr size_t kQ8_0BlockBytes = 34;
constexpr size_t kQ8_0BlockElems = 32;
size_t q8_0_bytes(size_t numel);

// ---------------------------------------------------------------- Device
enum class DeviceType {
  CPU,
  CUDA,
  HIP,
  Unknown,
};

struct Device {
  DeviceType type{DeviceType::CPU};
  int index{0};

  static Device cpu() { return {DeviceType::CPU, 0}; }
  static Device cuda(int idx) { return {DeviceType::CUDA, idx}; }
  static Device hip(int idx) { return {DeviceType::HIP, idx}; }

  std::string to_string() const;
  bool operator==(const Device& other) const = default;
};

// ---------------------------------------------------------------- Shape
class Shape {
 public:
  Shape() = default;
  explicit Shape(std::vector<int64_t> dims);

  size_t rank() const { return dims_.size(); }
  int64_t dim(size_t i) const;
  const std::vector<int64_t>& dims() const;
  bool empty() const { return dims_.empty(); }
  bool has_dynamic_dim() const;
  expected<size_t, Status> numel() const;
  std::string to_string() const;
  bool operator==(const Shape& other) const = default;

 private:
  std::vector<int64_t> dims_;
};

// ---------------------------------------------------------------- Tensor
// Physical data container bound to a graph ValueId.  Owns host storage, HIP
// device storage, or views external storage.  Move-only.
// Byte order of a tensor's storage.  Raw: the dtype's own layout (GGUF blocks for
// Q8_0).  Q8_0Tiled: the Q8_0 16-row tiles of mle_q8_0_tile, which a HipExecutor
// puts in place of a Linear-only weight's raw bytes when asked to
// (HipExecutor::tile_weights with release_raw; no counterpart in the reference).
enum class StorageLayout { Raw = 0, Q8_0Tiled = 1 };

class Tensor {
 public:
  Tensor() = default;
  Tensor(std::string name, Shape shape, DType dtype, Device device = Device::cpu());
  ~Tensor();

  Tensor(const Tensor&) = delete;
  Tensor& operator=(const Tensor&) = delete;
  Tensor(Tensor&& other) noexcept;
  Tensor& operator=(Tensor&& other) noexcept;

  const std::string& name() const;
  const Shape& shape() const;
  DType dtype() const;
  const Device& device() const;

  expected<size_t, Status> numel() const;
  expected<size_t, Status> nbytes() const;
  size_t allocated_bytes() const;

  bool is_allocated() const;
  void* data();
  const void* data() const;

  Status allocate_cpu();
  Status allocate_cpu_bytes(size_t bytes);
  Status bind_cpu_data(void* data, size_t bytes);
  // HIP device storage on device index device().index (hipMalloc / hipFree).
  Status allocate_hip();
  Status allocate_hip_bytes(size_t bytes);
  Status bind_hip_data(void* data, size_t bytes);
  Status release();

  StorageLayout storage_layout() const { return layout_; }
  // Whether the device storage was allocated by this tensor (allocate_hip*), as
  // opposed to bound (bind_hip_data) or absent.
  bool owns_hip_storage() const { return hip_ != nullptr; }
  // Replaces owned device storage by `data` (hipMalloc'd, `bytes` long, now owned
  // by the tensor and freed by release()) holding the same values in `layout`.
  // The old storage is freed with hipFree, so no launch may still read it.
  // InvalidArgument unless the tensor owns HIP storage and `data` is not null.
  Status adopt_hip_bytes(void* data, size_t bytes, StorageLayout layout);

 private:
  std::string name_;
  Shape shape_;
  DType dtype_{DType::Unknown};
  Device device_{Device::cpu()};
  std::vector<std::byte> host_;
  void* external_{nullptr};
  size_t external_bytes_{0};
  void* hip_{nullptr};
  size_t hip_bytes_{0};
  StorageLayout layout_{StorageLayout::Raw};
};

}  // namespace minillm
