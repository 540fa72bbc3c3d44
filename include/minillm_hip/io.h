// io.h -- GGUF reading and the weight loader of the HIP backend.
//
// Mirrors the reference's GGUF layer and weight loader
// (include/minillm/io/gguf_format.h:12-56, gguf_parser.h:19-115,
// gguf_weight_loader.h:17-80) with the same names, wire-format enums and
// semantics, and adds the HIP branch the reference has for CUDA
// (src/io/gguf_weight_loader.cpp:100-156, 526-541):
//   * Q8_0 GGUF tensors bound to HIP Q8_0 tensors are copied host-to-device as
//     raw 34-byte blocks (ceil(numel/32)*34 bytes, no conversion), exactly the
//     bytes the reference's CPU and CUDA paths keep;
//   * BF16 tensors stay BF16 (raw copy); every other type becomes Float32 on the
//     host (F16/BF16 decoded, F32 copied) and is copied to the device.
// Tensor data comes from a read-only mmap view of the file, as in the reference
// (gguf_parser.h:91-97), with buffered reads when the file cannot be mapped; the
// HIP branch copies a tensor's bytes to the device straight from the view.
// Difference: the model-config extraction (WeightLoader::extract_config) is not
// part of this path.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <string_view>
#include <unordered_map>
#include <variant>
#include <vector>

#include "minillm_hip/graph.h"
#include "minillm_hip/runtime.h"

namespace minillm {

// GGUF metadata value type tags (wire format).
enum class GgufValueType : uint32_t {
  UINT8 = 0,
  INT8 = 1,
  UINT16 = 2,
  INT16 = 3,
  UINT32 = 4,
  INT32 = 5,
  FLOAT32 = 6,
  BOOL = 7,
  STRING = 8,
  ARRAY = 9,
  UINT64 = 10,
  INT64 = 11,
  FLOAT64 = 12,
};

// GGML tensor element types (wire format); the ones this engine knows.
enum class GgmlDataType : uint32_t {
  F32 = 0,
  F16 = 1,
  Q4_0 = 2,
  Q4_1 = 3,
  Q8_0 = 8,
  BF16 = 30,
};

constexpr uint32_t kGgufVersion = 3;
constexpr uint32_t kGgufDefaultAlignment = 32;

// Bytes per element (F32 4, F16 / BF16 2) or per block (Q8_0 34); 0 for the
// types this engine does not read (Q4_0, Q4_1, unknown).
size_t ggml_dtype_size(GgmlDataType dt);
// Elements per block: 1 for F32 / F16 / BF16, 32 for Q8_0; 0 otherwise.
size_t ggml_blck_size(GgmlDataType dt);
std::string_view ggml_dtype_name(GgmlDataType dt);
// Engine dtype: F32 -> Float32, F16 -> Float16, BF16 -> BFloat16, Q8_0 -> Q8_0;
// others Unsupported.
expected<DType, Status> map_ggml_dtype(GgmlDataType dt);

struct MetadataArray;
using MetadataValue = std::variant<uint8_t, int8_t, uint16_t, int16_t, uint32_t, int32_t,
                                   uint64_t, int64_t, float, double, bool, std::string,
                                   MetadataArray>;
struct MetadataArray {
  std::vector<MetadataValue> elements;
};

struct GGUFTensorInfo {
  std::string name;
  GgmlDataType dtype{GgmlDataType::F32};
  std::vector<int64_t> dimensions;  // row-major: outermost first (GGUF stores innermost first)
  uint64_t offset{0};               // from the start of the data section

  expected<size_t, Status> num_elements() const;
  // Raw byte size: ceil(numel / blck) * dtype_size (Q8_0: ceil(numel/32)*34).
  expected<size_t, Status> bytes() const;
};

struct GGUFFile {
  uint32_t version{0};
  uint64_t tensor_count{0};
  uint64_t metadata_kv_count{0};
  uint64_t data_offset{0};  // absolute file offset of the (aligned) data section
  uint32_t alignment{kGgufDefaultAlignment};
  std::string source_path;
  std::unordered_map<std::string, MetadataValue> metadata;
  std::vector<GGUFTensorInfo> tensor_infos;

  const GGUFTensorInfo* find_tensor(std::string_view name) const;
};

expected<MetadataValue, Status> get_metadata(
    const std::unordered_map<std::string, MetadataValue>& meta, std::string_view key);

template <typename T>
T get_metadata_or(const std::unordered_map<std::string, MetadataValue>& meta,
                  std::string_view key, T default_val) {
  auto it = meta.find(std::string(key));
  if (it == meta.end()) return default_val;
  if (auto* v = std::get_if<T>(&it->second)) return *v;
  return default_val;
}

expected<size_t, Status> get_metadata_array_size(
    const std::unordered_map<std::string, MetadataValue>& meta, std::string_view key);

// GGUF v3 reader.  Errors: missing file / short read -> IOError; bad magic,
// zero or > 8 dimensions, zero dimension, oversized counts -> InvalidArgument;
// version != 3 or an unknown metadata type -> Unsupported; a tensor whose byte
// range lies past the end of the file -> OutOfRange.
class GGUFParser {
 public:
  static expected<GGUFFile, Status> parse(const std::string& filename);
  // Reads `byte_count` bytes of tensor data at data_offset + tensor_offset.
  static Status read_tensor_data(const std::string& filename, uint64_t data_offset,
                                 uint64_t tensor_offset, void* dst, size_t byte_count);
};

// Weights loaded once and bound (non-owning) into any number of contexts.
class SharedWeightStore {
 public:
  SharedWeightStore() = default;
  SharedWeightStore(const SharedWeightStore&) = delete;
  SharedWeightStore& operator=(const SharedWeightStore&) = delete;
  SharedWeightStore(SharedWeightStore&&) noexcept = default;
  SharedWeightStore& operator=(SharedWeightStore&&) noexcept = default;

  // Binds every graph Constant that has a loaded tensor (same shape, same
  // device, dtype equal or a Q8_0 / BF16 tensor serving a Float32 value).
  Status bind(const Graph& graph, RuntimeContext& ctx) const;

  Tensor* get(const std::string& value_name) const;
  size_t tensor_count() const { return storage_by_gguf_name_.size(); }
  size_t alias_count() const { return aliases_by_value_name_.size(); }
  size_t total_bytes() const { return total_bytes_; }

 private:
  friend class WeightLoader;
  std::unordered_map<std::string, std::unique_ptr<Tensor>> storage_by_gguf_name_;
  std::unordered_map<std::string, Tensor*> aliases_by_value_name_;
  size_t total_bytes_ = 0;
};

class WeightLoader {
 public:
  explicit WeightLoader(std::string gguf_path);

  expected<GGUFFile, Status> open();

  // Loads every GGUF tensor whose mapped name is a graph Constant into the
  // tensor already bound to that value in `ctx` (host or HIP storage).
  Status load_weights(const GGUFFile& file, const Graph& graph, RuntimeContext& ctx) const;

  // Allocates and loads each needed GGUF tensor once, on the device of the
  // graph value (HIP: Q8_0 and BF16 keep their raw bytes, others become Float32).
  expected<SharedWeightStore, Status> load_shared_weights(const GGUFFile& file,
                                                          const Graph& graph) const;

  // GGUF tensor name -> graph value name ("blk.3.ffn_up.weight" ->
  // "layer_3.up_proj.weight", "token_embd.weight" -> "tok_embeddings.weight").
  static expected<std::string, Status> gguf_name_to_value_name(const std::string& gguf_name,
                                                               int layer_index = 0);

  // F32 / F16 / BF16 / Q8_0 source data to fp32 (Q8_0: value = (float)q * d).
  static Status dequantize_to_f32(GgmlDataType src_dtype, const void* src, float* dst,
                                  size_t num_elements);

 private:
  std::string gguf_path_;
};

}  // namespace minillm
