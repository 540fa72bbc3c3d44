// io.cpp -- GGUF reader and weight loader (see include/minillm_hip/io.h).
#include "minillm_hip/io.h"
#include "minillm_hip/runtime.h"

#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>

namespace minillm {

// ---------------------------------------------------------------- GGML types
size_t ggml_dtype_size(GgmlDataType dt) {
  switch (dt) {
    case GgmlDataType::F32: return 4;
    case GgmlDataType::F16:
    case GgmlDataType::BF16: return 2;
    case GgmlDataType::Q8_0: return kQ8_0BlockBytes;
    default: return 0;
  }
}

size_t ggml_blck_size(GgmlDataType dt) {
  switch (dt) {
    case GgmlDataType::F32:
    case GgmlDataType::F16:
    case GgmlDataType::BF16: return 1;
    case GgmlDataType::Q8_0: return kQ8_0BlockElems;
    default: return 0;
  }
}

std::string_view ggml_dtype_name(GgmlDataType dt) {
  switch (dt) {
    case GgmlDataType::F32: return "F32";
    case GgmlDataType::F16: return "F16";
    case GgmlDataType::BF16: return "BF16";
    case GgmlDataType::Q8_0: return "Q8_0";
    default: return "UNKNOWN";
  }
}

expected<DType, Status> map_ggml_dtype(GgmlDataType dt) {
  switch (dt) {
    case GgmlDataType::F32: return DType::Float32;
    case GgmlDataType::F16: return DType::Float16;
    case GgmlDataType::BF16: return DType::BFloat16;
    case GgmlDataType::Q8_0: return DType::Q8_0;
    default:
      return unexpected(Status::unsupported("unsupported GGML dtype " +
                                            std::string(ggml_dtype_name(dt)) +
                                            " (only F32/F16/BF16/Q8_0 are supported)"));
  }
}

// ---------------------------------------------------------------- tensor info
expected<size_t, Status> GGUFTensorInfo::num_elements() const {
  size_t n = 1;
  for (int64_t d : dimensions) {
    if (d <= 0)
      return unexpected(Status::invalid_argument("invalid non-positive dimension for tensor: " +
                                                 name));
    if (n > std::numeric_limits<size_t>::max() / static_cast<size_t>(d))
      return unexpected(Status::invalid_argument("numel overflow for tensor: " + name));
    n *= static_cast<size_t>(d);
  }
  return n;
}

expected<size_t, Status> GGUFTensorInfo::bytes() const {
  auto n = num_elements();
  if (!n) return unexpected(n.error());
  const size_t blck = ggml_blck_size(dtype), unit = ggml_dtype_size(dtype);
  if (blck == 0 || unit == 0)
    return unexpected(
        Status::unsupported("unsupported GGML dtype for tensor byte size: " + name));
  const size_t blocks = *n / blck + (*n % blck != 0);
  if (blocks > std::numeric_limits<size_t>::max() / unit)
    return unexpected(Status::invalid_argument("byte size overflow for tensor: " + name));
  return blocks * unit;
}

const GGUFTensorInfo* GGUFFile::find_tensor(std::string_view name) const {
  for (const auto& ti : tensor_infos)
    if (ti.name == name) return &ti;
  return nullptr;
}

expected<MetadataValue, Status> get_metadata(
    const std::unordered_map<std::string, MetadataValue>& meta, std::string_view key) {
  auto it = meta.find(std::string(key));
  if (it == meta.end())
    return unexpected(Status::not_found("metadata key not found: " + std::string(key)));
  return it->second;
}

expected<size_t, Status> get_metadata_array_size(
    const std::unordered_map<std::string, MetadataValue>& meta, std::string_view key) {
  auto it = meta.find(std::string(key));
  if (it == meta.end())
    return unexpected(Status::not_found("metadata key not found: " + std::string(key)));
  auto* arr = std::get_if<MetadataArray>(&it->second);
  if (!arr)
    return unexpected(Status::type_error("metadata key is not an array: " + std::string(key)));
  return arr->elements.size();
}

// ---------------------------------------------------------------- parser
namespace {

constexpr uint64_t kMaxArrayLen = uint64_t(16) << 20;  // metadata array elements
constexpr uint64_t kMaxTensors = uint64_t(1) << 20;
constexpr uint32_t kMaxDims = 8;

struct FileCloser {
  void operator()(std::FILE* f) const {
    if (f) std::fclose(f);
  }
};
using FilePtr = std::unique_ptr<std::FILE, FileCloser>;

uint64_t file_size(std::FILE* f) {
  const auto here = ftello(f);
  fseeko(f, 0, SEEK_END);
  const auto end = ftello(f);
  fseeko(f, here, SEEK_SET);
  return end < 0 ? 0 : static_cast<uint64_t>(end);
}

// Sequential little-endian reads with the byte position tracked.
class Reader {
 public:
  Reader(std::FILE* f, uint64_t size) : f_(f), size_(size) {}

  uint64_t pos() const { return pos_; }
  uint64_t remaining() const { return size_ - pos_; }

  Status raw(void* dst, size_t n, const char* what) {
    if (n > remaining() || std::fread(dst, 1, n, f_) != n)
      return Status::io_error(std::string("unexpected end of GGUF file reading ") + what);
    pos_ += n;
    return Status::make_ok();
  }

  template <typename T>
  expected<T, Status> le(const char* what) {
    unsigned char b[sizeof(T)];
    auto st = raw(b, sizeof(T), what);
    if (!st.ok()) return unexpected(st);
    uint64_t v = 0;
    for (size_t i = 0; i < sizeof(T); ++i) v |= static_cast<uint64_t>(b[i]) << (8 * i);
    T out;
    if constexpr (sizeof(T) == 8) {
      std::memcpy(&out, &v, 8);
    } else {
      const auto narrow = static_cast<uint32_t>(v);
      if constexpr (sizeof(T) == 4) {
        std::memcpy(&out, &narrow, 4);
      } else if constexpr (sizeof(T) == 2) {
        const auto h = static_cast<uint16_t>(narrow);
        std::memcpy(&out, &h, 2);
      } else {
        const auto c = static_cast<uint8_t>(narrow);
        std::memcpy(&out, &c, 1);
      }
    }
    return out;
  }

  expected<std::string, Status> string(const char* what) {
    auto n = le<uint64_t>(what);
    if (!n) return unexpected(n.error());
    if (*n > remaining())
      return unexpected(Status::io_error(std::string("GGUF string runs past the end of file: ") +
                                         what));
    std::string s(static_cast<size_t>(*n), '\0');
    auto st = raw(s.data(), s.size(), what);
    if (!st.ok()) return unexpected(st);
    return s;
  }

 private:
  std::FILE* f_;
  uint64_t size_;
  uint64_t pos_ = 0;
};

expected<MetadataValue, Status> read_value(Reader& r, GgufValueType type, int depth) {
  switch (type) {
    case GgufValueType::UINT8: { auto v = r.le<uint8_t>("u8"); if (!v) return unexpected(v.error()); return MetadataValue(*v); }
    case GgufValueType::INT8: { auto v = r.le<int8_t>("i8"); if (!v) return unexpected(v.error()); return MetadataValue(*v); }
    case GgufValueType::UINT16: { auto v = r.le<uint16_t>("u16"); if (!v) return unexpected(v.error()); return MetadataValue(*v); }
    case GgufValueType::INT16: { auto v = r.le<int16_t>("i16"); if (!v) return unexpected(v.error()); return MetadataValue(*v); }
    case GgufValueType::UINT32: { auto v = r.le<uint32_t>("u32"); if (!v) return unexpected(v.error()); return MetadataValue(*v); }
    case GgufValueType::INT32: { auto v = r.le<int32_t>("i32"); if (!v) return unexpected(v.error()); return MetadataValue(*v); }
    case GgufValueType::UINT64: { auto v = r.le<uint64_t>("u64"); if (!v) return unexpected(v.error()); return MetadataValue(*v); }
    case GgufValueType::INT64: { auto v = r.le<int64_t>("i64"); if (!v) return unexpected(v.error()); return MetadataValue(*v); }
    case GgufValueType::FLOAT32: { auto v = r.le<float>("f32"); if (!v) return unexpected(v.error()); return MetadataValue(*v); }
    case GgufValueType::FLOAT64: { auto v = r.le<double>("f64"); if (!v) return unexpected(v.error()); return MetadataValue(*v); }
    case GgufValueType::BOOL: {
      auto v = r.le<uint8_t>("bool");
      if (!v) return unexpected(v.error());
      return MetadataValue(*v != 0);
    }
    case GgufValueType::STRING: {
      auto v = r.string("metadata string");
      if (!v) return unexpected(v.error());
      return MetadataValue(std::move(*v));
    }
    case GgufValueType::ARRAY: {
      if (depth > 0)
        return unexpected(Status::unsupported("nested GGUF metadata arrays are not supported"));
      auto et = r.le<uint32_t>("array type");
      if (!et) return unexpected(et.error());
      auto n = r.le<uint64_t>("array length");
      if (!n) return unexpected(n.error());
      if (*n > kMaxArrayLen)
        return unexpected(
            Status::invalid_argument("GGUF metadata array too long: " + std::to_string(*n)));
      MetadataArray arr;
      arr.elements.reserve(static_cast<size_t>(*n));
      for (uint64_t i = 0; i < *n; ++i) {
        auto e = read_value(r, static_cast<GgufValueType>(*et), depth + 1);
        if (!e) return unexpected(e.error());
        arr.elements.push_back(std::move(*e));
      }
      return MetadataValue(std::move(arr));
    }
  }
  return unexpected(Status::unsupported("unsupported GGUF metadata type: " +
                                        std::to_string(static_cast<uint32_t>(type))));
}

}  // namespace

expected<GGUFFile, Status> GGUFParser::parse(const std::string& filename) {
  FilePtr f(std::fopen(filename.c_str(), "rb"));
  if (!f) return unexpected(Status::io_error("cannot open file: " + filename));
  const uint64_t size = file_size(f.get());
  Reader r(f.get(), size);

  char magic[4];
  if (!r.raw(magic, 4, "magic").ok() || std::memcmp(magic, "GGUF", 4) != 0)
    return unexpected(Status::invalid_argument("invalid GGUF file: magic number mismatch"));

  GGUFFile file;
  file.source_path = filename;
  auto version = r.le<uint32_t>("version");
  if (!version) return unexpected(version.error());
  file.version = *version;
  if (file.version != kGgufVersion)
    return unexpected(Status::unsupported("unsupported GGUF version " +
                                          std::to_string(file.version) + " (expected " +
                                          std::to_string(kGgufVersion) + ")"));
  auto tc = r.le<uint64_t>("tensor count");
  if (!tc) return unexpected(tc.error());
  auto kc = r.le<uint64_t>("metadata count");
  if (!kc) return unexpected(kc.error());
  file.tensor_count = *tc;
  file.metadata_kv_count = *kc;
  if (file.tensor_count > kMaxTensors)
    return unexpected(Status::invalid_argument("GGUF tensor count too large: " +
                                               std::to_string(file.tensor_count)));

  for (uint64_t i = 0; i < file.metadata_kv_count; ++i) {
    auto key = r.string("metadata key");
    if (!key) return unexpected(key.error());
    auto type = r.le<uint32_t>("metadata type");
    if (!type) return unexpected(type.error());
    auto value = read_value(r, static_cast<GgufValueType>(*type), 0);
    if (!value) return unexpected(value.error());
    file.metadata.insert_or_assign(std::move(*key), std::move(*value));
  }

  file.tensor_infos.reserve(static_cast<size_t>(file.tensor_count));
  for (uint64_t i = 0; i < file.tensor_count; ++i) {
    GGUFTensorInfo ti;
    auto name = r.string("tensor name");
    if (!name) return unexpected(name.error());
    ti.name = std::move(*name);
    auto nd = r.le<uint32_t>("tensor rank");
    if (!nd) return unexpected(nd.error());
    if (*nd == 0 || *nd > kMaxDims)
      return unexpected(Status::invalid_argument("GGUF tensor has invalid dimension count: " +
                                                 std::to_string(*nd)));
    ti.dimensions.assign(*nd, 0);
    for (uint32_t d = 0; d < *nd; ++d) {  // GGUF lists the innermost dimension first
      auto dim = r.le<uint64_t>("tensor dimension");
      if (!dim) return unexpected(dim.error());
      if (*dim == 0 || *dim > static_cast<uint64_t>(std::numeric_limits<int64_t>::max()))
        return unexpected(Status::invalid_argument("GGUF tensor has invalid dimension: " +
                                                   std::to_string(*dim)));
      ti.dimensions[*nd - 1 - d] = static_cast<int64_t>(*dim);
    }
    auto dt = r.le<uint32_t>("tensor type");
    if (!dt) return unexpected(dt.error());
    ti.dtype = static_cast<GgmlDataType>(*dt);
    auto off = r.le<uint64_t>("tensor offset");
    if (!off) return unexpected(off.error());
    ti.offset = *off;
    file.tensor_infos.push_back(std::move(ti));
  }

  auto it = file.metadata.find("general.alignment");
  if (it != file.metadata.end()) {
    if (auto* a = std::get_if<uint32_t>(&it->second)) file.alignment = *a;
  }
  if (file.alignment == 0)
    return unexpected(Status::invalid_argument("GGUF general.alignment must be positive"));
  const uint64_t pos = r.pos();
  file.data_offset = pos + (file.alignment - pos % file.alignment) % file.alignment;
  return file;
}

namespace {

// Read-only mapping of a whole GGUF file (the reference's mmap view,
// gguf_parser.h:91-97).  open() returns null when the file cannot be mapped;
// callers then stream the bytes with buffered reads.
class MappedFile {
 public:
  static std::unique_ptr<MappedFile> open(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return nullptr;
    struct stat st {};
    if (::fstat(fd, &st) != 0 || st.st_size <= 0) {
      ::close(fd);
      return nullptr;
    }
    void* p = ::mmap(nullptr, static_cast<size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);  // the mapping keeps the file
    if (p == MAP_FAILED) return nullptr;
    return std::unique_ptr<MappedFile>(new MappedFile(p, static_cast<size_t>(st.st_size)));
  }
  ~MappedFile() { ::munmap(base_, size_); }
  MappedFile(const MappedFile&) = delete;
  MappedFile& operator=(const MappedFile&) = delete;
  // Bytes [at, at + n) of the file, or null when the range is outside it.
  const std::byte* view(uint64_t at, uint64_t n) const {
    if (at > size_ || n > size_ - at) return nullptr;
    return static_cast<const std::byte*>(base_) + at;
  }

 private:
  MappedFile(void* base, size_t size) : base_(base), size_(size) {}
  void* base_;
  size_t size_;
};

}  // namespace

Status GGUFParser::read_tensor_data(const std::string& filename, uint64_t data_offset,
                                    uint64_t tensor_offset, void* dst, size_t byte_count) {
  if (data_offset > std::numeric_limits<uint64_t>::max() - tensor_offset)
    return Status::out_of_range("tensor offset overflow for: " + filename);
  if (auto map = MappedFile::open(filename)) {  // mmap fast path
    const std::byte* src = map->view(data_offset + tensor_offset, byte_count);
    if (!src) return Status::out_of_range("tensor byte range exceeds GGUF file bounds: " + filename);
    std::memcpy(dst, src, byte_count);
    return Status::make_ok();
  }
  FilePtr f(std::fopen(filename.c_str(), "rb"));
  if (!f) return Status::io_error("cannot open file: " + filename);
  const uint64_t at = data_offset + tensor_offset, size = file_size(f.get());
  if (at > size || byte_count > size - at)
    return Status::out_of_range("tensor byte range exceeds GGUF file bounds: " + filename);
  if (at > static_cast<uint64_t>(std::numeric_limits<off_t>::max()) ||
      fseeko(f.get(), static_cast<off_t>(at), SEEK_SET) != 0)
    return Status::io_error("cannot seek to tensor data in: " + filename);
  if (std::fread(dst, 1, byte_count, f.get()) != byte_count)
    return Status::io_error("short read of tensor data from: " + filename);
  return Status::make_ok();
}

// ---------------------------------------------------------------- weight loader
namespace {

// IEEE binary16 -> binary32, exact (subnormals scaled by 2^-24, Inf kept, NaN quiet).
float half_to_float(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h >> 15) << 31;
  const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
  float mag;
  if (e == 0) {
    mag = static_cast<float>(m) * 0x1p-24f;
  } else if (e == 31) {
    uint32_t bits = 0x7f800000u | (m ? 0x00400000u | (m << 13) : 0u);
    std::memcpy(&mag, &bits, 4);
  } else {
    uint32_t bits = ((e + 112u) << 23) | (m << 13);
    std::memcpy(&mag, &bits, 4);
  }
  uint32_t out;
  std::memcpy(&out, &mag, 4);
  out |= sign;
  float r;
  std::memcpy(&r, &out, 4);
  return r;
}

float bfloat_to_float(uint16_t b) {
  const uint32_t bits = static_cast<uint32_t>(b) << 16;
  float r;
  std::memcpy(&r, &bits, 4);
  return r;
}

Status hip_copy(void* dst, const void* src, size_t bytes, const char* what) {
  const hipError_t e = hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
  if (e == hipSuccess) return Status::make_ok();
  return Status::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Reads a tensor's raw bytes from the file (streaming fallback of the mmap view).
expected<std::vector<std::byte>, Status> read_raw(const std::string& path, const GGUFFile& file,
                                                   const GGUFTensorInfo& ti) {
  auto nbytes = ti.bytes();
  if (!nbytes) return unexpected(nbytes.error());
  std::vector<std::byte> raw(*nbytes);
  auto st = GGUFParser::read_tensor_data(path, file.data_offset, ti.offset, raw.data(),
                                         raw.size());
  if (!st.ok()) return unexpected(st);
  return raw;
}

// Raw-byte payloads (Q8_0 -> Q8_0, BF16 -> BFloat16) are copied as stored; any
// other pair is decoded to fp32.  Mirrors the reference's load_tensor_from_gguf
// (src/io/gguf_weight_loader.cpp:85-191) with HIP in place of CUDA.
// The tensor's bytes: a view into the mapped file when there is one (no host
// copy; the HIP branch copies straight from it, as the reference's CUDA branch
// copies from its raw view), else a buffer read from the file.
struct RawBytes {
  std::vector<std::byte> owned;
  const std::byte* ptr = nullptr;
  size_t n = 0;
  const std::byte* data() const { return ptr; }
  size_t size() const { return n; }
};

expected<RawBytes, Status> tensor_bytes(const std::string& path, const GGUFFile& file,
                                        const GGUFTensorInfo& ti, const MappedFile* map) {
  RawBytes r;
  if (map) {
    auto nbytes = ti.bytes();
    if (!nbytes) return unexpected(nbytes.error());
    if (file.data_offset > std::numeric_limits<uint64_t>::max() - ti.offset)
      return unexpected(Status::out_of_range("tensor offset overflow for: " + path));
    r.ptr = map->view(file.data_offset + ti.offset, *nbytes);
    if (!r.ptr)
      return unexpected(
          Status::out_of_range("tensor byte range exceeds GGUF file bounds: " + path));
    r.n = *nbytes;
    return r;
  }
  auto raw = read_raw(path, file, ti);
  if (!raw) return unexpected(raw.error());
  r.owned = std::move(*raw);
  r.ptr = r.owned.data();
  r.n = r.owned.size();
  return r;
}

Status load_tensor(const std::string& path, const GGUFFile& file, const GGUFTensorInfo& ti,
                   Tensor& tensor, const MappedFile* map) {
  if (!tensor.is_allocated()) return Status::runtime_error("tensor not allocated: " + tensor.name());
  // Storage re-tiled in place (HipExecutor::tile_weights) holds 16-row tiles;
  // raw GGUF bytes written into it would be read as tiles.  Refilling it needs
  // a fresh allocation, which resets the layout to Raw.
  if (tensor.storage_layout() != StorageLayout::Raw)
    return Status::invalid_argument("tensor " + tensor.name() +
                                    " holds Q8_0 16-row tiles; reallocate it before loading "
                                    "raw GGUF bytes into it");
  auto raw = tensor_bytes(path, file, ti, map);
  if (!raw) return raw.error();
  auto numel = ti.num_elements();
  if (!numel) return numel.error();
  const bool hip = tensor.device().type == DeviceType::HIP;
  const char* where = hip ? "HIP " : "";

  const bool raw_q8 = ti.dtype == GgmlDataType::Q8_0 && tensor.dtype() == DType::Q8_0;
  const bool raw_bf16 = ti.dtype == GgmlDataType::BF16 && tensor.dtype() == DType::BFloat16;
  if (tensor.dtype() == DType::BFloat16 && !raw_bf16)
    return Status::unsupported("native BF16 weight load requires a BF16 GGUF tensor: " +
                               tensor.name());
  if (raw_q8 || raw_bf16) {
    const size_t need = raw->size();
    if (tensor.allocated_bytes() < need)
      return Status::out_of_range(std::string(where) + ggml_dtype_name(ti.dtype).data() +
                                  " tensor storage too small for " + tensor.name());
    if (hip) return hip_copy(tensor.data(), raw->data(), need, "copy GGUF weight to HIP tensor failed");
    std::memcpy(tensor.data(), raw->data(), need);
    return Status::make_ok();
  }
  if (tensor.dtype() != DType::Float32)
    return Status::unsupported(
        "GGUF weight loader supports Float32, native BF16, and native Q8_0 tensors only: " +
        tensor.name());
  if (*numel > std::numeric_limits<size_t>::max() / sizeof(float))
    return Status::invalid_argument("weight byte size overflow for tensor " + tensor.name());
  if (tensor.allocated_bytes() < *numel * sizeof(float))
    return Status::out_of_range(std::string(where) + "F32 tensor storage too small for " +
                                tensor.name());
  if (!hip) {
    return WeightLoader::dequantize_to_f32(ti.dtype, raw->data(),
                                           static_cast<float*>(tensor.data()), *numel);
  }
  if (ti.dtype == GgmlDataType::Q8_0) {
    // Raw blocks to the device, dequantised there (hip::dequantize_q8_0): the
    // host touches 34 bytes per 32 elements instead of 128, and decodes nothing.
    void* dev_raw = nullptr;
    hipError_t e = hipMalloc(&dev_raw, raw->size());
    if (e != hipSuccess)
      return Status::runtime_error(std::string("HIP staging allocation for ") + tensor.name() +
                                   " failed: " + hipGetErrorString(e));
    Status st = hip_copy(dev_raw, raw->data(), raw->size(), "copy GGUF weight to HIP tensor failed");
    if (st.ok())
      st = hip::dequantize_q8_0(static_cast<const uint8_t*>(dev_raw),
                                static_cast<float*>(tensor.data()),
                                static_cast<int64_t>(*numel), nullptr);
    if (st.ok()) {
      e = hipStreamSynchronize(nullptr);
      if (e != hipSuccess) st = Status::runtime_error(std::string("HIP dequantize failed: ") + hipGetErrorString(e));
    }
    (void)hipFree(dev_raw);
    return st;
  }
  std::vector<float> staging(*numel);
  TRY(WeightLoader::dequantize_to_f32(ti.dtype, raw->data(), staging.data(), *numel));
  return hip_copy(tensor.data(), staging.data(), *numel * sizeof(float),
                  "copy GGUF weight to HIP tensor failed");
}

Status check_compatible(const Tensor& tensor, const Value& value) {
  if (tensor.shape() != value.shape)
    return Status::shape_mismatch("shared weight shape mismatch for " + value.name +
                                  ": tensor " + tensor.shape().to_string() + " vs value " +
                                  value.shape.to_string());
  // Packed weights serve Float32 graph values: kernels dispatch on the physical dtype.
  const bool dtype_ok = tensor.dtype() == value.dtype ||
                        (value.dtype == DType::Float32 &&
                         (tensor.dtype() == DType::Q8_0 || tensor.dtype() == DType::BFloat16));
  if (!dtype_ok) return Status::type_error("shared weight dtype mismatch for " + value.name);
  if (!(tensor.device() == value.device))
    return Status::runtime_error("shared weight device mismatch for " + value.name +
                                 ": tensor " + tensor.device().to_string() + " vs value " +
                                 value.device.to_string());
  return Status::make_ok();
}

// value name -> GGUF name, with the tied-embedding fallback for lm_head.
std::unordered_map<std::string, std::string> value_to_gguf(const GGUFFile& file) {
  std::unordered_map<std::string, std::string> map;
  for (const auto& ti : file.tensor_infos) {
    auto v = WeightLoader::gguf_name_to_value_name(ti.name);
    if (v) map[*v] = ti.name;
  }
  if (!map.count("lm_head.weight") && map.count("tok_embeddings.weight"))
    map["lm_head.weight"] = map["tok_embeddings.weight"];
  return map;
}

}  // namespace

Tensor* SharedWeightStore::get(const std::string& value_name) const {
  auto it = aliases_by_value_name_.find(value_name);
  return it == aliases_by_value_name_.end() ? nullptr : it->second;
}

Status SharedWeightStore::bind(const Graph& graph, RuntimeContext& ctx) const {
  for (const auto& v : graph.values()) {
    if (v.kind != ValueKind::Constant) continue;
    Tensor* t = get(v.name);
    if (!t) continue;
    TRY(check_compatible(*t, v));
    TRY(ctx.bind(v.id, t));
  }
  return Status::make_ok();
}

WeightLoader::WeightLoader(std::string gguf_path) : gguf_path_(std::move(gguf_path)) {}

expected<GGUFFile, Status> WeightLoader::open() { return GGUFParser::parse(gguf_path_); }

expected<std::string, Status> WeightLoader::gguf_name_to_value_name(const std::string& gguf_name,
                                                                    int layer_index) {
  (void)layer_index;
  // GGUF tensor names and the graph value names they bind to (the naming
  // contract of the reference's graph builder).
  static const std::pair<const char*, const char*> kLayer[] = {
      {"attn_norm.weight", "attn_norm.weight"},   {"attn_q.weight", "q_proj.weight"},
      {"attn_k.weight", "k_proj.weight"},         {"attn_v.weight", "v_proj.weight"},
      {"attn_q_norm.weight", "q_norm.weight"},    {"attn_k_norm.weight", "k_norm.weight"},
      {"attn_output.weight", "o_proj.weight"},    {"ffn_norm.weight", "ffn_norm.weight"},
      {"ffn_gate.weight", "gate_proj.weight"},    {"ffn_up.weight", "up_proj.weight"},
      {"ffn_down.weight", "down_proj.weight"},
  };
  static const std::pair<const char*, const char*> kGlobal[] = {
      {"token_embd.weight", "tok_embeddings.weight"},
      {"output_norm.weight", "output_norm.weight"},
      {"output.weight", "lm_head.weight"},
  };
  if (gguf_name.rfind("blk.", 0) == 0) {
    const size_t dot = gguf_name.find('.', 4);
    if (dot != std::string::npos) {
      const std::string idx = gguf_name.substr(4, dot - 4);
      if (idx.empty() || idx.find_first_not_of("0123456789") != std::string::npos)
        return unexpected(
            Status::invalid_argument("non-numeric layer index in GGUF tensor: " + gguf_name));
      if (idx.size() > 9)
        return unexpected(
            Status::invalid_argument("invalid layer index in GGUF tensor: " + gguf_name));
      const std::string suffix = gguf_name.substr(dot + 1);
      for (const auto& [g, v] : kLayer)
        if (suffix == g) return "layer_" + std::to_string(std::stoi(idx)) + "." + v;
    }
  }
  for (const auto& [g, v] : kGlobal)
    if (gguf_name == g) return std::string(v);
  return unexpected(Status::not_found("no mapping for GGUF tensor: " + gguf_name));
}

Status WeightLoader::dequantize_to_f32(GgmlDataType src_dtype, const void* src, float* dst,
                                       size_t num_elements) {
  const auto* b = static_cast<const uint8_t*>(src);
  switch (src_dtype) {
    case GgmlDataType::F32:
      std::memcpy(dst, src, num_elements * sizeof(float));
      return Status::make_ok();
    case GgmlDataType::F16:
      for (size_t i = 0; i < num_elements; ++i)
        dst[i] = half_to_float(static_cast<uint16_t>(b[2 * i] | (b[2 * i + 1] << 8)));
      return Status::make_ok();
    case GgmlDataType::BF16:
      for (size_t i = 0; i < num_elements; ++i)
        dst[i] = bfloat_to_float(static_cast<uint16_t>(b[2 * i] | (b[2 * i + 1] << 8)));
      return Status::make_ok();
    case GgmlDataType::Q8_0:
      for (size_t i = 0; i < num_elements; ++i) {
        const uint8_t* blk = b + (i / kQ8_0BlockElems) * kQ8_0BlockBytes;
        const float d = half_to_float(static_cast<uint16_t>(blk[0] | (blk[1] << 8)));
        dst[i] = static_cast<float>(static_cast<int8_t>(blk[2 + i % kQ8_0BlockElems])) * d;
      }
      return Status::make_ok();
    default:
      return Status::unsupported("cannot dequantize GGML dtype " +
                                 std::string(ggml_dtype_name(src_dtype)));
  }
}

Status WeightLoader::load_weights(const GGUFFile& file, const Graph& graph,
                                  RuntimeContext& ctx) const {
  const auto names = value_to_gguf(file);
  const auto map = MappedFile::open(gguf_path_);  // null: streamed reads
  for (const auto& v : graph.values()) {
    if (v.kind != ValueKind::Constant) continue;
    auto it = names.find(v.name);
    if (it == names.end()) continue;
    const GGUFTensorInfo* ti = file.find_tensor(it->second);
    Tensor* t = ctx.get(v.id);
    if (!t) return Status::runtime_error("tensor not found in RuntimeContext for value: " + v.name);
    TRY(load_tensor(gguf_path_, file, *ti, *t, map.get()));
  }
  return Status::make_ok();
}

expected<SharedWeightStore, Status> WeightLoader::load_shared_weights(const GGUFFile& file,
                                                                      const Graph& graph) const {
  const auto names = value_to_gguf(file);
  const auto map = MappedFile::open(gguf_path_);  // null: streamed reads
  SharedWeightStore store;
  for (const auto& v : graph.values()) {
    if (v.kind != ValueKind::Constant) continue;
    auto it = names.find(v.name);
    if (it == names.end()) continue;
    const std::string& gguf_name = it->second;
    const GGUFTensorInfo* ti = file.find_tensor(gguf_name);
    if (!ti) return unexpected(Status::not_found("GGUF tensor not found for value: " + v.name));

    Tensor* shared = nullptr;
    auto existing = store.storage_by_gguf_name_.find(gguf_name);
    if (existing == store.storage_by_gguf_name_.end()) {
      // Packed formats stay packed (the kernels consume them); the rest is fp32.
      DType dt = DType::Float32;
      if (ti->dtype == GgmlDataType::Q8_0) dt = DType::Q8_0;
      if (ti->dtype == GgmlDataType::BF16) dt = DType::BFloat16;
      auto tensor = std::make_unique<Tensor>(v.name, v.shape, dt, v.device);
      size_t loaded = 0;
      Status st;
      if (dt == DType::Q8_0) {
        auto raw = ti->bytes();
        if (!raw) return unexpected(raw.error());
        st = v.device.type == DeviceType::HIP ? tensor->allocate_hip_bytes(*raw)
                                              : tensor->allocate_cpu_bytes(*raw);
        loaded = *raw;
      } else {
        st = v.device.type == DeviceType::HIP ? tensor->allocate_hip() : tensor->allocate_cpu();
        auto nb = tensor->nbytes();
        if (!nb) return unexpected(nb.error());
        loaded = *nb;
      }
      if (!st.ok()) return unexpected(st);
      st = load_tensor(gguf_path_, file, *ti, *tensor, map.get());
      if (!st.ok()) return unexpected(st);
      shared = tensor.get();
      store.total_bytes_ += loaded;
      store.storage_by_gguf_name_[gguf_name] = std::move(tensor);
    } else {
      shared = existing->second.get();
      auto st = check_compatible(*shared, v);
      if (!st.ok()) return unexpected(st);
    }
    store.aliases_by_value_name_[v.name] = shared;
  }
  return store;
}

}  // namespace minillm
