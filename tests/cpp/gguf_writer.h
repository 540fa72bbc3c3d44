// gguf_writer.h -- builds small GGUF v3 files for the loader tests (test
// infrastructure; the product only reads GGUF).  Layout per the GGUF v3 spec:
// magic, version, tensor count, metadata count, metadata key/type/value
// records, tensor infos (name, rank, dims innermost first, type, offset), zero
// padding to the alignment, then the tensor data, each tensor starting on an
// alignment boundary.
#pragma once

#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

struct GgufWriter {
  struct TensorRec {
    std::string name;
    std::vector<int64_t> dims;  // row-major, outermost first
    uint32_t type;
    std::vector<uint8_t> data;
  };

  uint32_t version = 3;
  uint32_t alignment = 32;
  std::string magic = "GGUF";
  std::vector<uint8_t> kv;
  uint64_t n_kv = 0;
  std::vector<TensorRec> tensors;

  static void put(std::vector<uint8_t>& o, const void* p, size_t n) {
    const auto* b = static_cast<const uint8_t*>(p);
    o.insert(o.end(), b, b + n);
  }
  template <typename T>
  static void put_le(std::vector<uint8_t>& o, T v) {
    uint8_t b[sizeof(T)];
    std::memcpy(b, &v, sizeof(T));  // the test hosts are little-endian
    put(o, b, sizeof(T));
  }
  static void put_str(std::vector<uint8_t>& o, const std::string& s) {
    put_le<uint64_t>(o, s.size());
    put(o, s.data(), s.size());
  }

  void kv_u32(const std::string& k, uint32_t v) {
    put_str(kv, k);
    put_le<uint32_t>(kv, 4);
    put_le<uint32_t>(kv, v);
    ++n_kv;
  }
  void kv_f32(const std::string& k, float v) {
    put_str(kv, k);
    put_le<uint32_t>(kv, 6);
    put_le<float>(kv, v);
    ++n_kv;
  }
  void kv_str(const std::string& k, const std::string& v) {
    put_str(kv, k);
    put_le<uint32_t>(kv, 8);
    put_str(kv, v);
    ++n_kv;
  }
  void kv_str_array(const std::string& k, const std::vector<std::string>& v) {
    put_str(kv, k);
    put_le<uint32_t>(kv, 9);
    put_le<uint32_t>(kv, 8);
    put_le<uint64_t>(kv, v.size());
    for (const auto& s : v) put_str(kv, s);
    ++n_kv;
  }
  void tensor(const std::string& name, std::vector<int64_t> dims, uint32_t type,
              std::vector<uint8_t> data) {
    tensors.push_back({name, std::move(dims), type, std::move(data)});
  }

  std::vector<uint8_t> bytes() const {
    std::vector<uint8_t> o;
    put(o, magic.data(), 4);
    put_le<uint32_t>(o, version);
    put_le<uint64_t>(o, tensors.size());
    put_le<uint64_t>(o, n_kv);
    put(o, kv.data(), kv.size());
    uint64_t off = 0;
    std::vector<uint64_t> offs;
    for (const auto& t : tensors) {
      offs.push_back(off);
      off += (t.data.size() + alignment - 1) / alignment * alignment;
    }
    for (size_t i = 0; i < tensors.size(); ++i) {
      const auto& t = tensors[i];
      put_str(o, t.name);
      put_le<uint32_t>(o, static_cast<uint32_t>(t.dims.size()));
      for (size_t d = t.dims.size(); d-- > 0;) put_le<uint64_t>(o, static_cast<uint64_t>(t.dims[d]));
      put_le<uint32_t>(o, t.type);
      put_le<uint64_t>(o, offs[i]);
    }
    while (o.size() % alignment) o.push_back(0);
    for (const auto& t : tensors) {
      put(o, t.data.data(), t.data.size());
      while (o.size() % alignment) o.push_back(0);
    }
    return o;
  }

  // Writes the file; returns its path (under TMPDIR or /tmp).
  std::string write(const std::string& stem) const {
    const char* dir = std::getenv("TMPDIR");
    std::string path = std::string(dir && *dir ? dir : "/tmp") + "/" + stem + "_" +
                       std::to_string(static_cast<long>(getpid())) + ".gguf";
    const auto b = bytes();
    std::FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(b.data(), 1, b.size(), f) != b.size()) {
      std::fprintf(stderr, "cannot write %s\n", path.c_str());
      std::abort();
    }
    std::fclose(f);
    return path;
  }
};
