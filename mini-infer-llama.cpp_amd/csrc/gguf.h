// gguf.h -- read-only GGUF v3 model files (the format src/gguf.cpp:259-436
// parses): memory-mapped, metadata keys and the tensor table, every tensor's
// data resolved to an address inside the mapping. Tensor types F32, F16 and
// Q8_0 only, as the engine.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace mi {

enum GgufValueType : uint32_t {
  kGgufU8 = 0, kGgufI8 = 1, kGgufU16 = 2, kGgufI16 = 3, kGgufU32 = 4, kGgufI32 = 5,
  kGgufF32 = 6, kGgufBool = 7, kGgufString = 8, kGgufArray = 9, kGgufU64 = 10,
  kGgufI64 = 11, kGgufF64 = 12,
};

enum GgufTensorType : uint32_t { kGgufTF32 = 0, kGgufTF16 = 1, kGgufTQ8_0 = 8 };

struct GgufValue {
  uint32_t type = 0;
  uint64_t u = 0;  // unsigned, signed (two's complement) and bool scalars
  double f = 0;    // F32 / F64
  std::string s;
  uint32_t arr_type = 0;  // arrays: element type and count (elements are skipped)
  uint64_t arr_n = 0;
};

struct GgufTensor {
  std::string name;
  int n_dims = 0;
  int64_t ne[4] = {1, 1, 1, 1};
  uint32_t type = 0;
  uint64_t offset = 0;  // within the data section
  const uint8_t* data = nullptr;
  size_t nbytes = 0;
  size_t row_bytes = 0;  // bytes of one ne[0] row
};

class GgufFile {
 public:
  GgufFile() = default;
  GgufFile(const GgufFile&) = delete;
  GgufFile& operator=(const GgufFile&) = delete;
  ~GgufFile();

  // Returns false with a message in *err on any malformed or unsupported input.
  bool open(const char* path, std::string* err);
  void close();

  bool get_u32(const char* key, uint32_t* v) const;
  bool get_f32(const char* key, float* v) const;
  const GgufValue* find_kv(const char* key) const;
  const GgufTensor* find_tensor(const char* name) const;
  size_t alignment() const { return alignment_; }
  const std::vector<GgufTensor>& tensors() const { return tensors_; }

 private:
  void* map_ = nullptr;
  size_t size_ = 0;
  int fd_ = -1;
  size_t alignment_ = 32;
  std::unordered_map<std::string, GgufValue> kv_;
  std::vector<GgufTensor> tensors_;
  std::unordered_map<std::string, size_t> index_;
};

}  // namespace mi
