// gguf.cpp -- GGUF v3 reader (format of src/gguf.cpp:259-436: magic, version 3,
// u64 tensor and key counts, typed keys, the tensor table, a data section at
// the next multiple of general.alignment (default 32)).
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>

namespace mi {
namespace {

class Cursor {
 public:
  Cursor(const uint8_t* p, size_t n) : p_(p), n_(n) {}
  bool ok() const { return ok_; }
  size_t pos() const { return off_; }
  bool bytes(void* dst, size_t k) {
    if (!ok_ || k > n_ - off_) return ok_ = false;
    std::memcpy(dst, p_ + off_, k);
    off_ += k;
    return true;
  }
  bool skip(uint64_t k) {
    if (!ok_ || k > n_ - off_) return ok_ = false;
    off_ += (size_t)k;
    return true;
  }
  template <typename T>
  bool get(T* v) { return bytes(v, sizeof(T)); }
  bool str(std::string* s) {
    uint64_t len = 0;
    if (!get(&len) || len > n_ - off_) return ok_ = false;
    s->assign(reinterpret_cast<const char*>(p_ + off_), (size_t)len);
    off_ += (size_t)len;
    return true;
  }

 private:
  const uint8_t* p_;
  size_t n_;
  size_t off_ = 0;
  bool ok_ = true;
};

size_t scalar_size(uint32_t t) {
  switch (t) {
    case kGgufU8: case kGgufI8: case kGgufBool: return 1;
    case kGgufU16: case kGgufI16: return 2;
    case kGgufU32: case kGgufI32: case kGgufF32: return 4;
    case kGgufU64: case kGgufI64: case kGgufF64: return 8;
    default: return 0;
  }
}

bool read_scalar(Cursor& c, uint32_t t, GgufValue* v) {
  const size_t k = scalar_size(t);
  if (k == 0) return false;
  uint8_t raw[8] = {0};
  if (!c.bytes(raw, k)) return false;
  if (t == kGgufF32) {
    float f;
    std::memcpy(&f, raw, 4);
    v->f = f;
  } else if (t == kGgufF64) {
    std::memcpy(&v->f, raw, 8);
  } else {
    uint64_t u = 0;
    std::memcpy(&u, raw, k);
    v->u = u;
  }
  return true;
}

bool read_value(Cursor& c, uint32_t t, GgufValue* v) {
  v->type = t;
  if (t == kGgufString) return c.str(&v->s);
  if (t == kGgufArray) {
    if (!c.get(&v->arr_type) || !c.get(&v->arr_n)) return false;
    if (v->arr_type == kGgufString) {
      for (uint64_t i = 0; i < v->arr_n; i++) {
        uint64_t len = 0;
        if (!c.get(&len) || !c.skip(len)) return false;
      }
      return true;
    }
    const size_t k = scalar_size(v->arr_type);
    if (k == 0 || v->arr_n > (uint64_t)1 << 40) return false;  // nested arrays are not used
    return c.skip(v->arr_n * k);
  }
  return read_scalar(c, t, v);
}

size_t type_row_bytes(uint32_t t, int64_t ne0) {
  switch (t) {
    case kGgufTF32: return (size_t)ne0 * 4;
    case kGgufTF16: return (size_t)ne0 * 2;
    case kGgufTQ8_0: return (size_t)(ne0 / 32) * 34;
    default: return 0;
  }
}

}  // namespace

GgufFile::~GgufFile() { close(); }

void GgufFile::close() {
  if (map_) munmap(map_, size_);
  if (fd_ >= 0) ::close(fd_);
  map_ = nullptr;
  fd_ = -1;
  size_ = 0;
  kv_.clear();
  tensors_.clear();
  index_.clear();
}

bool GgufFile::open(const char* path, std::string* err) {
  close();
  auto fail = [&](const std::string& m) {
    if (err) *err = m;
    close();
    return false;
  };
  fd_ = ::open(path, O_RDONLY);
  if (fd_ < 0) return fail(std::string("cannot open '") + path + "': " + std::strerror(errno));
  struct stat st {};
  if (fstat(fd_, &st) != 0) return fail(std::string("fstat: ") + std::strerror(errno));
  size_ = (size_t)st.st_size;
  if (size_ < 24) return fail("file too small to be a GGUF file");
  map_ = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
  if (map_ == MAP_FAILED) {
    map_ = nullptr;
    return fail(std::string("mmap: ") + std::strerror(errno));
  }
  const uint8_t* base = static_cast<const uint8_t*>(map_);
  Cursor c(base, size_);
  char magic[4];
  uint32_t version = 0;
  uint64_t n_tensors = 0, n_kv = 0;
  if (!c.bytes(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return fail("not a GGUF file (bad magic)");
  if (!c.get(&version) || version != 3) return fail("unsupported GGUF version (only v3 is read)");
  if (!c.get(&n_tensors) || !c.get(&n_kv)) return fail("truncated GGUF header");
  for (uint64_t i = 0; i < n_kv; i++) {
    std::string key;
    uint32_t t = 0;
    GgufValue v;
    if (!c.str(&key) || !c.get(&t) || !read_value(c, t, &v)) return fail("truncated or corrupt metadata table");
    kv_[key] = std::move(v);
  }
  const GgufValue* al = find_kv("general.alignment");
  if (al && al->type == kGgufU32) alignment_ = (size_t)al->u;
  if (alignment_ == 0 || (alignment_ & (alignment_ - 1)) != 0)
    return fail("invalid general.alignment (must be a non-zero power of two)");
  for (uint64_t i = 0; i < n_tensors; i++) {
    GgufTensor t;
    uint32_t nd = 0;
    if (!c.str(&t.name) || !c.get(&nd) || nd == 0 || nd > 4) return fail("corrupt tensor table");
    t.n_dims = (int)nd;
    for (uint32_t d = 0; d < nd; d++) {
      uint64_t v = 0;
      if (!c.get(&v) || v == 0 || v > ((uint64_t)1 << 40)) return fail("corrupt tensor table: " + t.name);
      t.ne[d] = (int64_t)v;
    }
    if (!c.get(&t.type) || !c.get(&t.offset)) return fail("corrupt tensor table");
    if (t.type != kGgufTF32 && t.type != kGgufTF16 && t.type != kGgufTQ8_0)
      return fail("unsupported tensor type: name=" + t.name + " type_id=" + std::to_string(t.type));
    if (t.type == kGgufTQ8_0 && t.ne[0] % 32 != 0) return fail("Q8_0 row length not a multiple of 32: " + t.name);
    tensors_.push_back(std::move(t));
  }
  if (!c.ok()) return fail("truncated GGUF file while parsing header tables");
  const size_t data = (c.pos() + alignment_ - 1) / alignment_ * alignment_;
  if (data > size_) return fail("data section start exceeds file size");
  for (size_t i = 0; i < tensors_.size(); i++) {
    GgufTensor& t = tensors_[i];
    t.row_bytes = type_row_bytes(t.type, t.ne[0]);
    t.nbytes = t.row_bytes * (size_t)(t.ne[1] * t.ne[2] * t.ne[3]);
    if (t.offset > size_ - data || t.nbytes > size_ - data - t.offset)
      return fail("tensor '" + t.name + "' data extends past end of file");
    t.data = base + data + t.offset;
    index_[t.name] = i;
  }
  return true;
}

const GgufValue* GgufFile::find_kv(const char* key) const {
  auto it = kv_.find(key);
  return it == kv_.end() ? nullptr : &it->second;
}

bool GgufFile::get_u32(const char* key, uint32_t* v) const {
  const GgufValue* e = find_kv(key);
  if (!e || e->type != kGgufU32) return false;
  *v = (uint32_t)e->u;
  return true;
}

bool GgufFile::get_f32(const char* key, float* v) const {
  const GgufValue* e = find_kv(key);
  if (!e || e->type != kGgufF32) return false;
  *v = (float)e->f;
  return true;
}

const GgufTensor* GgufFile::find_tensor(const char* name) const {
  auto it = index_.find(name);
  return it == index_.end() ? nullptr : &tensors_[it->second];
}

}  // namespace mi
