// GGUF model files (v2 and v3): header, metadata, tensor table and memory-mapped
// tensor bytes, with the checks and messages of the reference's reader
// (src/runtime/gguf_reader.cpp, interface include/toyllm/runtime/gguf_reader.hpp).
//
// Layout: magic "GGUF" (u32 0x46554747), version u32, tensor count u64,
// metadata count u64; metadata entries (key string, value type u32, value);
// tensor entries (name string, rank u32, dims u64[rank] innermost first, ggml
// type u32, offset u64 relative to the data section); the data section starts
// at the first multiple of general.alignment (default 32) after the tables.
// Strings are a u64 length and bytes; arrays an element type u32, a u64 count
// and the elements.  All little-endian.
#pragma once

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "kraken/hip_context.hpp"

namespace kraken::gguf {

using hip::Result;
using hip::Status;

// GGUF metadata value types 0..12.
enum class ValueKind : std::uint32_t {
  uint8 = 0, int8, uint16, int16, uint32, int32, float32, boolean, string, array, uint64, int64,
  float64,
};

struct MetadataValue {
  ValueKind kind{ValueKind::string};
  ValueKind array_kind{ValueKind::string};  // element type when kind == array
  // Scalars: unsigned kinds in u, signed in i, floats in f, bool in b, string in s.
  std::uint64_t u{0};
  std::int64_t i{0};
  double f{0.0};
  bool b{false};
  std::string s;
  // Arrays: one of these holds the elements, by element kind as for scalars.
  std::vector<std::uint64_t> ua;
  std::vector<std::int64_t> ia;
  std::vector<double> fa;
  std::vector<bool> ba;
  std::vector<std::string> sa;
  std::uint64_t count{0};
};

struct TensorInfo {
  std::string name;
  std::vector<std::uint64_t> shape;  // innermost dimension first
  std::uint32_t type{0};             // ggml type id
  std::uint64_t offset{0};           // from the data section
  std::uint64_t absolute_offset{0};  // from the file start
  std::uint64_t byte_size{0};
};

struct File {
  std::string path;
  std::uint32_t version{0};
  std::uint64_t tensor_count{0};
  std::uint64_t metadata_count{0};
  std::uint64_t file_size{0};
  std::uint64_t alignment{32};
  std::uint64_t data_offset{0};
  std::vector<TensorInfo> tensors;
  std::unordered_map<std::string, MetadataValue> metadata;
};

namespace detail {

constexpr std::uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian
constexpr std::uint64_t kDefaultAlignment = 32;

// A read-only mapping of a whole file, closed on destruction.
class Mapping {
 public:
  Mapping() = default;
  Mapping(const Mapping&) = delete;
  Mapping& operator=(const Mapping&) = delete;
  ~Mapping() {
    if (data_ != nullptr) {
      (void)::munmap(const_cast<unsigned char*>(data_), static_cast<std::size_t>(size_));
    }
    if (fd_ >= 0) {
      (void)::close(fd_);
    }
  }
  // Empty message on success.
  std::string open(const std::string& path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) {
      return "failed to open GGUF data file: " + path;
    }
    struct stat st {};
    if (::fstat(fd_, &st) != 0 || st.st_size <= 0) {
      return "invalid GGUF data file size: " + path;
    }
    size_ = static_cast<std::uint64_t>(st.st_size);
    void* m = ::mmap(nullptr, static_cast<std::size_t>(size_), PROT_READ, MAP_PRIVATE, fd_, 0);
    if (m == MAP_FAILED) {
      return "failed to mmap GGUF data file: " + path;
    }
    data_ = static_cast<const unsigned char*>(m);
    return {};
  }
  [[nodiscard]] const unsigned char* data() const { return data_; }
  [[nodiscard]] std::uint64_t size() const { return size_; }

 private:
  int fd_{-1};
  const unsigned char* data_{nullptr};
  std::uint64_t size_{0};
};

// Bounded little-endian cursor; a read past the end throws with its position.
class Cursor {
 public:
  Cursor(const unsigned char* data, std::uint64_t size) : data_(data), size_(size) {}
  [[nodiscard]] std::uint64_t position() const { return pos_; }

  template <typename T>
  T pod() {
    need(sizeof(T));
    T v;
    std::memcpy(&v, data_ + pos_, sizeof(T));
    pos_ += sizeof(T);
    return v;
  }
  std::string string() {
    const auto n = pod<std::uint64_t>();
    need(n);
    std::string s(reinterpret_cast<const char*>(data_ + pos_), static_cast<std::size_t>(n));
    pos_ += n;
    return s;
  }
  [[noreturn]] void fail(const std::string& what) const {
    throw std::runtime_error(what + " at byte " + std::to_string(pos_));
  }

 private:
  void need(std::uint64_t n) const {
    if (n > size_ || pos_ > size_ - n) {
      fail("unexpected end of GGUF file");
    }
  }
  const unsigned char* data_;
  std::uint64_t size_;
  std::uint64_t pos_{0};
};

inline ValueKind value_kind(std::uint32_t t) {
  if (t > 12) {
    throw std::runtime_error("unsupported GGUF metadata value type: " + std::to_string(t));
  }
  return static_cast<ValueKind>(t);
}

// Reads one scalar of `kind` into the matching field of `v`.
inline void read_scalar(Cursor& c, ValueKind kind, MetadataValue& v) {
  switch (kind) {
    case ValueKind::uint8: v.u = c.pod<std::uint8_t>(); break;
    case ValueKind::int8: v.i = c.pod<std::int8_t>(); break;
    case ValueKind::uint16: v.u = c.pod<std::uint16_t>(); break;
    case ValueKind::int16: v.i = c.pod<std::int16_t>(); break;
    case ValueKind::uint32: v.u = c.pod<std::uint32_t>(); break;
    case ValueKind::int32: v.i = c.pod<std::int32_t>(); break;
    case ValueKind::float32: v.f = c.pod<float>(); break;
    case ValueKind::boolean: v.b = c.pod<std::uint8_t>() != 0; break;
    case ValueKind::string: v.s = c.string(); break;
    case ValueKind::uint64: v.u = c.pod<std::uint64_t>(); break;
    case ValueKind::int64: v.i = c.pod<std::int64_t>(); break;
    case ValueKind::float64: v.f = c.pod<double>(); break;
    case ValueKind::array: throw std::runtime_error("nested GGUF arrays are not supported");
  }
}

inline bool is_unsigned(ValueKind k) {
  return k == ValueKind::uint8 || k == ValueKind::uint16 || k == ValueKind::uint32 ||
         k == ValueKind::uint64;
}
inline bool is_signed(ValueKind k) {
  return k == ValueKind::int8 || k == ValueKind::int16 || k == ValueKind::int32 ||
         k == ValueKind::int64;
}
inline bool is_float(ValueKind k) { return k == ValueKind::float32 || k == ValueKind::float64; }

inline MetadataValue read_value(Cursor& c) {
  MetadataValue v;
  v.kind = value_kind(c.pod<std::uint32_t>());
  if (v.kind != ValueKind::array) {
    read_scalar(c, v.kind, v);
    return v;
  }
  v.array_kind = value_kind(c.pod<std::uint32_t>());
  if (v.array_kind == ValueKind::array) {
    throw std::runtime_error("nested GGUF arrays are not supported");
  }
  v.count = c.pod<std::uint64_t>();
  for (std::uint64_t n = 0; n < v.count; ++n) {
    MetadataValue e;
    read_scalar(c, v.array_kind, e);
    if (is_unsigned(v.array_kind)) {
      v.ua.push_back(e.u);
    } else if (is_signed(v.array_kind)) {
      v.ia.push_back(e.i);
    } else if (is_float(v.array_kind)) {
      v.fa.push_back(e.f);
    } else if (v.array_kind == ValueKind::boolean) {
      v.ba.push_back(e.b);
    } else {
      v.sa.push_back(std::move(e.s));
    }
  }
  return v;
}

inline std::uint64_t align_up(std::uint64_t value, std::uint64_t alignment) {
  if (alignment == 0) {
    throw std::runtime_error("GGUF alignment must be non-zero");
  }
  const std::uint64_t r = value % alignment;
  if (r == 0) {
    return value;
  }
  if (value > std::numeric_limits<std::uint64_t>::max() - (alignment - r)) {
    throw std::runtime_error("GGUF alignment overflow");
  }
  return value + (alignment - r);
}

// ggml's block layouts by type id: (values per block, bytes per block); {0, 0}
// marks ids that are unassigned or retired, which are rejected.
struct Layout {
  std::uint64_t block;
  std::uint64_t bytes;
};
inline Layout type_layout(std::uint32_t type) {
  static const Layout table[] = {
    {1, 4},    {1, 2},     {32, 18},  {32, 20},  {0, 0},    {0, 0},    {32, 22},  {32, 24},
    {32, 34},  {32, 36},   {256, 84}, {256, 110}, {256, 144}, {256, 176}, {256, 210}, {256, 292},
    {256, 66}, {256, 74},  {256, 98}, {256, 50},  {32, 18},   {256, 110}, {256, 82},  {256, 136},
    {1, 1},    {1, 2},     {1, 4},    {1, 8},     {1, 8},     {256, 56},  {1, 2},     {0, 0},
    {0, 0},    {0, 0},     {256, 54}, {256, 66},  {0, 0},     {0, 0},     {0, 0},     {32, 17},
    {64, 36},  {128, 18},
  };
  if (type >= sizeof(table) / sizeof(table[0]) || table[type].block == 0) {
    throw std::runtime_error("unsupported GGML tensor type: " + std::to_string(type));
  }
  return table[type];
}

inline std::uint64_t tensor_bytes_of(const TensorInfo& t) {
  std::uint64_t elements = 1;
  for (const std::uint64_t d : t.shape) {
    if (d != 0 && elements > std::numeric_limits<std::uint64_t>::max() / d) {
      throw std::runtime_error("GGUF tensor shape product overflow");
    }
    elements *= d;
  }
  const Layout l = type_layout(t.type);
  if (elements % l.block != 0) {
    throw std::runtime_error("GGUF tensor element count is not divisible by block size: " +
                             t.name);
  }
  const std::uint64_t blocks = elements / l.block;
  if (l.bytes != 0 && blocks > std::numeric_limits<std::uint64_t>::max() / l.bytes) {
    throw std::runtime_error("GGUF tensor byte size overflow: " + t.name);
  }
  return blocks * l.bytes;
}

}  // namespace detail

// read_gguf_file (gguf_reader.cpp:548-620): parses the header and tables and
// checks every tensor's byte range against the file size.
[[nodiscard]] inline Result<File> read_file(const std::string& path) {
  detail::Mapping m;
  const std::string err = m.open(path);
  if (!err.empty()) {
    return Status::invalid_argument(err);
  }
  try {
    detail::Cursor c(m.data(), m.size());
    if (c.pod<std::uint32_t>() != detail::kMagic) {
      return Status::invalid_argument("not a GGUF file: " + path);
    }
    File f;
    f.path = path;
    f.file_size = m.size();
    f.version = c.pod<std::uint32_t>();
    if (f.version < 2 || f.version > 3) {
      return Status::invalid_argument("unsupported GGUF version: " + std::to_string(f.version));
    }
    f.tensor_count = c.pod<std::uint64_t>();
    f.metadata_count = c.pod<std::uint64_t>();
    for (std::uint64_t n = 0; n < f.metadata_count; ++n) {
      std::string key = c.string();
      f.metadata.emplace(std::move(key), detail::read_value(c));
    }
    const auto a = f.metadata.find("general.alignment");
    f.alignment = a != f.metadata.end() && detail::is_unsigned(a->second.kind)
                    ? a->second.u
                    : detail::kDefaultAlignment;
    for (std::uint64_t n = 0; n < f.tensor_count; ++n) {
      TensorInfo t;
      t.name = c.string();
      const auto rank = c.pod<std::uint32_t>();
      if (rank == 0 || rank > 4) {
        return Status::invalid_argument("invalid GGUF tensor rank for " + t.name);
      }
      for (std::uint32_t d = 0; d < rank; ++d) {
        t.shape.push_back(c.pod<std::uint64_t>());
      }
      t.type = c.pod<std::uint32_t>();
      t.offset = c.pod<std::uint64_t>();
      t.byte_size = detail::tensor_bytes_of(t);
      f.tensors.push_back(std::move(t));
    }
    f.data_offset = detail::align_up(c.position(), f.alignment);
    if (f.data_offset > f.file_size) {
      return Status::invalid_argument("GGUF data offset exceeds file size");
    }
    for (TensorInfo& t : f.tensors) {
      if (t.offset > f.file_size - f.data_offset) {
        return Status::invalid_argument("GGUF tensor offset exceeds file size: " + t.name);
      }
      t.absolute_offset = f.data_offset + t.offset;
      if (t.byte_size != 0 && t.byte_size > f.file_size - t.absolute_offset) {
        return Status::invalid_argument("GGUF tensor byte range exceeds file size: " + t.name);
      }
    }
    return f;
  } catch (const std::exception& e) {
    return Status::invalid_argument(e.what());
  }
}

[[nodiscard]] inline const TensorInfo* find_tensor(const File& f, const std::string& name) {
  for (const TensorInfo& t : f.tensors) {
    if (t.name == name) {
      return &t;
    }
  }
  return nullptr;
}

[[nodiscard]] inline const MetadataValue* find_metadata(const File& f, const std::string& key) {
  const auto it = f.metadata.find(key);
  return it == f.metadata.end() ? nullptr : &it->second;
}

// gguf_get_i64 (gguf_reader.cpp:830-848): any integer kind that fits int64.
[[nodiscard]] inline Result<std::int64_t> get_i64(const File& f, const std::string& key) {
  const MetadataValue* v = find_metadata(f, key);
  if (v == nullptr) {
    return Status::invalid_argument("missing GGUF metadata key: " + key);
  }
  if (detail::is_signed(v->kind)) {
    return v->i;
  }
  if (detail::is_unsigned(v->kind)) {
    if (v->u > static_cast<std::uint64_t>(std::numeric_limits<std::int64_t>::max())) {
      return Status::invalid_argument("GGUF metadata integer overflows int64: " + key);
    }
    return static_cast<std::int64_t>(v->u);
  }
  return Status::invalid_argument("GGUF metadata key is not integer: " + key);
}

// gguf_get_f64 (gguf_reader.cpp:850-865): any numeric kind.
[[nodiscard]] inline Result<double> get_f64(const File& f, const std::string& key) {
  const MetadataValue* v = find_metadata(f, key);
  if (v == nullptr) {
    return Status::invalid_argument("missing GGUF metadata key: " + key);
  }
  if (detail::is_float(v->kind)) {
    return v->f;
  }
  if (detail::is_signed(v->kind)) {
    return static_cast<double>(v->i);
  }
  if (detail::is_unsigned(v->kind)) {
    return static_cast<double>(v->u);
  }
  return Status::invalid_argument("GGUF metadata key is not numeric: " + key);
}

[[nodiscard]] inline Result<std::string> get_string(const File& f, const std::string& key) {
  const MetadataValue* v = find_metadata(f, key);
  if (v == nullptr) {
    return Status::invalid_argument("missing GGUF metadata key: " + key);
  }
  if (v->kind != ValueKind::string) {
    return Status::invalid_argument("GGUF metadata key is not string: " + key);
  }
  return v->s;
}

// GgufMappedData (gguf_reader.cpp:447-520): the file mapped once, tensor byte
// views into it.  The size must match the one read with the tables.
class MappedData {
 public:
  [[nodiscard]] static Result<MappedData> open(const File& f) {
    MappedData d;
    d.map_ = std::make_unique<detail::Mapping>();
    const std::string err = d.map_->open(f.path);
    if (!err.empty()) {
      return Status::invalid_argument(err);
    }
    if (d.map_->size() != f.file_size) {
      return Status::invalid_argument("GGUF data file size changed after metadata read: " +
                                      f.path);
    }
    return d;
  }
  [[nodiscard]] bool valid() const { return map_ != nullptr && map_->data() != nullptr; }
  [[nodiscard]] Result<std::pair<const unsigned char*, std::size_t>> tensor_bytes(
    const TensorInfo& t) const {
    if (!valid()) {
      return Status::invalid_argument("GGUF mapped data is not initialized");
    }
    if (t.byte_size > std::numeric_limits<std::size_t>::max()) {
      return Status::invalid_argument("GGUF tensor byte size exceeds size_t: " + t.name);
    }
    if (t.absolute_offset > map_->size() || t.byte_size > map_->size() - t.absolute_offset) {
      return Status::invalid_argument("GGUF tensor byte range exceeds mapped file: " + t.name);
    }
    return std::make_pair(map_->data() + t.absolute_offset, static_cast<std::size_t>(t.byte_size));
  }

 private:
  std::unique_ptr<detail::Mapping> map_;
};

}  // namespace kraken::gguf
