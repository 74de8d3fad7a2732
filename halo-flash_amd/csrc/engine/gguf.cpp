// GGUF reader (format: magic "GGUF", version 2 or 3, tensor and metadata counts, metadata key / typed value
// pairs, tensor infos, a data section aligned to general.alignment) and the model loader on top of it.
//
// Validation rules follow the reference's reader (src/core/gguf.cpp:358-760) so that the same files open and the
// same files are refused: counts bounded by the bytes left (13 bytes per metadata entry, 32 per tensor info) and a
// 128 MiB budget for host-side descriptors; keys and tensor names 1..65535 bytes; unknown value types, nested
// arrays and booleans other than 0 / 1 refused; general.alignment an unsigned power of two <= 2^32 - 1; duplicate
// keys or tensor names refused; 1..8 dimensions; the encoded size of every tensor nonzero and its first dimension a
// whole number of blocks; tensor offsets aligned and every extent inside the file.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <bit>
#include <cstdio>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include "engine.hpp"
#include "halo_gguf.h"

using namespace halo::engine;

namespace {

struct TypeInfo {
  std::uint32_t block;  // values per block (1 for plain types)
  std::uint32_t bytes;  // bytes per block
};

// Block geometry of the GGML storage types.
bool LookupType(std::uint32_t type, TypeInfo* info) {
  switch (type) {
    case HALO_GGML_F32: *info = {1, 4}; return true;
    case HALO_GGML_I32: *info = {1, 4}; return true;
    case HALO_GGML_F16: *info = {1, 2}; return true;
    case HALO_GGML_BF16: *info = {1, 2}; return true;
    case HALO_GGML_Q4_0: *info = {32, 18}; return true;
    case HALO_GGML_Q4_1: *info = {32, 20}; return true;
    case HALO_GGML_Q5_0: *info = {32, 22}; return true;
    case HALO_GGML_Q5_1: *info = {32, 24}; return true;
    case HALO_GGML_Q8_0: *info = {32, 34}; return true;
    case HALO_GGML_Q8_1: *info = {32, 36}; return true;
    case HALO_GGML_IQ4_NL: *info = {32, 18}; return true;
    case HALO_GGML_Q2_K: *info = {256, 84}; return true;
    case HALO_GGML_Q3_K: *info = {256, 110}; return true;
    case HALO_GGML_Q4_K: *info = {256, 144}; return true;
    case HALO_GGML_Q5_K: *info = {256, 176}; return true;
    case HALO_GGML_Q6_K: *info = {256, 210}; return true;
    case HALO_GGML_Q8_K: *info = {256, 292}; return true;
    case HALO_GGML_IQ2_XXS: *info = {256, 66}; return true;
    case HALO_GGML_IQ3_S: *info = {256, 110}; return true;
    case HALO_GGML_IQ4_XS: *info = {256, 136}; return true;
    default: return false;
  }
}

std::uint64_t EncodedBytes(std::uint32_t type, std::uint64_t elements) {
  TypeInfo ti;
  if (!LookupType(type, &ti) || elements % ti.block != 0) return 0;
  const std::uint64_t blocks = elements / ti.block;
  if (blocks > std::numeric_limits<std::uint64_t>::max() / ti.bytes) return 0;
  return blocks * ti.bytes;
}

const char* TypeName(std::uint32_t type) {
  switch (type) {
    case HALO_GGML_F32: return "F32";
    case HALO_GGML_F16: return "F16";
    case HALO_GGML_Q4_0: return "Q4_0";
    case HALO_GGML_Q4_1: return "Q4_1";
    case HALO_GGML_Q5_0: return "Q5_0";
    case HALO_GGML_Q5_1: return "Q5_1";
    case HALO_GGML_Q8_0: return "Q8_0";
    case HALO_GGML_Q8_1: return "Q8_1";
    case HALO_GGML_Q2_K: return "Q2_K";
    case HALO_GGML_Q3_K: return "Q3_K";
    case HALO_GGML_Q4_K: return "Q4_K";
    case HALO_GGML_Q5_K: return "Q5_K";
    case HALO_GGML_Q6_K: return "Q6_K";
    case HALO_GGML_Q8_K: return "Q8_K";
    case HALO_GGML_IQ2_XXS: return "IQ2_XXS";
    case HALO_GGML_IQ4_NL: return "IQ4_NL";
    case HALO_GGML_IQ3_S: return "IQ3_S";
    case HALO_GGML_IQ4_XS: return "IQ4_XS";
    case HALO_GGML_I32: return "I32";
    case HALO_GGML_BF16: return "BF16";
    default: return "UNKNOWN";
  }
}

// A metadata value. Scalars are widened as the reference stores them: unsigned integers to u64, signed integers to
// i64, floats to f64. Arrays of u32 / u64 / bool become u64 lists, of i32 / i64 i64 lists, of f32 / f64 f64 lists,
// of strings string lists; arrays of 8- and 16-bit integers are skipped (the value carries no elements).
struct Value {
  enum Kind { kU64, kI64, kF64, kBool, kStr, kStrArr, kU64Arr, kI64Arr, kF64Arr, kSkipped };
  std::uint32_t type = 0;      // GGUF value type
  std::uint32_t elem_type = 0; // arrays: element type
  std::uint64_t length = 0;    // arrays: element count
  Kind kind = kU64;
  std::uint64_t u = 0;
  std::int64_t i = 0;
  double f = 0.0;
  std::string_view s;
  std::vector<std::string_view> sa;
  std::vector<std::uint64_t> ua;
  std::vector<std::int64_t> ia;
  std::vector<double> fa;
};

struct Tensor {
  std::string_view name;
  std::uint32_t type = 0, n_dims = 0;
  std::uint64_t dims[8] = {};
  std::uint64_t offset = 0, size_bytes = 0;
  const std::uint8_t* data = nullptr;

  std::uint64_t Elements() const {
    std::uint64_t n = 1;
    for (std::uint32_t k = 0; k < n_dims; ++k) {
      if (dims[k] == 0 || n > std::numeric_limits<std::uint64_t>::max() / dims[k]) return 0;
      n *= dims[k];
    }
    return n_dims ? n : 0;
  }
};

// Bounds-checked cursor over the file bytes.
class Cursor {
 public:
  Cursor(const std::uint8_t* p, std::size_t n) : p_(p), n_(n) {}
  template <typename T>
  bool Pod(T* out) {
    if (at_ > n_ || n_ - at_ < sizeof(T)) return false;
    std::memcpy(out, p_ + at_, sizeof(T));
    at_ += sizeof(T);
    return true;
  }
  bool Str(std::string_view* out) {
    std::uint64_t len;
    if (!Pod(&len) || at_ > n_ || len > n_ - at_) return false;
    *out = std::string_view(reinterpret_cast<const char*>(p_ + at_), static_cast<std::size_t>(len));
    at_ += static_cast<std::size_t>(len);
    return true;
  }
  bool Skip(std::uint64_t bytes) {
    if (at_ > n_ || bytes > n_ - at_) return false;
    at_ += static_cast<std::size_t>(bytes);
    return true;
  }
  std::size_t at() const { return at_; }
  std::size_t left() const { return at_ <= n_ ? n_ - at_ : 0; }

 private:
  const std::uint8_t* p_;
  std::size_t n_;
  std::size_t at_ = 0;
};

}  // namespace

struct halo_gguf {
  const std::uint8_t* data = nullptr;
  std::size_t size = 0;
  void* map = nullptr;
  int fd = -1;
  std::uint32_t version = 0;
  std::uint64_t alignment = 32;
  std::unordered_map<std::string_view, Value> meta;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string_view, std::size_t> index;
  std::vector<std::unique_ptr<halo_gguf>> shards;  // split sets: the shards own the mappings

  ~halo_gguf() {
    if (map != nullptr) munmap(map, size);
    if (fd >= 0) close(fd);
  }

  const Value* Find(const char* key) const {
    if (key == nullptr) return nullptr;
    auto it = meta.find(std::string_view(key));
    return it == meta.end() ? nullptr : &it->second;
  }
  // A skipped array reads as the integer 0 through the integer getters, as in the reference (its value variant
  // stays default-initialized).
  bool U32(const char* key, std::uint32_t* out) const {
    const Value* v = Find(key);
    if (v == nullptr) return false;
    if (v->kind == Value::kSkipped) return *out = 0, true;
    if (v->kind == Value::kU64 && v->u <= 0xFFFFFFFFull) return *out = static_cast<std::uint32_t>(v->u), true;
    if (v->kind == Value::kI64 && v->i >= 0 && v->i <= 0xFFFFFFFFll) return *out = static_cast<std::uint32_t>(v->i), true;
    return false;
  }
  bool U64(const char* key, std::uint64_t* out) const {
    const Value* v = Find(key);
    if (v == nullptr) return false;
    if (v->kind == Value::kSkipped) return *out = 0, true;
    if (v->kind == Value::kU64) return *out = v->u, true;
    if (v->kind == Value::kI64 && v->i >= 0) return *out = static_cast<std::uint64_t>(v->i), true;
    return false;
  }
  bool Str(const char* key, std::string_view* out) const {
    const Value* v = Find(key);
    if (v == nullptr || v->kind != Value::kStr) return false;
    *out = v->s;
    return true;
  }

  bool Parse(std::string* why);
};

bool halo_gguf::Parse(std::string* why) {
  auto fail = [&](const char* msg) {
    if (why->empty()) *why = msg;
    return false;
  };
  if (size < 24) return fail("file too small for a GGUF header");
  if (std::memcmp(data, "GGUF", 4) != 0) return fail("bad GGUF magic");
  Cursor c(data, size);
  c.Skip(4);
  std::uint64_t n_tensors = 0, n_meta = 0;
  if (!c.Pod(&version)) return fail("truncated version");
  if (version != 2 && version != 3) return fail("unsupported GGUF version");
  if (!c.Pod(&n_tensors) || !c.Pod(&n_meta)) return fail("truncated counts");
  // host descriptor budget
  std::size_t budget = std::size_t{128} << 20;
  auto charge = [&](std::uint64_t count, std::size_t each) {
    if (count > budget / each) return false;
    budget -= static_cast<std::size_t>(count) * each;
    return true;
  };
  // per-entry charges of the reference reader (its descriptor sizes, 40 and 72 bytes, plus slack), so that the
  // same counts pass
  if (n_meta > c.left() / 13 || n_tensors > c.left() / 32 || !charge(n_meta, 40 + 64) || !charge(n_tensors, 72 + 128))
    return fail("descriptor counts exceed the file or the memory budget");
  meta.reserve(static_cast<std::size_t>(n_meta));
  for (std::uint64_t m = 0; m < n_meta; ++m) {
    std::string_view key;
    if (!c.Str(&key)) return fail("truncated metadata key");
    if (key.empty() || key.size() > 65535 || !charge(key.size(), 1)) return fail("metadata key out of limits");
    Value v;
    if (!c.Pod(&v.type)) return fail("truncated metadata type");
    if (v.type > HALO_GGUF_F64) return fail("unknown metadata type");
    bool ok = true;
    switch (v.type) {
      case HALO_GGUF_U8: { std::uint8_t x; ok = c.Pod(&x); v.u = x; v.kind = Value::kU64; break; }
      case HALO_GGUF_I8: { std::int8_t x; ok = c.Pod(&x); v.i = x; v.kind = Value::kI64; break; }
      case HALO_GGUF_U16: { std::uint16_t x; ok = c.Pod(&x); v.u = x; v.kind = Value::kU64; break; }
      case HALO_GGUF_I16: { std::int16_t x; ok = c.Pod(&x); v.i = x; v.kind = Value::kI64; break; }
      case HALO_GGUF_U32: { std::uint32_t x; ok = c.Pod(&x); v.u = x; v.kind = Value::kU64; break; }
      case HALO_GGUF_I32: { std::int32_t x; ok = c.Pod(&x); v.i = x; v.kind = Value::kI64; break; }
      case HALO_GGUF_U64: { ok = c.Pod(&v.u); v.kind = Value::kU64; break; }
      case HALO_GGUF_I64: { ok = c.Pod(&v.i); v.kind = Value::kI64; break; }
      case HALO_GGUF_F32: { float x; ok = c.Pod(&x); v.f = x; v.kind = Value::kF64; break; }
      case HALO_GGUF_F64: { ok = c.Pod(&v.f); v.kind = Value::kF64; break; }
      case HALO_GGUF_BOOL: {
        std::uint8_t x;
        ok = c.Pod(&x) && x <= 1;
        v.u = x;
        v.kind = Value::kBool;
        break;
      }
      case HALO_GGUF_STRING: ok = c.Str(&v.s) && charge(v.s.size(), 1); v.kind = Value::kStr; break;
      case HALO_GGUF_ARRAY: {
        if (!c.Pod(&v.elem_type) || !c.Pod(&v.length)) return fail("truncated array header");
        if (v.elem_type > HALO_GGUF_F64 || v.elem_type == HALO_GGUF_ARRAY) return fail("bad array element type");
        // least bytes an element can take (a string: its 8-byte length)
        static constexpr std::uint32_t kMinBytes[] = {1, 1, 2, 2, 4, 4, 4, 1, 8, 0, 8, 8, 8};
        if (v.length > c.left() / kMinBytes[v.elem_type] ||
            !charge(v.length, v.elem_type == HALO_GGUF_STRING ? sizeof(std::string_view) : 8))
          return fail("array length exceeds the file or the memory budget");
        const std::size_t n = static_cast<std::size_t>(v.length);
        switch (v.elem_type) {
          case HALO_GGUF_STRING:
            v.kind = Value::kStrArr;
            v.sa.resize(n);
            for (std::size_t a = 0; a < n && ok; ++a) ok = c.Str(&v.sa[a]) && charge(v.sa[a].size(), 1);
            break;
          case HALO_GGUF_F32:
          case HALO_GGUF_F64:
            v.kind = Value::kF64Arr;
            v.fa.resize(n);
            for (std::size_t a = 0; a < n && ok; ++a) {
              if (v.elem_type == HALO_GGUF_F32) {
                float x;
                ok = c.Pod(&x);
                v.fa[a] = x;
              } else {
                ok = c.Pod(&v.fa[a]);
              }
            }
            break;
          case HALO_GGUF_U32:
          case HALO_GGUF_U64:
          case HALO_GGUF_BOOL:
            v.kind = Value::kU64Arr;
            v.ua.resize(n);
            for (std::size_t a = 0; a < n && ok; ++a) {
              if (v.elem_type == HALO_GGUF_U32) {
                std::uint32_t x;
                ok = c.Pod(&x);
                v.ua[a] = x;
              } else if (v.elem_type == HALO_GGUF_BOOL) {
                std::uint8_t x;
                ok = c.Pod(&x) && x <= 1;
                v.ua[a] = x;
              } else {
                ok = c.Pod(&v.ua[a]);
              }
            }
            break;
          case HALO_GGUF_I32:
          case HALO_GGUF_I64:
            v.kind = Value::kI64Arr;
            v.ia.resize(n);
            for (std::size_t a = 0; a < n && ok; ++a) {
              if (v.elem_type == HALO_GGUF_I32) {
                std::int32_t x;
                ok = c.Pod(&x);
                v.ia[a] = x;
              } else {
                ok = c.Pod(&v.ia[a]);
              }
            }
            break;
          default:  // 8- and 16-bit integers: skipped
            v.kind = Value::kSkipped;
            ok = c.Skip(v.length * (v.elem_type <= HALO_GGUF_I8 ? 1u : 2u));
            break;
        }
        break;
      }
      default: return fail("unknown metadata type");
    }
    if (!ok) return fail("truncated or invalid metadata value");
    if (key == "general.alignment") {
      if (v.kind != Value::kU64 || !std::has_single_bit(v.u) || v.u > 0xFFFFFFFFull)
        return fail("invalid general.alignment");
      alignment = v.u;
    }
    if (!meta.emplace(key, std::move(v)).second) return fail("duplicate metadata key");
  }
  tensors.reserve(static_cast<std::size_t>(n_tensors));
  index.reserve(static_cast<std::size_t>(n_tensors));
  for (std::uint64_t t = 0; t < n_tensors; ++t) {
    Tensor x;
    if (!c.Str(&x.name)) return fail("truncated tensor name");
    if (x.name.empty() || x.name.size() > 65535 || !charge(x.name.size(), 1)) return fail("tensor name out of limits");
    if (!c.Pod(&x.n_dims) || x.n_dims == 0 || x.n_dims > 8) return fail("bad tensor dimension count");
    for (std::uint32_t k = 0; k < x.n_dims; ++k)
      if (!c.Pod(&x.dims[k])) return fail("truncated tensor dimensions");
    if (!c.Pod(&x.type)) return fail("truncated tensor type");
    if (x.type > 0xFFFF) return fail("bad tensor type");
    TypeInfo ti{0, 0};
    const bool known = LookupType(x.type, &ti);
    x.size_bytes = EncodedBytes(x.type, x.Elements());
    if (x.size_bytes == 0 || (known && ti.block > 1 && x.dims[0] % ti.block != 0))
      return fail("invalid tensor shape or unsupported storage type");
    if (!c.Pod(&x.offset)) return fail("truncated tensor offset");
    if (!index.emplace(x.name, tensors.size()).second) return fail("duplicate tensor name");
    tensors.push_back(x);
  }
  if (tensors.empty()) return c.at() <= size;  // no data section
  const std::size_t pad = static_cast<std::size_t>((alignment - c.at() % alignment) % alignment);
  if (c.at() > size || pad > size - c.at()) return fail("data section out of the file");
  const std::size_t base = c.at() + pad;
  for (Tensor& x : tensors) {
    if (x.offset % alignment != 0 || x.offset > size - base || x.size_bytes > size - base - x.offset)
      return fail("tensor extent or alignment is invalid");
    x.data = data + base + x.offset;
  }
  return true;
}

namespace {

std::unique_ptr<halo_gguf> OpenMapped(const std::string& path, std::string* why) {
  const int fd = open(path.c_str(), O_RDONLY);
  if (fd < 0) return *why = "cannot open " + path, nullptr;
  struct stat st{};
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    close(fd);
    return *why = "empty or unreadable file " + path, nullptr;
  }
  void* p = mmap(nullptr, static_cast<std::size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
  if (p == MAP_FAILED) {
    close(fd);
    return *why = "cannot map " + path, nullptr;
  }
  madvise(p, static_cast<std::size_t>(st.st_size), MADV_SEQUENTIAL);
  auto g = std::make_unique<halo_gguf>();
  g->map = p;
  g->fd = fd;
  g->data = static_cast<const std::uint8_t*>(p);
  g->size = static_cast<std::size_t>(st.st_size);
  try {
    if (!g->Parse(why)) return nullptr;
  } catch (const std::bad_alloc&) {
    return *why = "insufficient memory for GGUF descriptors", nullptr;
  }
  return g;
}

// <prefix>-<i>-of-<n>.gguf with decimal fields; returns false for any other file name.
bool SplitName(const std::string& file, std::string* prefix, std::size_t* iw, std::size_t* nw) {
  const std::string ext = ".gguf";
  if (file.size() <= ext.size() || file.compare(file.size() - ext.size(), ext.size(), ext) != 0) return false;
  const std::string stem = file.substr(0, file.size() - ext.size());
  const std::size_t of = stem.rfind("-of-");
  if (of == std::string::npos) return false;
  const std::string count = stem.substr(of + 4);
  const std::size_t dash = stem.rfind('-', of == 0 ? 0 : of - 1);
  if (dash == std::string::npos || dash >= of) return false;
  const std::string index = stem.substr(dash + 1, of - dash - 1);
  auto digits = [](const std::string& s) {
    return !s.empty() && std::all_of(s.begin(), s.end(), [](char ch) { return ch >= '0' && ch <= '9'; });
  };
  if (!digits(index) || !digits(count)) return false;
  *prefix = stem.substr(0, dash);
  *iw = index.size();
  *nw = count.size();
  return true;
}

std::unique_ptr<halo_gguf> OpenSplit(const std::string& path, std::unique_ptr<halo_gguf> first, std::uint32_t n,
                                     std::string* why) {
  std::uint32_t no;
  std::uint64_t total;
  if (!first->U32("split.no", &no) || no >= n || !first->U64("split.tensors.count", &total))
    return *why = "invalid split GGUF metadata in " + path, nullptr;
  const std::size_t slash = path.find_last_of('/');
  const std::string dir = slash == std::string::npos ? "" : path.substr(0, slash + 1);
  const std::string file = slash == std::string::npos ? path : path.substr(slash + 1);
  std::string prefix;
  std::size_t iw, nw;
  if (!SplitName(file, &prefix, &iw, &nw)) return *why = "split GGUF file name is not <name>-i-of-n.gguf", nullptr;
  auto shard_path = [&](std::uint32_t i) {
    char a[32], b[32];
    std::snprintf(a, sizeof a, "%0*u", static_cast<int>(iw), i + 1);
    std::snprintf(b, sizeof b, "%0*u", static_cast<int>(nw), n);
    return dir + prefix + "-" + a + "-of-" + b + ".gguf";
  };
  std::vector<std::unique_ptr<halo_gguf>> shards(n);
  shards[no] = std::move(first);
  for (std::uint32_t i = 0; i < n; ++i) {
    if (shards[i]) continue;
    std::string w;
    shards[i] = OpenMapped(shard_path(i), &w);
    if (!shards[i]) return *why = w.empty() ? "cannot open split shard " + shard_path(i) : w, nullptr;
  }
  std::string_view arch;
  const bool has_arch = shards[0]->Str("general.architecture", &arch);
  for (std::uint32_t i = 0; i < n; ++i) {
    std::uint32_t sno, scount;
    std::string_view sa;
    const bool sarch = shards[i]->Str("general.architecture", &sa);
    if (!shards[i]->U32("split.no", &sno) || sno != i || !shards[i]->U32("split.count", &scount) || scount != n ||
        shards[i]->version != shards[0]->version || (sarch && (!has_arch || sa != arch)))
      return *why = "inconsistent split GGUF shard " + shard_path(i), nullptr;
  }
  auto g = std::make_unique<halo_gguf>();
  g->version = shards[0]->version;
  g->alignment = shards[0]->alignment;
  g->meta = shards[0]->meta;
  std::uint64_t count = 0;
  for (const auto& s : shards) {
    count += s->tensors.size();
    g->size += s->size;
  }
  if (count != total) return *why = "split GGUF tensor count mismatch", nullptr;
  g->tensors.reserve(static_cast<std::size_t>(count));
  for (const auto& s : shards)
    for (const Tensor& t : s->tensors) {
      if (!g->index.emplace(t.name, g->tensors.size()).second)
        return *why = "duplicate tensor across split GGUF shards", nullptr;
      g->tensors.push_back(t);
    }
  g->shards = std::move(shards);
  return g;
}

void Export(const Tensor& t, halo_gguf_tensor* out) {
  *out = halo_gguf_tensor{};
  out->name = t.name.data();
  out->name_len = t.name.size();
  out->type = t.type;
  out->n_dims = t.n_dims;
  for (std::uint32_t k = 0; k < t.n_dims; ++k) out->dims[k] = t.dims[k];
  out->offset = t.offset;
  out->data = t.data;
  out->size_bytes = t.size_bytes;
}

}  // namespace

extern "C" {

uint64_t halo_ggml_encoded_bytes(uint32_t type, uint64_t elements) { return EncodedBytes(type, elements); }

int halo_gguf_open_file(const char* path, halo_gguf** out, char* err, size_t errlen) {
  if (path == nullptr || out == nullptr) return SetErr(err, errlen, "null argument"), -1;
  *out = nullptr;
  std::string why;
  auto g = OpenMapped(path, &why);
  if (!g) return SetErr(err, errlen, "%s", why.empty() ? "malformed or truncated GGUF" : why.c_str()), -1;
  std::uint32_t n = 1;
  if (g->Find("split.count") != nullptr && (!g->U32("split.count", &n) || n == 0 || n > 65535))
    return SetErr(err, errlen, "invalid GGUF split count"), -1;
  if (n > 1) {
    g = OpenSplit(path, std::move(g), n, &why);
    if (!g) return SetErr(err, errlen, "%s", why.c_str()), -1;
  }
  *out = g.release();
  return 0;
}

int halo_gguf_open_memory(const void* data, size_t size, halo_gguf** out, char* err, size_t errlen) {
  if (out == nullptr) return SetErr(err, errlen, "null argument"), -1;
  *out = nullptr;
  if (data == nullptr || size < 24) return SetErr(err, errlen, "invalid memory buffer for GGUF"), -1;
  auto g = std::make_unique<halo_gguf>();
  g->data = static_cast<const std::uint8_t*>(data);
  g->size = size;
  std::string why;
  try {
    if (!g->Parse(&why)) return SetErr(err, errlen, "%s", why.empty() ? "malformed or truncated GGUF" : why.c_str()), -1;
  } catch (const std::bad_alloc&) {
    return SetErr(err, errlen, "insufficient memory for GGUF descriptors"), -1;
  }
  *out = g.release();
  return 0;
}

void halo_gguf_close(halo_gguf* g) { delete g; }
uint32_t halo_gguf_version(const halo_gguf* g) { return g ? g->version : 0; }
uint64_t halo_gguf_alignment(const halo_gguf* g) { return g ? g->alignment : 0; }
uint64_t halo_gguf_tensor_count(const halo_gguf* g) { return g ? g->tensors.size() : 0; }
uint64_t halo_gguf_metadata_count(const halo_gguf* g) { return g ? g->meta.size() : 0; }

int halo_gguf_tensor_at(const halo_gguf* g, uint64_t i, halo_gguf_tensor* out) {
  if (g == nullptr || out == nullptr || i >= g->tensors.size()) return -1;
  Export(g->tensors[static_cast<std::size_t>(i)], out);
  return 0;
}

int halo_gguf_find_tensor(const halo_gguf* g, const char* name, halo_gguf_tensor* out) {
  if (g == nullptr || name == nullptr || out == nullptr) return -1;
  auto it = g->index.find(std::string_view(name));
  if (it == g->index.end()) return -1;
  Export(g->tensors[it->second], out);
  return 0;
}

int halo_gguf_metadata_type(const halo_gguf* g, const char* key) {
  const Value* v = g ? g->Find(key) : nullptr;
  return v ? static_cast<int>(v->type) : -1;
}
int halo_gguf_metadata_key_at(const halo_gguf* g, uint64_t i, const char** key, size_t* len) {
  if (g == nullptr || key == nullptr || len == nullptr || i >= g->meta.size()) return -1;
  auto it = g->meta.begin();
  std::advance(it, static_cast<std::ptrdiff_t>(i));
  *key = it->first.data();
  *len = it->first.size();
  return 0;
}
int halo_gguf_get_i64(const halo_gguf* g, const char* key, int64_t* out) {
  const Value* v = g ? g->Find(key) : nullptr;
  if (v == nullptr || out == nullptr || v->kind != Value::kI64) return -1;
  *out = v->i;
  return 0;
}
int halo_gguf_get_f64(const halo_gguf* g, const char* key, double* out) {
  const Value* v = g ? g->Find(key) : nullptr;
  if (v == nullptr || out == nullptr || v->kind != Value::kF64) return -1;
  *out = v->f;
  return 0;
}
int halo_gguf_get_u32(const halo_gguf* g, const char* key, uint32_t* out) {
  return g && out && g->U32(key, out) ? 0 : -1;
}
int halo_gguf_get_u64(const halo_gguf* g, const char* key, uint64_t* out) {
  return g && out && g->U64(key, out) ? 0 : -1;
}
int halo_gguf_get_f32(const halo_gguf* g, const char* key, float* out) {
  const Value* v = g ? g->Find(key) : nullptr;
  if (v == nullptr || out == nullptr || v->kind != Value::kF64) return -1;
  *out = static_cast<float>(v->f);
  return 0;
}
int halo_gguf_get_bool(const halo_gguf* g, const char* key, int* out) {
  const Value* v = g ? g->Find(key) : nullptr;
  if (v == nullptr || out == nullptr || v->kind != Value::kBool) return -1;
  *out = static_cast<int>(v->u);
  return 0;
}
int halo_gguf_get_string(const halo_gguf* g, const char* key, const char** data, size_t* len) {
  std::string_view s;
  if (g == nullptr || data == nullptr || len == nullptr || !g->Str(key, &s)) return -1;
  *data = s.data();
  *len = s.size();
  return 0;
}
int halo_gguf_get_array_info(const halo_gguf* g, const char* key, uint32_t* elem_type, uint64_t* length) {
  const Value* v = g ? g->Find(key) : nullptr;
  if (v == nullptr || v->type != HALO_GGUF_ARRAY || elem_type == nullptr || length == nullptr) return -1;
  *elem_type = v->elem_type;
  *length = v->length;
  return 0;
}
int halo_gguf_get_array_u64(const halo_gguf* g, const char* key, uint64_t i, uint64_t* out) {
  const Value* v = g ? g->Find(key) : nullptr;
  if (v == nullptr || out == nullptr) return -1;
  if (v->kind == Value::kU64Arr && i < v->ua.size()) return *out = v->ua[static_cast<std::size_t>(i)], 0;
  if (v->kind == Value::kI64Arr && i < v->ia.size() && v->ia[static_cast<std::size_t>(i)] >= 0)
    return *out = static_cast<std::uint64_t>(v->ia[static_cast<std::size_t>(i)]), 0;
  return -1;
}
int halo_gguf_get_array_i64(const halo_gguf* g, const char* key, uint64_t i, int64_t* out) {
  const Value* v = g ? g->Find(key) : nullptr;
  if (v == nullptr || out == nullptr || v->kind != Value::kI64Arr || i >= v->ia.size()) return -1;
  *out = v->ia[static_cast<std::size_t>(i)];
  return 0;
}
int halo_gguf_get_array_f64(const halo_gguf* g, const char* key, uint64_t i, double* out) {
  const Value* v = g ? g->Find(key) : nullptr;
  if (v == nullptr || out == nullptr || v->kind != Value::kF64Arr || i >= v->fa.size()) return -1;
  *out = v->fa[static_cast<std::size_t>(i)];
  return 0;
}
int halo_gguf_get_array_string(const halo_gguf* g, const char* key, uint64_t i, const char** data, size_t* len) {
  const Value* v = g ? g->Find(key) : nullptr;
  if (v == nullptr || data == nullptr || len == nullptr || v->kind != Value::kStrArr || i >= v->sa.size()) return -1;
  *data = v->sa[static_cast<std::size_t>(i)].data();
  *len = v->sa[static_cast<std::size_t>(i)].size();
  return 0;
}

size_t halo_gguf_quantization_label(const halo_gguf* g, char* out, size_t len) {
  std::string label = "unknown";
  if (g != nullptr) {
    std::map<std::uint32_t, std::uint64_t> by_type;
    std::uint64_t total = 0;
    for (const Tensor& t : g->tensors) {
      const std::uint64_t n = t.Elements();
      by_type[t.type] += n;
      total += n;
    }
    if (!by_type.empty() && total != 0) {
      auto best = by_type.begin();
      for (auto it = by_type.begin(); it != by_type.end(); ++it)
        if (it->second > best->second) best = it;
      label = TypeName(best->first);
      if (best->second * 5 < total * 4) label += " mixed";
    }
  }
  if (out != nullptr && len > 0) {
    const std::size_t n = std::min(len - 1, label.size());
    std::memcpy(out, label.data(), n);
    out[n] = '\0';
  }
  return label.size();
}

int halo_gguf_upload_q8_0(halo_engine* eng, const halo_gguf_tensor* t, uint64_t row0, uint32_t rows, int8_t* qs,
                          uint16_t* d, uint32_t qstride, void* staging, size_t staging_bytes, char* err,
                          size_t errlen) {
  if (eng == nullptr || t == nullptr || t->data == nullptr || qs == nullptr || d == nullptr || staging == nullptr)
    return SetErr(err, errlen, "null argument"), -1;
  if (t->type != HALO_GGML_Q8_0) return SetErr(err, errlen, "tensor is %s, not Q8_0", TypeName(t->type)), -1;
  const std::uint64_t cols = t->dims[0];
  std::uint64_t all_rows = 1;
  for (std::uint32_t k = 1; k < t->n_dims; ++k) all_rows *= t->dims[k];
  if (cols == 0 || cols % 32 != 0)
    return SetErr(err, errlen, "Q8_0 tensor with %llu columns (must be a positive multiple of 32)",
                  static_cast<unsigned long long>(cols)),
           -1;
  if (qstride < cols || qstride % 16 != 0)
    return SetErr(err, errlen, "qstride %u must be >= the %llu columns and a multiple of 16", qstride,
                  static_cast<unsigned long long>(cols)),
           -1;
  if (cols > 0xFFFFFFFFull || row0 > all_rows || rows > all_rows - row0)
    return SetErr(err, errlen, "rows [%llu, %llu) outside the tensor's %llu", static_cast<unsigned long long>(row0),
                  static_cast<unsigned long long>(row0 + rows), static_cast<unsigned long long>(all_rows)),
           -1;
  const std::uint64_t row_bytes = cols / 32 * 34;
  const std::uint64_t per = staging_bytes / row_bytes;
  if (per == 0) return SetErr(err, errlen, "staging of %zu bytes holds no row of %llu bytes", staging_bytes,
                              static_cast<unsigned long long>(row_bytes)), -1;
  halo_device* dev = halo_engine_device(eng);
  halo_buffer st{};
  st.device = staging;
  st.bytes = staging_bytes;
  const auto* src = static_cast<const std::uint8_t*>(t->data) + row0 * row_bytes;
  for (std::uint64_t r = 0; r < rows;) {
    const std::uint32_t n = static_cast<std::uint32_t>(std::min<std::uint64_t>(per, rows - r));
    // the copy is ordered after the previous chunk's repack on the device stream and complete on return
    if (halo_upload(dev, &st, 0, src + r * row_bytes, n * row_bytes, err, errlen) != 0) return -1;
    if (halo_op_repack_q8_0(eng, staging, qs + r * qstride, d + r * (cols / 32), n, static_cast<std::uint32_t>(cols),
                            qstride, err, errlen) != 0)
      return -1;
    r += n;
  }
  return halo_synchronize(dev, err, errlen);
}

}  // extern "C"

// ---- model loading ---------------------------------------------------------------------------------------------

namespace {

struct LoadItem {
  std::uint32_t layer;        // UINT32_MAX: model-level tensor
  const char* model_name;     // halo_model_tensor name
  std::string gguf_name;
  std::uint32_t row0, rows;   // row range of the model tensor this GGUF tensor fills
  halo_model_tensor_view view;
  halo_gguf_tensor t;
};

std::uint64_t RowsOf(const halo_gguf_tensor& t) {
  std::uint64_t r = 1;
  for (std::uint32_t k = 1; k < t.n_dims; ++k) r *= t.dims[k];
  return r;
}

}  // namespace

extern "C" {

int halo_model_config_from_gguf(const halo_gguf* g, halo_model_config* cfg, char* err, size_t errlen) {
  if (g == nullptr || cfg == nullptr) return SetErr(err, errlen, "null argument"), -1;
  std::string_view arch;
  if (!g->Str("general.architecture", &arch)) return SetErr(err, errlen, "general.architecture missing"), -1;
  const std::string p = std::string(arch) + ".";
  halo_model_config c = *cfg;
  struct {
    const char* key;
    std::uint32_t* dst;
  } u32[] = {{"block_count", &c.layers},
             {"embedding_length", &c.hidden},
             {"full_attention_interval", &c.attn_interval},
             {"attention.head_count", &c.q_heads},
             {"attention.head_count_kv", &c.kv_heads},
             {"attention.key_length", &c.head_dim},
             {"rope.dimension_count", &c.rotary_dim},
             {"ssm.conv_kernel", &c.conv_kernel},
             {"ssm.state_size", &c.gdn_head_dim},
             {"ssm.group_count", &c.gdn_k_heads},
             {"ssm.time_step_rank", &c.gdn_v_heads},
             {"expert_count", &c.n_experts},
             {"expert_used_count", &c.n_used},
             {"expert_feed_forward_length", &c.expert_ff},
             {"expert_shared_feed_forward_length", &c.shared_ff}};
  for (const auto& e : u32)
    if (!g->U32((p + e.key).c_str(), e.dst)) return SetErr(err, errlen, "metadata %s%s missing", p.c_str(), e.key), -1;
  float f;
  c.rope_theta = halo_gguf_get_f32(g, (p + "rope.freq_base").c_str(), &f) == 0 ? f : 10000000.0f;
  c.rms_eps = halo_gguf_get_f32(g, (p + "attention.layer_norm_rms_epsilon").c_str(), &f) == 0 ? f : 1e-6f;
  halo_gguf_tensor emb;
  if (halo_gguf_find_tensor(g, "token_embd.weight", &emb) != 0 || emb.n_dims != 2 || emb.dims[1] > 0xFFFFFFFFull)
    return SetErr(err, errlen, "token_embd.weight missing or not 2-D"), -1;
  c.vocab = static_cast<std::uint32_t>(emb.dims[1]);
  *cfg = c;
  return 0;
}

int halo_model_load_gguf(halo_model* m, const halo_gguf* g, char* err, size_t errlen) {
  if (m == nullptr || g == nullptr) return SetErr(err, errlen, "null argument"), -1;
  halo_engine* eng = halo_model_engine_of(m);
  halo_device* dev = halo_engine_device(eng);
  std::vector<LoadItem> items;
  auto add = [&](std::uint32_t layer, const char* mn, std::string gn, std::uint32_t row0 = 0,
                 std::uint32_t rows = 0) {
    LoadItem it{};
    it.layer = layer;
    it.model_name = mn;
    it.gguf_name = std::move(gn);
    it.row0 = row0;
    it.rows = rows;
    items.push_back(std::move(it));
  };
  add(UINT32_MAX, "embd", "token_embd.weight");
  add(UINT32_MAX, "head", "output.weight");
  add(UINT32_MAX, "out_norm", "output_norm.weight");
  for (std::uint32_t l = 0;; ++l) {
    halo_model_tensor_view probe;
    if (halo_model_tensor(m, l, "attn_norm", &probe, nullptr, 0) != 0) break;
    const std::string b = "blk." + std::to_string(l) + ".";
    add(l, "attn_norm", b + "attn_norm.weight");
    add(l, "ffn_norm", b + "post_attention_norm.weight");
    add(l, "router", b + "ffn_gate_inp.weight");
    add(l, "shared_gate", b + "ffn_gate_inp_shexp.weight");
    add(l, "gate", b + "ffn_gate_exps.weight");
    add(l, "up", b + "ffn_up_exps.weight");
    add(l, "down", b + "ffn_down_exps.weight");
    add(l, "sgate", b + "ffn_gate_shexp.weight");
    add(l, "sup", b + "ffn_up_shexp.weight");
    add(l, "sdown", b + "ffn_down_shexp.weight");
    if (halo_model_tensor(m, l, "qkv", &probe, nullptr, 0) == 0) {
      halo_model_tensor_view ab;
      if (halo_model_tensor(m, l, "ab", &ab, err, errlen) != 0) return -1;
      add(l, "qkv", b + "attn_qkv.weight");
      add(l, "z", b + "attn_gate.weight");
      add(l, "ab", b + "ssm_alpha.weight", 0, ab.rows / 2);
      add(l, "ab", b + "ssm_beta.weight", ab.rows / 2, ab.rows / 2);
      add(l, "out", b + "ssm_out.weight");
      add(l, "conv_w", b + "ssm_conv1d.weight");
      add(l, "a", b + "ssm_a");
      add(l, "dt", b + "ssm_dt.bias");
      add(l, "norm_w", b + "ssm_norm.weight");
    } else {
      add(l, "qg", b + "attn_q.weight");
      add(l, "k", b + "attn_k.weight");
      add(l, "v", b + "attn_v.weight");
      add(l, "o", b + "attn_output.weight");
      add(l, "q_norm", b + "attn_q_norm.weight");
      add(l, "k_norm", b + "attn_k_norm.weight");
    }
  }
  // check everything before copying anything
  std::uint64_t max_row_bytes = 0;
  for (LoadItem& it : items) {
    if (halo_model_tensor(m, it.layer, it.model_name, &it.view, err, errlen) != 0) return -1;
    if (it.rows == 0) it.rows = it.view.rows;
    if (halo_gguf_find_tensor(g, it.gguf_name.c_str(), &it.t) != 0)
      return SetErr(err, errlen, "tensor %s missing from the checkpoint", it.gguf_name.c_str()), -1;
    if (it.view.kind == HALO_TENSOR_Q8) {
      if (it.t.type != HALO_GGML_Q8_0 || it.t.dims[0] != it.view.cols || RowsOf(it.t) != it.rows)
        return SetErr(err, errlen, "%s: %s [%llu x %llu], the model needs Q8_0 [%u x %u]", it.gguf_name.c_str(),
                      TypeName(it.t.type), static_cast<unsigned long long>(RowsOf(it.t)),
                      static_cast<unsigned long long>(it.t.dims[0]), it.rows, it.view.cols),
               -1;
      max_row_bytes = std::max<std::uint64_t>(max_row_bytes, it.t.dims[0] / 32 * 34);
    } else {
      const std::uint64_t n = static_cast<std::uint64_t>(it.rows) * it.view.cols;
      std::uint64_t elems = 1;
      for (std::uint32_t k = 0; k < it.t.n_dims; ++k) elems *= it.t.dims[k];
      if (it.t.type != HALO_GGML_F32 || elems != n)
        return SetErr(err, errlen, "%s: %s with %llu values, the model needs F32 with %llu", it.gguf_name.c_str(),
                      TypeName(it.t.type), static_cast<unsigned long long>(elems), static_cast<unsigned long long>(n)),
               -1;
    }
  }
  const std::size_t staging_bytes = std::max<std::size_t>(std::size_t{64} << 20, max_row_bytes);
  halo_buffer staging{};
  if (halo_alloc(dev, staging_bytes, &staging, err, errlen) != 0) return -1;
  int rc = 0;
  for (const LoadItem& it : items) {
    if (it.view.kind == HALO_TENSOR_Q8) {
      auto* qs = static_cast<std::int8_t*>(it.view.data) + static_cast<std::size_t>(it.row0) * it.view.qstride;
      auto* d = static_cast<std::uint16_t*>(it.view.scales) + static_cast<std::size_t>(it.row0) * (it.view.cols / 32);
      rc = halo_gguf_upload_q8_0(eng, &it.t, 0, it.rows, qs, d, it.view.qstride, staging.device, staging.bytes, err,
                                 errlen);
    } else {
      halo_buffer dst{};
      dst.device = it.view.data;
      dst.bytes = static_cast<std::size_t>(it.t.size_bytes);
      rc = halo_upload(dev, &dst, 0, it.t.data, dst.bytes, err, errlen);
    }
    if (rc != 0) break;
  }
  halo_free(dev, &staging);
  return rc;
}

}  // extern "C"
