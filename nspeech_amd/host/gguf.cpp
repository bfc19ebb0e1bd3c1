// GGUF reader: see gguf.h and include/nspeech_gguf.h.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <limits>

#include "nspeech_gguf.h"

namespace nspeech {
namespace rocm {
namespace gguf {

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read as a little-endian u32
constexpr int kMaxArrayDepth = 4;

[[noreturn]] void bad(const std::string& what) { throw Error("gguf: " + what); }

// Bounds-checked little-endian reader over the file image.
class Cursor {
 public:
  Cursor(const uint8_t* p, uint64_t n, uint32_t version) : p_(p), n_(n), v1_(version == 1) {}
  uint64_t pos() const { return off_; }
  uint64_t left() const { return n_ - off_; }
  void need(uint64_t k, const char* what) const {
    if (k > left()) bad(std::string("truncated file while reading ") + what);
  }
  template <class T>
  T get(const char* what) {
    need(sizeof(T), what);
    T v;
    std::memcpy(&v, p_ + off_, sizeof(T));
    off_ += sizeof(T);
    return v;
  }
  // counts and lengths: u64, or u32 in version 1
  uint64_t count(const char* what) { return v1_ ? get<uint32_t>(what) : get<uint64_t>(what); }
  std::string str(const char* what) {
    const uint64_t len = count(what);
    need(len, what);
    std::string s(reinterpret_cast<const char*>(p_ + off_), (size_t)len);
    off_ += len;
    return s;
  }
  void set_version(uint32_t v) { v1_ = v == 1; }

 private:
  const uint8_t* p_;
  uint64_t n_;
  uint64_t off_ = 0;
  bool v1_;
};

// Smallest encoded size of one value of `type` (bounds array lengths before
// anything is allocated for them).
uint64_t min_size(uint32_t type, bool v1) {
  switch (type) {
    case U8: case I8: case BOOL: return 1;
    case U16: case I16: return 2;
    case U32: case I32: case F32: return 4;
    case U64: case I64: case F64: return 8;
    case STRING: return v1 ? 4 : 8;
    case ARRAY: return v1 ? 8 : 12;
  }
  return 1;
}

Value read_value(Cursor& c, uint32_t type, bool v1, int depth) {
  Value v;
  v.type = type;
  switch (type) {
    case U8: v.u = c.get<uint8_t>("u8"); break;
    case I8: v.i = c.get<int8_t>("i8"); break;
    case U16: v.u = c.get<uint16_t>("u16"); break;
    case I16: v.i = c.get<int16_t>("i16"); break;
    case U32: v.u = c.get<uint32_t>("u32"); break;
    case I32: v.i = c.get<int32_t>("i32"); break;
    case U64: v.u = c.get<uint64_t>("u64"); break;
    case I64: v.i = c.get<int64_t>("i64"); break;
    case F32: v.f = c.get<float>("f32"); break;
    case F64: v.f = c.get<double>("f64"); break;
    case BOOL: {
      const uint8_t b = c.get<uint8_t>("bool");
      if (b > 1) bad("bool value " + std::to_string(b));
      v.u = b;
      break;
    }
    case STRING: v.s = c.str("string value"); break;
    case ARRAY: {
      if (depth >= kMaxArrayDepth) bad("arrays nested deeper than " + std::to_string(kMaxArrayDepth));
      v.elem_type = c.get<uint32_t>("array type");
      if (v.elem_type > F64) bad("unknown array element type " + std::to_string(v.elem_type));
      const uint64_t n = c.count("array length");
      if (n > c.left() / min_size(v.elem_type, v1)) bad("array length " + std::to_string(n) + " exceeds the file");
      v.arr.reserve((size_t)n);
      for (uint64_t k = 0; k < n; ++k) v.arr.push_back(read_value(c, v.elem_type, v1, depth + 1));
      break;
    }
    default: bad("unknown metadata value type " + std::to_string(type));
  }
  return v;
}

}  // namespace

bool Value::is_int() const {
  return type == U8 || type == I8 || type == U16 || type == I16 || type == U32 || type == I32 || type == U64 ||
         type == I64 || type == BOOL;
}

int64_t Value::as_int() const {
  if (type == I8 || type == I16 || type == I32 || type == I64) return i;
  if (type == U8 || type == U16 || type == U32 || type == BOOL) return (int64_t)u;
  if (type == U64) {
    if (u > (uint64_t)std::numeric_limits<int64_t>::max()) throw Error("gguf: u64 value does not fit in int64");
    return (int64_t)u;
  }
  throw Error("gguf: value is not an integer");
}

double Value::as_float() const {
  if (type == F32 || type == F64) return f;
  throw Error("gguf: value is not a float");
}

bool ggml_type_layout(uint32_t type, uint64_t* block, uint64_t* type_size) {
  // {id, block elements, bytes per block}: ggml's type traits for the
  // types GGUF files of this stack carry
  static const struct {
    uint32_t id;
    uint64_t block, bytes;
  } kTypes[] = {{0, 1, 4},    {1, 1, 2},     {2, 32, 18},   {3, 32, 20},   {6, 32, 22},
                {7, 32, 24},  {8, 32, 34},   {9, 32, 36},   {10, 256, 84}, {11, 256, 110},
                {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292}, {30, 1, 2}};
  for (const auto& t : kTypes)
    if (t.id == type) {
      *block = t.block;
      *type_size = t.bytes;
      return true;
    }
  return false;
}

const char* ggml_type_name(uint32_t type) {
  switch (type) {
    case 0: return "f32";
    case 1: return "f16";
    case 2: return "q4_0";
    case 3: return "q4_1";
    case 6: return "q5_0";
    case 7: return "q5_1";
    case 8: return "q8_0";
    case 9: return "q8_1";
    case 10: return "q2_k";
    case 11: return "q3_k";
    case 12: return "q4_k";
    case 13: return "q5_k";
    case 14: return "q6_k";
    case 15: return "q8_k";
    case 30: return "bf16";
  }
  return "unknown";
}

Content Content::read(const uint8_t* data, uint64_t size, std::shared_ptr<void> keepalive) {
  if (!data && size) bad("null buffer");
  Content ct;
  ct.keep_ = std::move(keepalive);
  ct.base_ = data;
  ct.size_ = size;
  Cursor c(data, size, 3);
  if (c.get<uint32_t>("magic") != kMagic) bad("not a GGUF file (bad magic)");
  ct.version_ = c.get<uint32_t>("version");
  if (ct.version_ < 1 || ct.version_ > 3) bad("unsupported GGUF version " + std::to_string(ct.version_));
  const bool v1 = ct.version_ == 1;
  c.set_version(ct.version_);
  const uint64_t n_tensors = c.count("tensor count");
  const uint64_t n_kv = c.count("metadata count");
  // every entry takes at least a few bytes: reject counts the file cannot hold
  if (n_kv > c.left() / (v1 ? 8 : 12)) bad("metadata count " + std::to_string(n_kv) + " exceeds the file");
  for (uint64_t k = 0; k < n_kv; ++k) {
    std::string key = c.str("metadata key");
    const uint32_t type = c.get<uint32_t>("metadata type");
    Value v = read_value(c, type, v1, 0);
    if (ct.meta_index_.count(key)) bad("duplicate metadata key '" + key + "'");
    ct.meta_index_[key] = ct.metadata_.size();
    ct.metadata_.emplace_back(std::move(key), std::move(v));
  }
  if (const Value* a = ct.find_metadata("general.alignment")) {
    if (!a->is_int()) bad("general.alignment is not an integer");
    const int64_t al = a->as_int();
    if (al <= 0 || al > (1 << 20) || (al & (al - 1)) != 0) bad("general.alignment " + std::to_string(al));
    ct.alignment_ = (uint64_t)al;
  }
  if (n_tensors > c.left() / (v1 ? 20 : 28)) bad("tensor count " + std::to_string(n_tensors) + " exceeds the file");
  ct.tensors_.reserve((size_t)n_tensors);
  for (uint64_t k = 0; k < n_tensors; ++k) {
    TensorInfo t;
    t.name = c.str("tensor name");
    const uint32_t nd = c.get<uint32_t>("tensor n_dims");
    if (nd < 1 || nd > 4) bad("tensor '" + t.name + "' has " + std::to_string(nd) + " dimensions");
    std::vector<uint64_t> ne(nd);
    for (uint32_t d = 0; d < nd; ++d) ne[d] = v1 ? c.get<uint32_t>("tensor dim") : c.get<uint64_t>("tensor dim");
    t.type = c.get<uint32_t>("tensor type");
    t.offset = c.get<uint64_t>("tensor offset");
    uint64_t block = 0, tsize = 0;
    if (!ggml_type_layout(t.type, &block, &tsize))
      bad("tensor '" + t.name + "' has unknown ggml type " + std::to_string(t.type));
    uint64_t nelem = 1;
    for (uint64_t d : ne) {
      if (d != 0 && nelem > std::numeric_limits<uint64_t>::max() / d) bad("tensor '" + t.name + "' size overflows");
      nelem *= d;
    }
    if (ne[0] % block != 0)
      bad("tensor '" + t.name + "': innermost dimension " + std::to_string(ne[0]) + " is not a multiple of the " +
          ggml_type_name(t.type) + " block (" + std::to_string(block) + ")");
    if (nelem / block > std::numeric_limits<uint64_t>::max() / tsize) bad("tensor '" + t.name + "' size overflows");
    t.nbytes = nelem / block * tsize;
    t.shape.assign(ne.rbegin(), ne.rend());  // outermost first
    if (ct.tensor_index_.count(t.name)) bad("duplicate tensor name '" + t.name + "'");
    ct.tensor_index_[t.name] = ct.tensors_.size();
    ct.tensors_.push_back(std::move(t));
  }
  const uint64_t end = c.pos();
  ct.data_offset_ = (end + ct.alignment_ - 1) / ct.alignment_ * ct.alignment_;
  if (ct.data_offset_ > size && !ct.tensors_.empty()) bad("data section starts past the end of the file");
  for (const TensorInfo& t : ct.tensors_) {
    if (t.offset % ct.alignment_ != 0)
      bad("tensor '" + t.name + "' offset " + std::to_string(t.offset) + " is not aligned to " +
          std::to_string(ct.alignment_));
    const uint64_t room = size - ct.data_offset_;
    if (t.offset > room || t.nbytes > room - t.offset)
      bad("tensor '" + t.name + "' data (" + std::to_string(t.nbytes) + " bytes at " + std::to_string(t.offset) +
          ") lies past the end of the file");
  }
  return ct;
}

Content Content::open(const std::string& path) {
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) bad("cannot open '" + path + "': " + std::strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    const int e = errno;
    ::close(fd);
    bad("cannot stat '" + path + "': " + std::strerror(e));
  }
  const uint64_t size = (uint64_t)st.st_size;
  if (size == 0) {
    ::close(fd);
    bad("'" + path + "' is empty");
  }
  void* p = mmap(nullptr, (size_t)size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (p == MAP_FAILED) bad("cannot map '" + path + "': " + std::strerror(errno));
  std::shared_ptr<void> keep(p, [size](void* q) { munmap(q, (size_t)size); });
  return read(static_cast<const uint8_t*>(p), size, keep);
}

const Value* Content::find_metadata(const std::string& key) const {
  auto it = meta_index_.find(key);
  return it == meta_index_.end() ? nullptr : &metadata_[it->second].second;
}

const TensorInfo* Content::find_tensor(const std::string& name) const {
  auto it = tensor_index_.find(name);
  return it == tensor_index_.end() ? nullptr : &tensors_[it->second];
}

Tensor Content::upload(const TensorInfo& t, const RocmDevice& device) const {
  return Tensor::from_host(device, tensor_data(t), {(size_t)t.nbytes}, DType::U8);
}

Tensor Content::get(const std::vector<uint64_t>& shape, const std::string& name, const RocmDevice& device,
                    uint32_t* type) const {
  const TensorInfo* t = find_tensor(name);
  if (!t) throw Error("cannot find tensor " + name);
  if (t->shape != shape) {
    auto fmt = [](const std::vector<uint64_t>& s) {
      std::string r = "[";
      for (size_t k = 0; k < s.size(); ++k) r += (k ? ", " : "") + std::to_string(s[k]);
      return r + "]";
    };
    throw Error("shape mismatch for " + name + ", got " + fmt(t->shape) + ", expected " + fmt(shape));
  }
  if (type) *type = t->type;
  return upload(*t, device);
}

}  // namespace gguf
}  // namespace rocm
}  // namespace nspeech

// ------------------------------------------------------------------ C ABI --

using nspeech::rocm::Error;
using namespace nspeech::rocm::gguf;

struct nsr_gguf {
  Content content;
};

namespace {

thread_local std::string g_gguf_error;

nsr_status gguf_fail(nsr_status st, const std::string& msg) {
  g_gguf_error = msg;
  return st;
}

template <class F>
nsr_status guarded(F&& f) {
  try {
    return f();
  } catch (const Error& e) {
    return gguf_fail(NSR_ERR_BAD_ARG, e.what());
  } catch (const std::bad_alloc&) {
    return gguf_fail(NSR_ERR_BAD_ARG, "gguf: out of host memory");
  } catch (const std::exception& e) {
    return gguf_fail(NSR_ERR_BAD_ARG, std::string("gguf: ") + e.what());
  }
}

void fill(const nsr_gguf* g, const TensorInfo& t, nsr_gguf_tensor* out) {
  std::memset(out, 0, sizeof(*out));
  out->name = t.name.c_str();
  out->type = t.type;
  out->n_dims = (uint32_t)t.shape.size();
  for (int d = 0; d < 4; ++d) out->shape[d] = d < (int)t.shape.size() ? (int64_t)t.shape[d] : 1;
  out->offset = g->content.data_offset() + t.offset;
  out->nbytes = t.nbytes;
  out->data = g->content.tensor_data(t);
}

const Value* meta(const nsr_gguf* g, const char* key) {
  if (!g || !key) throw Error("gguf: null argument");
  const Value* v = g->content.find_metadata(key);
  if (!v) throw Error(std::string("gguf: no metadata key '") + key + "'");
  return v;
}

const Value* array_elem(const nsr_gguf* g, const char* key, uint64_t i) {
  const Value* v = meta(g, key);
  if (v->type != ARRAY) throw Error(std::string("gguf: '") + key + "' is not an array");
  if (i >= v->arr.size()) throw Error(std::string("gguf: index out of range for '") + key + "'");
  return &v->arr[i];
}

}  // namespace

extern "C" {

const char* nsr_gguf_last_error(void) { return g_gguf_error.c_str(); }

nsr_status nsr_gguf_open(const char* path, nsr_gguf** out) {
  if (!path || !out) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  *out = nullptr;
  return guarded([&] {
    *out = new nsr_gguf{Content::open(path)};
    return NSR_OK;
  });
}

nsr_status nsr_gguf_open_buffer(const void* data, uint64_t size, nsr_gguf** out) {
  if (!out || (!data && size)) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  *out = nullptr;
  return guarded([&] {
    *out = new nsr_gguf{Content::read(static_cast<const uint8_t*>(data), size)};
    return NSR_OK;
  });
}

void nsr_gguf_close(nsr_gguf* g) { delete g; }

uint32_t nsr_gguf_version(const nsr_gguf* g) { return g ? g->content.version() : 0; }
uint64_t nsr_gguf_alignment(const nsr_gguf* g) { return g ? g->content.alignment() : 0; }
uint64_t nsr_gguf_data_offset(const nsr_gguf* g) { return g ? g->content.data_offset() : 0; }
int64_t nsr_gguf_tensor_count(const nsr_gguf* g) { return g ? (int64_t)g->content.tensor_infos().size() : 0; }
int64_t nsr_gguf_metadata_count(const nsr_gguf* g) { return g ? (int64_t)g->content.metadata().size() : 0; }

nsr_status nsr_gguf_tensor_at(const nsr_gguf* g, int64_t index, nsr_gguf_tensor* out) {
  if (!g || !out) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  if (index < 0 || index >= (int64_t)g->content.tensor_infos().size())
    return gguf_fail(NSR_ERR_BAD_ARG, "gguf: tensor index out of range");
  fill(g, g->content.tensor_infos()[(size_t)index], out);
  return NSR_OK;
}

nsr_status nsr_gguf_find_tensor(const nsr_gguf* g, const char* name, nsr_gguf_tensor* out) {
  if (!g || !name || !out) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  const TensorInfo* t = g->content.find_tensor(name);
  if (!t) return gguf_fail(NSR_ERR_BAD_ARG, std::string("cannot find tensor ") + name);
  fill(g, *t, out);
  return NSR_OK;
}

nsr_status nsr_gguf_upload(const nsr_gguf* g, const nsr_gguf_tensor* t, void* device_dst, nsr_stream_t stream) {
  if (!g || !t || !device_dst || !t->data) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  // the descriptor must be one this handle filled in (its bytes lie in the file)
  const TensorInfo* info = g->content.find_tensor(t->name ? t->name : "");
  if (!info || g->content.tensor_data(*info) != t->data || info->nbytes != t->nbytes)
    return gguf_fail(NSR_ERR_BAD_ARG, "gguf: tensor descriptor does not belong to this file");
  if (t->nbytes == 0) return NSR_OK;
  hipError_t e = hipMemcpyAsync(device_dst, t->data, (size_t)t->nbytes, hipMemcpyHostToDevice, (hipStream_t)stream);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return gguf_fail(NSR_ERR_HIP, std::string("gguf upload: ") + hipGetErrorString(e));
  }
  return NSR_OK;
}

nsr_status nsr_gguf_metadata_at(const nsr_gguf* g, int64_t index, const char** key, uint32_t* value_type) {
  if (!g || !key || !value_type) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  if (index < 0 || index >= (int64_t)g->content.metadata().size())
    return gguf_fail(NSR_ERR_BAD_ARG, "gguf: metadata index out of range");
  const auto& kv = g->content.metadata()[(size_t)index];
  *key = kv.first.c_str();
  *value_type = kv.second.type;
  return NSR_OK;
}

nsr_status nsr_gguf_get_int(const nsr_gguf* g, const char* key, int64_t* out) {
  if (!out) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  return guarded([&] {
    *out = meta(g, key)->as_int();
    return NSR_OK;
  });
}

nsr_status nsr_gguf_get_float(const nsr_gguf* g, const char* key, double* out) {
  if (!out) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  return guarded([&] {
    *out = meta(g, key)->as_float();
    return NSR_OK;
  });
}

nsr_status nsr_gguf_get_string(const nsr_gguf* g, const char* key, const char** out) {
  if (!out) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  return guarded([&] {
    const Value* v = meta(g, key);
    if (v->type != STRING) throw Error(std::string("gguf: '") + key + "' is not a string");
    *out = v->s.c_str();
    return NSR_OK;
  });
}

nsr_status nsr_gguf_get_array(const nsr_gguf* g, const char* key, uint32_t* elem_type, uint64_t* count) {
  if (!elem_type || !count) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  return guarded([&] {
    const Value* v = meta(g, key);
    if (v->type != ARRAY) throw Error(std::string("gguf: '") + key + "' is not an array");
    *elem_type = v->elem_type;
    *count = v->arr.size();
    return NSR_OK;
  });
}

nsr_status nsr_gguf_get_array_int(const nsr_gguf* g, const char* key, uint64_t i, int64_t* out) {
  if (!out) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  return guarded([&] {
    *out = array_elem(g, key, i)->as_int();
    return NSR_OK;
  });
}

nsr_status nsr_gguf_get_array_float(const nsr_gguf* g, const char* key, uint64_t i, double* out) {
  if (!out) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  return guarded([&] {
    *out = array_elem(g, key, i)->as_float();
    return NSR_OK;
  });
}

nsr_status nsr_gguf_get_array_string(const nsr_gguf* g, const char* key, uint64_t i, const char** out) {
  if (!out) return gguf_fail(NSR_ERR_BAD_ARG, "gguf: null argument");
  return guarded([&] {
    const Value* v = array_elem(g, key, i);
    if (v->type != STRING) throw Error(std::string("gguf: '") + key + "' is not an array of strings");
    *out = v->s.c_str();
    return NSR_OK;
  });
}

}  // extern "C"
