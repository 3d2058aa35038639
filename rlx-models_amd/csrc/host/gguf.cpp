// GGUF checkpoint reader: the on-disk step in front of the packed-weight
// kernels.  It parses a GGUF file's header (version 2 or 3: magic, counts,
// metadata key/values, tensor infos, aligned data section) and hands each
// packed tensor to the device without dequantising it, as the reference's
// `GgufLoader::take_packed` / `take_packed_metadata` do
// (crates/rlx-models-core/src/weight_loader.rs:1360-1486; ggml type ->
// QuantScheme map :497-565) with the streamed upload of
// crates/rlx-qwen3/src/high_level_runner.rs:474-499 (one reused scratch per
// tensor instead of borrowing the whole mapping).
//
// The container parser itself is the external crate `rlx_gguf` (^0.2.19,
// not in the reference tree); this file restates the published GGUF layout:
//   u32 magic "GGUF", u32 version, u64 tensor_count, u64 kv_count,
//   kv_count x { string key, u32 type, value },
//   tensor_count x { string name, u32 n_dims, u64 dims[n_dims] (innermost
//                    first), u32 ggml_type, u64 offset (from the data start) },
//   data start = header end rounded up to general.alignment (default 32).
// Strings are u64 length + bytes; arrays are u32 element type + u64 count +
// elements.  All little-endian.
//
// Uploads read the file with pread (up to 8 threads per buffer) into two
// pinned staging buffers (hipHostMalloc) and copy each filled buffer to the
// device on the caller's stream while the other one is refilled, so the host
// never holds more than the two buffers, whatever the tensor size.
#include <fcntl.h>
#include <hip/hip_runtime_api.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstdint>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "file_io.hpp"
#include "rlxq.h"

namespace {

using rlxq::pread_all;

enum : uint32_t {
  GT_U8 = 0, GT_I8 = 1, GT_U16 = 2, GT_I16 = 3, GT_U32 = 4, GT_I32 = 5, GT_F32 = 6, GT_BOOL = 7,
  GT_STR = 8, GT_ARR = 9, GT_U64 = 10, GT_I64 = 11, GT_F64 = 12
};

int scalar_bytes(uint32_t t) {
  switch (t) {
    case GT_U8: case GT_I8: case GT_BOOL: return 1;
    case GT_U16: case GT_I16: return 2;
    case GT_U32: case GT_I32: case GT_F32: return 4;
    case GT_U64: case GT_I64: case GT_F64: return 8;
    default: return 0;
  }
}

// ggml tensor types with a fixed block layout: elements per block and bytes
// per block (ggml's type traits; blocks run along the innermost dimension).
struct TypeLayout { int32_t id; int32_t block; int32_t bytes; };
constexpr TypeLayout kLayouts[] = {
    {0, 1, 4},       // F32
    {1, 1, 2},       // F16
    {2, 32, 18},     // Q4_0
    {3, 32, 20},     // Q4_1
    {6, 32, 22},     // Q5_0
    {7, 32, 24},     // Q5_1
    {8, 32, 34},     // Q8_0
    {9, 32, 36},     // Q8_1
    {10, 256, 84},   // Q2_K
    {11, 256, 110},  // Q3_K
    {12, 256, 144},  // Q4_K
    {13, 256, 176},  // Q5_K
    {14, 256, 210},  // Q6_K
    {15, 256, 292},  // Q8_K
    {24, 1, 1},      // I8
    {25, 1, 2},      // I16
    {26, 1, 4},      // I32
    {27, 1, 8},      // I64
    {28, 1, 8},      // F64
    {30, 1, 2},      // BF16
};

const TypeLayout* layout_of(int32_t t) {
  for (const auto& l : kLayouts)
    if (l.id == t) return &l;
  return nullptr;
}

// ggml type -> rlxq scheme for the types whose packed bytes the kernels read
// as stored (ggml_type_to_quant_scheme, weight_loader.rs:497-565); 0 for the
// rest.  Q4_1 stays packed unconditionally: the reference's opt-in
// (`RLX_GGUF_PACKED_Q4_1`, :556-565) exists because its GPU backends cannot
// dequantise Q4_1, which these kernels do.
int scheme_of(int32_t t) {
  switch (t) {
    case 2: return RLXQ_GGUF_Q4_0;
    case 3: return RLXQ_GGUF_Q4_1;
    case 8: return RLXQ_GGUF_Q8_0;
    case 10: return RLXQ_GGUF_Q2_K;
    case 11: return RLXQ_GGUF_Q3_K;
    case 12: return RLXQ_GGUF_Q4_K;
    case 13: return RLXQ_GGUF_Q5_K;
    case 14: return RLXQ_GGUF_Q6_K;
    case 15: return RLXQ_GGUF_Q8_K;
    default: return 0;
  }
}

struct Meta {
  std::string key;
  uint32_t type = 0;       // value type (GT_ARR for arrays)
  uint32_t elem = 0;       // element type of an array, else = type
  uint64_t count = 1;      // elements (1 for a scalar)
  std::vector<uint8_t> raw;          // numeric values, little-endian, packed
  std::vector<std::string> strs;     // string values
};

struct Tensor {
  std::string name;
  int32_t type = 0;
  int32_t n_dims = 0;
  int64_t dims[4] = {1, 1, 1, 1};   // innermost first, as stored
  uint64_t rel = 0;                 // offset from the data start
  int64_t nbytes = -1;              // -1: no fixed block layout for the type
  bool taken = false;
};


}  // namespace

struct rlxq_gguf {
  int fd = -1;
  uint64_t file_size = 0;
  uint32_t version = 0;
  uint32_t alignment = 32;
  uint64_t data_start = 0;
  std::vector<Meta> meta;
  std::unordered_map<std::string, size_t> meta_idx;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> tensor_idx;
  std::string err;
  rlxq::StagedUpload up;

  int fail(int code, const std::string& msg) {
    err = msg;
    return code;
  }
};

namespace {

// Sequential reader over pread with a 1 MiB window; every read is bounds
// checked against the file size.
class Reader {
 public:
  Reader(int fd, uint64_t size) : fd_(fd), size_(size), buf_(1 << 20) {}
  uint64_t pos() const { return pos_; }
  bool read(void* dst, uint64_t n) {
    if (n > size_ - std::min(pos_, size_)) return false;
    uint8_t* d = static_cast<uint8_t*>(dst);
    while (n) {
      if (pos_ < win_ || pos_ >= win_ + win_len_) {
        const ssize_t r = pread(fd_, buf_.data(), buf_.size(), (off_t)pos_);
        if (r <= 0) return false;
        win_ = pos_;
        win_len_ = (size_t)r;
      }
      const uint64_t off = pos_ - win_;
      const uint64_t take = std::min<uint64_t>(n, win_len_ - off);
      std::memcpy(d, buf_.data() + off, take);
      d += take;
      pos_ += take;
      n -= take;
    }
    return true;
  }
  template <class T>
  bool get(T& v) { return read(&v, sizeof v); }
  bool str(std::string& s) {
    uint64_t n;
    if (!get(n) || n > (uint64_t(1) << 30) || n > size_ - pos_) return false;
    s.resize(n);
    return read(s.data(), n);
  }
  uint64_t left() const { return size_ > pos_ ? size_ - pos_ : 0; }

 private:
  int fd_;
  uint64_t size_, pos_ = 0, win_ = 0;
  size_t win_len_ = 0;
  std::vector<uint8_t> buf_;
};

int parse(rlxq_gguf* g) {
  Reader r(g->fd, g->file_size);
  uint32_t magic = 0, version = 0;
  if (!r.get(magic) || magic != 0x46554747u) return g->fail(RLXQ_E_FORMAT, "gguf: bad magic (not a GGUF file)");
  if (!r.get(version)) return g->fail(RLXQ_E_FORMAT, "gguf: truncated header");
  if (version != 2 && version != 3)
    return g->fail(RLXQ_E_FORMAT, "gguf: unsupported version " + std::to_string(version) + " (2 and 3 are read)");
  g->version = version;
  uint64_t nt = 0, nkv = 0;
  if (!r.get(nt) || !r.get(nkv)) return g->fail(RLXQ_E_FORMAT, "gguf: truncated header");
  // every entry takes more than 8 bytes: counts beyond that are corrupt
  if (nt > r.left() / 8 || nkv > r.left() / 8) return g->fail(RLXQ_E_FORMAT, "gguf: counts exceed the file");

  g->meta.resize(nkv);
  for (uint64_t i = 0; i < nkv; i++) {
    Meta& m = g->meta[i];
    if (!r.str(m.key) || !r.get(m.type)) return g->fail(RLXQ_E_FORMAT, "gguf: truncated metadata");
    m.elem = m.type;
    m.count = 1;
    if (m.type == GT_ARR) {
      if (!r.get(m.elem) || !r.get(m.count)) return g->fail(RLXQ_E_FORMAT, "gguf: truncated metadata array");
      if (m.elem == GT_ARR) return g->fail(RLXQ_E_FORMAT, "gguf: nested array in " + m.key);
    }
    if (m.elem == GT_STR) {
      if (m.count > r.left() / 8) return g->fail(RLXQ_E_FORMAT, "gguf: array exceeds the file in " + m.key);
      m.strs.resize(m.count);
      for (auto& s : m.strs)
        if (!r.str(s)) return g->fail(RLXQ_E_FORMAT, "gguf: truncated string in " + m.key);
    } else {
      const int sb = scalar_bytes(m.elem);
      if (!sb) return g->fail(RLXQ_E_FORMAT, "gguf: unknown value type " + std::to_string(m.elem) + " in " + m.key);
      if (m.count > r.left() / sb) return g->fail(RLXQ_E_FORMAT, "gguf: array exceeds the file in " + m.key);
      m.raw.resize(m.count * sb);
      if (!r.read(m.raw.data(), m.raw.size())) return g->fail(RLXQ_E_FORMAT, "gguf: truncated value in " + m.key);
    }
    if (!g->meta_idx.emplace(m.key, i).second) return g->fail(RLXQ_E_FORMAT, "gguf: duplicate key " + m.key);
  }
  auto it = g->meta_idx.find("general.alignment");
  if (it != g->meta_idx.end()) {
    const Meta& m = g->meta[it->second];
    if (m.type != GT_U32) return g->fail(RLXQ_E_FORMAT, "gguf: general.alignment is not a u32");
    uint32_t a;
    std::memcpy(&a, m.raw.data(), 4);
    if (a == 0 || (a & (a - 1))) return g->fail(RLXQ_E_FORMAT, "gguf: general.alignment is not a power of two");
    g->alignment = a;
  }

  g->tensors.resize(nt);
  for (uint64_t i = 0; i < nt; i++) {
    Tensor& t = g->tensors[i];
    uint32_t nd = 0;
    if (!r.str(t.name) || !r.get(nd)) return g->fail(RLXQ_E_FORMAT, "gguf: truncated tensor info");
    if (nd == 0 || nd > 4) return g->fail(RLXQ_E_FORMAT, "gguf: tensor " + t.name + " has " + std::to_string(nd) + " dims (1..4)");
    t.n_dims = (int32_t)nd;
    uint64_t elems = 1;
    bool big = false;
    for (uint32_t d = 0; d < nd; d++) {
      uint64_t v;
      if (!r.get(v)) return g->fail(RLXQ_E_FORMAT, "gguf: truncated tensor info");
      t.dims[d] = (int64_t)(v & ((uint64_t(1) << 62) - 1));
      if (v >= (uint64_t(1) << 62) || __builtin_mul_overflow(elems, v, &elems)) big = true;
    }
    uint32_t ty;
    if (!r.get(ty) || !r.get(t.rel)) return g->fail(RLXQ_E_FORMAT, "gguf: truncated tensor info");
    if (big || elems >= (uint64_t(1) << 62)) return g->fail(RLXQ_E_FORMAT, "gguf: tensor " + t.name + " is too large");
    t.type = (int32_t)ty;
    if (const TypeLayout* l = layout_of(t.type)) {
      // (blocks x bytes per block, checked: 8-byte types could wrap)
      uint64_t nb = 0;
      if (t.dims[0] % l->block == 0 &&
          !__builtin_mul_overflow(elems / l->block, (uint64_t)l->bytes, &nb) && nb < (uint64_t(1) << 62))
        t.nbytes = (int64_t)nb;
      else if (t.dims[0] % l->block == 0)
        return g->fail(RLXQ_E_FORMAT, "gguf: tensor " + t.name + " is too large");
    }
    if (!g->tensor_idx.emplace(t.name, i).second) return g->fail(RLXQ_E_FORMAT, "gguf: duplicate tensor " + t.name);
  }
  const uint64_t a = g->alignment;
  g->data_start = (r.pos() + a - 1) / a * a;
  return RLXQ_OK;
}

Tensor* tensor_at(rlxq_gguf* g, const char* name, int* rc) {
  if (!name) {
    *rc = g->fail(RLXQ_E_NULL, "gguf: tensor name is null");
    return nullptr;
  }
  auto it = g->tensor_idx.find(name);
  if (it == g->tensor_idx.end()) {
    *rc = g->fail(RLXQ_E_NOTFOUND, std::string("tensor missing: ") + name);
    return nullptr;
  }
  *rc = RLXQ_OK;
  return &g->tensors[it->second];
}

// The tensor's byte range in the file, checked against the file size.
int data_range(rlxq_gguf* g, const Tensor& t, uint64_t* off, uint64_t* len) {
  if (t.nbytes < 0)
    return g->fail(RLXQ_E_FORMAT, "gguf: tensor " + t.name + ": ggml type " + std::to_string(t.type) +
                                      " has no fixed block layout here, or its rows are not whole blocks");
  if (t.rel % g->alignment) return g->fail(RLXQ_E_FORMAT, "gguf: tensor " + t.name + " is not aligned");
  const uint64_t o = g->data_start + t.rel, n = (uint64_t)t.nbytes;
  if (o < g->data_start || o > g->file_size || n > g->file_size - o)
    return g->fail(RLXQ_E_IO, "gguf: tensor " + t.name + " data lies past the end of the file");
  *off = o;
  *len = n;
  return RLXQ_OK;
}

const Meta* meta_at(const rlxq_gguf* g, int64_t i) {
  return (g && i >= 0 && (uint64_t)i < g->meta.size()) ? &g->meta[(size_t)i] : nullptr;
}

// Element j of a numeric value as int64 or double.
bool meta_int(const Meta& m, uint64_t j, int64_t* v) {
  const uint8_t* p = m.raw.data() + j * scalar_bytes(m.elem);
  switch (m.elem) {
    case GT_U8: *v = *p; return true;
    case GT_I8: *v = (int8_t)*p; return true;
    case GT_BOOL: *v = *p != 0; return true;
    case GT_U16: { uint16_t x; std::memcpy(&x, p, 2); *v = x; return true; }
    case GT_I16: { int16_t x; std::memcpy(&x, p, 2); *v = x; return true; }
    case GT_U32: { uint32_t x; std::memcpy(&x, p, 4); *v = x; return true; }
    case GT_I32: { int32_t x; std::memcpy(&x, p, 4); *v = x; return true; }
    case GT_U64: { uint64_t x; std::memcpy(&x, p, 8); if (x > (uint64_t)INT64_MAX) return false; *v = (int64_t)x; return true; }
    case GT_I64: { int64_t x; std::memcpy(&x, p, 8); *v = x; return true; }
    default: return false;
  }
}

bool meta_float(const Meta& m, uint64_t j, double* v) {
  const uint8_t* p = m.raw.data() + j * scalar_bytes(m.elem);
  if (m.elem == GT_F32) { float x; std::memcpy(&x, p, 4); *v = x; return true; }
  if (m.elem == GT_F64) { std::memcpy(v, p, 8); return true; }
  int64_t i;
  if (!meta_int(m, j, &i)) return false;
  *v = (double)i;
  return true;
}

}  // namespace

extern "C" {

int rlxq_gguf_open(const char* path, rlxq_gguf** out) {
  if (!out) return RLXQ_E_NULL;
  *out = nullptr;
  if (!path) return RLXQ_E_NULL;
  auto* g = new (std::nothrow) rlxq_gguf();
  if (!g) return RLXQ_E_NOMEM;
  g->fd = open(path, O_RDONLY | O_CLOEXEC);
  struct stat st;
  if (g->fd < 0 || fstat(g->fd, &st) != 0) {
    g->fail(RLXQ_E_IO, std::string("gguf: cannot open ") + path + ": " + std::strerror(errno));
    *out = g;   // the handle carries the message; rlxq_gguf_close frees it
    return RLXQ_E_IO;
  }
  g->file_size = (uint64_t)st.st_size;
  const int rc = parse(g);
  *out = g;
  return rc;
}

void rlxq_gguf_close(rlxq_gguf* g) {
  if (!g) return;
  if (g->fd >= 0) close(g->fd);
  delete g;   // (the staging buffers wait for their last copies)
}

const char* rlxq_gguf_last_error(const rlxq_gguf* g) { return g ? g->err.c_str() : ""; }

int rlxq_gguf_version(const rlxq_gguf* g) { return g ? (int)g->version : RLXQ_E_NULL; }

int64_t rlxq_gguf_data_offset(const rlxq_gguf* g) { return g ? (int64_t)g->data_start : RLXQ_E_NULL; }

int64_t rlxq_gguf_tensor_count(const rlxq_gguf* g) { return g ? (int64_t)g->tensors.size() : RLXQ_E_NULL; }

int64_t rlxq_gguf_find_tensor(const rlxq_gguf* g, const char* name) {
  if (!g || !name) return RLXQ_E_NULL;
  auto it = g->tensor_idx.find(name);
  return it == g->tensor_idx.end() ? RLXQ_E_NOTFOUND : (int64_t)it->second;
}

int rlxq_gguf_tensor_info(const rlxq_gguf* g, int64_t i, rlxq_gguf_tensor* info) {
  if (!g || !info) return RLXQ_E_NULL;
  if (i < 0 || (uint64_t)i >= g->tensors.size()) return RLXQ_E_NOTFOUND;
  const Tensor& t = g->tensors[(size_t)i];
  info->name = t.name.c_str();
  info->ggml_type = t.type;
  info->n_dims = t.n_dims;
  for (int d = 0; d < 4; d++) info->dims[d] = t.dims[d];
  info->offset = g->data_start + t.rel;
  info->nbytes = t.nbytes;
  info->scheme = scheme_of(t.type);
  return RLXQ_OK;
}

int rlxq_gguf_take_packed(rlxq_gguf* g, const char* name, int* scheme, int64_t shape[4], int* n_dims,
                          int64_t* nbytes) {
  if (!g) return RLXQ_E_NULL;
  g->err.clear();
  if (!scheme || !shape || !n_dims || !nbytes) return g->fail(RLXQ_E_NULL, "gguf: null output pointer");
  int rc;
  Tensor* t = tensor_at(g, name, &rc);
  if (!t) return rc;
  if (t->taken) return g->fail(RLXQ_E_TAKEN, std::string("weight already taken: ") + name);
  *scheme = scheme_of(t->type);
  *n_dims = t->n_dims;
  for (int d = 0; d < 4; d++) shape[d] = d < t->n_dims ? t->dims[t->n_dims - 1 - d] : 1;
  *nbytes = t->nbytes;
  if (!*scheme) return RLXQ_OK;   // stored in a form that does not stay packed: not taken
  if (t->nbytes < 0 || rlxq_row_bytes(*scheme, t->dims[0]) < 0)
    return g->fail(RLXQ_E_SHAPE, std::string("gguf: tensor ") + name + ": rows are not whole blocks");
  t->taken = true;
  return RLXQ_OK;
}

int rlxq_gguf_read(rlxq_gguf* g, const char* name, void* dst, size_t cap) {
  if (!g) return RLXQ_E_NULL;
  g->err.clear();
  if (!dst) return g->fail(RLXQ_E_NULL, "gguf: destination is null");
  int rc;
  const Tensor* t = tensor_at(g, name, &rc);
  if (!t) return rc;
  uint64_t off, len;
  if ((rc = data_range(g, *t, &off, &len))) return rc;
  if (len > cap) return g->fail(RLXQ_E_SHAPE, std::string("gguf: ") + name + " needs " + std::to_string(len) + " bytes");
  if (!pread_all(g->fd, dst, len, off)) return g->fail(RLXQ_E_IO, std::string("gguf: read failed for ") + name);
  return RLXQ_OK;
}

int rlxq_gguf_upload(rlxq_gguf* g, const char* name, void* dst, size_t cap, void* stream) {
  if (!g) return RLXQ_E_NULL;
  g->err.clear();
  if (!dst) return g->fail(RLXQ_E_NULL, "gguf: destination is null");
  int rc;
  const Tensor* t = tensor_at(g, name, &rc);
  if (!t) return rc;
  uint64_t off, len;
  if ((rc = data_range(g, *t, &off, &len))) return rc;
  if (len > cap) return g->fail(RLXQ_E_SHAPE, std::string("gguf: ") + name + " needs " + std::to_string(len) + " bytes");
  std::string why;
  if ((rc = g->up.run(g->fd, off, len, dst, stream, &why)))
    return g->fail(rc, std::string("gguf: ") + name + ": " + why);
  return RLXQ_OK;
}

int64_t rlxq_gguf_meta_count(const rlxq_gguf* g) { return g ? (int64_t)g->meta.size() : RLXQ_E_NULL; }

int64_t rlxq_gguf_meta_find(const rlxq_gguf* g, const char* key) {
  if (!g || !key) return RLXQ_E_NULL;
  auto it = g->meta_idx.find(key);
  return it == g->meta_idx.end() ? RLXQ_E_NOTFOUND : (int64_t)it->second;
}

const char* rlxq_gguf_meta_key(const rlxq_gguf* g, int64_t i) {
  const Meta* m = meta_at(g, i);
  return m ? m->key.c_str() : nullptr;
}

int rlxq_gguf_meta_type(const rlxq_gguf* g, int64_t i, int* type, int* elem_type, uint64_t* count) {
  const Meta* m = meta_at(g, i);
  if (!m) return g ? RLXQ_E_NOTFOUND : RLXQ_E_NULL;
  if (type) *type = (int)m->type;
  if (elem_type) *elem_type = (int)m->elem;
  if (count) *count = m->count;
  return RLXQ_OK;
}

int rlxq_gguf_meta_int(const rlxq_gguf* g, int64_t i, uint64_t j, int64_t* v) {
  const Meta* m = meta_at(g, i);
  if (!m || !v) return (!g || !v) ? RLXQ_E_NULL : RLXQ_E_NOTFOUND;
  if (j >= m->count || m->elem == GT_STR || !meta_int(*m, j, v)) return RLXQ_E_DTYPE;
  return RLXQ_OK;
}

int rlxq_gguf_meta_float(const rlxq_gguf* g, int64_t i, uint64_t j, double* v) {
  const Meta* m = meta_at(g, i);
  if (!m || !v) return (!g || !v) ? RLXQ_E_NULL : RLXQ_E_NOTFOUND;
  if (j >= m->count || m->elem == GT_STR || !meta_float(*m, j, v)) return RLXQ_E_DTYPE;
  return RLXQ_OK;
}

int rlxq_gguf_meta_str(const rlxq_gguf* g, int64_t i, uint64_t j, const char** s, uint64_t* len) {
  const Meta* m = meta_at(g, i);
  if (!m || !s) return (!g || !s) ? RLXQ_E_NULL : RLXQ_E_NOTFOUND;
  if (j >= m->count || m->elem != GT_STR) return RLXQ_E_DTYPE;
  *s = m->strs[(size_t)j].c_str();
  if (len) *len = m->strs[(size_t)j].size();
  return RLXQ_OK;
}

}  // extern "C"
