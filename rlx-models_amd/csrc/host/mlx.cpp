// MLX checkpoint reader: the on-disk step in front of the MLX affine / MXFP4
// kernels.  An mlx-community checkpoint is a directory of safetensors files
// (one, or shards listed by model.safetensors.index.json) plus config.json,
// whose "quantization" block gives the packing ({"group_size": g, "bits": b,
// "mode": "affine" | "mxfp4"}, with optional per-layer overrides or `false`
// for a layer left unquantized).  A quantized Linear `key` is stored as three
// tensors: `key.weight` (U32 codes, LSB first, [out, in * bits / 32]),
// `key.scales` and `key.biases` ([out, in / group]; no biases for MXFP4,
// whose scales are E8M0 bytes).  This restates the reference's
// MlxLoader::take_packed_mlx (crates/rlx-models-core/src/weight_loader.rs:
// 906-1012, consumed by load_proj, standard_decoder.rs:590-645); the reader
// underneath is the external crate rlx-mlx-io (absent), restated from the
// published safetensors layout:
//   u64 header length n (little-endian), n bytes of JSON:
//   { "name": {"dtype": "F32", "shape": [..], "data_offsets": [b, e]}, ...,
//     "__metadata__": {...} }, then the data, offsets relative to its start.
// The bytes are handed to the device as stored (rlxq_mlx_upload: pread into
// pinned staging, copies on the caller's stream); scale slabs stored as F16
// can be read converted to f32 (the kernels take F32 or BF16 slabs).
#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "file_io.hpp"
#include "rlxq.h"

namespace {

// ---------------------------------------------------------------- JSON
// A small JSON reader for safetensors headers and config files: objects keep
// their key order; numbers keep the exact integer when they have one.
struct Json {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  double num = 0.0;
  bool is_int = false;
  int64_t i = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;

  const Json* get(const std::string& k) const {
    if (kind != OBJ) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

class JsonParser {
 public:
  JsonParser(const char* p, size_t n) : p_(p), end_(p + n) {}
  bool parse(Json& out) {
    if (!value(out, 0)) return false;
    ws();
    return p_ == end_;
  }
  std::string error() const { return err_; }

 private:
  const char* p_;
  const char* end_;
  std::string err_;

  bool fail(const char* m) {
    if (err_.empty()) err_ = m;
    return false;
  }
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if ((size_t)(end_ - p_) < n || std::memcmp(p_, s, n)) return fail("bad literal");
    p_ += n;
    return true;
  }
  static int hex(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
  }
  void utf8(uint32_t cp, std::string& s) {
    if (cp < 0x80) {
      s += (char)cp;
    } else if (cp < 0x800) {
      s += (char)(0xC0 | (cp >> 6));
      s += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += (char)(0xE0 | (cp >> 12));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    } else {
      s += (char)(0xF0 | (cp >> 18));
      s += (char)(0x80 | ((cp >> 12) & 0x3F));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool u4(uint32_t& v) {
    if (end_ - p_ < 4) return fail("truncated \\u escape");
    v = 0;
    for (int k = 0; k < 4; k++) {
      const int h = hex(*p_++);
      if (h < 0) return fail("bad \\u escape");
      v = v << 4 | (uint32_t)h;
    }
    return true;
  }
  bool string(std::string& s) {
    if (p_ >= end_ || *p_ != '"') return fail("expected a string");
    p_++;
    while (true) {
      if (p_ >= end_) return fail("unterminated string");
      const char c = *p_++;
      if (c == '"') return true;
      if ((unsigned char)c < 0x20) return fail("control character in a string");
      if (c != '\\') {
        s += c;
        continue;
      }
      if (p_ >= end_) return fail("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!u4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {   // surrogate pair
            uint32_t lo;
            if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
            p_ += 2;
            if (!u4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(cp, s);
          break;
        }
        default: return fail("bad escape");
      }
    }
  }
  bool number(Json& v) {
    const char* s = p_;
    if (p_ < end_ && *p_ == '-') p_++;
    const char* digits = p_;
    while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
    if (p_ == digits) return fail("bad number");
    bool integral = true;
    if (p_ < end_ && *p_ == '.') {
      integral = false;
      p_++;
      const char* f = p_;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
      if (p_ == f) return fail("bad number");
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      integral = false;
      p_++;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) p_++;
      const char* x = p_;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
      if (p_ == x) return fail("bad number");
    }
    const std::string text(s, p_);
    v.kind = Json::NUM;
    v.num = std::strtod(text.c_str(), nullptr);
    if (integral && p_ - digits <= 18) {
      v.is_int = true;
      v.i = std::strtoll(text.c_str(), nullptr, 10);
    }
    return true;
  }
  bool value(Json& v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p_ >= end_) return fail("unexpected end");
    const char c = *p_;
    if (c == '{') {
      p_++;
      v.kind = Json::OBJ;
      ws();
      if (p_ < end_ && *p_ == '}') {
        p_++;
        return true;
      }
      while (true) {
        ws();
        std::pair<std::string, Json> kv;
        if (!string(kv.first)) return false;
        ws();
        if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
        p_++;
        if (!value(kv.second, depth + 1)) return false;
        v.obj.push_back(std::move(kv));
        ws();
        if (p_ < end_ && *p_ == ',') {
          p_++;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          p_++;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      p_++;
      v.kind = Json::ARR;
      ws();
      if (p_ < end_ && *p_ == ']') {
        p_++;
        return true;
      }
      while (true) {
        v.arr.emplace_back();
        if (!value(v.arr.back(), depth + 1)) return false;
        ws();
        if (p_ < end_ && *p_ == ',') {
          p_++;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          p_++;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Json::STR;
      return string(v.str);
    }
    if (c == 't') {
      v.kind = Json::BOOL;
      v.b = true;
      return lit("true");
    }
    if (c == 'f') {
      v.kind = Json::BOOL;
      return lit("false");
    }
    if (c == 'n') return lit("null");
    return number(v);
  }
};

// ---------------------------------------------------------------- tensors
struct Dtype {
  const char* name;
  int32_t code;   // rlxq_mlx_dtype
  int32_t bytes;
};
constexpr Dtype kDtypes[] = {
    {"BOOL", RLXQ_ST_BOOL, 1}, {"U8", RLXQ_ST_U8, 1},       {"I8", RLXQ_ST_I8, 1},
    {"U16", RLXQ_ST_U16, 2},   {"I16", RLXQ_ST_I16, 2},     {"F16", RLXQ_ST_F16, 2},
    {"BF16", RLXQ_ST_BF16, 2}, {"U32", RLXQ_ST_U32, 4},     {"I32", RLXQ_ST_I32, 4},
    {"F32", RLXQ_ST_F32, 4},   {"U64", RLXQ_ST_U64, 8},     {"I64", RLXQ_ST_I64, 8},
    {"F64", RLXQ_ST_F64, 8},   {"F8_E4M3", RLXQ_ST_F8_E4M3, 1}, {"F8_E5M2", RLXQ_ST_F8_E5M2, 1},
};
const Dtype* dtype_of(const std::string& s) {
  for (const auto& d : kDtypes)
    if (s == d.name) return &d;
  return nullptr;
}

struct File {
  std::string path;
  int fd = -1;
  uint64_t size = 0, data_start = 0;
};

struct Tensor {
  std::string name;
  int32_t dtype = 0, dbytes = 0, n_dims = 0;
  int64_t shape[8] = {1, 1, 1, 1, 1, 1, 1, 1};
  int file = 0;
  uint64_t off = 0, nbytes = 0;   // absolute file offset, length
};

struct Quant {
  bool on = false;
  int bits = 0, group = 0;
  bool mxfp4 = false;
};

}  // namespace

struct rlxq_mlx {
  std::vector<File> files;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> idx;
  std::unordered_map<std::string, bool> taken;
  Quant quant;                                    // the checkpoint-wide block
  std::map<std::string, Quant> layer_quant;       // per-layer entries
  std::vector<std::string> layer_off;             // layers left unquantized
  std::string err;
  rlxq::StagedUpload up;

  int fail(int code, const std::string& msg) {
    err = msg;
    return code;
  }
  ~rlxq_mlx() {
    for (auto& f : files)
      if (f.fd >= 0) close(f.fd);
  }
};

namespace {

bool read_text(const std::string& path, std::string& out, uint64_t cap) {
  const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return false;
  struct stat st;
  if (fstat(fd, &st) != 0 || (uint64_t)st.st_size > cap) {
    close(fd);
    return false;
  }
  out.resize((size_t)st.st_size);
  const bool ok = rlxq::pread_all(fd, out.data(), out.size(), 0);
  close(fd);
  return ok;
}

bool json_int(const Json* v, int64_t& out) {
  if (!v || v->kind != Json::NUM || !v->is_int) return false;
  out = v->i;
  return true;
}

// One quantization entry: {"group_size": g, "bits": b[, "mode": m]}.
bool parse_quant(const Json& q, Quant& out) {
  int64_t g = 0, b = 0;
  if (!json_int(q.get("group_size"), g) || !json_int(q.get("bits"), b)) return false;
  if (g <= 0 || g > (1 << 20) || b <= 0 || b > 32) return false;
  out.on = true;
  out.group = (int)g;
  out.bits = (int)b;
  const Json* m = q.get("mode");
  out.mxfp4 = m && m->kind == Json::STR && m->str == "mxfp4";
  return true;
}

int add_file(rlxq_mlx* h, const std::string& path) {
  File f;
  f.path = path;
  f.fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  struct stat st;
  if (f.fd < 0 || fstat(f.fd, &st) != 0) {
    if (f.fd >= 0) close(f.fd);
    return h->fail(RLXQ_E_IO, "safetensors: cannot open " + path + ": " + std::strerror(errno));
  }
  f.size = (uint64_t)st.st_size;
  h->files.push_back(f);
  const int fi = (int)h->files.size() - 1;
  uint64_t n = 0;
  if (f.size < 8 || !rlxq::pread_all(f.fd, &n, 8, 0))
    return h->fail(RLXQ_E_FORMAT, "safetensors: " + path + ": truncated header length");
  if (n == 0 || n > f.size - 8 || n > (uint64_t(100) << 20))
    return h->fail(RLXQ_E_FORMAT, "safetensors: " + path + ": header length " + std::to_string(n) +
                                      " does not fit the file");
  std::string text(n, '\0');
  if (!rlxq::pread_all(f.fd, text.data(), n, 8))
    return h->fail(RLXQ_E_IO, "safetensors: " + path + ": header read failed");
  Json root;
  JsonParser jp(text.data(), text.size());
  if (!jp.parse(root) || root.kind != Json::OBJ)
    return h->fail(RLXQ_E_FORMAT, "safetensors: " + path + ": header is not a JSON object (" + jp.error() + ")");
  h->files[fi].data_start = 8 + n;
  const uint64_t data_len = f.size - (8 + n);
  for (const auto& kv : root.obj) {
    if (kv.first == "__metadata__") continue;
    const Json& e = kv.second;
    const Json* dt = e.get("dtype");
    const Json* sh = e.get("shape");
    const Json* of = e.get("data_offsets");
    const std::string where = "safetensors: " + path + ": tensor " + kv.first;
    if (!dt || dt->kind != Json::STR || !sh || sh->kind != Json::ARR || !of || of->kind != Json::ARR ||
        of->arr.size() != 2)
      return h->fail(RLXQ_E_FORMAT, where + ": needs dtype, shape and data_offsets");
    const Dtype* d = dtype_of(dt->str);
    if (!d) return h->fail(RLXQ_E_FORMAT, where + ": unknown dtype " + dt->str);
    if (sh->arr.size() > 8) return h->fail(RLXQ_E_FORMAT, where + ": more than 8 dims");
    Tensor t;
    t.name = kv.first;
    t.dtype = d->code;
    t.dbytes = d->bytes;
    t.n_dims = (int32_t)sh->arr.size();
    t.file = fi;
    uint64_t elems = 1;
    for (size_t k = 0; k < sh->arr.size(); k++) {
      int64_t v;
      if (!json_int(&sh->arr[k], v) || v < 0) return h->fail(RLXQ_E_FORMAT, where + ": bad shape");
      t.shape[k] = v;
      if (__builtin_mul_overflow(elems, (uint64_t)v, &elems)) return h->fail(RLXQ_E_FORMAT, where + ": too large");
    }
    int64_t b, en;
    if (!json_int(&of->arr[0], b) || !json_int(&of->arr[1], en) || b < 0 || en < b || (uint64_t)en > data_len)
      return h->fail(RLXQ_E_FORMAT, where + ": data_offsets outside the data section");
    uint64_t want;
    if (__builtin_mul_overflow(elems, (uint64_t)d->bytes, &want) || want != (uint64_t)(en - b))
      return h->fail(RLXQ_E_FORMAT, where + ": data_offsets do not match dtype and shape");
    t.off = 8 + n + (uint64_t)b;
    t.nbytes = want;
    if (!h->idx.emplace(t.name, h->tensors.size()).second)
      return h->fail(RLXQ_E_FORMAT, where + ": tensor appears twice");
    h->tensors.push_back(std::move(t));
  }
  return RLXQ_OK;
}

int read_config(rlxq_mlx* h, const std::string& dir) {
  std::string text;
  const std::string path = dir + "/config.json";
  struct stat st;
  if (stat(path.c_str(), &st) != 0) return RLXQ_OK;   // no config: nothing is quantized
  if (!read_text(path, text, uint64_t(64) << 20)) return h->fail(RLXQ_E_IO, "mlx: cannot read " + path);
  Json root;
  JsonParser jp(text.data(), text.size());
  if (!jp.parse(root) || root.kind != Json::OBJ)
    return h->fail(RLXQ_E_FORMAT, "mlx: " + path + " is not a JSON object (" + jp.error() + ")");
  // Only an mlx-lm `quantization` object holding bits or group_size marks
  // an MLX-quantized checkpoint (dir_is_mlx_quant,
  // crates/rlx-models-core/src/weight_registry.rs:27-41); GPTQ / AWQ / fp8
  // `quantization_config` blocks belong to the plain safetensors path, so
  // without the marker every tensor is read as stored.
  const Json* q = root.get("quantization");
  if (!q || q->kind != Json::OBJ || (!q->get("bits") && !q->get("group_size"))) return RLXQ_OK;
  if (!parse_quant(*q, h->quant))
    return h->fail(RLXQ_E_FORMAT, "mlx: " + path + ": quantization needs integer group_size and bits");
  for (const auto& kv : q->obj) {
    if (kv.second.kind == Json::OBJ) {
      Quant lq;
      if (!parse_quant(kv.second, lq))
        return h->fail(RLXQ_E_FORMAT, "mlx: " + path + ": quantization entry " + kv.first + " is malformed");
      h->layer_quant[kv.first] = lq;
    } else if (kv.second.kind == Json::BOOL && !kv.second.b) {
      h->layer_off.push_back(kv.first);
    }
  }
  return RLXQ_OK;
}

bool ends_with(const std::string& s, const char* suf) {
  const size_t n = std::strlen(suf);
  return s.size() >= n && !s.compare(s.size() - n, n, suf);
}

int open_dir(rlxq_mlx* h, const std::string& dir) {
  int rc;
  if ((rc = read_config(h, dir))) return rc;
  std::vector<std::string> shards;
  std::string text;
  const std::string index = dir + "/model.safetensors.index.json";
  struct stat st;
  if (stat(index.c_str(), &st) == 0) {
    if (!read_text(index, text, uint64_t(256) << 20)) return h->fail(RLXQ_E_IO, "mlx: cannot read " + index);
    Json root;
    JsonParser jp(text.data(), text.size());
    const Json* wm = nullptr;
    if (!jp.parse(root) || !(wm = root.get("weight_map")) || wm->kind != Json::OBJ)
      return h->fail(RLXQ_E_FORMAT, "mlx: " + index + " has no weight_map object");
    for (const auto& kv : wm->obj) {
      if (kv.second.kind != Json::STR || kv.second.str.find('/') != std::string::npos)
        return h->fail(RLXQ_E_FORMAT, "mlx: " + index + ": bad shard name for " + kv.first);
      if (std::find(shards.begin(), shards.end(), kv.second.str) == shards.end()) shards.push_back(kv.second.str);
    }
  } else {
    DIR* d = opendir(dir.c_str());
    if (!d) return h->fail(RLXQ_E_IO, "mlx: cannot list " + dir);
    while (dirent* e = readdir(d))
      if (ends_with(e->d_name, ".safetensors")) shards.push_back(e->d_name);
    closedir(d);
    std::sort(shards.begin(), shards.end());
  }
  if (shards.empty()) return h->fail(RLXQ_E_NOTFOUND, "mlx: no safetensors files in " + dir);
  for (const auto& s : shards)
    if ((rc = add_file(h, dir + "/" + s))) return rc;
  return RLXQ_OK;
}

const Tensor* find(const rlxq_mlx* h, const std::string& name) {
  auto it = h->idx.find(name);
  return it == h->idx.end() ? nullptr : &h->tensors[it->second];
}

// The quantization that applies to layer `key`: a per-layer entry whose name
// is the key (or the key with a leading "model." removed), else the
// checkpoint-wide block; `false` entries switch it off.
Quant quant_for(const rlxq_mlx* h, const std::string& key) {
  std::vector<std::string> names = {key};
  if (key.rfind("model.", 0) == 0) names.push_back(key.substr(6));
  for (const auto& n : names) {
    if (std::find(h->layer_off.begin(), h->layer_off.end(), n) != h->layer_off.end()) return Quant{};
    auto it = h->layer_quant.find(n);
    if (it != h->layer_quant.end()) return it->second;
  }
  return h->quant;
}

float f16_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = s;
    } else {   // subnormal: m * 2^-24
      float v = std::ldexp((float)m, -24);
      std::memcpy(&bits, &v, 4);
      bits |= s;
    }
  } else if (e == 31) {
    bits = s | 0x7F800000u | (m << 13);
  } else {
    bits = s | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

}  // namespace

extern "C" {

int rlxq_mlx_open(const char* path, rlxq_mlx** out) {
  if (!out) return RLXQ_E_NULL;
  *out = nullptr;
  if (!path) return RLXQ_E_NULL;
  auto* h = new (std::nothrow) rlxq_mlx();
  if (!h) return RLXQ_E_NOMEM;
  *out = h;   // the handle carries the message even on failure
  struct stat st;
  if (stat(path, &st) != 0) return h->fail(RLXQ_E_IO, std::string("mlx: cannot open ") + path);
  const std::string p(path);
  if (S_ISDIR(st.st_mode)) return open_dir(h, p);
  // a single safetensors file: config.json from its directory, if any
  const size_t slash = p.rfind('/');
  int rc = read_config(h, slash == std::string::npos ? "." : p.substr(0, slash));
  if (rc) return rc;
  return add_file(h, p);
}

void rlxq_mlx_close(rlxq_mlx* h) { delete h; }

const char* rlxq_mlx_last_error(const rlxq_mlx* h) { return h ? h->err.c_str() : ""; }

int rlxq_mlx_quantization(const rlxq_mlx* h, int* bits, int* group_size, int* mode) {
  if (!h || !bits || !group_size || !mode) return RLXQ_E_NULL;
  *bits = h->quant.on ? h->quant.bits : 0;
  *group_size = h->quant.on ? h->quant.group : 0;
  *mode = h->quant.on ? (h->quant.mxfp4 ? RLXQ_MLX_MODE_MXFP4 : RLXQ_MLX_MODE_AFFINE) : RLXQ_MLX_MODE_NONE;
  return RLXQ_OK;
}

int64_t rlxq_mlx_tensor_count(const rlxq_mlx* h) { return h ? (int64_t)h->tensors.size() : RLXQ_E_NULL; }

int64_t rlxq_mlx_find_tensor(const rlxq_mlx* h, const char* name) {
  if (!h || !name) return RLXQ_E_NULL;
  auto it = h->idx.find(name);
  return it == h->idx.end() ? RLXQ_E_NOTFOUND : (int64_t)it->second;
}

int rlxq_mlx_tensor_info(const rlxq_mlx* h, int64_t i, rlxq_mlx_tensor* info) {
  if (!h || !info) return RLXQ_E_NULL;
  if (i < 0 || (uint64_t)i >= h->tensors.size()) return RLXQ_E_NOTFOUND;
  const Tensor& t = h->tensors[(size_t)i];
  info->name = t.name.c_str();
  info->dtype = t.dtype;
  info->n_dims = t.n_dims;
  for (int d = 0; d < 8; d++) info->shape[d] = t.shape[d];
  info->nbytes = (int64_t)t.nbytes;
  info->file = h->files[(size_t)t.file].path.c_str();
  info->offset = t.off;
  return RLXQ_OK;
}

int rlxq_mlx_take_packed(rlxq_mlx* h, const char* key, rlxq_mlx_packed* out) {
  if (!h) return RLXQ_E_NULL;
  h->err.clear();
  if (!key || !out) return h->fail(RLXQ_E_NULL, "mlx: null argument");
  std::memset(out, 0, sizeof *out);
  const std::string k(key);
  const Tensor* w = find(h, k + ".weight");
  if (!w) return h->fail(RLXQ_E_NOTFOUND, "mlx: no tensor " + k + ".weight");
  const Tensor* s = find(h, k + ".scales");
  const Quant q = quant_for(h, k);
  // (the reference's Ok(None): a Linear stored dense, or a packing these
  // kernels do not read, stays with the caller's dense path and is not taken)
  if (!q.on || !s || w->dtype != RLXQ_ST_U32 || w->n_dims != 2) return RLXQ_OK;
  int scheme = 0;
  if (q.mxfp4) scheme = (q.bits == 4 && q.group == 32) ? RLXQ_MLX_MXFP4 : 0;
  else if (q.group == 32 || q.group == 64 || q.group == 128)
    scheme = q.bits == 4 ? RLXQ_MLX_AFFINE4 : (q.bits == 8 ? RLXQ_MLX_AFFINE8 : 0);
  if (!scheme) return RLXQ_OK;
  const Tensor* b = q.mxfp4 ? nullptr : find(h, k + ".biases");
  if (!q.mxfp4 && !b) return h->fail(RLXQ_E_NOTFOUND, "mlx: affine Linear " + k + " has no .biases");
  if (h->taken.count(k)) return h->fail(RLXQ_E_TAKEN, "weight already taken: " + k);
  const int64_t n = w->shape[0], kin = w->shape[1] * 32 / q.bits;
  const int64_t groups = kin / q.group;
  if (n <= 0 || kin <= 0 || kin % q.group || s->n_dims != 2 || s->shape[0] != n || s->shape[1] != groups)
    return h->fail(RLXQ_E_SHAPE, "mlx: " + k + ": scales are not [out, in / group_size]");
  const bool s_ok = q.mxfp4 ? s->dtype == RLXQ_ST_U8
                            : (s->dtype == RLXQ_ST_F32 || s->dtype == RLXQ_ST_BF16 || s->dtype == RLXQ_ST_F16);
  if (!s_ok) return h->fail(RLXQ_E_DTYPE, "mlx: " + k + ": scale dtype not readable");
  if (b && (b->n_dims != 2 || b->shape[0] != n || b->shape[1] != groups || b->dtype != s->dtype))
    return h->fail(RLXQ_E_SHAPE, "mlx: " + k + ": biases do not match the scales");
  out->scheme = scheme;
  out->bits = q.bits;
  out->group_size = q.group;
  out->out_features = n;
  out->in_features = kin;
  out->codes = w->name.c_str();
  out->scales = s->name.c_str();
  out->biases = b ? b->name.c_str() : nullptr;
  out->codes_nbytes = (int64_t)w->nbytes;
  out->scales_nbytes = (int64_t)s->nbytes;
  out->biases_nbytes = b ? (int64_t)b->nbytes : 0;
  out->slab_dtype = s->dtype;
  h->taken[k] = true;
  return RLXQ_OK;
}

int rlxq_mlx_read(rlxq_mlx* h, const char* name, void* dst, size_t cap) {
  if (!h) return RLXQ_E_NULL;
  h->err.clear();
  if (!name || !dst) return h->fail(RLXQ_E_NULL, "mlx: null argument");
  const Tensor* t = find(h, name);
  if (!t) return h->fail(RLXQ_E_NOTFOUND, std::string("mlx: no tensor ") + name);
  if (t->nbytes > cap) return h->fail(RLXQ_E_SHAPE, std::string("mlx: ") + name + " needs " + std::to_string(t->nbytes) + " bytes");
  if (!rlxq::pread_all(h->files[(size_t)t->file].fd, dst, t->nbytes, t->off))
    return h->fail(RLXQ_E_IO, std::string("mlx: read failed for ") + name);
  return RLXQ_OK;
}

int rlxq_mlx_read_f32(rlxq_mlx* h, const char* name, float* dst, size_t count) {
  if (!h) return RLXQ_E_NULL;
  h->err.clear();
  if (!name || !dst) return h->fail(RLXQ_E_NULL, "mlx: null argument");
  const Tensor* t = find(h, name);
  if (!t) return h->fail(RLXQ_E_NOTFOUND, std::string("mlx: no tensor ") + name);
  if (t->dtype != RLXQ_ST_F32 && t->dtype != RLXQ_ST_F16 && t->dtype != RLXQ_ST_BF16)
    return h->fail(RLXQ_E_DTYPE, std::string("mlx: ") + name + " is not F32, F16 or BF16");
  const uint64_t elems = t->nbytes / (uint64_t)t->dbytes;
  if (elems > count) return h->fail(RLXQ_E_SHAPE, std::string("mlx: ") + name + " has " + std::to_string(elems) + " elements");
  if (t->dtype == RLXQ_ST_F32) return rlxq_mlx_read(h, name, dst, count * 4);
  std::vector<uint16_t> raw((size_t)elems);
  if (!rlxq::pread_all(h->files[(size_t)t->file].fd, raw.data(), t->nbytes, t->off))
    return h->fail(RLXQ_E_IO, std::string("mlx: read failed for ") + name);
  for (uint64_t i = 0; i < elems; i++) {
    if (t->dtype == RLXQ_ST_F16) {
      dst[i] = f16_to_f32(raw[i]);
    } else {
      const uint32_t bits = (uint32_t)raw[i] << 16;
      std::memcpy(&dst[i], &bits, 4);
    }
  }
  return RLXQ_OK;
}

int rlxq_mlx_upload(rlxq_mlx* h, const char* name, void* dst, size_t cap, void* stream) {
  if (!h) return RLXQ_E_NULL;
  h->err.clear();
  if (!name || !dst) return h->fail(RLXQ_E_NULL, "mlx: null argument");
  const Tensor* t = find(h, name);
  if (!t) return h->fail(RLXQ_E_NOTFOUND, std::string("mlx: no tensor ") + name);
  if (t->nbytes > cap) return h->fail(RLXQ_E_SHAPE, std::string("mlx: ") + name + " needs " + std::to_string(t->nbytes) + " bytes");
  std::string why;
  const int rc = h->up.run(h->files[(size_t)t->file].fd, t->off, t->nbytes, dst, stream, &why);
  return rc ? h->fail(rc, std::string("mlx: ") + name + ": " + why) : RLXQ_OK;
}

}  // extern "C"
