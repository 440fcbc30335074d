// nf4_loader.hip - shard loader: the on-disk NF4 format of AethelStream's
// shard_engine read from mmap'd safetensors files, dequantized on the device.
//
// Mirrors shard_engine/src/loader.rs (ShardLoader::new / load_layer /
// load_param), shard_engine/src/index.rs (IndexStore, TensorInfo) and the
// error kinds of shard_engine/src/error.rs:5-28.  The NF4 branch of
// load_param keeps the reference's checks and their order (loader.rs:93-161):
// packed bounds, the three required nf4_* fields, absmax bounds, 4-byte
// absmax alignment; then dequant_nf4_alloc semantics (n = 2 * packed bytes,
// nf4.rs:98-107) on the device.  The index may also carry the double-quant
// extension written by aethelstream_amd.shard (nf4_absmax_q_offset/_length,
// nf4_absmax_scale_offset/_length, nf4_dq_group); the reference loader does
// not know those fields.
#include "abi_common.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <vector>

namespace nf4s {

// ---------------------------------------------------------------------------
// Minimal JSON (objects, arrays, strings, integers, true/false/null).
// ---------------------------------------------------------------------------
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0.0;
  long long inum = 0;
  bool is_int = false;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
  const Json *get(const char *key) const {
    for (const auto &kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

class JsonParser {
 public:
  JsonParser(const char *s, size_t n) : p_(s), end_(s + n) {}
  bool parse(Json &out, std::string &err) {
    ws();
    if (!value(out, 0)) {
      err = err_.empty() ? "invalid JSON" : err_;
      return false;
    }
    ws();
    if (p_ != end_) {
      err = "trailing characters after JSON value";
      return false;
    }
    return true;
  }

 private:
  const char *p_, *end_;
  std::string err_;
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
  }
  bool fail_(const char *m) {
    if (err_.empty()) err_ = m;
    return false;
  }
  bool lit(const char *w) {
    const size_t n = strlen(w);
    if ((size_t)(end_ - p_) < n || memcmp(p_, w, n) != 0) return fail_("unexpected token");
    p_ += n;
    return true;
  }
  bool string(std::string &s) {
    if (p_ >= end_ || *p_ != '"') return fail_("expected string");
    ++p_;
    while (p_ < end_ && *p_ != '"') {
      char c = *p_++;
      if (c == '\\') {
        if (p_ >= end_) return fail_("bad escape");
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
            if (end_ - p_ < 4) return fail_("bad unicode escape");
            unsigned v = 0;
            for (int i = 0; i < 4; ++i) {
              const char h = *p_++;
              v <<= 4;
              if (h >= '0' && h <= '9') v |= h - '0';
              else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
              else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
              else return fail_("bad unicode escape");
            }
            if (v < 0x80) {
              s += (char)v;
            } else if (v < 0x800) {
              s += (char)(0xc0 | (v >> 6));
              s += (char)(0x80 | (v & 0x3f));
            } else {
              s += (char)(0xe0 | (v >> 12));
              s += (char)(0x80 | ((v >> 6) & 0x3f));
              s += (char)(0x80 | (v & 0x3f));
            }
            break;
          }
          default: return fail_("bad escape");
        }
      } else {
        s += c;
      }
    }
    if (p_ >= end_) return fail_("unterminated string");
    ++p_;
    return true;
  }
  bool number(Json &j) {
    const char *s = p_;
    if (p_ < end_ && (*p_ == '-' || *p_ == '+')) ++p_;
    bool frac = false;
    while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                         *p_ == '-' || *p_ == '+')) {
      if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') frac = true;
      ++p_;
    }
    if (p_ == s) return fail_("expected value");
    const std::string t(s, p_);
    j.kind = Json::Num;
    j.num = strtod(t.c_str(), nullptr);
    j.is_int = !frac;
    if (j.is_int) j.inum = strtoll(t.c_str(), nullptr, 10);
    return true;
  }
  bool value(Json &j, int depth) {
    if (depth > 64) return fail_("JSON nested too deeply");
    ws();
    if (p_ >= end_) return fail_("unexpected end of JSON");
    const char c = *p_;
    if (c == '{') {
      ++p_;
      j.kind = Json::Obj;
      ws();
      if (p_ < end_ && *p_ == '}') { ++p_; return true; }
      while (true) {
        ws();
        std::string k;
        if (!string(k)) return false;
        ws();
        if (p_ >= end_ || *p_ != ':') return fail_("expected ':'");
        ++p_;
        Json v;
        if (!value(v, depth + 1)) return false;
        j.obj.emplace_back(std::move(k), std::move(v));
        ws();
        if (p_ < end_ && *p_ == ',') { ++p_; continue; }
        if (p_ < end_ && *p_ == '}') { ++p_; return true; }
        return fail_("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p_;
      j.kind = Json::Arr;
      ws();
      if (p_ < end_ && *p_ == ']') { ++p_; return true; }
      while (true) {
        Json v;
        if (!value(v, depth + 1)) return false;
        j.arr.push_back(std::move(v));
        ws();
        if (p_ < end_ && *p_ == ',') { ++p_; continue; }
        if (p_ < end_ && *p_ == ']') { ++p_; return true; }
        return fail_("expected ',' or ']'");
      }
    }
    if (c == '"') {
      j.kind = Json::Str;
      return string(j.str);
    }
    if (c == 't') { j.kind = Json::Bool; j.b = true; return lit("true"); }
    if (c == 'f') { j.kind = Json::Bool; j.b = false; return lit("false"); }
    if (c == 'n') { j.kind = Json::Null; return lit("null"); }
    return number(j);
  }
};

// ---------------------------------------------------------------------------
// Index (shard_engine/src/index.rs:7-34)
// ---------------------------------------------------------------------------
struct TensorInfo {
  std::string file_path;
  int64_t byte_offset = 0, byte_length = 0;
  std::vector<int64_t> shape;
  std::string dtype, precision;
  bool has_absmax_offset = false, has_absmax_length = false, has_block_size = false;
  int64_t absmax_offset = 0, absmax_length = 0, block_size = 0;
  // double-quant extension
  bool dq = false;
  int64_t q_offset = 0, q_length = 0, scale_offset = 0, scale_length = 0, dq_group = 0;
};

struct MappedFile {
  const uint8_t *data = nullptr;
  size_t size = 0;
  ~MappedFile() {
    if (data != nullptr && size > 0) munmap(const_cast<uint8_t *>(data), size);
  }
};

}  // namespace nf4s

struct nf4s_loader {
  std::string model_dir;
  std::map<std::string, nf4s::TensorInfo> index;
  std::map<std::string, std::string> registry;
  std::map<std::string, std::unique_ptr<nf4s::MappedFile>> mmap_cache;
};

namespace nf4s {

static bool read_file(const std::string &path, std::string &out, int &err) {
  const int fd = open(path.c_str(), O_RDONLY);
  if (fd < 0) {
    err = errno;
    return false;
  }
  struct stat st;
  if (fstat(fd, &st) != 0) {
    err = errno;
    close(fd);
    return false;
  }
  out.resize((size_t)st.st_size);
  size_t got = 0;
  while (got < out.size()) {
    const ssize_t r = read(fd, &out[got], out.size() - got);
    if (r <= 0) {
      err = r < 0 ? errno : EIO;
      close(fd);
      return false;
    }
    got += (size_t)r;
  }
  close(fd);
  return true;
}

// A usize field of TensorInfo (index.rs:7-34).  Absent or null leaves
// `present` false (Option::None); anything but a non-negative integer is the
// error serde reports for a usize (index.rs:282-284 maps it to Json).
static bool get_usize(const Json &j, const char *key, int64_t &v, bool &present,
                      std::string &err) {
  present = false;
  const Json *f = j.get(key);
  if (f == nullptr || f->kind == Json::Null) return true;
  if (f->kind != Json::Num || !f->is_int) {
    err = std::string("invalid type for field `") + key + "`, expected usize";
    return false;
  }
  if (f->inum < 0) {
    err = "invalid value: integer `" + std::to_string(f->inum) + "`, expected usize";
    return false;
  }
  v = f->inum;
  present = true;
  return true;
}

static bool require_usize(const Json &j, const char *key, int64_t &v, std::string &err) {
  bool present = false;
  if (!get_usize(j, key, v, present, err)) return false;
  if (!present) err = std::string("missing field `") + key + "`";
  return present;
}

// Deserializes one TensorInfo; missing required fields and negative sizes
// are a JSON error, as serde would report them (index.rs:282-284).
static bool parse_info(const Json &j, TensorInfo &t, std::string &err) {
  if (j.kind != Json::Obj) { err = "tensor entry is not an object"; return false; }
  const Json *fp = j.get("file_path"), *dt = j.get("dtype"), *pr = j.get("precision"),
             *sh = j.get("shape");
  if (fp == nullptr || fp->kind != Json::Str) { err = "missing field `file_path`"; return false; }
  if (!require_usize(j, "byte_offset", t.byte_offset, err)) return false;
  if (!require_usize(j, "byte_length", t.byte_length, err)) return false;
  if (sh == nullptr || sh->kind != Json::Arr) { err = "missing field `shape`"; return false; }
  for (const Json &d : sh->arr) {
    if (d.kind != Json::Num || !d.is_int) { err = "invalid shape entry, expected usize"; return false; }
    if (d.inum < 0) {
      err = "invalid value: integer `" + std::to_string(d.inum) + "`, expected usize";
      return false;
    }
    t.shape.push_back(d.inum);
  }
  if (dt == nullptr || dt->kind != Json::Str) { err = "missing field `dtype`"; return false; }
  if (pr == nullptr || pr->kind != Json::Str) { err = "missing field `precision`"; return false; }
  t.file_path = fp->str;
  t.dtype = dt->str;
  t.precision = pr->str;
  if (!get_usize(j, "nf4_absmax_offset", t.absmax_offset, t.has_absmax_offset, err) ||
      !get_usize(j, "nf4_absmax_length", t.absmax_length, t.has_absmax_length, err) ||
      !get_usize(j, "nf4_block_size", t.block_size, t.has_block_size, err))
    return false;
  bool dq[5];
  if (!get_usize(j, "nf4_absmax_q_offset", t.q_offset, dq[0], err) ||
      !get_usize(j, "nf4_absmax_q_length", t.q_length, dq[1], err) ||
      !get_usize(j, "nf4_absmax_scale_offset", t.scale_offset, dq[2], err) ||
      !get_usize(j, "nf4_absmax_scale_length", t.scale_length, dq[3], err) ||
      !get_usize(j, "nf4_dq_group", t.dq_group, dq[4], err))
    return false;
  t.dq = dq[0] && dq[1] && dq[2] && dq[3] && dq[4];
  return true;
}

static int32_t io_fail(const std::string &what, int err) {
  return fail(NF4S_ERR_IO, "I/O error: %s: %s", what.c_str(), strerror(err));
}

static int32_t get_mmap(nf4s_loader *L, const std::string &file, const MappedFile **out) {
  auto it = L->mmap_cache.find(file);
  if (it == L->mmap_cache.end()) {
    const std::string path = L->model_dir + "/" + file;
    const int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) return io_fail(path, errno);
    struct stat st;
    if (fstat(fd, &st) != 0) {
      const int e = errno;
      close(fd);
      return io_fail(path, e);
    }
    std::unique_ptr<MappedFile> m(new (std::nothrow) MappedFile());
    if (!m) {
      close(fd);
      return fail(NF4S_ERR_IO, "I/O error: out of host memory");
    }
    m->size = (size_t)st.st_size;
    if (m->size > 0) {
      void *p = mmap(nullptr, m->size, PROT_READ, MAP_PRIVATE, fd, 0);
      if (p == MAP_FAILED) {
        const int e = errno;
        close(fd);
        return io_fail(path, e);
      }
      m->data = static_cast<const uint8_t *>(p);
    }
    close(fd);
    it = L->mmap_cache.emplace(file, std::move(m)).first;
  }
  *out = it->second.get();
  return NF4S_OK;
}

static int32_t malformed(const std::string &name, const char *fmt, ...) {
  char detail[384];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(detail, sizeof(detail), fmt, ap);
  va_end(ap);
  return fail(NF4S_ERR_MALFORMED_INDEX, "malformed index entry '%s': %s", name.c_str(), detail);
}

static int32_t lookup(nf4s_loader *L, const char *name, const TensorInfo **out) {
  if (name == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "parameter name is NULL");
  auto it = L->index.find(name);
  if (it == L->index.end())  // error.rs:17-18
    return fail(NF4S_ERR_PARAM_NOT_FOUND, "parameter '%s' not found in shard index", name);
  *out = &it->second;
  return NF4S_OK;
}

static bool is_nf4(const TensorInfo &t) { return t.precision == "nf4"; }

// off + len > size without the wrap of the sum (parse_info keeps both >= 0).
static bool beyond(int64_t off, int64_t len, uint64_t size) {
  return (uint64_t)off > size || (uint64_t)len > size - (uint64_t)off;
}

// The NF4 checks of loader.rs:93-151 (bounds, required fields, alignment),
// extended to the double-quant fields.
static int32_t check_nf4(const std::string &name, const TensorInfo &t, const MappedFile &m) {
  const uint64_t sz = m.size;
  if (beyond(t.byte_offset, t.byte_length, sz))
    return malformed(name, "packed data out of bounds: offset %lld + length %lld > mmap %llu",
                     (long long)t.byte_offset, (long long)t.byte_length, (unsigned long long)sz);
  if (t.dq) {
    if (t.dq_group <= 0 || (t.dq_group & (t.dq_group - 1)) != 0)
      return malformed(name, "nf4_dq_group must be a power of two");
    if (beyond(t.q_offset, t.q_length, sz))
      return malformed(name, "absmax codes out of bounds: offset %lld + length %lld > mmap %llu",
                       (long long)t.q_offset, (long long)t.q_length, (unsigned long long)sz);
    if (beyond(t.scale_offset, t.scale_length, sz))
      return malformed(name, "absmax scales out of bounds: offset %lld + length %lld > mmap %llu",
                       (long long)t.scale_offset, (long long)t.scale_length,
                       (unsigned long long)sz);
    if (t.scale_offset % 4 != 0)
      return malformed(name, "absmax scale offset %lld is not 4-byte aligned",
                       (long long)t.scale_offset);
    if (!t.has_block_size) return malformed(name, "missing nf4_block_size");
    return NF4S_OK;
  }
  if (!t.has_absmax_offset) return malformed(name, "missing nf4_absmax_offset");
  if (!t.has_absmax_length) return malformed(name, "missing nf4_absmax_length");
  if (!t.has_block_size) return malformed(name, "missing nf4_block_size");
  if (beyond(t.absmax_offset, t.absmax_length, sz))
    return malformed(name, "absmax data out of bounds: offset %lld + length %lld > mmap %llu",
                     (long long)t.absmax_offset, (long long)t.absmax_length,
                     (unsigned long long)sz);
  if (t.absmax_offset % 4 != 0)
    return malformed(name, "absmax offset %lld is not 4-byte aligned", (long long)t.absmax_offset);
  return NF4S_OK;
}

// Bytes of the fp32 parts that are read: the reference views an absmax
// byte range as floor(len / 4) floats (loader.rs:158-161).
static int64_t f32_bytes(int64_t len) { return len / 4 * 4; }

static int64_t round_up(int64_t x) { return (x + 255) / 256 * 256; }

// Staging layout of one NF4 parameter: packed bytes, then the absmax part,
// then the double-quant scales, each at a 256-byte boundary.
struct Staging {
  int64_t am_off, sc_off, bytes, am_bytes, sc_bytes;
};

static Staging staging_of(const TensorInfo &t) {
  Staging g;
  g.am_bytes = t.dq ? t.q_length : f32_bytes(t.absmax_length);
  g.sc_bytes = t.dq ? f32_bytes(t.scale_length) : 0;
  g.am_off = round_up(t.byte_length);
  g.sc_off = g.am_off + round_up(g.am_bytes);
  g.bytes = g.sc_off + round_up(g.sc_bytes);
  return g;
}

}  // namespace nf4s

using namespace nf4s;

extern "C" {

// ShardLoader::new (loader.rs:44-50) -> IndexStore::load (index.rs:279-295).
int32_t nf4s_loader_open(const char *model_dir, nf4s_loader **out) {
  clear_error();
  if (model_dir == nullptr || out == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad loader_open args");
  *out = nullptr;
  std::unique_ptr<nf4s_loader> L(new (std::nothrow) nf4s_loader());
  if (!L) return fail(NF4S_ERR_IO, "I/O error: out of host memory");
  L->model_dir = model_dir;
  std::string text, err;
  int e = 0;
  const std::string ipath = L->model_dir + "/shard_index.json";
  if (!read_file(ipath, text, e)) return io_fail(ipath, e);
  Json idx;
  if (!JsonParser(text.data(), text.size()).parse(idx, err) || idx.kind != Json::Obj)
    return fail(NF4S_ERR_JSON, "JSON parse error: %s: %s", ipath.c_str(),
                err.empty() ? "expected an object" : err.c_str());
  for (const auto &kv : idx.obj) {
    TensorInfo t;
    if (!parse_info(kv.second, t, err))
      return fail(NF4S_ERR_JSON, "JSON parse error: %s: entry '%s': %s", ipath.c_str(),
                  kv.first.c_str(), err.c_str());
    L->index[kv.first] = std::move(t);
  }
  const std::string rpath = L->model_dir + "/layer_registry.json";
  if (!read_file(rpath, text, e)) return io_fail(rpath, e);
  Json reg;
  if (!JsonParser(text.data(), text.size()).parse(reg, err) || reg.kind != Json::Obj)
    return fail(NF4S_ERR_JSON, "JSON parse error: %s: %s", rpath.c_str(),
                err.empty() ? "expected an object" : err.c_str());
  for (const auto &kv : reg.obj) {
    if (kv.second.kind != Json::Str)
      return fail(NF4S_ERR_JSON, "JSON parse error: %s: value of '%s' is not a string",
                  rpath.c_str(), kv.first.c_str());
    L->registry[kv.first] = kv.second.str;
  }
  *out = L.release();
  return NF4S_OK;
}

int32_t nf4s_loader_close(nf4s_loader *L) {
  clear_error();
  delete L;
  return NF4S_OK;
}

int32_t nf4s_loader_param_info(nf4s_loader *L, const char *name, nf4s_param_info *out) {
  clear_error();
  if (L == nullptr || out == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "bad args");
  const TensorInfo *t;
  int32_t rc = lookup(L, name, &t);
  if (rc != NF4S_OK) return rc;
  memset(out, 0, sizeof(*out));
  out->ndim = (int32_t)t->shape.size();
  if (out->ndim > 8) return malformed(name, "more than 8 dimensions");
  int64_t numel = 1;
  for (int i = 0; i < out->ndim; ++i) {
    out->shape[i] = t->shape[i];
    if (__builtin_mul_overflow(numel, t->shape[i], &numel))
      return malformed(name, "shape element count overflows 64 bits");
  }
  out->numel = numel;
  out->byte_length = t->byte_length;
  snprintf(out->precision_str, sizeof(out->precision_str), "%s", t->precision.c_str());
  snprintf(out->dtype_str, sizeof(out->dtype_str), "%s", t->dtype.c_str());
  if (is_nf4(*t)) {
    out->precision = t->dq ? 2 : 1;
    out->block_size = (int32_t)t->block_size;
    out->absmax_len = t->dq ? t->q_length : t->absmax_length / 4;
    out->scale_len = t->dq ? t->scale_length / 4 : 0;
    out->dq_group = t->dq ? (int32_t)t->dq_group : 0;
    if (t->byte_length > INT64_MAX / 2)
      return malformed(name, "byte_length %lld too large", (long long)t->byte_length);
    out->out_elems = 2 * t->byte_length;  // nf4.rs:103
  } else {
    out->precision = 0;
    out->out_elems = t->byte_length / 2;
  }
  return NF4S_OK;
}

// ShardLoader::load_layer (loader.rs:53-75): the whole shard file of a layer.
// Returns a pointer into the loader's read-only mapping, valid until close.
int32_t nf4s_loader_load_layer(nf4s_loader *L, uint32_t layer, const uint8_t **data,
                               int64_t *len) {
  clear_error();
  if (L == nullptr || data == nullptr || len == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad args");
  auto it = L->registry.find(std::to_string(layer));
  if (it == L->registry.end())  // error.rs:13-14, index.rs:298-304
    return fail(NF4S_ERR_LAYER_NOT_FOUND, "layer index %u not found in layer registry", layer);
  const MappedFile *m;
  const int32_t rc = get_mmap(L, it->second, &m);
  if (rc != NF4S_OK) return rc;
  *data = m->data;
  *len = (int64_t)m->size;
  return NF4S_OK;
}

// Device staging bytes nf4s_loader_load_param_f16 needs for `name` (0 for an
// fp16 entry, which is copied straight into the output).  An NF4 entry is
// checked against its shard file first, as the load does, so its lengths are
// bounded by the file size before they are summed.
int32_t nf4s_loader_staging_size(nf4s_loader *L, const char *name, int64_t *bytes) {
  clear_error();
  if (L == nullptr || bytes == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "bad args");
  *bytes = 0;
  const TensorInfo *t;
  int32_t rc = lookup(L, name, &t);
  if (rc != NF4S_OK) return rc;
  if (!is_nf4(*t)) return NF4S_OK;
  const MappedFile *m;
  rc = get_mmap(L, t->file_path, &m);
  if (rc != NF4S_OK) return rc;
  rc = check_nf4(name, *t, *m);
  if (rc != NF4S_OK) return rc;
  *bytes = staging_of(*t).bytes;
  return NF4S_OK;
}

// ShardLoader::load_param (loader.rs:78-206) into a device f16 buffer of
// out_len elements: NF4 entries are copied into the caller's device staging
// buffer and dequantized on the device (dequant_nf4_alloc semantics: 2 *
// packed bytes elements); fp16 entries are copied (loader.rs:179-198).
// Allocates nothing and never synchronizes the device.
int32_t nf4s_loader_load_param_f16(nf4s_loader *L, const char *name, uint16_t *out,
                                   int64_t out_len, void *staging, int64_t staging_bytes,
                                   void *stream) {
  clear_error();
  if (L == nullptr || out == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "bad args");
  const TensorInfo *t;
  int32_t rc = lookup(L, name, &t);
  if (rc != NF4S_OK) return rc;
  const MappedFile *m;
  rc = get_mmap(L, t->file_path, &m);
  if (rc != NF4S_OK) return rc;
  hipStream_t s = as_stream(stream);
  if (!is_nf4(*t)) {
    if (beyond(t->byte_offset, t->byte_length, m->size))
      return malformed(name, "tensor data out of bounds: offset %lld + length %lld > mmap %llu",
                       (long long)t->byte_offset, (long long)t->byte_length,
                       (unsigned long long)m->size);
    if (out_len < 0 || out_len < t->byte_length / 2 + t->byte_length % 2)
      return fail(NF4S_ERR_INVALID_ARGUMENT, "output holds %lld elements, need %lld",
                  (long long)out_len, (long long)(t->byte_length / 2));
    const hipError_t e = hipMemcpyAsync(out, m->data + t->byte_offset, (size_t)t->byte_length,
                                        hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return fail(NF4S_ERR_HIP, "hipMemcpyAsync: %s", hipGetErrorString(e));
    return NF4S_OK;
  }
  rc = check_nf4(name, *t, *m);
  if (rc != NF4S_OK) return rc;
  const int64_t n = 2 * t->byte_length;
  if (out_len < n)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "output holds %lld elements, need %lld",
                (long long)out_len, (long long)n);
  const Staging g = staging_of(*t);
  if (staging == nullptr || staging_bytes < g.bytes)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "staging holds %lld bytes, need %lld",
                (long long)(staging == nullptr ? 0 : staging_bytes), (long long)g.bytes);
  if (!aligned(staging, 16)) return fail(NF4S_ERR_MISALIGNED, "staging must be 16-byte aligned");
  uint8_t *st = static_cast<uint8_t *>(staging);
  hipError_t e = hipMemcpyAsync(st, m->data + t->byte_offset, (size_t)t->byte_length,
                                hipMemcpyHostToDevice, s);
  if (e == hipSuccess && g.am_bytes > 0)
    e = hipMemcpyAsync(st + g.am_off, m->data + (t->dq ? t->q_offset : t->absmax_offset),
                       (size_t)g.am_bytes, hipMemcpyHostToDevice, s);
  if (e == hipSuccess && g.sc_bytes > 0)
    e = hipMemcpyAsync(st + g.sc_off, m->data + t->scale_offset, (size_t)g.sc_bytes,
                       hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return fail(NF4S_ERR_HIP, "hipMemcpyAsync: %s", hipGetErrorString(e));
  nf4s_tensor d{};
  d.packed = st;
  d.packed_len = t->byte_length;
  d.block_size = (int32_t)t->block_size;
  if (t->dq) {
    d.absmax_q = st + g.am_off;
    d.absmax_scale = reinterpret_cast<const float *>(st + g.sc_off);
    d.absmax_len = t->q_length;
    d.scale_len = t->scale_length / 4;
    d.dq_group = (int32_t)t->dq_group;
  } else {
    d.absmax = reinterpret_cast<const float *>(st + g.am_off);
    d.absmax_len = t->absmax_length / 4;  // loader.rs:160
  }
  // dequant_nf4_alloc (nf4.rs:98-107) -> dequant_nf4_into checks (nf4.rs:46-57)
  return nf4s_dequant_f16(&d, n, out, stream);
}

// The raw NF4 payload of a parameter copied into caller device buffers of the
// given byte capacities (the device-resident weight provider keeps NF4 on the
// device instead of f32).  The fp32 parts copy floor(length / 4) floats, as
// many as the reference reads (loader.rs:158-161); `scale` may be NULL for
// an entry without double-quant.
int32_t nf4s_loader_load_param_nf4(nf4s_loader *L, const char *name, uint8_t *packed,
                                   int64_t packed_bytes, void *absmax_or_q, int64_t absmax_bytes,
                                   float *scale, int64_t scale_bytes, void *stream) {
  clear_error();
  if (L == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "bad args");
  const TensorInfo *t;
  int32_t rc = lookup(L, name, &t);
  if (rc != NF4S_OK) return rc;
  if (!is_nf4(*t)) return malformed(name, "precision is %s, not nf4", t->precision.c_str());
  const MappedFile *m;
  rc = get_mmap(L, t->file_path, &m);
  if (rc != NF4S_OK) return rc;
  rc = check_nf4(name, *t, *m);
  if (rc != NF4S_OK) return rc;
  const Staging g = staging_of(*t);
  if (packed == nullptr || absmax_or_q == nullptr || (t->dq && scale == nullptr))
    return fail(NF4S_ERR_INVALID_ARGUMENT, "NULL destination buffer");
  if (packed_bytes < t->byte_length || absmax_bytes < g.am_bytes || scale_bytes < g.sc_bytes)
    return fail(NF4S_ERR_INVALID_ARGUMENT,
                "destination too small: packed %lld < %lld, absmax %lld < %lld or scale %lld < %lld",
                (long long)packed_bytes, (long long)t->byte_length, (long long)absmax_bytes,
                (long long)g.am_bytes, (long long)scale_bytes, (long long)g.sc_bytes);
  hipStream_t s = as_stream(stream);
  hipError_t e = hipMemcpyAsync(packed, m->data + t->byte_offset, (size_t)t->byte_length,
                                hipMemcpyHostToDevice, s);
  const int64_t am_off = t->dq ? t->q_offset : t->absmax_offset;
  if (e == hipSuccess && g.am_bytes > 0)
    e = hipMemcpyAsync(absmax_or_q, m->data + am_off, (size_t)g.am_bytes, hipMemcpyHostToDevice,
                       s);
  if (e == hipSuccess && g.sc_bytes > 0)
    e = hipMemcpyAsync(scale, m->data + t->scale_offset, (size_t)g.sc_bytes,
                       hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return fail(NF4S_ERR_HIP, "hipMemcpyAsync: %s", hipGetErrorString(e));
  return NF4S_OK;
}

}  // extern "C"

namespace nf4s {

// Placement of one NF4 parameter's parts in a layer blob: packed bytes, the
// absmax part (fp32 or uint8 codes), the double-quant scales, each at the
// next 256-byte boundary after the previous part.
static int32_t place_entry(nf4s_loader *L, const char *name, int64_t at, nf4s_blob_entry &e,
                           const TensorInfo **info, const MappedFile **map, int64_t *end) {
  const TensorInfo *t;
  int32_t rc = lookup(L, name, &t);
  if (rc != NF4S_OK) return rc;
  if (!is_nf4(*t)) return malformed(name, "precision is %s, not nf4", t->precision.c_str());
  const MappedFile *m;
  rc = get_mmap(L, t->file_path, &m);
  if (rc != NF4S_OK) return rc;
  rc = check_nf4(name, *t, *m);
  if (rc != NF4S_OK) return rc;
  if (t->block_size <= 0 || t->block_size > 0x7fffffff || t->dq_group > 0x7fffffff)
    return malformed(name, "nf4_block_size %lld or nf4_dq_group %lld out of range",
                     (long long)t->block_size, (long long)t->dq_group);
  const Staging g = staging_of(*t);
  e = nf4s_blob_entry{};
  e.packed_off = at;
  e.packed_len = t->byte_length;
  e.absmax_off = at + g.am_off;
  e.absmax_len = t->dq ? t->q_length : g.am_bytes / 4;
  e.scale_off = t->dq ? at + g.sc_off : 0;
  e.scale_len = g.sc_bytes / 4;
  e.block_size = (int32_t)t->block_size;
  e.dq_group = t->dq ? (int32_t)t->dq_group : 0;
  *info = t;
  *map = m;
  *end = at + g.bytes;
  return NF4S_OK;
}

}  // namespace nf4s

extern "C" {

// The bytes a FlowCast pinned slot holds for one layer (ready.rs:27-30):
// the raw NF4 payloads of `count` parameters packed into one host blob, so
// that one asynchronous H2D copy moves the layer.
int32_t nf4s_loader_pack_layer(nf4s_loader *L, const char *const *names, int32_t count,
                               void *dst, int64_t dst_bytes, nf4s_blob_entry *entries,
                               int64_t *bytes) {
  clear_error();
  if (L == nullptr || names == nullptr || entries == nullptr || bytes == nullptr || count < 0)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad pack_layer args");
  *bytes = 0;
  int64_t at = 0;
  for (int32_t i = 0; i < count; ++i) {
    const TensorInfo *t;
    const MappedFile *m;
    int64_t end = 0;
    const int32_t rc = place_entry(L, names[i], at, entries[i], &t, &m, &end);
    if (rc != NF4S_OK) return rc;
    at = end;
  }
  *bytes = at;
  if (dst == nullptr) return NF4S_OK;
  if (dst_bytes < at)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "blob holds %lld bytes, need %lld",
                (long long)dst_bytes, (long long)at);
  uint8_t *out = static_cast<uint8_t *>(dst);
  memset(out, 0, (size_t)at);  // alignment gaps
  for (int32_t i = 0; i < count; ++i) {
    const TensorInfo *t;
    const MappedFile *m;
    int64_t end = 0;
    nf4s_blob_entry e;
    const int32_t rc = place_entry(L, names[i], entries[i].packed_off, e, &t, &m, &end);
    if (rc != NF4S_OK) return rc;
    memcpy(out + e.packed_off, m->data + t->byte_offset, (size_t)e.packed_len);
    const int64_t am_bytes = t->dq ? e.absmax_len : 4 * e.absmax_len;
    memcpy(out + e.absmax_off, m->data + (t->dq ? t->q_offset : t->absmax_offset),
           (size_t)am_bytes);
    if (e.scale_len > 0)
      memcpy(out + e.scale_off, m->data + t->scale_offset, (size_t)(4 * e.scale_len));
  }
  return NF4S_OK;
}

// Descriptor of blob entry `e` inside a copy of the blob at `base`.
int32_t nf4s_blob_tensor(const nf4s_blob_entry *e, const void *base, nf4s_tensor *out) {
  clear_error();
  if (e == nullptr || base == nullptr || out == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad blob_tensor args");
  const uint8_t *b = static_cast<const uint8_t *>(base);
  *out = nf4s_tensor{};
  out->packed = b + e->packed_off;
  out->packed_len = e->packed_len;
  if (e->dq_group > 0) {
    out->absmax_q = b + e->absmax_off;
    out->absmax_scale = reinterpret_cast<const float *>(b + e->scale_off);
    out->scale_len = e->scale_len;
  } else {
    out->absmax = reinterpret_cast<const float *>(b + e->absmax_off);
  }
  out->absmax_len = e->absmax_len;
  out->block_size = e->block_size;
  out->dq_group = e->dq_group;
  return NF4S_OK;
}

}  // extern "C"
