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
  void *staging = nullptr;  // device bytes for packed + absmax payloads
  int64_t staging_bytes = 0;
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

static bool get_int(const Json *j, int64_t &v) {
  if (j == nullptr || j->kind != Json::Num || !j->is_int) return false;
  v = j->inum;
  return true;
}

// Deserializes one TensorInfo; missing required fields are a JSON error, as
// serde would report them (index.rs:282-284).
static bool parse_info(const Json &j, TensorInfo &t, std::string &err) {
  if (j.kind != Json::Obj) { err = "tensor entry is not an object"; return false; }
  const Json *fp = j.get("file_path"), *dt = j.get("dtype"), *pr = j.get("precision"),
             *sh = j.get("shape");
  if (fp == nullptr || fp->kind != Json::Str) { err = "missing field `file_path`"; return false; }
  if (!get_int(j.get("byte_offset"), t.byte_offset) || t.byte_offset < 0) {
    err = "missing field `byte_offset`";
    return false;
  }
  if (!get_int(j.get("byte_length"), t.byte_length) || t.byte_length < 0) {
    err = "missing field `byte_length`";
    return false;
  }
  if (sh == nullptr || sh->kind != Json::Arr) { err = "missing field `shape`"; return false; }
  for (const Json &d : sh->arr) {
    int64_t v;
    if (!get_int(&d, v) || v < 0) { err = "invalid shape entry"; return false; }
    t.shape.push_back(v);
  }
  if (dt == nullptr || dt->kind != Json::Str) { err = "missing field `dtype`"; return false; }
  if (pr == nullptr || pr->kind != Json::Str) { err = "missing field `precision`"; return false; }
  t.file_path = fp->str;
  t.dtype = dt->str;
  t.precision = pr->str;
  t.has_absmax_offset = get_int(j.get("nf4_absmax_offset"), t.absmax_offset);
  t.has_absmax_length = get_int(j.get("nf4_absmax_length"), t.absmax_length);
  t.has_block_size = get_int(j.get("nf4_block_size"), t.block_size);
  t.dq = get_int(j.get("nf4_absmax_q_offset"), t.q_offset) &&
         get_int(j.get("nf4_absmax_q_length"), t.q_length) &&
         get_int(j.get("nf4_absmax_scale_offset"), t.scale_offset) &&
         get_int(j.get("nf4_absmax_scale_length"), t.scale_length) &&
         get_int(j.get("nf4_dq_group"), t.dq_group);
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

// The NF4 checks of loader.rs:93-151 (bounds, required fields, alignment),
// extended to the double-quant fields.
static int32_t check_nf4(const std::string &name, const TensorInfo &t, const MappedFile &m) {
  const uint64_t sz = m.size;
  if ((uint64_t)t.byte_offset + (uint64_t)t.byte_length > sz)
    return malformed(name, "packed data out of bounds: offset %lld + length %lld > mmap %llu",
                     (long long)t.byte_offset, (long long)t.byte_length, (unsigned long long)sz);
  if (t.dq) {
    if (t.dq_group <= 0 || (t.dq_group & (t.dq_group - 1)) != 0)
      return malformed(name, "nf4_dq_group must be a power of two");
    if ((uint64_t)t.q_offset + (uint64_t)t.q_length > sz)
      return malformed(name, "absmax codes out of bounds: offset %lld + length %lld > mmap %llu",
                       (long long)t.q_offset, (long long)t.q_length, (unsigned long long)sz);
    if ((uint64_t)t.scale_offset + (uint64_t)t.scale_length > sz)
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
  if ((uint64_t)t.absmax_offset + (uint64_t)t.absmax_length > sz)
    return malformed(name, "absmax data out of bounds: offset %lld + length %lld > mmap %llu",
                     (long long)t.absmax_offset, (long long)t.absmax_length,
                     (unsigned long long)sz);
  if (t.absmax_offset % 4 != 0)
    return malformed(name, "absmax offset %lld is not 4-byte aligned", (long long)t.absmax_offset);
  return NF4S_OK;
}

static int32_t ensure_staging(nf4s_loader *L, int64_t bytes) {
  if (bytes <= L->staging_bytes) return NF4S_OK;
  if (L->staging != nullptr) {
    // A previous call's kernels may still read the old buffer.
    (void)hipDeviceSynchronize();
    (void)hipFree(L->staging);
    L->staging = nullptr;
    L->staging_bytes = 0;
  }
  const hipError_t e = hipMalloc(&L->staging, (size_t)bytes);
  if (e != hipSuccess) return fail(NF4S_ERR_HIP, "staging hipMalloc: %s", hipGetErrorString(e));
  L->staging_bytes = bytes;
  return NF4S_OK;
}

static int64_t round_up(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace nf4s

using namespace nf4s;

extern "C" {

// ShardLoader::new (loader.rs:44-50) -> IndexStore::load (index.rs:279-295).
int32_t nf4s_loader_open(const char *model_dir, nf4s_loader **out) {
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
  if (L == nullptr) return NF4S_OK;
  if (L->staging != nullptr) {
    (void)hipDeviceSynchronize();
    (void)hipFree(L->staging);
  }
  delete L;
  return NF4S_OK;
}

int32_t nf4s_loader_param_info(nf4s_loader *L, const char *name, nf4s_param_info *out) {
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
    numel *= t->shape[i];
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

// ShardLoader::load_param (loader.rs:78-206) into a device f16 buffer of
// out_len elements: NF4 entries are dequantized on the device
// (dequant_nf4_alloc semantics: 2 * packed bytes elements); fp16 entries are
// copied (loader.rs:179-198).  Uses the loader's device staging buffer: one
// stream at a time per loader (the reference's loader needs &mut self).
int32_t nf4s_loader_load_param_f16(nf4s_loader *L, const char *name, uint16_t *out,
                                   int64_t out_len, void *stream) {
  if (L == nullptr || out == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "bad args");
  const TensorInfo *t;
  int32_t rc = lookup(L, name, &t);
  if (rc != NF4S_OK) return rc;
  const MappedFile *m;
  rc = get_mmap(L, t->file_path, &m);
  if (rc != NF4S_OK) return rc;
  hipStream_t s = as_stream(stream);
  if (!is_nf4(*t)) {
    if ((uint64_t)t->byte_offset + (uint64_t)t->byte_length > m->size)
      return malformed(name, "tensor data out of bounds: offset %lld + length %lld > mmap %llu",
                       (long long)t->byte_offset, (long long)t->byte_length,
                       (unsigned long long)m->size);
    if (out_len * 2 < t->byte_length)
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
  const int64_t am_bytes = t->dq ? t->q_length : t->absmax_length;
  const int64_t sc_bytes = t->dq ? t->scale_length : 0;
  const int64_t o_am = round_up(t->byte_length);
  const int64_t o_sc = o_am + round_up(am_bytes);
  rc = ensure_staging(L, o_sc + round_up(sc_bytes));
  if (rc != NF4S_OK) return rc;
  uint8_t *st = static_cast<uint8_t *>(L->staging);
  hipError_t e = hipMemcpyAsync(st, m->data + t->byte_offset, (size_t)t->byte_length,
                                hipMemcpyHostToDevice, s);
  if (e == hipSuccess && am_bytes > 0)
    e = hipMemcpyAsync(st + o_am, m->data + (t->dq ? t->q_offset : t->absmax_offset),
                       (size_t)am_bytes, hipMemcpyHostToDevice, s);
  if (e == hipSuccess && sc_bytes > 0)
    e = hipMemcpyAsync(st + o_sc, m->data + t->scale_offset, (size_t)sc_bytes,
                       hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return fail(NF4S_ERR_HIP, "hipMemcpyAsync: %s", hipGetErrorString(e));
  nf4s_tensor d{};
  d.packed = st;
  d.packed_len = t->byte_length;
  d.block_size = (int32_t)t->block_size;
  if (t->dq) {
    d.absmax_q = st + o_am;
    d.absmax_scale = reinterpret_cast<const float *>(st + o_sc);
    d.absmax_len = t->q_length;
    d.scale_len = t->scale_length / 4;
    d.dq_group = (int32_t)t->dq_group;
  } else {
    d.absmax = reinterpret_cast<const float *>(st + o_am);
    d.absmax_len = t->absmax_length / 4;  // loader.rs:160
  }
  // dequant_nf4_alloc (nf4.rs:98-107) -> dequant_nf4_into checks (nf4.rs:46-57)
  return nf4s_dequant_f16(&d, n, out, stream);
}

// The raw NF4 payload of a parameter copied into caller device buffers (the
// device-resident weight provider keeps NF4 on the device instead of f32).
// Buffers may be NULL when the entry has no such part.
int32_t nf4s_loader_load_param_nf4(nf4s_loader *L, const char *name, uint8_t *packed,
                                   void *absmax_or_q, float *scale, void *stream) {
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
  if (packed == nullptr || absmax_or_q == nullptr || (t->dq && scale == nullptr))
    return fail(NF4S_ERR_INVALID_ARGUMENT, "NULL destination buffer");
  hipStream_t s = as_stream(stream);
  hipError_t e = hipMemcpyAsync(packed, m->data + t->byte_offset, (size_t)t->byte_length,
                                hipMemcpyHostToDevice, s);
  const int64_t am_off = t->dq ? t->q_offset : t->absmax_offset;
  const int64_t am_len = t->dq ? t->q_length : t->absmax_length;
  if (e == hipSuccess && am_len > 0)
    e = hipMemcpyAsync(absmax_or_q, m->data + am_off, (size_t)am_len, hipMemcpyHostToDevice, s);
  if (e == hipSuccess && t->dq && t->scale_length > 0)
    e = hipMemcpyAsync(scale, m->data + t->scale_offset, (size_t)t->scale_length,
                       hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return fail(NF4S_ERR_HIP, "hipMemcpyAsync: %s", hipGetErrorString(e));
  return NF4S_OK;
}

}  // extern "C"
