// lux3d_weights.cpp -- GGUF and safetensors readers (the C ABI of
// include/lux3d_weights.h). Host code only: the file is mapped read-only and
// parsed in place; tensor data is never copied here.
//
// GGUF layout (the public ggml GGUF specification, versions 1-3):
//   u32 magic "GGUF", u32 version,
//   tensor count and metadata count (u32 in v1, u64 from v2),
//   metadata: {string key, u32 type, value},
//   tensor infos: {string name, u32 n_dims, dims (u32 in v1, u64 from v2),
//                  u32 ggml type, u64 offset},
//   padding to `general.alignment` (default 32), then the tensor data;
//   strings are {length (u32 in v1, u64 from v2), bytes}.
// Dims are stored innermost first; candle's reader and writer reverse them,
// so the shape here is reversed to candle order.
//
// safetensors layout: u64 header size N, N bytes of JSON
// {name: {"dtype", "shape", "data_offsets": [begin, end]}, "__metadata__": {}},
// then the data; offsets are relative to the byte after the header.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "lux3d_fused.h"
#include "lux3d_weights.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

// A read-only mapping of a whole file.
struct Mapping {
  const uint8_t *base = nullptr;
  size_t size = 0;
  Mapping() = default;
  Mapping(const Mapping &) = delete;
  Mapping &operator=(const Mapping &) = delete;
  ~Mapping() {
    if (base && size) munmap(const_cast<uint8_t *>(base), size);
  }
  bool open(const char *path) {
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(LUX3D_ERR_VALUE, "cannot open %s", path), false;
    struct stat st;
    if (fstat(fd, &st) != 0) {
      ::close(fd);
      return fail(LUX3D_ERR_VALUE, "cannot stat %s", path), false;
    }
    size = (size_t)st.st_size;
    if (size == 0) {
      ::close(fd);
      return fail(LUX3D_ERR_VALUE, "%s is empty", path), false;
    }
    void *p = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (p == MAP_FAILED) {
      size = 0;
      return fail(LUX3D_ERR_VALUE, "cannot map %s", path), false;
    }
    base = static_cast<const uint8_t *>(p);
    return true;
  }
};

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
  const uint8_t *p;
  size_t n, pos = 0;
  bool bad = false;
  bool need(size_t k) {
    if (bad || k > n - pos) bad = true;
    return !bad;
  }
  template <typename T> T get() {
    T v{};
    if (need(sizeof(T))) {
      std::memcpy(&v, p + pos, sizeof(T));
      pos += sizeof(T);
    }
    return v;
  }
  const uint8_t *take(size_t k) {
    if (!need(k)) return nullptr;
    const uint8_t *r = p + pos;
    pos += k;
    return r;
  }
};

// ---------------------------------------------------------------------------
// GGUF
// ---------------------------------------------------------------------------

size_t gguf_scalar_size(uint32_t t) {
  switch (t) {
    case LUX3D_GGUF_U8: case LUX3D_GGUF_I8: case LUX3D_GGUF_BOOL: return 1;
    case LUX3D_GGUF_U16: case LUX3D_GGUF_I16: return 2;
    case LUX3D_GGUF_U32: case LUX3D_GGUF_I32: case LUX3D_GGUF_F32: return 4;
    case LUX3D_GGUF_U64: case LUX3D_GGUF_I64: case LUX3D_GGUF_F64: return 8;
  }
  return 0;
}

// ggml block size (elements) and bytes per block for the types read here
bool ggml_block(uint32_t t, uint64_t &blk, uint64_t &bytes) {
  switch (t) {
    case LUX3D_GGML_F32: blk = 1; bytes = 4; return true;
    case LUX3D_GGML_F16: case LUX3D_GGML_BF16: blk = 1; bytes = 2; return true;
    case LUX3D_GGML_Q8_0: blk = 32; bytes = 34; return true;
  }
  return false;
}

struct GgufMeta {
  std::string key;
  uint32_t type = 0, elem_type = 0;
  const void *value = nullptr;
  uint64_t count = 0;
};

struct GgufTensor {
  std::string name;
  uint32_t type = 0;
  std::vector<int64_t> shape;  // candle order
  uint64_t offset = 0, nbytes = 0;
  const void *data = nullptr;
};

}  // namespace

struct lux3d_gguf {
  Mapping map;
  uint32_t version = 0;
  std::vector<GgufMeta> meta;
  std::vector<GgufTensor> tensors;
  std::map<std::string, int64_t> by_name, meta_by_key;
};

namespace {

bool read_string(Cursor &c, uint32_t version, std::string *out, const uint8_t **raw = nullptr,
                 uint64_t *len_out = nullptr) {
  const uint64_t len = version == 1 ? c.get<uint32_t>() : c.get<uint64_t>();
  const uint8_t *b = c.take(len);
  if (!b) return false;
  if (out) out->assign(reinterpret_cast<const char *>(b), (size_t)len);
  if (raw) *raw = b;
  if (len_out) *len_out = len;
  return true;
}

// Skips (and for the top level records) one metadata value of type t.
bool read_value(Cursor &c, uint32_t version, uint32_t t, GgufMeta *m, int depth) {
  if (depth > 8) return false;
  if (t == LUX3D_GGUF_STRING) {
    const uint8_t *raw;
    uint64_t len;
    if (!read_string(c, version, nullptr, &raw, &len)) return false;
    if (m) m->value = raw, m->count = len;
    return true;
  }
  if (t == LUX3D_GGUF_ARRAY) {
    const uint32_t et = c.get<uint32_t>();
    const uint64_t count = version == 1 ? c.get<uint32_t>() : c.get<uint64_t>();
    if (c.bad) return false;
    if (m) m->elem_type = et, m->count = count, m->value = nullptr;
    const size_t es = gguf_scalar_size(et);
    if (es) {
      if (count > (c.n - c.pos) / es) return false;
      if (m) m->value = c.p + c.pos;
      c.pos += (size_t)(count * es);
      return true;
    }
    if (et != LUX3D_GGUF_STRING && et != LUX3D_GGUF_ARRAY) return false;
    if (count > c.n - c.pos) return false;  // every element takes at least one byte
    for (uint64_t i = 0; i < count; ++i)
      if (!read_value(c, version, et, nullptr, depth + 1)) return false;
    return true;
  }
  const size_t es = gguf_scalar_size(t);
  if (!es) return false;
  const uint8_t *b = c.take(es);
  if (!b) return false;
  if (m) m->value = b, m->count = 1;
  return true;
}

int gguf_parse(lux3d_gguf *g, const char *path) {
  Cursor c{g->map.base, g->map.size};
  const uint32_t magic = c.get<uint32_t>();
  if (c.bad || magic != 0x46554747u) return fail(LUX3D_ERR_VALUE, "%s: not a GGUF file (bad magic)", path);
  g->version = c.get<uint32_t>();
  if (g->version < 1 || g->version > 3)
    return fail(LUX3D_ERR_VALUE, "%s: unsupported GGUF version %u", path, g->version);
  const uint64_t n_tensors = g->version == 1 ? c.get<uint32_t>() : c.get<uint64_t>();
  const uint64_t n_meta = g->version == 1 ? c.get<uint32_t>() : c.get<uint64_t>();
  if (c.bad) return fail(LUX3D_ERR_VALUE, "%s: truncated GGUF header", path);
  // each record takes more than 8 bytes: no count beyond what the file can hold
  if (n_meta > g->map.size / 8 || n_tensors > g->map.size / 8)
    return fail(LUX3D_ERR_VALUE, "%s: GGUF counts exceed the file size", path);
  g->meta.resize((size_t)n_meta);
  for (uint64_t i = 0; i < n_meta; ++i) {
    GgufMeta &m = g->meta[(size_t)i];
    if (!read_string(c, g->version, &m.key)) return fail(LUX3D_ERR_VALUE, "%s: truncated metadata key", path);
    m.type = c.get<uint32_t>();
    if (c.bad || !read_value(c, g->version, m.type, &m, 0))
      return fail(LUX3D_ERR_VALUE, "%s: bad or truncated value of metadata `%s`", path, m.key.c_str());
    g->meta_by_key[m.key] = (int64_t)i;
  }
  uint64_t alignment = 32;
  auto it = g->meta_by_key.find("general.alignment");
  if (it != g->meta_by_key.end()) {
    const GgufMeta &m = g->meta[(size_t)it->second];
    if (m.type == LUX3D_GGUF_U32) {
      uint32_t a;
      std::memcpy(&a, m.value, 4);
      alignment = a;
    } else if (m.type == LUX3D_GGUF_U64) {
      std::memcpy(&alignment, m.value, 8);
    } else {
      return fail(LUX3D_ERR_VALUE, "%s: general.alignment is not an unsigned integer", path);
    }
    if (alignment == 0 || alignment > (1u << 30))
      return fail(LUX3D_ERR_VALUE, "%s: general.alignment %llu out of range", path, (unsigned long long)alignment);
  }
  g->tensors.resize((size_t)n_tensors);
  for (uint64_t i = 0; i < n_tensors; ++i) {
    GgufTensor &t = g->tensors[(size_t)i];
    if (!read_string(c, g->version, &t.name)) return fail(LUX3D_ERR_VALUE, "%s: truncated tensor info", path);
    const uint32_t nd = c.get<uint32_t>();
    if (c.bad || nd > LUX3D_WEIGHTS_MAX_RANK)
      return fail(LUX3D_ERR_VALUE, "%s: tensor `%s` has %u dims", path, t.name.c_str(), nd);
    std::vector<uint64_t> dims(nd);
    for (uint32_t d = 0; d < nd; ++d) dims[d] = g->version == 1 ? c.get<uint32_t>() : c.get<uint64_t>();
    t.type = c.get<uint32_t>();
    t.offset = c.get<uint64_t>();
    if (c.bad) return fail(LUX3D_ERR_VALUE, "%s: truncated tensor info of `%s`", path, t.name.c_str());
    uint64_t elems = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      if (dims[d] > (1ull << 40) || (dims[d] && elems > (1ull << 50) / dims[d]))
        return fail(LUX3D_ERR_VALUE, "%s: tensor `%s` is too large", path, t.name.c_str());
      elems *= dims[d];
    }
    t.shape.assign(dims.rbegin(), dims.rend());
    uint64_t blk, bytes;
    if (ggml_block(t.type, blk, bytes)) {
      // blocks run along the innermost dim: its length must be whole blocks
      if (elems % blk || (nd > 0 && dims[0] % blk))
        return fail(LUX3D_ERR_VALUE, "%s: tensor `%s` rows of %llu elements are not whole blocks of %llu", path,
                    t.name.c_str(), (unsigned long long)(nd ? dims[0] : 1), (unsigned long long)blk);
      t.nbytes = elems / blk * bytes;
    }
    if (g->by_name.count(t.name)) return fail(LUX3D_ERR_VALUE, "%s: duplicate tensor `%s`", path, t.name.c_str());
    g->by_name[t.name] = (int64_t)i;
  }
  const uint64_t data0 = (c.pos + alignment - 1) / alignment * alignment;
  for (GgufTensor &t : g->tensors) {
    if (data0 > g->map.size || t.offset > g->map.size - data0 || t.nbytes > g->map.size - data0 - t.offset)
      return fail(LUX3D_ERR_VALUE, "%s: data of tensor `%s` lies past the end of the file", path, t.name.c_str());
    t.data = g->map.base + data0 + t.offset;
  }
  return LUX3D_OK;
}

// ---------------------------------------------------------------------------
// safetensors: a JSON reader for the header
// ---------------------------------------------------------------------------

struct Json {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  double num = 0;
  bool is_int = false;
  int64_t i = 0;
  std::string s;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
};

struct JsonParser {
  const char *p, *end;
  int depth = 0;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(const char *w) {
    const size_t n = std::strlen(w);
    if ((size_t)(end - p) < n || std::memcmp(p, w, n)) return false;
    p += n;
    return true;
  }
  static void utf8(std::string &o, uint32_t cp) {
    if (cp < 0x80) {
      o += (char)cp;
    } else if (cp < 0x800) {
      o += (char)(0xC0 | (cp >> 6));
      o += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      o += (char)(0xE0 | (cp >> 12));
      o += (char)(0x80 | ((cp >> 6) & 0x3F));
      o += (char)(0x80 | (cp & 0x3F));
    } else {
      o += (char)(0xF0 | (cp >> 18));
      o += (char)(0x80 | ((cp >> 12) & 0x3F));
      o += (char)(0x80 | ((cp >> 6) & 0x3F));
      o += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t &v) {
    if (end - p < 4) return false;
    v = 0;
    for (int k = 0; k < 4; ++k) {
      const char ch = *p++;
      v <<= 4;
      if (ch >= '0' && ch <= '9') v |= (uint32_t)(ch - '0');
      else if (ch >= 'a' && ch <= 'f') v |= (uint32_t)(ch - 'a' + 10);
      else if (ch >= 'A' && ch <= 'F') v |= (uint32_t)(ch - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool str(std::string &o) {
    if (p >= end || *p != '"') return false;
    ++p;
    while (p < end && *p != '"') {
      if ((unsigned char)*p < 0x20) return false;
      if (*p != '\\') {
        o += *p++;
        continue;
      }
      if (++p >= end) return false;
      const char e = *p++;
      switch (e) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            uint32_t lo;
            if (end - p < 6 || p[0] != '\\' || p[1] != 'u') return false;
            p += 2;
            if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(o, cp);
          break;
        }
        default: return false;
      }
    }
    if (p >= end) return false;
    ++p;
    return true;
  }
  bool number(Json &v) {
    const char *s0 = p;
    if (p < end && *p == '-') ++p;
    bool frac = false;
    while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) {
      if (*p == '.' || *p == 'e' || *p == 'E') frac = true;
      ++p;
    }
    if (p == s0) return false;
    const std::string t(s0, p);
    char *e = nullptr;
    v.kind = Json::NUM;
    v.num = std::strtod(t.c_str(), &e);
    if (!e || *e) return false;
    if (!frac) {
      errno = 0;
      v.i = std::strtoll(t.c_str(), &e, 10);
      v.is_int = errno == 0 && e && !*e;
    }
    return true;
  }
  bool value(Json &v) {
    if (++depth > 64) return false;
    ws();
    if (p >= end) return false;
    bool ok;
    if (*p == '{') {
      ++p;
      v.kind = Json::OBJ;
      ws();
      ok = true;
      if (p < end && *p == '}') {
        ++p;
      } else {
        for (;;) {
          std::string k;
          ws();
          if (!str(k)) { ok = false; break; }
          ws();
          if (p >= end || *p != ':') { ok = false; break; }
          ++p;
          Json child;
          if (!value(child)) { ok = false; break; }
          v.obj.emplace_back(std::move(k), std::move(child));
          ws();
          if (p < end && *p == ',') { ++p; continue; }
          if (p < end && *p == '}') { ++p; break; }
          ok = false;
          break;
        }
      }
    } else if (*p == '[') {
      ++p;
      v.kind = Json::ARR;
      ws();
      ok = true;
      if (p < end && *p == ']') {
        ++p;
      } else {
        for (;;) {
          Json child;
          if (!value(child)) { ok = false; break; }
          v.arr.push_back(std::move(child));
          ws();
          if (p < end && *p == ',') { ++p; continue; }
          if (p < end && *p == ']') { ++p; break; }
          ok = false;
          break;
        }
      }
    } else if (*p == '"') {
      v.kind = Json::STR;
      ok = str(v.s);
    } else if (lit("true")) {
      v.kind = Json::BOOL, v.b = true, ok = true;
    } else if (lit("false")) {
      v.kind = Json::BOOL, v.b = false, ok = true;
    } else if (lit("null")) {
      v.kind = Json::NUL, ok = true;
    } else {
      ok = number(v);
    }
    --depth;
    return ok;
  }
};

const Json *member(const Json &o, const char *k) {
  for (const auto &kv : o.obj)
    if (kv.first == k) return &kv.second;
  return nullptr;
}

// safetensors dtype name -> (lux3d dtype or -1, element bytes or 0)
void st_dtype(const std::string &s, int &dt, uint64_t &bytes) {
  static const struct { const char *name; int dt; uint64_t bytes; } k[] = {
      {"F32", LUX3D_F32, 4}, {"BF16", LUX3D_BF16, 2}, {"F16", LUX3D_F16, 2}, {"I32", LUX3D_I32, 4},
      {"I64", LUX3D_I64, 8}, {"U8", LUX3D_U8, 1},     {"I8", LUX3D_I8, 1},   {"F64", -1, 8},
      {"BOOL", -1, 1},       {"U16", -1, 2},          {"I16", -1, 2},        {"U32", -1, 4},
      {"U64", -1, 8},        {"F8_E4M3", -1, 1},      {"F8_E5M2", -1, 1}};
  for (const auto &e : k)
    if (s == e.name) {
      dt = e.dt;
      bytes = e.bytes;
      return;
    }
  dt = -1;
  bytes = 0;
}

}  // namespace

struct lux3d_safetensors {
  Mapping map;
  std::vector<GgufTensor> tensors;  // type = lux3d dtype (or -1 as uint32)
  std::map<std::string, int64_t> by_name;
  std::map<std::string, std::string> meta;
};

namespace {

int st_parse(lux3d_safetensors *s, const char *path) {
  Cursor c{s->map.base, s->map.size};
  const uint64_t hlen = c.get<uint64_t>();
  if (c.bad || hlen > s->map.size - 8)
    return fail(LUX3D_ERR_VALUE, "%s: safetensors header size %llu exceeds the file", path, (unsigned long long)hlen);
  const char *h = reinterpret_cast<const char *>(s->map.base + 8);
  JsonParser jp{h, h + hlen};
  Json root;
  if (!jp.value(root) || root.kind != Json::OBJ)
    return fail(LUX3D_ERR_VALUE, "%s: the safetensors header is not a JSON object", path);
  jp.ws();
  if (jp.p != jp.end) return fail(LUX3D_ERR_VALUE, "%s: trailing bytes after the safetensors header", path);
  const uint64_t data0 = 8 + hlen, dsize = s->map.size - data0;
  for (const auto &kv : root.obj) {
    if (kv.first == "__metadata__") {
      if (kv.second.kind != Json::OBJ) return fail(LUX3D_ERR_VALUE, "%s: __metadata__ is not an object", path);
      for (const auto &m : kv.second.obj) {
        if (m.second.kind != Json::STR)
          return fail(LUX3D_ERR_VALUE, "%s: __metadata__ value of `%s` is not a string", path, m.first.c_str());
        s->meta[m.first] = m.second.s;
      }
      continue;
    }
    const Json &t = kv.second;
    const Json *dt = t.kind == Json::OBJ ? member(t, "dtype") : nullptr;
    const Json *sh = t.kind == Json::OBJ ? member(t, "shape") : nullptr;
    const Json *off = t.kind == Json::OBJ ? member(t, "data_offsets") : nullptr;
    if (!dt || dt->kind != Json::STR || !sh || sh->kind != Json::ARR || !off || off->kind != Json::ARR ||
        off->arr.size() != 2 || !off->arr[0].is_int || !off->arr[1].is_int)
      return fail(LUX3D_ERR_VALUE, "%s: malformed entry for tensor `%s`", path, kv.first.c_str());
    if (sh->arr.size() > LUX3D_WEIGHTS_MAX_RANK)
      return fail(LUX3D_ERR_VALUE, "%s: tensor `%s` has rank %zu", path, kv.first.c_str(), sh->arr.size());
    GgufTensor e;
    e.name = kv.first;
    uint64_t elems = 1;
    for (const Json &d : sh->arr) {
      if (!d.is_int || d.i < 0 || d.i > (1ll << 40) || (d.i && elems > (1ull << 50) / (uint64_t)d.i))
        return fail(LUX3D_ERR_VALUE, "%s: bad shape of tensor `%s`", path, kv.first.c_str());
      e.shape.push_back(d.i);
      elems *= (uint64_t)d.i;
    }
    int ldt;
    uint64_t eb;
    st_dtype(dt->s, ldt, eb);
    e.type = (uint32_t)ldt;
    const int64_t b0 = off->arr[0].i, b1 = off->arr[1].i;
    if (b0 < 0 || b1 < b0 || (uint64_t)b1 > dsize)
      return fail(LUX3D_ERR_VALUE, "%s: data of tensor `%s` lies outside the file", path, kv.first.c_str());
    if (eb && (uint64_t)(b1 - b0) != elems * eb)
      return fail(LUX3D_ERR_VALUE, "%s: tensor `%s` holds %lld bytes for %llu elements of %s", path, kv.first.c_str(),
                  (long long)(b1 - b0), (unsigned long long)elems, dt->s.c_str());
    e.offset = (uint64_t)b0;
    e.nbytes = (uint64_t)(b1 - b0);
    e.data = s->map.base + data0 + b0;
    s->by_name[e.name] = (int64_t)s->tensors.size();
    s->tensors.push_back(std::move(e));
  }
  return LUX3D_OK;
}

void fill(const GgufTensor &t, int32_t dtype, lux3d_weights_tensor_t *out) {
  std::memset(out, 0, sizeof(*out));
  out->name = t.name.c_str();
  out->dtype = dtype;
  out->rank = (int32_t)t.shape.size();
  for (size_t d = 0; d < t.shape.size(); ++d) out->shape[d] = t.shape[d];
  out->data = t.data;
  out->nbytes = t.nbytes;
}

}  // namespace

extern "C" {

const char *lux3d_weights_last_error(void) { return g_error.c_str(); }

lux3d_gguf_t *lux3d_gguf_open(const char *path) {
  if (!path) return fail(LUX3D_ERR_NULL, "lux3d_gguf_open: NULL path"), nullptr;
  auto *g = new lux3d_gguf;
  if (!g->map.open(path) || gguf_parse(g, path) != LUX3D_OK) {
    delete g;
    return nullptr;
  }
  g_error.clear();
  return g;
}

void lux3d_gguf_close(lux3d_gguf_t *g) { delete g; }

uint32_t lux3d_gguf_version(const lux3d_gguf_t *g) { return g ? g->version : 0; }

int64_t lux3d_gguf_tensor_count(const lux3d_gguf_t *g) { return g ? (int64_t)g->tensors.size() : 0; }

int64_t lux3d_gguf_find(const lux3d_gguf_t *g, const char *name) {
  if (!g || !name) return -1;
  auto it = g->by_name.find(name);
  return it == g->by_name.end() ? -1 : it->second;
}

int lux3d_gguf_tensor(const lux3d_gguf_t *g, int64_t index, lux3d_weights_tensor_t *out) {
  if (!g || !out) return fail(LUX3D_ERR_NULL, "lux3d_gguf_tensor: NULL argument");
  if (index < 0 || index >= (int64_t)g->tensors.size())
    return fail(LUX3D_ERR_SHAPE, "lux3d_gguf_tensor: index %lld out of range", (long long)index);
  const GgufTensor &t = g->tensors[(size_t)index];
  fill(t, (int32_t)t.type, out);
  return LUX3D_OK;
}

int64_t lux3d_gguf_metadata_count(const lux3d_gguf_t *g) { return g ? (int64_t)g->meta.size() : 0; }

int lux3d_gguf_metadata(const lux3d_gguf_t *g, int64_t index, const char **key, int32_t *type, int32_t *elem_type,
                        const void **value, uint64_t *count) {
  if (!g) return fail(LUX3D_ERR_NULL, "lux3d_gguf_metadata: NULL handle");
  if (index < 0 || index >= (int64_t)g->meta.size())
    return fail(LUX3D_ERR_SHAPE, "lux3d_gguf_metadata: index %lld out of range", (long long)index);
  const GgufMeta &m = g->meta[(size_t)index];
  if (key) *key = m.key.c_str();
  if (type) *type = (int32_t)m.type;
  if (elem_type) *elem_type = (int32_t)m.elem_type;
  if (value) *value = m.value;
  if (count) *count = m.count;
  return LUX3D_OK;
}

int64_t lux3d_gguf_metadata_find(const lux3d_gguf_t *g, const char *key) {
  if (!g || !key) return -1;
  auto it = g->meta_by_key.find(key);
  return it == g->meta_by_key.end() ? -1 : it->second;
}

lux3d_safetensors_t *lux3d_safetensors_open(const char *path) {
  if (!path) return fail(LUX3D_ERR_NULL, "lux3d_safetensors_open: NULL path"), nullptr;
  auto *s = new lux3d_safetensors;
  if (!s->map.open(path) || st_parse(s, path) != LUX3D_OK) {
    delete s;
    return nullptr;
  }
  g_error.clear();
  return s;
}

void lux3d_safetensors_close(lux3d_safetensors_t *s) { delete s; }

int64_t lux3d_safetensors_tensor_count(const lux3d_safetensors_t *s) {
  return s ? (int64_t)s->tensors.size() : 0;
}

int64_t lux3d_safetensors_find(const lux3d_safetensors_t *s, const char *name) {
  if (!s || !name) return -1;
  auto it = s->by_name.find(name);
  return it == s->by_name.end() ? -1 : it->second;
}

int lux3d_safetensors_tensor(const lux3d_safetensors_t *s, int64_t index, lux3d_weights_tensor_t *out) {
  if (!s || !out) return fail(LUX3D_ERR_NULL, "lux3d_safetensors_tensor: NULL argument");
  if (index < 0 || index >= (int64_t)s->tensors.size())
    return fail(LUX3D_ERR_SHAPE, "lux3d_safetensors_tensor: index %lld out of range", (long long)index);
  const GgufTensor &t = s->tensors[(size_t)index];
  fill(t, (int32_t)t.type, out);
  return LUX3D_OK;
}

const char *lux3d_safetensors_metadata(const lux3d_safetensors_t *s, const char *key) {
  if (!s || !key) return nullptr;
  auto it = s->meta.find(key);
  return it == s->meta.end() ? nullptr : it->second.c_str();
}

}  // extern "C"
