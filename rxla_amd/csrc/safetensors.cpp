// safetensors checkpoints: memory-mapped reader and device upload with the
// dtype rules of rxla-safetensors (crates/rxla-safetensors/src/model.rs:340-440):
// U8 storage takes U8 tensors verbatim; F32 / F16 / BF16 storage takes any of
// F32 / F16 / BF16 (widening exactly, narrowing with round-to-nearest-even).
//
// File format: u64 little-endian header length n, n bytes of UTF-8 JSON
// {"name": {"dtype": "U8", "shape": [..], "data_offsets": [begin, end]}, ...,
//  "__metadata__": {"key": "value", ...}}, then the data section; offsets are
// relative to the data section. Every tensor is checked at open: known shape,
// offsets inside the data section, end - begin = numel * element size, and no
// two tensors overlap. Nothing is read from the payload until an upload.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "internal.h"

namespace rxw8 {
namespace {

struct TensorEntry {
  std::string name;
  std::string st_dtype;  // safetensors dtype string
  int dtype = 0;         // rxw8 dtype, 0 when not representable
  std::vector<int64_t> shape;
  int64_t numel = 0;            // validated: numel * element size <= INT64_MAX
  uint64_t begin = 0, end = 0;  // relative to the data section
};

// Minimal JSON reader for the header: objects, arrays, strings (with the
// standard escapes, \u as UTF-8), non-negative integers, true/false/null.
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  uint64_t num = 0;
  bool neg_or_frac = false;  // a number this reader does not represent exactly
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
};

struct Parser {
  const char *p, *e;
  std::string err;
  int depth = 0;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool fail_at(const char *what) {
    if (err.empty()) err = what;
    return false;
  }
  bool lit(const char *s) {
    const size_t n = std::strlen(s);
    if ((size_t)(e - p) < n || std::memcmp(p, s, n) != 0) return fail_at("bad literal");
    p += n;
    return true;
  }
  static void put_utf8(std::string &s, uint32_t c) {
    if (c < 0x80) {
      s += (char)c;
    } else if (c < 0x800) {
      s += (char)(0xC0 | (c >> 6));
      s += (char)(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      s += (char)(0xE0 | (c >> 12));
      s += (char)(0x80 | ((c >> 6) & 0x3F));
      s += (char)(0x80 | (c & 0x3F));
    } else {
      s += (char)(0xF0 | (c >> 18));
      s += (char)(0x80 | ((c >> 12) & 0x3F));
      s += (char)(0x80 | ((c >> 6) & 0x3F));
      s += (char)(0x80 | (c & 0x3F));
    }
  }
  bool hex4(uint32_t *v) {
    if (e - p < 4) return fail_at("short \\u escape");
    uint32_t r = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p++;
      r <<= 4;
      if (c >= '0' && c <= '9') r |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') r |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') r |= (uint32_t)(c - 'A' + 10);
      else return fail_at("bad \\u escape");
    }
    *v = r;
    return true;
  }
  bool string(std::string *out) {
    if (p >= e || *p != '"') return fail_at("expected string");
    ++p;
    while (p < e && *p != '"') {
      const char c = *p++;
      if ((unsigned char)c < 0x20) return fail_at("control character in string");
      if (c != '\\') {
        *out += c;
        continue;
      }
      if (p >= e) return fail_at("unterminated escape");
      const char x = *p++;
      switch (x) {
        case '"': *out += '"'; break;
        case '\\': *out += '\\'; break;
        case '/': *out += '/'; break;
        case 'b': *out += '\b'; break;
        case 'f': *out += '\f'; break;
        case 'n': *out += '\n'; break;
        case 'r': *out += '\r'; break;
        case 't': *out += '\t'; break;
        case 'u': {
          uint32_t c0;
          if (!hex4(&c0)) return false;
          if (c0 >= 0xD800 && c0 < 0xDC00) {  // surrogate pair
            uint32_t c1;
            if (e - p < 2 || p[0] != '\\' || p[1] != 'u') return fail_at("lone surrogate");
            p += 2;
            if (!hex4(&c1) || c1 < 0xDC00 || c1 >= 0xE000) return fail_at("bad surrogate pair");
            c0 = 0x10000 + ((c0 - 0xD800) << 10) + (c1 - 0xDC00);
          }
          put_utf8(*out, c0);
          break;
        }
        default: return fail_at("bad escape");
      }
    }
    if (p >= e) return fail_at("unterminated string");
    ++p;
    return true;
  }
  bool value(Json *v) {
    if (++depth > 64) return fail_at("nesting too deep");
    ws();
    if (p >= e) return fail_at("unexpected end");
    bool ok = true;
    if (*p == '{') {
      v->kind = Json::Obj;
      ++p;
      ws();
      if (p < e && *p == '}') {
        ++p;
      } else {
        for (;;) {
          ws();
          std::string k;
          if (!string(&k)) return false;
          ws();
          if (p >= e || *p != ':') return fail_at("expected ':'");
          ++p;
          Json child;
          if (!value(&child)) return false;
          v->obj.emplace_back(std::move(k), std::move(child));
          ws();
          if (p < e && *p == ',') {
            ++p;
            continue;
          }
          if (p < e && *p == '}') {
            ++p;
            break;
          }
          return fail_at("expected ',' or '}'");
        }
      }
    } else if (*p == '[') {
      v->kind = Json::Arr;
      ++p;
      ws();
      if (p < e && *p == ']') {
        ++p;
      } else {
        for (;;) {
          Json child;
          if (!value(&child)) return false;
          v->arr.push_back(std::move(child));
          ws();
          if (p < e && *p == ',') {
            ++p;
            continue;
          }
          if (p < e && *p == ']') {
            ++p;
            break;
          }
          return fail_at("expected ',' or ']'");
        }
      }
    } else if (*p == '"') {
      v->kind = Json::Str;
      ok = string(&v->str);
    } else if (*p == 't') {
      v->kind = Json::Bool;
      ok = lit("true");
    } else if (*p == 'f') {
      v->kind = Json::Bool;
      ok = lit("false");
    } else if (*p == 'n') {
      ok = lit("null");
    } else if (*p == '-' || (*p >= '0' && *p <= '9')) {
      v->kind = Json::Num;
      if (*p == '-') {
        v->neg_or_frac = true;
        ++p;
      }
      if (p >= e || *p < '0' || *p > '9') return fail_at("bad number");
      uint64_t r = 0;
      while (p < e && *p >= '0' && *p <= '9') {
        const uint64_t d = (uint64_t)(*p++ - '0');
        if (r > (UINT64_MAX - d) / 10) v->neg_or_frac = true;  // overflow: not exact
        r = r * 10 + d;
      }
      if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) {
        v->neg_or_frac = true;
        while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' ||
                         *p == '+' || *p == '-'))
          ++p;
      }
      v->num = r;
    } else {
      return fail_at("unexpected character");
    }
    --depth;
    return ok;
  }
};

int dtype_of(const std::string &s, size_t *elem) {
  struct D {
    const char *n;
    int dt;
    size_t sz;
  };
  static const D table[] = {{"U8", RXW8_U8, 1},    {"I8", 0, 1},      {"BOOL", 0, 1},
                            {"I16", 0, 2},          {"U16", 0, 2},     {"F16", RXW8_F16, 2},
                            {"BF16", RXW8_BF16, 2}, {"I32", RXW8_I32, 4}, {"U32", 0, 4},
                            {"F32", RXW8_F32, 4},   {"I64", 0, 8},     {"U64", 0, 8},
                            {"F64", 0, 8},          {"F8_E4M3", 0, 1}, {"F8_E5M2", 0, 1}};
  for (const D &d : table)
    if (s == d.n) {
      *elem = d.sz;
      return d.dt;
    }
  *elem = 0;
  return -1;
}

// f16 / bf16 <-> f32, bit-exact: widening is exact; narrowing rounds to
// nearest, ties to even, with subnormals, infinities and NaN preserved.
float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {  // subnormal: normalise
      int e = -1;
      do {
        ++e;
        man <<= 1;
      } while (!(man & 0x400u));
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u)  // inf or NaN (keep NaN quiet and non-zero)
    return sign | (ax > 0x7F800000u ? (uint16_t)(0x7E00u | ((ax >> 13) & 0x3FFu)) : 0x7C00u);
  if (ax >= 0x477FF000u) return sign | 0x7C00u;  // rounds past 65504: infinity
  if (ax < 0x33000001u) return sign;             // below half the smallest subnormal
  const int e = (int)(ax >> 23) - 127;
  if (e < -14) {  // subnormal result: shift the full significand, round to even
    const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    const int shift = -e - 14 + 13;  // 14..24
    uint32_t r = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return sign | (uint16_t)r;
  }
  uint32_t r = ((uint32_t)(e + 15) << 10) | ((ax >> 13) & 0x3FFu);
  const uint32_t rem = ax & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;  // may carry into the exponent
  return sign | (uint16_t)r;
}

float bf16_to_f32(uint16_t b) {
  const uint32_t bits = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

uint16_t f32_to_bf16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);  // quiet NaN
  x += 0x7FFFu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

}  // namespace

struct SafeTensors {
  void *map = nullptr;
  size_t map_bytes = 0;
  const uint8_t *data = nullptr;  // start of the data section
  uint64_t data_bytes = 0;
  std::vector<TensorEntry> tensors;
  std::map<std::string, size_t> index;
  std::vector<std::pair<std::string, std::string>> metadata;
};

static int open_file(const char *path, SafeTensors *st) {
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return fail(RXW8_NOT_FOUND, "cannot open \"%s\"", path);
  struct stat sb;
  if (fstat(fd, &sb) != 0 || !S_ISREG(sb.st_mode)) {
    ::close(fd);
    return fail(RXW8_INVALID_ARGUMENT, "\"%s\" is not a regular file", path);
  }
  const size_t bytes = (size_t)sb.st_size;
  if (bytes < 8) {
    ::close(fd);
    return fail(RXW8_DATA_LOSS, "\"%s\": %zu bytes, too short for a safetensors header", path, bytes);
  }
  void *m = mmap(nullptr, bytes, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return fail(RXW8_RESOURCE_EXHAUSTED, "mmap of \"%s\" failed", path);
  st->map = m;
  st->map_bytes = bytes;
  return RXW8_OK;
}

static int parse_header(const char *path, SafeTensors *st) {
  const uint8_t *base = (const uint8_t *)st->map;
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | base[i];
  if (n > st->map_bytes - 8)
    return fail(RXW8_DATA_LOSS, "\"%s\": header length %llu exceeds the file", path,
                (unsigned long long)n);
  Parser ps{(const char *)base + 8, (const char *)base + 8 + n, {}, 0};
  Json root;
  if (!ps.value(&root)) return fail(RXW8_DATA_LOSS, "\"%s\": header JSON: %s", path, ps.err.c_str());
  ps.ws();
  if (ps.p != ps.e) return fail(RXW8_DATA_LOSS, "\"%s\": trailing bytes after the header JSON", path);
  if (root.kind != Json::Obj) return fail(RXW8_DATA_LOSS, "\"%s\": header is not an object", path);
  st->data = base + 8 + n;
  st->data_bytes = st->map_bytes - 8 - n;
  for (auto &kv : root.obj) {
    const Json &v = kv.second;
    if (kv.first == "__metadata__") {
      if (v.kind != Json::Obj) return fail(RXW8_DATA_LOSS, "\"%s\": __metadata__ is not an object", path);
      for (auto &m : v.obj) {
        if (m.second.kind != Json::Str)
          return fail(RXW8_DATA_LOSS, "\"%s\": metadata \"%s\" is not a string", path, m.first.c_str());
        st->metadata.emplace_back(m.first, m.second.str);
      }
      continue;
    }
    if (v.kind != Json::Obj) return fail(RXW8_DATA_LOSS, "\"%s\": tensor \"%s\" is not an object", path, kv.first.c_str());
    const Json *dt = nullptr, *shape = nullptr, *offs = nullptr;
    for (auto &f : v.obj) {
      if (f.first == "dtype") dt = &f.second;
      else if (f.first == "shape") shape = &f.second;
      else if (f.first == "data_offsets") offs = &f.second;
    }
    if (!dt || dt->kind != Json::Str || !shape || shape->kind != Json::Arr || !offs ||
        offs->kind != Json::Arr || offs->arr.size() != 2)
      return fail(RXW8_DATA_LOSS, "\"%s\": tensor \"%s\" needs dtype, shape and data_offsets", path,
                  kv.first.c_str());
    TensorEntry t;
    t.name = kv.first;
    t.st_dtype = dt->str;
    size_t elem = 0;
    const int code = dtype_of(dt->str, &elem);
    if (code < 0)
      return fail(RXW8_DATA_LOSS, "\"%s\": tensor \"%s\" has unknown dtype \"%s\"", path, kv.first.c_str(),
                  dt->str.c_str());
    t.dtype = code;
    if (shape->arr.size() > RXW8_MAX_RANK)
      return fail(RXW8_UNIMPLEMENTED, "\"%s\": tensor \"%s\" has rank %zu > %d", path, kv.first.c_str(),
                  shape->arr.size(), RXW8_MAX_RANK);
    // element count with checked multiplication: any count whose bytes
    // exceed INT64_MAX is rejected (it cannot match a data section anyway),
    // so the product never wraps and later int64 arithmetic on it is exact
    uint64_t numel = 1;
    bool zero = false;
    for (const Json &d : shape->arr) {
      if (d.kind != Json::Num || d.neg_or_frac || d.num > (uint64_t)INT64_MAX)
        return fail(RXW8_DATA_LOSS, "\"%s\": tensor \"%s\" has a bad dimension", path, kv.first.c_str());
      t.shape.push_back((int64_t)d.num);
      zero = zero || d.num == 0;
    }
    for (int64_t d : t.shape) {
      if (zero) {
        numel = 0;
        break;
      }
      if (elem == 0 || (uint64_t)d > (uint64_t)INT64_MAX / elem / numel)
        return fail(RXW8_DATA_LOSS, "\"%s\": tensor \"%s\" has more than INT64_MAX bytes", path,
                    kv.first.c_str());
      numel *= (uint64_t)d;
    }
    t.numel = (int64_t)numel;
    for (const Json &o : offs->arr)
      if (o.kind != Json::Num || o.neg_or_frac)
        return fail(RXW8_DATA_LOSS, "\"%s\": tensor \"%s\" has bad data_offsets", path, kv.first.c_str());
    t.begin = offs->arr[0].num;
    t.end = offs->arr[1].num;
    if (t.begin > t.end || t.end > st->data_bytes || numel * elem != t.end - t.begin)
      return fail(RXW8_DATA_LOSS, "\"%s\": tensor \"%s\": data_offsets [%llu, %llu) do not hold %s %s elements inside %llu bytes",
                  path, kv.first.c_str(), (unsigned long long)t.begin, (unsigned long long)t.end,
                  "its", dt->str.c_str(), (unsigned long long)st->data_bytes);
    if (st->index.count(t.name))
      return fail(RXW8_DATA_LOSS, "\"%s\": tensor \"%s\" appears twice", path, t.name.c_str());
    st->index[t.name] = st->tensors.size();
    st->tensors.push_back(std::move(t));
  }
  // no two payloads may overlap
  std::vector<const TensorEntry *> order;
  for (const TensorEntry &t : st->tensors)
    if (t.end > t.begin) order.push_back(&t);
  std::sort(order.begin(), order.end(),
            [](const TensorEntry *a, const TensorEntry *b) { return a->begin < b->begin; });
  for (size_t i = 1; i < order.size(); ++i)
    if (order[i]->begin < order[i - 1]->end)
      return fail(RXW8_DATA_LOSS, "\"%s\": tensors \"%s\" and \"%s\" overlap", path,
                  order[i - 1]->name.c_str(), order[i]->name.c_str());
  return RXW8_OK;
}

static void close_st(SafeTensors *st) {
  if (st->map) munmap(st->map, st->map_bytes);
  delete st;
}

// Convert n elements of a source dtype into a destination dtype on the host.
static int convert(const uint8_t *src, int sdt, void *dst, int ddt, int64_t n) {
  auto to_f32 = [&](int64_t i) -> float {
    if (sdt == RXW8_F32) {
      float f;
      std::memcpy(&f, src + 4 * i, 4);
      return f;
    }
    uint16_t h;
    std::memcpy(&h, src + 2 * i, 2);
    return sdt == RXW8_F16 ? f16_to_f32(h) : bf16_to_f32(h);
  };
  if (ddt == RXW8_F32) {
    float *o = (float *)dst;
    for (int64_t i = 0; i < n; ++i) o[i] = to_f32(i);
  } else if (ddt == RXW8_BF16) {
    uint16_t *o = (uint16_t *)dst;
    for (int64_t i = 0; i < n; ++i) o[i] = f32_to_bf16(to_f32(i));
  } else if (ddt == RXW8_F16) {
    uint16_t *o = (uint16_t *)dst;
    for (int64_t i = 0; i < n; ++i) o[i] = f32_to_f16(to_f32(i));
  } else {
    return RXW8_UNIMPLEMENTED;
  }
  return RXW8_OK;
}

}  // namespace rxw8

using namespace rxw8;

struct rxw8_safetensors : rxw8::SafeTensors {};

extern "C" {

int rxw8_safetensors_open(const char *path, rxw8_safetensors **out) {
  if (!path || !out) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  auto *st = new rxw8_safetensors();
  int rc = open_file(path, st);
  if (rc == RXW8_OK) rc = parse_header(path, st);
  if (rc != RXW8_OK) {
    close_st(st);
    return rc;
  }
  *out = st;
  return RXW8_OK;
}

int rxw8_safetensors_close(rxw8_safetensors *st) {
  if (!st) return fail(RXW8_INVALID_ARGUMENT, "NULL handle");
  close_st(st);
  return RXW8_OK;
}

int rxw8_safetensors_num_tensors(rxw8_safetensors *st, int64_t *count) {
  if (!st || !count) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  *count = (int64_t)st->tensors.size();
  return RXW8_OK;
}

int rxw8_safetensors_tensor_info(rxw8_safetensors *st, int64_t index, const char **name, int *dtype,
                                 int64_t *dims, int *rank) {
  if (!st || !name || !dtype || !dims || !rank) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if (index < 0 || index >= (int64_t)st->tensors.size())
    return fail(RXW8_OUT_OF_RANGE, "tensor index %lld out of range", (long long)index);
  const TensorEntry &t = st->tensors[(size_t)index];
  *name = t.name.c_str();
  *dtype = t.dtype;
  *rank = (int)t.shape.size();
  for (size_t i = 0; i < t.shape.size(); ++i) dims[i] = t.shape[i];
  return RXW8_OK;
}

int rxw8_safetensors_find(rxw8_safetensors *st, const char *name, int64_t *index) {
  if (!st || !name || !index) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  auto it = st->index.find(name);
  if (it == st->index.end()) return fail(RXW8_NOT_FOUND, "missing tensor \"%s\"", name);
  *index = (int64_t)it->second;
  return RXW8_OK;
}

int rxw8_safetensors_metadata(rxw8_safetensors *st, const char *key, const char **value) {
  if (!st || !key || !value) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  for (auto &kv : st->metadata)
    if (kv.first == key) {
      *value = kv.second.c_str();
      return RXW8_OK;
    }
  return fail(RXW8_NOT_FOUND, "no metadata key \"%s\"", key);
}

int rxw8_safetensors_upload(rxw8_safetensors *st, int64_t index, rxw8_buffer *dst, int64_t offset) {
  if (!st || !dst) return fail(RXW8_INVALID_ARGUMENT, "NULL argument");
  if (index < 0 || index >= (int64_t)st->tensors.size())
    return fail(RXW8_OUT_OF_RANGE, "tensor index %lld out of range", (long long)index);
  const TensorEntry &t = st->tensors[(size_t)index];
  const int64_t numel = t.numel;
  const int ddt = dst->dtype;
  const bool floaty = [](int d) { return d == RXW8_F32 || d == RXW8_F16 || d == RXW8_BF16; }(ddt);
  const bool src_floaty = t.dtype == RXW8_F32 || t.dtype == RXW8_F16 || t.dtype == RXW8_BF16;
  if (!(t.dtype == ddt && t.dtype != 0) && !(floaty && src_floaty))
    return fail(RXW8_INVALID_ARGUMENT, "tensor \"%s\": incompatible checkpoint dtype %s for %s storage",
                t.name.c_str(), t.st_dtype.c_str(), dtype_name(ddt));
  const int64_t cap = (int64_t)dst->numel();
  if (offset < 0 || offset > cap || numel > cap - offset)
    return fail(RXW8_OUT_OF_RANGE, "tensor \"%s\": %lld elements at offset %lld exceed the buffer's %lld",
                t.name.c_str(), (long long)numel, (long long)offset, (long long)cap);
  if (numel == 0) return RXW8_OK;
  const size_t esz = dtype_size(ddt);
  const uint8_t *src = st->data + t.begin;
  Runtime *rt = dst->rt;
  std::vector<uint8_t> staged;
  const void *host = src;
  if (t.dtype != ddt) {
    staged.resize((size_t)numel * esz);
    int rc = convert(src, t.dtype, staged.data(), ddt, numel);
    if (rc) return fail(rc, "tensor \"%s\": unsupported conversion", t.name.c_str());
    host = staged.data();
  }
  std::lock_guard<std::recursive_mutex> g(rt->mu);
  RXW8_HIP(hipMemcpyAsync((char *)dst->ptr + (size_t)offset * esz, host, (size_t)numel * esz,
                          hipMemcpyHostToDevice, rt->stream));
  RXW8_HIP(hipStreamSynchronize(rt->stream));
  return RXW8_OK;
}

}  // extern "C"
