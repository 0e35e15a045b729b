// fmx_st_parse.cpp -- the weight-ingest format on the host: safetensors
// container headers and tensor byte ranges (the upload of a tensor into an
// fmx_array is fmx_safetensors.cpp).  Plain host C++ with no HIP, built with
// the sanitizers by the CPU test suite.
//
// Restates compute/safetensors.go (ParseSafetensorsHeader, :101-165; dtype sizes
// :21-37) and compute/loader.go (mlxgoDtype :13-42, TensorBytes :47-55, the
// per-tensor upload of LoadTensors :61-84).  The header is an 8-byte
// little-endian length followed by that many bytes of JSON: {name: {dtype,
// shape, data_offsets}} plus an optional __metadata__ string map.  Validation
// follows the reference: every dtype known, begin <= end, end within the data
// buffer, and end - begin equal to numel * dtype size; tensors are listed by
// (begin, name).  Keys repeated in the JSON keep their last value, as a Go map
// decode does; unknown fields of a tensor entry are ignored.
#include <algorithm>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/fmx.h"
#include "../../include/fmxq.h"
#include "fmxq_status.hpp"

using fmxq::fail;

struct fmx_st_header_ {
  struct Tensor {
    std::string name, dtype;
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;
  };
  std::vector<Tensor> tensors;
  std::map<std::string, int64_t> by_name;
  bool has_metadata = false;
  std::vector<std::pair<std::string, std::string>> metadata;
  uint64_t header_size = 0, data_start = 0;
};

namespace {

uint64_t st_dtype_size(const std::string& t) {
  static const std::map<std::string, uint64_t> sizes = {
      {"BOOL", 1}, {"U8", 1},  {"I8", 1},  {"F8_E5M2", 1}, {"F8_E4M3", 1},
      {"I16", 2},  {"U16", 2}, {"F16", 2}, {"BF16", 2},    {"I32", 4},
      {"U32", 4},  {"F32", 4}, {"F64", 8}, {"I64", 8},     {"U64", 8}};
  auto it = sizes.find(t);
  return it == sizes.end() ? 0 : it->second;
}

// A minimal JSON reader for the header: objects, arrays, strings (with every
// escape, \u pairs included), integers, null/true/false, and numbers skipped
// where their value is not needed.
struct Json {
  const char* p;
  const char* e;
  std::string err;

  bool fail_at(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool peek(char c) {
    ws();
    return p < e && *p == c;
  }
  bool eat(char c) {
    ws();
    if (p < e && *p == c) {
      ++p;
      return true;
    }
    return false;
  }
  bool literal(const char* lit) {
    ws();
    const size_t n = strlen(lit);
    if ((size_t)(e - p) >= n && memcmp(p, lit, n) == 0) {
      p += n;
      return true;
    }
    return false;
  }
  static void put_utf8(std::string& s, uint32_t c) {
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
  bool hex4(uint32_t* out) {
    if (e - p < 4) return fail_at("truncated \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = p[i];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return fail_at("bad \\u escape");
    }
    p += 4;
    *out = v;
    return true;
  }
  bool str(std::string* out) {
    if (!eat('"')) return fail_at("expected a string");
    std::string s;
    while (p < e && *p != '"') {
      const unsigned char c = (unsigned char)*p++;
      if (c < 0x20) return fail_at("control character in string");
      if (c != '\\') {
        s += (char)c;
        continue;
      }
      if (p >= e) return fail_at("truncated escape");
      const char k = *p++;
      switch (k) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t c1 = 0;
          if (!hex4(&c1)) return false;
          if (c1 >= 0xD800 && c1 < 0xDC00 && e - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            const char* save = p;
            p += 2;
            uint32_t c2 = 0;
            if (hex4(&c2) && c2 >= 0xDC00 && c2 < 0xE000) {
              c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
            } else {
              p = save;
              err.clear();
              c1 = 0xFFFD;
            }
          } else if (c1 >= 0xD800 && c1 < 0xE000) {
            c1 = 0xFFFD;  // lone surrogate
          }
          put_utf8(s, c1);
          break;
        }
        default: return fail_at("bad escape");
      }
    }
    if (p >= e) return fail_at("unterminated string");
    ++p;
    *out = std::move(s);
    return true;
  }
  // An integer literal (no fraction or exponent), as Go decodes into int/uint64.
  bool integer(int64_t* out, bool allow_negative) {
    ws();
    const char* q = p;
    bool neg = false;
    if (q < e && *q == '-') {
      neg = true;
      ++q;
    }
    if (q >= e || *q < '0' || *q > '9') return fail_at("expected an integer");
    if (*q == '0' && q + 1 < e && q[1] >= '0' && q[1] <= '9') return fail_at("bad number");
    uint64_t v = 0;
    while (q < e && *q >= '0' && *q <= '9') {
      const uint64_t d = (uint64_t)(*q - '0');
      if (v > (UINT64_MAX - d) / 10) return fail_at("integer out of range");
      v = v * 10 + d;
      ++q;
    }
    if (q < e && (*q == '.' || *q == 'e' || *q == 'E')) return fail_at("expected an integer");
    if (neg && !allow_negative) return fail_at("negative value");
    if (v > (uint64_t)INT64_MAX) return fail_at("integer out of range");
    p = q;
    *out = neg ? -(int64_t)v : (int64_t)v;
    return true;
  }
  bool number_skip() {
    ws();
    const char* q = p;
    if (q < e && *q == '-') ++q;
    if (q >= e || *q < '0' || *q > '9') return fail_at("bad number");
    while (q < e && ((*q >= '0' && *q <= '9') || *q == '.' || *q == 'e' || *q == 'E' ||
                     *q == '+' || *q == '-'))
      ++q;
    p = q;
    return true;
  }
  bool skip(int depth = 0) {
    if (depth > 64) return fail_at("nesting too deep");
    ws();
    if (p >= e) return fail_at("unexpected end");
    if (*p == '"') {
      std::string s;
      return str(&s);
    }
    if (*p == '{') {
      ++p;
      if (eat('}')) return true;
      do {
        std::string k;
        if (!str(&k) || !eat(':') || !skip(depth + 1)) return fail_at("bad object");
      } while (eat(','));
      return eat('}') || fail_at("expected '}'");
    }
    if (*p == '[') {
      ++p;
      if (eat(']')) return true;
      do {
        if (!skip(depth + 1)) return false;
      } while (eat(','));
      return eat(']') || fail_at("expected ']'");
    }
    if (literal("null") || literal("true") || literal("false")) return true;
    return number_skip();
  }
};

int parse_tensor(Json& j, const std::string& name, fmx_st_header_::Tensor* t) {
  t->name = name;
  if (j.literal("null")) return FMXQ_OK;  // zero value: rejected below for its dtype
  if (!j.eat('{'))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: tensor \"%s\": not an object",
                name.c_str());
  if (j.eat('}')) return FMXQ_OK;
  do {
    std::string key;
    if (!j.str(&key) || !j.eat(':'))
      return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: tensor \"%s\": %s", name.c_str(),
                  j.err.empty() ? "bad entry" : j.err.c_str());
    bool ok = true;
    if (key == "dtype") {
      if (j.literal("null")) t->dtype.clear();
      else ok = j.str(&t->dtype);
    } else if (key == "shape") {
      t->shape.clear();
      if (!j.literal("null")) {
        ok = j.eat('[');
        if (ok && !j.eat(']')) {
          do {
            int64_t d = 0;
            ok = j.integer(&d, true);
            if (ok) t->shape.push_back(d);
          } while (ok && j.eat(','));
          ok = ok && j.eat(']');
        }
      }
    } else if (key == "data_offsets") {
      // A two-element array: missing elements stay zero, extra ones are dropped.
      t->begin = t->end = 0;
      if (!j.literal("null")) {
        ok = j.eat('[');
        if (ok && !j.eat(']')) {
          int idx = 0;
          do {
            int64_t v = 0;
            ok = j.integer(&v, false);
            if (ok && idx == 0) t->begin = (uint64_t)v;
            if (ok && idx == 1) t->end = (uint64_t)v;
            ++idx;
          } while (ok && j.eat(','));
          ok = ok && j.eat(']');
        }
      }
    } else {
      ok = j.skip();
    }
    if (!ok)
      return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: tensor \"%s\": %s in \"%s\"",
                  name.c_str(), j.err.empty() ? "bad value" : j.err.c_str(), key.c_str());
  } while (j.eat(','));
  if (!j.eat('}'))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: tensor \"%s\": expected '}'",
                name.c_str());
  return FMXQ_OK;
}

int parse_metadata(Json& j, fmx_st_header_* h) {
  h->metadata.clear();
  if (j.literal("null")) {
    h->has_metadata = false;
    return FMXQ_OK;
  }
  if (!j.eat('{')) return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: __metadata__: not an object");
  h->has_metadata = true;
  std::map<std::string, size_t> at;
  if (j.eat('}')) return FMXQ_OK;
  do {
    std::string k, v;
    if (!j.str(&k) || !j.eat(':') || !j.str(&v))
      return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: __metadata__: %s",
                  j.err.empty() ? "values must be strings" : j.err.c_str());
    if (k.find('\0') != std::string::npos || v.find('\0') != std::string::npos)
      return fail(FMXQ_ERR_INVALID_ARGUMENT,
                  "safetensors: __metadata__: a key or value holds a NUL (\\u0000), which the "
                  "C-string accessors cannot return");
    auto it = at.find(k);
    if (it != at.end()) {
      h->metadata[it->second].second = v;
    } else {
      at[k] = h->metadata.size();
      h->metadata.emplace_back(k, v);
    }
  } while (j.eat(','));
  if (!j.eat('}')) return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: __metadata__: expected '}'");
  return FMXQ_OK;
}

int parse(const uint8_t* blob, uint64_t len, fmx_st_header_* h) {
  if (len < 8) return fail(FMXQ_ERR_SHAPE, "safetensors: buffer shorter than declared header");
  uint64_t hs = 0;
  for (int i = 7; i >= 0; --i) hs = (hs << 8) | blob[i];
  if (hs > len - 8) return fail(FMXQ_ERR_SHAPE, "safetensors: header length exceeds buffer");
  const uint64_t data_len = len - 8 - hs;
  h->header_size = hs;
  h->data_start = 8 + hs;
  Json j{reinterpret_cast<const char*>(blob) + 8, reinterpret_cast<const char*>(blob) + 8 + hs, {}};
  if (!j.eat('{')) return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: header JSON: not an object");
  std::vector<fmx_st_header_::Tensor> raw;
  std::map<std::string, size_t> seen;
  if (!j.eat('}')) {
    do {
      std::string name;
      if (!j.str(&name) || !j.eat(':'))
        return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: header JSON: %s",
                    j.err.empty() ? "bad key" : j.err.c_str());
      if (name == "__metadata__") {
        if (int rc = parse_metadata(j, h)) return rc;
        continue;
      }
      // Names leave through C strings (fmx_safetensors_tensor / _find): one that
      // decodes a NUL could not be found again by its own name.
      if (name.find('\0') != std::string::npos)
        return fail(FMXQ_ERR_INVALID_ARGUMENT,
                    "safetensors: a tensor name holds a NUL (\\u0000), which the C-string "
                    "accessors cannot return");
      fmx_st_header_::Tensor t;
      if (int rc = parse_tensor(j, name, &t)) return rc;
      auto it = seen.find(name);
      if (it != seen.end()) {
        raw[it->second] = std::move(t);
      } else {
        seen[name] = raw.size();
        raw.push_back(std::move(t));
      }
    } while (j.eat(','));
    if (!j.eat('}')) return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: header JSON: expected '}'");
  }
  j.ws();
  if (j.p != j.e) return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: header JSON: trailing data");

  for (const auto& t : raw) {
    const uint64_t size = st_dtype_size(t.dtype);
    if (!size)
      return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: tensor \"%s\" has unknown dtype \"%s\"",
                  t.name.c_str(), t.dtype.c_str());
    if (t.begin > t.end)
      return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: tensor \"%s\" has begin %llu > end %llu",
                  t.name.c_str(), (unsigned long long)t.begin, (unsigned long long)t.end);
    if (t.end > data_len)
      return fail(FMXQ_ERR_INVALID_ARGUMENT,
                  "safetensors: tensor \"%s\" range [%llu,%llu) exceeds data length %llu",
                  t.name.c_str(), (unsigned long long)t.begin, (unsigned long long)t.end,
                  (unsigned long long)data_len);
    // numel * size in unsigned arithmetic, as the reference computes it; a
    // negative axis can never match a real byte length.
    bool neg = false;
    unsigned __int128 want = size;
    for (int64_t d : t.shape) {
      neg |= d < 0;
      want *= (unsigned __int128)(uint64_t)d;
      if (want > (unsigned __int128)UINT64_MAX) neg = true;
    }
    if (neg || (uint64_t)want != t.end - t.begin)
      return fail(FMXQ_ERR_INVALID_ARGUMENT,
                  "safetensors: tensor \"%s\" byte length %llu does not match shape*dtype",
                  t.name.c_str(), (unsigned long long)(t.end - t.begin));
  }
  std::sort(raw.begin(), raw.end(), [](const fmx_st_header_::Tensor& a,
                                       const fmx_st_header_::Tensor& b) {
    return a.begin != b.begin ? a.begin < b.begin : a.name < b.name;
  });
  h->tensors = std::move(raw);
  for (size_t i = 0; i < h->tensors.size(); ++i) h->by_name[h->tensors[i].name] = (int64_t)i;
  return FMXQ_OK;
}

}  // namespace

extern "C" {

int fmx_safetensors_parse(const uint8_t* blob, uint64_t len, fmx_st_header** out) {
  if (!out) return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: null result");
  *out = nullptr;
  if (!blob && len) return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: null blob");
  auto* h = new fmx_st_header_;
  if (int rc = parse(blob, len, h)) {
    delete h;
    return rc;
  }
  *out = h;
  return FMXQ_OK;
}

void fmx_safetensors_free(fmx_st_header* h) { delete h; }

uint64_t fmx_safetensors_header_size(const fmx_st_header* h) { return h ? h->header_size : 0; }

uint64_t fmx_safetensors_data_start(const fmx_st_header* h) { return h ? h->data_start : 0; }

int64_t fmx_safetensors_count(const fmx_st_header* h) {
  return h ? (int64_t)h->tensors.size() : 0;
}

int fmx_safetensors_tensor(const fmx_st_header* h, int64_t i, const char** name,
                           const char** dtype, int* ndim, const int64_t** shape, uint64_t* begin,
                           uint64_t* end) {
  if (!h || i < 0 || i >= (int64_t)h->tensors.size())
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: tensor index %lld out of range",
                (long long)i);
  const auto& t = h->tensors[(size_t)i];
  if (name) *name = t.name.c_str();
  if (dtype) *dtype = t.dtype.c_str();
  if (ndim) *ndim = (int)t.shape.size();
  if (shape) *shape = t.shape.data();
  if (begin) *begin = t.begin;
  if (end) *end = t.end;
  return FMXQ_OK;
}

int64_t fmx_safetensors_find(const fmx_st_header* h, const char* name) {
  if (!h || !name) return -1;
  auto it = h->by_name.find(name);
  return it == h->by_name.end() ? -1 : it->second;
}

int64_t fmx_safetensors_metadata_count(const fmx_st_header* h) {
  return (h && h->has_metadata) ? (int64_t)h->metadata.size() : -1;
}

int fmx_safetensors_metadata(const fmx_st_header* h, int64_t i, const char** key,
                             const char** value) {
  if (!h || !h->has_metadata || i < 0 || i >= (int64_t)h->metadata.size())
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "safetensors: metadata index %lld out of range",
                (long long)i);
  if (key) *key = h->metadata[(size_t)i].first.c_str();
  if (value) *value = h->metadata[(size_t)i].second.c_str();
  return FMXQ_OK;
}

int fmx_safetensors_dtype(const char* tag, fmx_dtype* out) {
  static const std::map<std::string, fmx_dtype> m = {
      {"BOOL", FMX_BOOL},     {"U8", FMX_UINT8},    {"I8", FMX_INT8},   {"U16", FMX_UINT16},
      {"I16", FMX_INT16},     {"F16", FMX_FLOAT16}, {"BF16", FMX_BFLOAT16},
      {"U32", FMX_UINT32},    {"I32", FMX_INT32},   {"F32", FMX_FLOAT32}, {"U64", FMX_UINT64},
      {"I64", FMX_INT64},     {"F64", FMX_FLOAT64}};
  auto it = tag ? m.find(tag) : m.end();
  if (it == m.end())
    return fail(FMXQ_ERR_UNSUPPORTED, "safetensors: dtype \"%s\" has no array type",
                tag ? tag : "(null)");
  if (out) *out = it->second;
  return FMXQ_OK;
}

int fmx_safetensors_slice(uint64_t blob_len, uint64_t data_start, uint64_t begin, uint64_t end,
                          uint64_t* offset) {
  const uint64_t s = data_start + begin, e = data_start + end;
  if (e < s || e > blob_len || s < data_start || e < data_start)
    return fail(FMXQ_ERR_INVALID_ARGUMENT,
                "safetensors: range [%llu,%llu) out of bounds for %llu-byte blob",
                (unsigned long long)s, (unsigned long long)e, (unsigned long long)blob_len);
  if (offset) *offset = s;
  return FMXQ_OK;
}

}  // extern "C"
