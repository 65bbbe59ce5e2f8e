// Reader for .safetensors files and compressed-tensors metadata (see
// safetensors.hpp).  Every length, offset and count read from the file is
// checked before it is used, so a malformed file is an error, never an
// out-of-bounds access.
#include "safetensors.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>

namespace teeny {
namespace st {

const Json *Json::get(const std::string &key) const {
  if (kind != Object) return nullptr;
  for (const auto &kv : obj)
    if (kv.first == key) return &kv.second;
  return nullptr;
}

namespace {

constexpr int kMaxDepth = 64;

struct Parser {
  const char *p, *end;
  std::string *err;

  bool fail(const std::string &msg) {
    if (err->empty()) *err = "json: " + msg;
    return false;
  }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(const char *word) {
    const size_t n = std::strlen(word);
    if (static_cast<size_t>(end - p) < n || std::memcmp(p, word, n) != 0) return false;
    p += n;
    return true;
  }
  static void put_utf8(std::string &s, uint32_t cp) {
    if (cp < 0x80) {
      s += static_cast<char>(cp);
    } else if (cp < 0x800) {
      s += static_cast<char>(0xC0 | (cp >> 6));
      s += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += static_cast<char>(0xE0 | (cp >> 12));
      s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      s += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
      s += static_cast<char>(0xF0 | (cp >> 18));
      s += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
      s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      s += static_cast<char>(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t *out) {
    if (end - p < 4) return fail("truncated \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = p[i];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
      else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    p += 4;
    *out = v;
    return true;
  }
  bool string(std::string *out) {
    if (p >= end || *p != '"') return fail("expected a string");
    ++p;
    out->clear();
    while (true) {
      if (p >= end) return fail("unterminated string");
      const unsigned char c = static_cast<unsigned char>(*p++);
      if (c == '"') return true;
      if (c < 0x20) return fail("control character in string");
      if (c != '\\') {
        *out += static_cast<char>(c);
        continue;
      }
      if (p >= end) return fail("unterminated escape");
      const char e = *p++;
      switch (e) {
        case '"': *out += '"'; break;
        case '\\': *out += '\\'; break;
        case '/': *out += '/'; break;
        case 'b': *out += '\b'; break;
        case 'f': *out += '\f'; break;
        case 'n': *out += '\n'; break;
        case 'r': *out += '\r'; break;
        case 't': *out += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(&cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // high surrogate: a low one must follow
            uint32_t lo;
            if (end - p < 2 || p[0] != '\\' || p[1] != 'u') return fail("lone high surrogate");
            p += 2;
            if (!hex4(&lo)) return false;
            if (lo < 0xDC00 || lo >= 0xE000) return fail("bad low surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            return fail("lone low surrogate");
          }
          put_utf8(*out, cp);
          break;
        }
        default: return fail("bad escape");
      }
    }
  }
  bool number(Json *out) {
    const char *s = p;
    bool frac = false;
    if (p < end && *p == '-') ++p;
    if (p >= end) return fail("bad number");
    if (*p == '0') {
      ++p;
    } else if (*p >= '1' && *p <= '9') {
      while (p < end && *p >= '0' && *p <= '9') ++p;
    } else {
      return fail("bad number");
    }
    if (p < end && *p == '.') {
      frac = true;
      ++p;
      if (p >= end || *p < '0' || *p > '9') return fail("bad fraction");
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    if (p < end && (*p == 'e' || *p == 'E')) {
      frac = true;
      ++p;
      if (p < end && (*p == '+' || *p == '-')) ++p;
      if (p >= end || *p < '0' || *p > '9') return fail("bad exponent");
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    const std::string text(s, p);
    out->kind = Json::Number;
    out->num = std::strtod(text.c_str(), nullptr);
    out->integral = false;
    if (!frac) {
      errno = 0;
      char *e = nullptr;
      const long long v = std::strtoll(text.c_str(), &e, 10);
      if (errno == 0 && e != nullptr && *e == '\0') {
        out->integral = true;
        out->i = v;
      }
    }
    return true;
  }
  bool value(Json *out, int depth) {
    if (depth > kMaxDepth) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    const char c = *p;
    if (c == '{') {
      ++p;
      out->kind = Json::Object;
      ws();
      if (p < end && *p == '}') {
        ++p;
        return true;
      }
      while (true) {
        ws();
        std::string key;
        if (!string(&key)) return false;
        ws();
        if (p >= end || *p != ':') return fail("expected ':'");
        ++p;
        out->obj.emplace_back(std::move(key), Json());
        if (!value(&out->obj.back().second, depth + 1)) return false;
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == '}') {
          ++p;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p;
      out->kind = Json::Array;
      ws();
      if (p < end && *p == ']') {
        ++p;
        return true;
      }
      while (true) {
        out->arr.emplace_back();
        if (!value(&out->arr.back(), depth + 1)) return false;
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == ']') {
          ++p;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      out->kind = Json::String;
      return string(&out->str);
    }
    if (c == 't' && lit("true")) {
      out->kind = Json::Bool;
      out->b = true;
      return true;
    }
    if (c == 'f' && lit("false")) {
      out->kind = Json::Bool;
      out->b = false;
      return true;
    }
    if (c == 'n' && lit("null")) {
      out->kind = Json::Null;
      return true;
    }
    if (c == '-' || (c >= '0' && c <= '9')) return number(out);
    return fail("unexpected character");
  }
};

bool nonneg_int(const Json *j, int64_t *out) {
  if (j == nullptr || j->kind != Json::Number || !j->integral || j->i < 0) return false;
  *out = j->i;
  return true;
}

}  // namespace

bool parse_json(const char *text, size_t len, Json *out, std::string *err) {
  Parser ps{text, text + len, err};
  *out = Json();
  if (!ps.value(out, 0)) return false;
  ps.ws();
  if (ps.p != ps.end) return ps.fail("trailing characters");
  return true;
}

DType dtype_from_name(const std::string &n) {
  static const std::pair<const char *, DType> names[] = {
      {"F64", DType::F64}, {"F32", DType::F32}, {"F16", DType::F16}, {"BF16", DType::BF16},
      {"I64", DType::I64}, {"I32", DType::I32}, {"I16", DType::I16}, {"I8", DType::I8},
      {"U8", DType::U8},   {"BOOL", DType::BOOL}, {"F8_E4M3", DType::F8_E4M3}, {"F8_E5M2", DType::F8_E5M2}};
  for (const auto &kv : names)
    if (n == kv.first) return kv.second;
  return DType::Unknown;
}

size_t dtype_size(DType d) {
  switch (d) {
    case DType::F64: case DType::I64: return 8;
    case DType::F32: case DType::I32: return 4;
    case DType::F16: case DType::BF16: case DType::I16: return 2;
    case DType::I8: case DType::U8: case DType::BOOL: case DType::F8_E4M3: case DType::F8_E5M2: return 1;
    default: return 0;
  }
}

int64_t TensorEntry::numel() const {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}

File::~File() {
  if (mapping_ != nullptr) munmap(mapping_, size_);
}

bool File::open(const std::string &path, std::string *err) {
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    *err = "cannot open " + path;
    return false;
  }
  struct stat stb;
  if (fstat(fd, &stb) != 0 || stb.st_size < 0) {
    ::close(fd);
    *err = "cannot stat " + path;
    return false;
  }
  size_ = static_cast<size_t>(stb.st_size);
  if (size_ < 8) {
    ::close(fd);
    *err = path + ": shorter than the 8-byte header length";
    return false;
  }
  void *m = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) {
    *err = "cannot map " + path;
    return false;
  }
  mapping_ = m;
  base_ = static_cast<const uint8_t *>(m);
  return parse(err);
}

bool File::open_image(const uint8_t *data, size_t size, std::string *err) {
  base_ = data;
  size_ = size;
  if (data == nullptr || size < 8) {
    *err = "image shorter than the 8-byte header length";
    return false;
  }
  return parse(err);
}

const TensorEntry *File::find(const std::string &name) const {
  auto it = index_.find(name);
  return it == index_.end() ? nullptr : &tensors_[it->second];
}

bool File::parse(std::string *err) {
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | base_[i];
  // the safetensors format caps the header at 100 MB
  if (hlen == 0 || hlen > 100000000ull || hlen > size_ - 8) {
    *err = "header length " + std::to_string(hlen) + " does not fit the file";
    return false;
  }
  data_start_ = 8 + static_cast<size_t>(hlen);
  const uint64_t data_size = size_ - data_start_;
  Json root;
  if (!parse_json(reinterpret_cast<const char *>(base_ + 8), static_cast<size_t>(hlen), &root, err)) return false;
  if (root.kind != Json::Object) {
    *err = "header is not a JSON object";
    return false;
  }
  for (const auto &kv : root.obj) {
    if (kv.first == "__metadata__") {
      if (kv.second.kind != Json::Object) {
        *err = "__metadata__ is not an object";
        return false;
      }
      for (const auto &m : kv.second.obj) {
        if (m.second.kind != Json::String) {
          *err = "__metadata__ value of '" + m.first + "' is not a string";
          return false;
        }
        metadata_[m.first] = m.second.str;
      }
      continue;
    }
    const Json &t = kv.second;
    const Json *dt = t.get("dtype"), *sh = t.get("shape"), *off = t.get("data_offsets");
    if (t.kind != Json::Object || dt == nullptr || dt->kind != Json::String || sh == nullptr ||
        sh->kind != Json::Array || off == nullptr || off->kind != Json::Array || off->arr.size() != 2) {
      *err = "tensor '" + kv.first + "': needs dtype, shape and two data_offsets";
      return false;
    }
    TensorEntry e;
    e.name = kv.first;
    e.dtype_name = dt->str;
    e.dtype = dtype_from_name(dt->str);
    if (e.dtype == DType::Unknown) {
      *err = "tensor '" + kv.first + "': unknown dtype " + dt->str;
      return false;
    }
    uint64_t numel = 1;
    for (const Json &d : sh->arr) {
      int64_t v;
      if (!nonneg_int(&d, &v)) {
        *err = "tensor '" + kv.first + "': shape entries must be non-negative integers";
        return false;
      }
      if (v != 0 && numel > std::numeric_limits<uint64_t>::max() / static_cast<uint64_t>(v)) {
        *err = "tensor '" + kv.first + "': element count overflows";
        return false;
      }
      numel *= static_cast<uint64_t>(v);
      e.shape.push_back(v);
    }
    if (e.shape.size() > 8) {
      *err = "tensor '" + kv.first + "': more than 8 dimensions";
      return false;
    }
    int64_t b, en;
    if (!nonneg_int(&off->arr[0], &b) || !nonneg_int(&off->arr[1], &en) || b > en ||
        static_cast<uint64_t>(en) > data_size) {
      *err = "tensor '" + kv.first + "': data_offsets outside the data section";
      return false;
    }
    const size_t es = dtype_size(e.dtype);
    if (numel > data_size / es || static_cast<uint64_t>(en - b) != numel * es) {
      *err = "tensor '" + kv.first + "': data_offsets span " + std::to_string(en - b) + " bytes, shape and " +
             dt->str + " need " + std::to_string(numel * es);
      return false;
    }
    e.begin = static_cast<uint64_t>(b);
    e.end = static_cast<uint64_t>(en);
    if (index_.count(e.name) != 0) {
      *err = "tensor '" + kv.first + "' listed twice";
      return false;
    }
    index_[e.name] = tensors_.size();
    tensors_.push_back(std::move(e));
  }
  // compressed-tensors scheme (format.rs:52-126), when present
  auto it = metadata_.find("quantization_config");
  if (it != metadata_.end()) {
    Json q;
    std::string qerr;
    if (!parse_json(it->second.data(), it->second.size(), &q, &qerr) || q.kind != Json::Object) {
      *err = "quantization_config: " + (qerr.empty() ? std::string("not an object") : qerr);
      return false;
    }
    QuantConfig &c = qcfg_;
    c.present = true;
    if (const Json *v = q.get("quant_method"); v != nullptr && v->kind == Json::String) c.quant_method = v->str;
    if (const Json *v = q.get("format"); v != nullptr && v->kind == Json::String) c.format = v->str;
    if (const Json *ig = q.get("ignore"); ig != nullptr && ig->kind == Json::Array)
      for (const Json &s : ig->arr)
        if (s.kind == Json::String) c.ignore.push_back(s.str);
    const Json *groups = q.get("config_groups");
    if (groups == nullptr || groups->kind != Json::Object || groups->obj.empty()) {
      *err = "quantization_config: no config_groups";
      return false;
    }
    c.n_groups = static_cast<int>(groups->obj.size());
    const Json *w = groups->obj.front().second.get("weights");
    if (w == nullptr || w->kind != Json::Object) {
      *err = "quantization_config: config group without a weights block";
      return false;
    }
    int64_t nb = 0;
    if (!nonneg_int(w->get("num_bits"), &nb) || nb == 0 || nb > 64) {
      *err = "quantization_config: weights.num_bits missing or invalid";
      return false;
    }
    c.num_bits = static_cast<int>(nb);
    if (const Json *v = w->get("type"); v != nullptr && v->kind == Json::String) c.type = v->str;
    // WeightsConfig.symmetric is a required bool (format.rs:52-70): a file
    // without it does not state its zero points, so it is refused
    if (const Json *v = w->get("symmetric"); v != nullptr && v->kind == Json::Bool) {
      c.symmetric = v->b;
    } else {
      *err = "quantization_config: weights.symmetric missing or not a bool";
      return false;
    }
    if (const Json *v = w->get("strategy"); v != nullptr && v->kind == Json::String) c.strategy = v->str;
    int64_t v64;
    if (const Json *v = w->get("axis"); v != nullptr && v->kind != Json::Null) {
      if (!nonneg_int(v, &v64)) {
        *err = "quantization_config: weights.axis invalid";
        return false;
      }
      c.axis = v64;
    }
    if (const Json *v = w->get("group_size"); v != nullptr && v->kind != Json::Null) {
      if (!nonneg_int(v, &v64) || v64 == 0) {
        *err = "quantization_config: weights.group_size invalid";
        return false;
      }
      c.group_size = v64;
    }
  }
  return true;
}

}  // namespace st
}  // namespace teeny
