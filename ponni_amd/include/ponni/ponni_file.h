// Host-only reader/writer of the PONNI profile of Safetensors (".ponni").
//
// File layout (utils/ponni_safetensors.h:350-407 of the reference):
//   u64 little-endian header length N, then N bytes of JSON padded with spaces
//   to a multiple of 8, then the little-endian payload.  The JSON object holds
//   "__metadata__" (string values: ponni.profile_version "1",
//   ponni.model_fingerprint, ponni.schema_fingerprint,
//   ponni.payload_checksum_fnv1a64, ponni.source_framework, ponni.target) and
//   one descriptor {"dtype","shape","data_offsets"} per tensor; tensors are
//   stored in name order and must tile the payload exactly.
// Rejection messages keep the reference's wording because callers match on
// them (unit/core/test_template_coverage.cpp:559-686).
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <limits>
#include <map>
#include <sstream>
#include <string>
#include <utility>
#include <vector>

namespace ponni {

// FNV-1a 64-bit (offset basis 14695981039346656037, prime 1099511628211).
inline std::uint64_t ponni_fnv1a64(unsigned char const* data, std::size_t size) {
  std::uint64_t h = 0xcbf29ce484222325ull;
  for (std::size_t i = 0; i < size; i++) {
    h ^= data[i];
    h *= 0x100000001b3ull;
  }
  return h;
}

inline std::string ponni_fnv1a64_string(std::uint64_t value) {
  char text[32];
  std::snprintf(text, sizeof(text), "fnv1a64:%016llx", static_cast<unsigned long long>(value));
  return text;
}

namespace detail {

// A small JSON value tree: enough of RFC 8259 for Safetensors headers, with
// duplicate-key rejection and a nesting limit.
struct JsonValue {
  enum class Kind { null_value, boolean, number, string, array, object };
  Kind kind = Kind::null_value;
  bool boolean = false;
  std::string text;  // string contents, or the literal spelling of a number
  std::vector<JsonValue> array;
  std::map<std::string, JsonValue> object;

  JsonValue const* find(std::string const& key) const {
    auto it = object.find(key);
    return it == object.end() ? nullptr : &it->second;
  }
};

class JsonParser {
 public:
  JsonParser(char const* text, std::size_t size) : begin_(text), pos_(text), end_(text + size) {}

  bool parse(JsonValue& value, std::string& error) {
    skip_space();
    bool ok = parse_value(value, 0);
    if (ok) {
      skip_space();
      if (pos_ != end_) ok = set_error("unexpected characters after JSON value");
    }
    error = error_;
    return ok && error_.empty();
  }

 private:
  char const* begin_;
  char const* pos_;
  char const* end_;
  std::string error_;
  static constexpr int kMaxDepth = 64;

  bool set_error(std::string const& what) {
    if (error_.empty()) error_ = what + " at JSON byte " + std::to_string(pos_ - begin_);
    return false;
  }
  void skip_space() {
    while (pos_ != end_ && (*pos_ == ' ' || *pos_ == '\t' || *pos_ == '\n' || *pos_ == '\r')) ++pos_;
  }
  bool literal(char const* word) {
    std::size_t const n = std::strlen(word);
    if (static_cast<std::size_t>(end_ - pos_) < n || std::memcmp(pos_, word, n) != 0)
      return set_error(std::string("expected ") + word);
    pos_ += n;
    return true;
  }
  static void append_utf8(std::string& out, std::uint32_t cp) {
    if (cp < 0x80) {
      out += static_cast<char>(cp);
    } else if (cp < 0x800) {
      out += static_cast<char>(0xc0 | (cp >> 6));
      out += static_cast<char>(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
      out += static_cast<char>(0xe0 | (cp >> 12));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
      out += static_cast<char>(0x80 | (cp & 0x3f));
    } else {
      out += static_cast<char>(0xf0 | (cp >> 18));
      out += static_cast<char>(0x80 | ((cp >> 12) & 0x3f));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
      out += static_cast<char>(0x80 | (cp & 0x3f));
    }
  }
  bool hex4(std::uint32_t& cp) {
    if (end_ - pos_ < 4) return set_error("incomplete Unicode escape");
    cp = 0;
    for (int i = 0; i < 4; i++) {
      char const ch = *pos_++;
      int d = -1;
      if (ch >= '0' && ch <= '9') d = ch - '0';
      else if (ch >= 'a' && ch <= 'f') d = ch - 'a' + 10;
      else if (ch >= 'A' && ch <= 'F') d = ch - 'A' + 10;
      if (d < 0) return set_error("invalid Unicode escape");
      cp = cp * 16 + static_cast<std::uint32_t>(d);
    }
    return true;
  }
  bool parse_string(std::string& out) {
    if (pos_ == end_ || *pos_ != '"') return set_error("expected '\"'");
    ++pos_;
    while (pos_ != end_) {
      unsigned char const ch = static_cast<unsigned char>(*pos_++);
      if (ch == '"') return true;
      if (ch < 0x20) return set_error("unescaped control character in string");
      if (ch != '\\') {
        out += static_cast<char>(ch);
        continue;
      }
      if (pos_ == end_) return set_error("incomplete string escape");
      char const esc = *pos_++;
      switch (esc) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          std::uint32_t cp = 0;
          if (!hex4(cp)) return false;
          if (cp >= 0xd800 && cp <= 0xdbff) {
            if (end_ - pos_ < 2 || pos_[0] != '\\' || pos_[1] != 'u') return set_error("missing low Unicode surrogate");
            pos_ += 2;
            std::uint32_t lo = 0;
            if (!hex4(lo)) return false;
            if (lo < 0xdc00 || lo > 0xdfff) return set_error("invalid low Unicode surrogate");
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          } else if (cp >= 0xdc00 && cp <= 0xdfff) {
            return set_error("unpaired low Unicode surrogate");
          }
          append_utf8(out, cp);
          break;
        }
        default:
          return set_error("invalid string escape");
      }
    }
    return set_error("unterminated string");
  }
  bool parse_number(JsonValue& value) {
    char const* start = pos_;
    if (pos_ != end_ && *pos_ == '-') ++pos_;
    if (pos_ == end_) return set_error("incomplete number");
    if (*pos_ == '0') {
      ++pos_;
    } else if (*pos_ >= '1' && *pos_ <= '9') {
      while (pos_ != end_ && *pos_ >= '0' && *pos_ <= '9') ++pos_;
    } else {
      return set_error("invalid number");
    }
    if (pos_ != end_ && *pos_ == '.') {
      ++pos_;
      if (pos_ == end_ || *pos_ < '0' || *pos_ > '9') return set_error("invalid fractional number");
      while (pos_ != end_ && *pos_ >= '0' && *pos_ <= '9') ++pos_;
    }
    if (pos_ != end_ && (*pos_ == 'e' || *pos_ == 'E')) {
      ++pos_;
      if (pos_ != end_ && (*pos_ == '+' || *pos_ == '-')) ++pos_;
      if (pos_ == end_ || *pos_ < '0' || *pos_ > '9') return set_error("invalid exponent");
      while (pos_ != end_ && *pos_ >= '0' && *pos_ <= '9') ++pos_;
    }
    value.kind = JsonValue::Kind::number;
    value.text.assign(start, pos_);
    return true;
  }
  bool parse_value(JsonValue& value, int depth) {
    if (depth > kMaxDepth) return set_error("JSON nesting limit exceeded");
    if (pos_ == end_) return set_error("expected JSON value");
    char const ch = *pos_;
    if (ch == '{') {
      ++pos_;
      value.kind = JsonValue::Kind::object;
      skip_space();
      if (pos_ != end_ && *pos_ == '}') {
        ++pos_;
        return true;
      }
      while (true) {
        skip_space();
        std::string key;
        if (!parse_string(key)) return false;
        skip_space();
        if (pos_ == end_ || *pos_ != ':') return set_error("expected ':'");
        ++pos_;
        skip_space();
        JsonValue item;
        if (!parse_value(item, depth + 1)) return false;
        if (!value.object.emplace(key, std::move(item)).second) return set_error("duplicate object key " + key);
        skip_space();
        if (pos_ != end_ && *pos_ == ',') {
          ++pos_;
          continue;
        }
        if (pos_ != end_ && *pos_ == '}') {
          ++pos_;
          return true;
        }
        return set_error("unterminated object");
      }
    }
    if (ch == '[') {
      ++pos_;
      value.kind = JsonValue::Kind::array;
      skip_space();
      if (pos_ != end_ && *pos_ == ']') {
        ++pos_;
        return true;
      }
      while (true) {
        skip_space();
        JsonValue item;
        if (!parse_value(item, depth + 1)) return false;
        value.array.push_back(std::move(item));
        skip_space();
        if (pos_ != end_ && *pos_ == ',') {
          ++pos_;
          continue;
        }
        if (pos_ != end_ && *pos_ == ']') {
          ++pos_;
          return true;
        }
        return set_error("unterminated array");
      }
    }
    if (ch == '"') {
      value.kind = JsonValue::Kind::string;
      return parse_string(value.text);
    }
    if (ch == 't') {
      value.kind = JsonValue::Kind::boolean;
      value.boolean = true;
      return literal("true");
    }
    if (ch == 'f') {
      value.kind = JsonValue::Kind::boolean;
      return literal("false");
    }
    if (ch == 'n') {
      value.kind = JsonValue::Kind::null_value;
      return literal("null");
    }
    if (ch == '-' || (ch >= '0' && ch <= '9')) return parse_number(value);
    return set_error("expected JSON value");
  }
};

inline bool parse_size(JsonValue const& v, std::size_t& out) {
  if (v.kind != JsonValue::Kind::number || v.text.empty()) return false;
  std::size_t r = 0;
  for (char ch : v.text) {
    if (ch < '0' || ch > '9') return false;
    std::size_t const d = static_cast<std::size_t>(ch - '0');
    if (r > (std::numeric_limits<std::size_t>::max() - d) / 10) return false;
    r = r * 10 + d;
  }
  out = r;
  return true;
}

inline std::size_t dtype_bytes(std::string const& dtype) {
  if (dtype == "BOOL" || dtype == "I8" || dtype == "U8") return 1;
  if (dtype == "F16" || dtype == "BF16" || dtype == "I16" || dtype == "U16") return 2;
  if (dtype == "F32" || dtype == "I32" || dtype == "U32") return 4;
  if (dtype == "F64" || dtype == "I64" || dtype == "U64") return 8;
  return 0;
}

inline bool element_count(std::vector<std::size_t> const& shape, std::size_t& n) {
  n = 1;
  for (std::size_t d : shape) {
    if (d != 0 && n > std::numeric_limits<std::size_t>::max() / d) return false;
    n *= d;
  }
  return true;
}

inline std::string json_quote(std::string const& s) {
  std::string out = "\"";
  for (unsigned char ch : s) {
    switch (ch) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\b': out += "\\b"; break;
      case '\f': out += "\\f"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      default:
        if (ch < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof(buf), "\\u%04x", ch);
          out += buf;
        } else {
          out += static_cast<char>(ch);
        }
    }
  }
  out += '"';
  return out;
}

}  // namespace detail

struct PonniTensorDescriptor {
  std::string name;
  std::string dtype;
  std::vector<std::size_t> shape;
  std::size_t data_begin = 0;
  std::size_t data_end = 0;
};

// A tensor a model expects; source_element_offset locates it in the caller's
// flattened storage when writing.
struct PonniTensorSpec {
  std::string name;
  std::string dtype;
  std::vector<std::size_t> shape;
  std::size_t source_element_offset = 0;
};

namespace detail {

// "ponni-tensor-schema-v1\n" + "name\tdtype\td0,d1,...\n" per tensor in name order.
inline std::string schema_fingerprint(std::vector<PonniTensorDescriptor> tensors) {
  std::sort(tensors.begin(), tensors.end(), [](auto const& l, auto const& r) { return l.name < r.name; });
  std::string text = "ponni-tensor-schema-v1\n";
  for (auto const& t : tensors) {
    text += t.name;
    text += '\t';
    text += t.dtype;
    text += '\t';
    for (std::size_t i = 0; i < t.shape.size(); i++) {
      if (i) text += ',';
      text += std::to_string(t.shape[i]);
    }
    text += '\n';
  }
  return ponni_fnv1a64_string(ponni_fnv1a64(reinterpret_cast<unsigned char const*>(text.data()), text.size()));
}

inline std::uint64_t read_u64_le(unsigned char const* p) {
  std::uint64_t v = 0;
  for (int i = 7; i >= 0; i--) v = (v << 8) | p[i];
  return v;
}

template <class T>
inline T read_le(unsigned char const* p) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "F32 or F64 only");
  using U = std::conditional_t<sizeof(T) == 4, std::uint32_t, std::uint64_t>;
  U u = 0;
  for (int i = static_cast<int>(sizeof(T)) - 1; i >= 0; i--) u = (u << 8) | p[i];
  T v;
  std::memcpy(&v, &u, sizeof(T));
  return v;
}

template <class T>
inline void append_le(std::vector<unsigned char>& out, T v) {
  using U = std::conditional_t<sizeof(T) == 4, std::uint32_t, std::uint64_t>;
  U u;
  std::memcpy(&u, &v, sizeof(T));
  for (std::size_t i = 0; i < sizeof(T); i++) out.push_back(static_cast<unsigned char>((u >> (8 * i)) & 0xff));
}

}  // namespace detail

class PonniFile {
 public:
  bool load(std::string const& path, std::string* error = nullptr) {
    bytes_.clear();
    tensors_.clear();
    metadata_.clear();
    data_offset_ = 0;
    std::ifstream in(path, std::ios::binary);
    if (!in) return fail("cannot open PONNI file: " + path, error);
    bytes_.assign(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
    if (in.bad()) return fail("cannot read PONNI file: " + path, error);
    return parse(error);
  }

  bool load_bytes(std::vector<unsigned char> bytes, std::string* error = nullptr) {
    bytes_ = std::move(bytes);
    tensors_.clear();
    metadata_.clear();
    data_offset_ = 0;
    return parse(error);
  }

  // Check the file against the tensors a model expects and its fingerprint.
  bool validate(std::vector<PonniTensorSpec> const& expected, std::string const& model_fingerprint,
                std::string* error = nullptr) const {
    auto const* fp = metadata("ponni.model_fingerprint");
    if (fp == nullptr || *fp != model_fingerprint) return fail("PONNI model fingerprint does not match this model", error);
    if (expected.size() != tensors_.size()) return fail("PONNI tensor count does not match this model", error);
    for (auto const& spec : expected) {
      auto const* t = find(spec.name);
      if (t == nullptr) return fail("PONNI file is missing tensor " + spec.name, error);
      if (t->dtype != spec.dtype) return fail("PONNI tensor dtype mismatch for " + spec.name, error);
      if (t->shape != spec.shape) return fail("PONNI tensor shape mismatch for " + spec.name, error);
    }
    return true;
  }

  PonniTensorDescriptor const* find(std::string const& name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
  }
  std::string const* metadata(std::string const& key) const {
    auto it = metadata_.find(key);
    return it == metadata_.end() ? nullptr : &it->second;
  }
  unsigned char const* tensor_data(PonniTensorDescriptor const& t) const {
    return bytes_.data() + data_offset_ + t.data_begin;
  }
  std::size_t tensor_count() const { return tensors_.size(); }

 private:
  std::vector<unsigned char> bytes_;
  std::size_t data_offset_ = 0;
  std::map<std::string, std::string> metadata_;
  std::map<std::string, PonniTensorDescriptor> tensors_;

  static bool fail(std::string const& message, std::string* error) {
    if (error) *error = message;
    return false;
  }

  bool parse(std::string* error) {
    using detail::JsonValue;
    if (bytes_.size() < 10) return fail("PONNI file is shorter than a Safetensors header", error);
    std::uint64_t const header = detail::read_u64_le(bytes_.data());
    if (header < 2 || header > 100u * 1024u * 1024u || header > bytes_.size() - 8)
      return fail("PONNI file has an invalid Safetensors header size", error);
    data_offset_ = 8 + static_cast<std::size_t>(header);
    JsonValue root;
    std::string perr;
    detail::JsonParser parser(reinterpret_cast<char const*>(bytes_.data() + 8), static_cast<std::size_t>(header));
    if (!parser.parse(root, perr)) return fail("invalid Safetensors JSON: " + perr, error);
    if (root.kind != JsonValue::Kind::object) return fail("Safetensors header root must be an object", error);
    std::size_t const payload = bytes_.size() - data_offset_;
    for (auto const& [name, value] : root.object) {
      if (name == "__metadata__") {
        if (value.kind != JsonValue::Kind::object) return fail("Safetensors metadata must be an object", error);
        for (auto const& [key, item] : value.object) {
          if (item.kind != JsonValue::Kind::string) return fail("Safetensors metadata values must be strings", error);
          metadata_.emplace(key, item.text);
        }
        continue;
      }
      if (value.kind != JsonValue::Kind::object)
        return fail("Safetensors tensor descriptor for " + name + " must be an object", error);
      auto const* dtype = value.find("dtype");
      auto const* shape = value.find("shape");
      auto const* offsets = value.find("data_offsets");
      if (!dtype || !shape || !offsets || dtype->kind != JsonValue::Kind::string ||
          shape->kind != JsonValue::Kind::array || offsets->kind != JsonValue::Kind::array ||
          offsets->array.size() != 2)
        return fail("incomplete Safetensors descriptor for " + name, error);
      PonniTensorDescriptor t;
      t.name = name;
      t.dtype = dtype->text;
      for (auto const& d : shape->array) {
        std::size_t v = 0;
        if (!detail::parse_size(d, v)) return fail("invalid Safetensors shape for " + name, error);
        t.shape.push_back(v);
      }
      if (!detail::parse_size(offsets->array[0], t.data_begin) || !detail::parse_size(offsets->array[1], t.data_end))
        return fail("invalid Safetensors offsets for " + name, error);
      std::size_t const es = detail::dtype_bytes(t.dtype);
      std::size_t n = 0;
      if (es == 0 || !detail::element_count(t.shape, n) || n > std::numeric_limits<std::size_t>::max() / es ||
          t.data_begin > t.data_end || t.data_end > payload || t.data_end - t.data_begin != n * es)
        return fail("Safetensors dtype, shape, and byte length disagree for " + name, error);
      tensors_.emplace(name, std::move(t));
    }
    if (metadata_.empty()) return fail("PONNI file has no Safetensors metadata", error);
    auto const* version = metadata("ponni.profile_version");
    auto const* model = metadata("ponni.model_fingerprint");
    auto const* schema = metadata("ponni.schema_fingerprint");
    auto const* checksum = metadata("ponni.payload_checksum_fnv1a64");
    if (!version || !model || !schema || !checksum) return fail("PONNI Safetensors metadata is incomplete", error);
    if (*version != "1") return fail("unsupported PONNI profile version " + *version, error);
    std::vector<PonniTensorDescriptor> physical;
    for (auto const& kv : tensors_) physical.push_back(kv.second);
    std::sort(physical.begin(), physical.end(), [](auto const& l, auto const& r) {
      return l.data_begin != r.data_begin ? l.data_begin < r.data_begin : l.data_end < r.data_end;
    });
    std::size_t cursor = 0;
    for (auto const& t : physical) {
      if (t.data_begin != cursor) return fail("Safetensors payload has a hole or overlap before " + t.name, error);
      cursor = t.data_end;
    }
    if (cursor != payload) return fail("Safetensors payload contains unindexed trailing bytes", error);
    if (*schema != detail::schema_fingerprint(physical))
      return fail("PONNI tensor-schema fingerprint does not match the Safetensors descriptors", error);
    std::string const actual = ponni_fnv1a64_string(ponni_fnv1a64(bytes_.data() + data_offset_, payload));
    if (*checksum != actual) return fail("PONNI payload checksum mismatch", error);
    return true;
  }
};

// Serialize `specs` (gathered from `source` at each spec's element offset)
// into a .ponni file; tensors are written in name order.
template <class Scalar>
inline bool write_ponni_file(std::string const& path, std::vector<PonniTensorSpec> specs,
                             std::string const& model_fingerprint, Scalar const* source, std::string* error = nullptr,
                             std::string const& target = "ponni", std::string const& source_framework = "ponni-cpp") {
  static_assert(std::is_same_v<Scalar, float> || std::is_same_v<Scalar, double>, "F32 or F64 payloads");
  auto fail = [&](std::string const& m) {
    if (error) *error = m;
    return false;
  };
  std::string const dtype = std::is_same_v<Scalar, double> ? "F64" : "F32";
  std::sort(specs.begin(), specs.end(), [](auto const& l, auto const& r) { return l.name < r.name; });
  std::vector<unsigned char> payload;
  std::vector<PonniTensorDescriptor> tensors;
  for (auto const& s : specs) {
    if (s.dtype != dtype) return fail("PONNI tensor dtype does not match the supplied scalar type");
    std::size_t n = 0;
    if (!detail::element_count(s.shape, n)) return fail("PONNI tensor shape overflows size_t");
    PonniTensorDescriptor t{s.name, s.dtype, s.shape, payload.size(), 0};
    for (std::size_t i = 0; i < n; i++) detail::append_le(payload, source[s.source_element_offset + i]);
    t.data_end = payload.size();
    tensors.push_back(std::move(t));
  }
  std::string header = "{\"__metadata__\":{\"ponni.profile_version\":\"1\",";
  header += "\"ponni.model_fingerprint\":" + detail::json_quote(model_fingerprint) + ",";
  header += "\"ponni.schema_fingerprint\":" + detail::json_quote(detail::schema_fingerprint(tensors)) + ",";
  header += "\"ponni.payload_checksum_fnv1a64\":" +
            detail::json_quote(ponni_fnv1a64_string(ponni_fnv1a64(payload.data(), payload.size()))) + ",";
  header += "\"ponni.source_framework\":" + detail::json_quote(source_framework) + ",";
  header += "\"ponni.target\":" + detail::json_quote(target) + "}";
  for (auto const& t : tensors) {
    header += "," + detail::json_quote(t.name) + ":{\"dtype\":" + detail::json_quote(t.dtype) + ",\"shape\":[";
    for (std::size_t i = 0; i < t.shape.size(); i++) {
      if (i) header += ",";
      header += std::to_string(t.shape[i]);
    }
    header += "],\"data_offsets\":[" + std::to_string(t.data_begin) + "," + std::to_string(t.data_end) + "]}";
  }
  header += "}";
  header.append((8 - header.size() % 8) % 8, ' ');
  std::vector<unsigned char> bytes;
  std::uint64_t const n = header.size();
  for (int i = 0; i < 8; i++) bytes.push_back(static_cast<unsigned char>((n >> (8 * i)) & 0xff));
  bytes.insert(bytes.end(), header.begin(), header.end());
  bytes.insert(bytes.end(), payload.begin(), payload.end());
  std::ofstream out(path, std::ios::binary | std::ios::trunc);
  if (!out) return fail("cannot open PONNI output file: " + path);
  out.write(reinterpret_cast<char const*>(bytes.data()), static_cast<std::streamsize>(bytes.size()));
  if (!out) return fail("cannot write PONNI output file: " + path);
  return true;
}

}  // namespace ponni
