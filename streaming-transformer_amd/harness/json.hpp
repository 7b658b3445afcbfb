// A small JSON value with a parser and a writer, enough for the benchmark driver: checkpoint
// and fixture manifests, configs, reset lists, the runtime's info() report and the result
// file. Objects keep their keys sorted (as the reference driver's nlohmann::json does), so
// two objects compare equal when they hold the same members. Numbers keep their source text
// when they are integers, so 64-bit counts and hashes of counts survive a round trip.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace stbench {

class Json {
 public:
  enum class Type { Null, Bool, Number, String, Array, Object };

  Json() = default;
  Json(std::nullptr_t) {}
  Json(bool b) : type_(Type::Bool), bool_(b) {}
  Json(double v) : type_(Type::Number), num_(v) {}
  Json(float v) : Json((double)v) {}
  Json(int v) : Json((long long)v) {}
  Json(long v) : Json((long long)v) {}
  Json(long long v) : type_(Type::Number), num_((double)v), int_(true), i_(v) {}
  Json(unsigned v) : Json((unsigned long long)v) {}
  Json(unsigned long v) : Json((unsigned long long)v) {}
  Json(unsigned long long v) : type_(Type::Number), num_((double)v), int_(true), unsigned_(true), u_(v) {}
  Json(const char* s) : type_(Type::String), str_(s) {}
  Json(std::string s) : type_(Type::String), str_(std::move(s)) {}

  static Json array() {
    Json j;
    j.type_ = Type::Array;
    return j;
  }
  static Json object() {
    Json j;
    j.type_ = Type::Object;
    return j;
  }
  static Json parse(const std::string& text);

  Type type() const { return type_; }
  bool is_null() const { return type_ == Type::Null; }
  bool is_object() const { return type_ == Type::Object; }
  bool is_array() const { return type_ == Type::Array; }
  bool is_string() const { return type_ == Type::String; }
  bool is_number() const { return type_ == Type::Number; }

  // Object access. operator[] inserts (turning null into an object); at() throws.
  Json& operator[](const std::string& key) {
    if (type_ == Type::Null) type_ = Type::Object;
    if (type_ != Type::Object) throw std::runtime_error("JSON value is not an object");
    return obj_[key];
  }
  const Json& at(const std::string& key) const {
    if (type_ != Type::Object) throw std::runtime_error("JSON value is not an object");
    auto it = obj_.find(key);
    if (it == obj_.end()) throw std::runtime_error("Missing JSON key: " + key);
    return it->second;
  }
  bool contains(const std::string& key) const { return type_ == Type::Object && obj_.count(key) != 0; }
  const std::map<std::string, Json>& items() const { return obj_; }

  // Array access.
  void push_back(Json v) {
    if (type_ == Type::Null) type_ = Type::Array;
    if (type_ != Type::Array) throw std::runtime_error("JSON value is not an array");
    arr_.push_back(std::move(v));
  }
  const Json& at(size_t i) const {
    if (type_ != Type::Array || i >= arr_.size()) throw std::runtime_error("JSON array index out of range");
    return arr_[i];
  }
  const std::vector<Json>& elements() const { return arr_; }
  size_t size() const { return type_ == Type::Array ? arr_.size() : type_ == Type::Object ? obj_.size() : 0; }

  // Scalars.
  double number() const {
    if (type_ != Type::Number) throw std::runtime_error("JSON value is not a number");
    return num_;
  }
  long long integer() const {
    if (type_ != Type::Number) throw std::runtime_error("JSON value is not a number");
    if (int_) return unsigned_ ? (long long)u_ : i_;
    if (num_ != std::floor(num_)) throw std::runtime_error("JSON number is not an integer");
    return (long long)num_;
  }
  unsigned long long uinteger() const {
    if (type_ == Type::Number && int_ && unsigned_) return u_;
    long long v = integer();
    if (v < 0) throw std::runtime_error("JSON number is negative");
    return (unsigned long long)v;
  }
  bool boolean() const {
    if (type_ != Type::Bool) throw std::runtime_error("JSON value is not a boolean");
    return bool_;
  }
  const std::string& str() const {
    if (type_ != Type::String) throw std::runtime_error("JSON value is not a string");
    return str_;
  }

  bool operator==(const Json& o) const {
    if (type_ != o.type_) return false;
    switch (type_) {
      case Type::Null: return true;
      case Type::Bool: return bool_ == o.bool_;
      case Type::Number:
        if (int_ && o.int_) return unsigned_ == o.unsigned_ ? (unsigned_ ? u_ == o.u_ : i_ == o.i_) : num_ == o.num_;
        return num_ == o.num_;
      case Type::String: return str_ == o.str_;
      case Type::Array: return arr_ == o.arr_;
      case Type::Object: return obj_ == o.obj_;
    }
    return false;
  }
  bool operator!=(const Json& o) const { return !(*this == o); }

  std::string dump(int indent = -1) const {
    std::string out;
    write(out, indent, 0);
    return out;
  }

 private:
  void write(std::string& out, int indent, int depth) const;
  static void write_string(std::string& out, const std::string& s);

  Type type_ = Type::Null;
  bool bool_ = false;
  double num_ = 0;
  bool int_ = false, unsigned_ = false;
  long long i_ = 0;
  unsigned long long u_ = 0;
  std::string str_;
  std::vector<Json> arr_;
  std::map<std::string, Json> obj_;
};

inline void Json::write_string(std::string& out, const std::string& s) {
  out += '"';
  for (unsigned char ch : s) {
    switch (ch) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      case '\b': out += "\\b"; break;
      case '\f': out += "\\f"; break;
      default:
        if (ch < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof buf, "\\u%04x", ch);
          out += buf;
        } else {
          out += (char)ch;
        }
    }
  }
  out += '"';
}

inline void Json::write(std::string& out, int indent, int depth) const {
  auto newline = [&](int d) {
    if (indent < 0) return;
    out += '\n';
    out.append((size_t)(indent * d), ' ');
  };
  switch (type_) {
    case Type::Null: out += "null"; break;
    case Type::Bool: out += bool_ ? "true" : "false"; break;
    case Type::Number: {
      if (int_) {
        out += unsigned_ ? std::to_string(u_) : std::to_string(i_);
      } else if (!std::isfinite(num_)) {
        out += "null";  // JSON has no inf / nan
      } else {
        char buf[32];
        std::snprintf(buf, sizeof buf, "%.17g", num_);
        out += buf;
      }
      break;
    }
    case Type::String: write_string(out, str_); break;
    case Type::Array: {
      if (arr_.empty()) {
        out += "[]";
        break;
      }
      out += '[';
      for (size_t i = 0; i < arr_.size(); i++) {
        if (i) out += ',';
        newline(depth + 1);
        arr_[i].write(out, indent, depth + 1);
      }
      newline(depth);
      out += ']';
      break;
    }
    case Type::Object: {
      if (obj_.empty()) {
        out += "{}";
        break;
      }
      out += '{';
      bool first = true;
      for (const auto& [k, v] : obj_) {
        if (!first) out += ',';
        first = false;
        newline(depth + 1);
        write_string(out, k);
        out += indent < 0 ? ":" : ": ";
        v.write(out, indent, depth + 1);
      }
      newline(depth);
      out += '}';
      break;
    }
  }
}

namespace detail {
struct Parser {
  const std::string& s;
  size_t p = 0;
  [[noreturn]] void fail(const char* what) const {
    throw std::runtime_error(std::string("JSON parse error: ") + what + " at offset " + std::to_string(p));
  }
  void ws() {
    while (p < s.size() && (s[p] == ' ' || s[p] == '\n' || s[p] == '\r' || s[p] == '\t')) p++;
  }
  bool take(char c) {
    ws();
    if (p < s.size() && s[p] == c) {
      p++;
      return true;
    }
    return false;
  }
  void expect(char c) {
    if (!take(c)) fail("unexpected character");
  }
  static void utf8(std::string& out, unsigned cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += (char)(0xE0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    } else {
      out += (char)(0xF0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3F));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    }
  }
  unsigned hex4() {
    if (p + 4 > s.size()) fail("short \\u escape");
    unsigned v = 0;
    for (int i = 0; i < 4; i++) {
      char c = s[p++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
      else fail("bad \\u escape");
    }
    return v;
  }
  std::string string() {
    expect('"');
    std::string out;
    while (true) {
      if (p >= s.size()) fail("unterminated string");
      char c = s[p++];
      if (c == '"') break;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (p >= s.size()) fail("unterminated escape");
      char e = s[p++];
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          unsigned cp = hex4();
          if (cp >= 0xDC00 && cp < 0xE000) fail("unpaired low surrogate");
          if (cp >= 0xD800 && cp < 0xDC00) {
            // A high surrogate must be followed by a \u escape holding a low surrogate.
            if (p + 6 > s.size() || s[p] != '\\' || s[p + 1] != 'u') fail("unpaired high surrogate");
            p += 2;
            const unsigned lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) fail("high surrogate without a low surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(out, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
    return out;
  }
  // A number in the JSON grammar: -?(0|[1-9][0-9]*)(.[0-9]+)?([eE][+-]?[0-9]+)?. The whole
  // token is checked against the grammar before it is converted, so "12-3", "1+" or "01" are
  // errors, not a prefix that parses.
  Json number() {
    const size_t start = p;
    auto digits = [&]() {
      const size_t d0 = p;
      while (p < s.size() && s[p] >= '0' && s[p] <= '9') p++;
      return p - d0;
    };
    if (p < s.size() && s[p] == '-') p++;
    if (p < s.size() && s[p] == '0') {
      p++;
    } else if (digits() == 0) {
      fail("bad number");
    }
    bool integral = true;
    if (p < s.size() && s[p] == '.') {
      p++;
      integral = false;
      if (digits() == 0) fail("bad number");
    }
    if (p < s.size() && (s[p] == 'e' || s[p] == 'E')) {
      p++;
      integral = false;
      if (p < s.size() && (s[p] == '+' || s[p] == '-')) p++;
      if (digits() == 0) fail("bad number");
    }
    const std::string t = s.substr(start, p - start);
    try {
      size_t used = 0;
      if (integral) {
        if (t[0] == '-') {
          const long long v = std::stoll(t, &used);
          if (used == t.size()) return Json(v);
        } else {
          const unsigned long long v = std::stoull(t, &used);
          if (used == t.size()) return Json(v);
        }
        fail("bad number");
      }
      return Json(real(t));
    } catch (const std::out_of_range&) {
      return Json(real(t));  // an integer beyond 64 bits keeps its double value
    } catch (const std::invalid_argument&) {
      fail("bad number");
    }
  }
  // A grammar-checked token as a double: underflow gives the nearest subnormal or zero, a
  // magnitude beyond the double range is an error.
  double real(const std::string& t) const {
    char* end = nullptr;
    const double v = std::strtod(t.c_str(), &end);
    if (end != t.c_str() + t.size()) fail("bad number");
    if (std::isinf(v)) fail("number out of range");
    return v;
  }
  static constexpr int kMaxDepth = 256;  // nesting limit: deeper documents are rejected
  int depth = 0;
  struct Nest {
    Parser& parser;
    explicit Nest(Parser& q) : parser(q) {
      if (++parser.depth > kMaxDepth) parser.fail("nesting too deep");
    }
    ~Nest() { parser.depth--; }
  };
  Json value() {
    ws();
    if (p >= s.size()) fail("unexpected end");
    char c = s[p];
    if (c == '{' || c == '[') {
      Nest nest(*this);
      return c == '{' ? object() : array();
    }
    return scalar(c);
  }
  Json object() {
    p++;
    Json o = Json::object();
    if (take('}')) return o;
    do {
      ws();
      std::string k = string();
      expect(':');
      o[k] = value();
    } while (take(','));
    expect('}');
    return o;
  }
  Json array() {
    p++;
    Json a = Json::array();
    if (take(']')) return a;
    do a.push_back(value());
    while (take(','));
    expect(']');
    return a;
  }
  Json scalar(char c) {
    if (c == '"') return Json(string());
    if (s.compare(p, 4, "true") == 0) {
      p += 4;
      return Json(true);
    }
    if (s.compare(p, 5, "false") == 0) {
      p += 5;
      return Json(false);
    }
    if (s.compare(p, 4, "null") == 0) {
      p += 4;
      return Json();
    }
    return number();
  }
};
}  // namespace detail

inline Json Json::parse(const std::string& text) {
  detail::Parser parser{text};
  Json v = parser.value();
  parser.ws();
  if (parser.p != text.size()) parser.fail("trailing characters");
  return v;
}

}  // namespace stbench
