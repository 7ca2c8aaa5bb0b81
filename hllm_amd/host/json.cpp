#include "json.hpp"

#include <cerrno>
#include <cstdlib>
#include <limits>

namespace hllm_rocm::json {

const Value* Value::find(std::string_view key) const {
  const Value* hit = nullptr;
  if (kind == Kind::kObject)
    for (const auto& [k, v] : object)
      if (k == key) hit = &v;
  return hit;
}

namespace {

class Reader {
 public:
  explicit Reader(std::string_view text) : s_(text) {}

  Value document() {
    Value v = value(0);
    skip_space();
    if (i_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  static constexpr int kMaxDepth = 256;

  [[noreturn]] void fail(const char* what) const {
    throw ParseError(std::string("JSON ") + what + " at offset " + std::to_string(i_));
  }
  void skip_space() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
  }
  char peek() {
    skip_space();
    if (i_ >= s_.size()) fail("ends early");
    return s_[i_];
  }
  void expect(char c) {
    if (peek() != c) fail("has an unexpected character");
    ++i_;
  }
  bool literal(std::string_view word) {
    if (s_.substr(i_, word.size()) != word) return false;
    i_ += word.size();
    return true;
  }

  Value value(int depth) {
    if (depth > kMaxDepth) fail("nests too deeply");
    Value v;
    const char c = peek();
    if (c == '{') {
      v.kind = Value::Kind::kObject;
      ++i_;
      if (peek() == '}') {
        ++i_;
        return v;
      }
      while (true) {
        if (peek() != '"') fail("expects a member name");
        std::string key = string();
        expect(':');
        v.object.emplace_back(std::move(key), value(depth + 1));
        const char d = peek();
        ++i_;
        if (d == '}') return v;
        if (d != ',') fail("expects ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = Value::Kind::kArray;
      ++i_;
      if (peek() == ']') {
        ++i_;
        return v;
      }
      while (true) {
        v.array.push_back(value(depth + 1));
        const char d = peek();
        ++i_;
        if (d == ']') return v;
        if (d != ',') fail("expects ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Value::Kind::kString;
      v.string = string();
      return v;
    }
    if (literal("true")) {
      v.kind = Value::Kind::kBool;
      v.boolean = true;
      return v;
    }
    if (literal("false")) {
      v.kind = Value::Kind::kBool;
      return v;
    }
    if (literal("null")) return v;
    return number();
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
  std::uint32_t hex4() {
    if (i_ + 4 > s_.size()) fail("has a short \\u escape");
    std::uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char h = s_[i_++];
      v <<= 4;
      if (h >= '0' && h <= '9') v |= h - '0';
      else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
      else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
      else fail("has a bad \\u escape");
    }
    return v;
  }
  std::string string() {
    ++i_;  // opening quote
    std::string out;
    while (true) {
      if (i_ >= s_.size()) fail("has an unterminated string");
      const unsigned char c = static_cast<unsigned char>(s_[i_++]);
      if (c == '"') return out;
      if (c < 0x20) fail("has a control character in a string");
      if (c != '\\') {
        out += static_cast<char>(c);
        continue;
      }
      if (i_ >= s_.size()) fail("has an unterminated escape");
      const char e = s_[i_++];
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
          std::uint32_t cp = hex4();
          if (cp >= 0xd800 && cp <= 0xdbff) {
            if (i_ + 2 > s_.size() || s_[i_] != '\\' || s_[i_ + 1] != 'u') fail("has a lone surrogate");
            i_ += 2;
            const std::uint32_t lo = hex4();
            if (lo < 0xdc00 || lo > 0xdfff) fail("has a bad surrogate pair");
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          } else if (cp >= 0xdc00 && cp <= 0xdfff) {
            fail("has a lone surrogate");
          }
          append_utf8(out, cp);
          break;
        }
        default: fail("has an unknown escape");
      }
    }
  }
  Value number() {
    const std::size_t start = i_;
    if (i_ < s_.size() && s_[i_] == '-') ++i_;
    auto digits = [&] {
      const std::size_t d0 = i_;
      while (i_ < s_.size() && s_[i_] >= '0' && s_[i_] <= '9') ++i_;
      return i_ - d0;
    };
    if (i_ >= s_.size() || s_[i_] < '0' || s_[i_] > '9') fail("has an invalid value");
    if (s_[i_] == '0') ++i_;
    else digits();
    bool integer = true;
    if (i_ < s_.size() && s_[i_] == '.') {
      ++i_;
      if (digits() == 0) fail("has a malformed fraction");
      integer = false;
    }
    if (i_ < s_.size() && (s_[i_] == 'e' || s_[i_] == 'E')) {
      ++i_;
      if (i_ < s_.size() && (s_[i_] == '+' || s_[i_] == '-')) ++i_;
      if (digits() == 0) fail("has a malformed exponent");
      integer = false;
    }
    const std::string text(s_.substr(start, i_ - start));
    Value v;
    v.kind = Value::Kind::kNumber;
    v.number = std::strtod(text.c_str(), nullptr);
    if (integer) {
      v.is_integer = true;
      errno = 0;
      if (text[0] == '-') {
        const long long x = std::strtoll(text.c_str(), nullptr, 10);
        if (errno == 0) v.signed_value = x;
        else v.is_integer = false;
      } else {
        const unsigned long long x = std::strtoull(text.c_str(), nullptr, 10);
        if (errno == 0) {
          v.is_unsigned = true;
          v.unsigned_value = x;
          v.signed_value = x <= static_cast<unsigned long long>(std::numeric_limits<std::int64_t>::max())
                               ? static_cast<std::int64_t>(x)
                               : 0;
        } else {
          v.is_integer = false;
        }
      }
    }
    return v;
  }

  std::string_view s_;
  std::size_t i_{0};
};

}  // namespace

Value parse(std::string_view text) { return Reader(text).document(); }

}  // namespace hllm_rocm::json
