// A small JSON reader for checkpoint metadata (Safetensors headers, model config files):
// RFC 8259 values into a tree, numbers kept as unsigned / signed / double as written.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace hllm_rocm::json {

class ParseError : public std::runtime_error {
 public:
  using std::runtime_error::runtime_error;
};

struct Value {
  enum class Kind { kNull, kBool, kNumber, kString, kArray, kObject };
  Kind kind{Kind::kNull};
  bool boolean{false};
  // Numbers: `is_unsigned` when written as a non-negative integer that fits 64 bits,
  // `is_integer` for any integer literal; `number` always holds the double value.
  bool is_unsigned{false}, is_integer{false};
  std::uint64_t unsigned_value{0};
  std::int64_t signed_value{0};
  double number{0.0};
  std::string string;
  std::vector<Value> array;
  std::vector<std::pair<std::string, Value>> object;  // in document order

  bool is_object() const { return kind == Kind::kObject; }
  bool is_array() const { return kind == Kind::kArray; }
  bool is_string() const { return kind == Kind::kString; }
  bool is_number() const { return kind == Kind::kNumber; }
  bool is_bool() const { return kind == Kind::kBool; }
  bool is_null() const { return kind == Kind::kNull; }
  // Object member or nullptr (the last one wins for duplicate keys, as most readers do).
  const Value* find(std::string_view key) const;
};

// Parses one complete document; throws ParseError on malformed input or trailing text.
Value parse(std::string_view text);

}  // namespace hllm_rocm::json
