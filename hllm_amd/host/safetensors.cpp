#include "safetensors.hpp"

#include <algorithm>
#include <fstream>
#include <limits>

#include "json.hpp"

namespace hllm_rocm::runtime {

std::size_t data_type_bytes(DataType d) noexcept {
  switch (d) {
    case DataType::kBool: case DataType::kU8: case DataType::kI8: return 1;
    case DataType::kI16: case DataType::kU16: case DataType::kF16: case DataType::kBF16: return 2;
    case DataType::kI32: case DataType::kU32: case DataType::kF32: return 4;
    case DataType::kI64: case DataType::kU64: case DataType::kF64: return 8;
  }
  return 0;
}

namespace {

constexpr std::size_t kHeaderLimit = 128u << 20;

std::string in_quotes(std::string_view s) { return "'" + std::string(s) + "'"; }

DataType dtype_of(const std::string& text, const std::string& name) {
  static const std::pair<const char*, DataType> kNames[] = {
      {"BOOL", DataType::kBool}, {"U8", DataType::kU8},     {"I8", DataType::kI8},   {"I16", DataType::kI16},
      {"U16", DataType::kU16},   {"I32", DataType::kI32},   {"U32", DataType::kU32}, {"I64", DataType::kI64},
      {"U64", DataType::kU64},   {"F16", DataType::kF16},   {"BF16", DataType::kBF16}, {"F32", DataType::kF32},
      {"F64", DataType::kF64}};
  for (const auto& [n, d] : kNames)
    if (text == n) return d;
  throw SafetensorsError("tensor " + in_quotes(name) + " has unsupported dtype " + in_quotes(text));
}

std::size_t size_field(const json::Value& v, const char* field, const std::string& name) {
  if (!v.is_number() || !v.is_unsigned) throw SafetensorsError("tensor " + in_quotes(name) + " has invalid " + field);
  if (v.unsigned_value > std::numeric_limits<std::size_t>::max())
    throw SafetensorsError("tensor " + in_quotes(name) + " has oversized " + field);
  return static_cast<std::size_t>(v.unsigned_value);
}

TensorMetadata record(const std::string& name, const json::Value& entry) {
  const json::Value* dtype = entry.find("dtype");
  const json::Value* shape = entry.find("shape");
  const json::Value* offsets = entry.find("data_offsets");
  if (!entry.is_object() || !dtype || !shape || !offsets)
    throw SafetensorsError("tensor " + in_quotes(name) + " has invalid metadata");
  if (!dtype->is_string() || !shape->is_array() || !offsets->is_array() || offsets->array.size() != 2)
    throw SafetensorsError("tensor " + in_quotes(name) + " has invalid metadata types");
  TensorMetadata t{name, dtype_of(dtype->string, name), {}, 0, 0};
  for (const json::Value& d : shape->array) t.shape.push_back(size_field(d, "shape", name));
  const std::size_t begin = size_field(offsets->array[0], "data offset", name);
  const std::size_t end = size_field(offsets->array[1], "data offset", name);
  if (end < begin) throw SafetensorsError("tensor " + in_quotes(name) + " has a reversed data range");
  std::size_t bytes = data_type_bytes(t.dtype);
  for (std::size_t d : t.shape) {
    if (d != 0 && bytes > std::numeric_limits<std::size_t>::max() / d)
      throw SafetensorsError("tensor " + in_quotes(name) + " byte length overflows");
    bytes *= d;
  }
  if (end - begin != bytes)
    throw SafetensorsError("tensor " + in_quotes(name) + " byte length is " + std::to_string(end - begin) +
                           ", expected " + std::to_string(bytes));
  t.data_offset = begin;
  t.byte_length = bytes;
  return t;
}

}  // namespace

SafetensorsFile::SafetensorsFile(std::filesystem::path path) : path_(std::move(path)) {
  std::error_code ec;
  const auto size = std::filesystem::file_size(path_, ec);
  if (ec) throw SafetensorsError("cannot determine Safetensors file size: " + path_.string());
  file_size_ = static_cast<std::size_t>(size);
  if (file_size_ < 8) throw SafetensorsError("Safetensors file is shorter than its header prefix");
  std::ifstream in(path_, std::ios::binary);
  if (!in) throw SafetensorsError("cannot open Safetensors file: " + path_.string());
  unsigned char prefix[8];
  in.read(reinterpret_cast<char*>(prefix), 8);
  std::uint64_t length = 0;
  for (int b = 7; b >= 0; --b) length = (length << 8) | prefix[b];
  if (length == 0 || length > kHeaderLimit) throw SafetensorsError("Safetensors file has an invalid header length");
  if (length > file_size_ - 8) throw SafetensorsError("Safetensors header extends beyond the file");
  header_size_ = 8 + static_cast<std::size_t>(length);
  std::string header(static_cast<std::size_t>(length), '\0');
  in.read(header.data(), static_cast<std::streamsize>(length));
  if (!in) throw SafetensorsError("cannot read complete Safetensors header");
  json::Value doc;
  try {
    doc = json::parse(header);
  } catch (const json::ParseError& e) {
    throw SafetensorsError(std::string("Safetensors file contains invalid JSON: ") + e.what());
  }
  if (!doc.is_object()) throw SafetensorsError("Safetensors header must be a JSON object");
  for (const auto& [name, entry] : doc.object)
    if (name != "__metadata__") tensors_.push_back(record(name, entry));
  if (tensors_.empty()) throw SafetensorsError("Safetensors file does not contain tensors");
  std::sort(tensors_.begin(), tensors_.end(), [](const auto& a, const auto& b) { return a.name < b.name; });
  for (std::size_t i = 1; i < tensors_.size(); ++i)
    if (tensors_[i].name == tensors_[i - 1].name)
      throw SafetensorsError("tensor " + in_quotes(tensors_[i].name) + " appears twice");
  std::vector<const TensorMetadata*> by_offset;
  for (const auto& t : tensors_) by_offset.push_back(&t);
  std::sort(by_offset.begin(), by_offset.end(),
            [](const TensorMetadata* a, const TensorMetadata* b) { return a->data_offset < b->data_offset; });
  const std::size_t data = file_size_ - header_size_;
  std::size_t covered = 0;
  for (const TensorMetadata* t : by_offset) {
    if (t->data_offset < covered) throw SafetensorsError("tensor " + in_quotes(t->name) + " overlaps an earlier tensor");
    if (t->data_offset > data || t->byte_length > data - t->data_offset)
      throw SafetensorsError("tensor " + in_quotes(t->name) + " extends beyond the data section");
    covered = t->data_offset + t->byte_length;
  }
}

const TensorMetadata& SafetensorsFile::tensor(std::string_view name) const {
  const auto it = std::lower_bound(tensors_.begin(), tensors_.end(), name,
                                   [](const TensorMetadata& t, std::string_view n) { return t.name < n; });
  if (it == tensors_.end() || it->name != name)
    throw SafetensorsError("tensor " + in_quotes(name) + " is not present in " + path_.string());
  return *it;
}

void SafetensorsFile::read(const TensorMetadata& t, std::size_t offset, void* out, std::size_t length) const {
  if (offset > t.byte_length || length > t.byte_length - offset)
    throw SafetensorsError("read past the end of tensor " + in_quotes(t.name));
  if (length == 0) return;
  std::ifstream in(path_, std::ios::binary);
  if (!in) throw SafetensorsError("cannot reopen Safetensors file: " + path_.string());
  in.seekg(static_cast<std::streamoff>(header_size_ + t.data_offset + offset));
  in.read(static_cast<char*>(out), static_cast<std::streamsize>(length));
  if (!in) throw SafetensorsError("cannot read tensor " + in_quotes(t.name));
}

}  // namespace hllm_rocm::runtime
