#include "safetensors.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>

#include "json.hpp"

namespace hllm_rocm::runtime {

namespace {

// Largest JSON header accepted: the reference reader's limit, so both accept the same files.
constexpr std::size_t kHeaderLimit = std::size_t{128} << 20;

struct DTypeName {
  const char* name;
  DataType type;
};
constexpr DTypeName kDTypes[] = {{"BOOL", DataType::kBool}, {"U8", DataType::kU8},     {"I8", DataType::kI8},
                                 {"I16", DataType::kI16},   {"U16", DataType::kU16},   {"I32", DataType::kI32},
                                 {"U32", DataType::kU32},   {"I64", DataType::kI64},   {"U64", DataType::kU64},
                                 {"F16", DataType::kF16},   {"BF16", DataType::kBF16}, {"F32", DataType::kF32},
                                 {"F64", DataType::kF64}};

[[noreturn]] void reject(const std::filesystem::path& path, const std::string& why) {
  throw SafetensorsError(path.filename().string() + ": " + why);
}

// One tensor record of the header, checked against the data section's size.
TensorMetadata record(const std::filesystem::path& path, const std::string& name, const json::Value& v,
                      std::size_t data_bytes) {
  const json::Value* dtype = v.find("dtype");
  const json::Value* shape = v.find("shape");
  const json::Value* offsets = v.find("data_offsets");
  if (!v.is_object() || !dtype || !dtype->is_string() || !shape || !shape->is_array() || !offsets ||
      !offsets->is_array() || offsets->array.size() != 2)
    reject(path, "record of '" + name + "' lacks dtype, shape or a data_offsets pair");
  TensorMetadata t{name, DataType::kU8, {}, 0, 0};
  const auto known = std::find_if(std::begin(kDTypes), std::end(kDTypes),
                                  [&](const DTypeName& d) { return dtype->string == d.name; });
  if (known == std::end(kDTypes)) reject(path, "'" + name + "' has element type '" + dtype->string + "'");
  t.dtype = known->type;
  std::size_t bytes = data_type_bytes(t.dtype);
  for (const json::Value& d : shape->array) {
    if (!d.is_number() || !d.is_unsigned) reject(path, "'" + name + "' has a dimension that is not a size");
    if (d.unsigned_value != 0 && bytes > SIZE_MAX / d.unsigned_value) reject(path, "'" + name + "' is too large");
    t.shape.push_back((std::size_t)d.unsigned_value);
    bytes *= (std::size_t)d.unsigned_value;
  }
  for (const json::Value& o : offsets->array)
    if (!o.is_number() || !o.is_unsigned) reject(path, "'" + name + "' has a data offset that is not a size");
  const std::uint64_t begin = offsets->array[0].unsigned_value, end = offsets->array[1].unsigned_value;
  if (end < begin) reject(path, "'" + name + "' has its data range reversed");
  if (end - begin != bytes) reject(path, "'" + name + "' spans " + std::to_string(end - begin) + " bytes, its shape " +
                                     std::to_string(bytes));
  if (end > data_bytes) reject(path, "'" + name + "' ends past the data section");
  t.data_offset = (std::size_t)begin;
  t.byte_length = bytes;
  return t;
}

}  // namespace

std::size_t data_type_bytes(DataType dtype) noexcept {
  switch (dtype) {
    case DataType::kBool:
    case DataType::kU8:
    case DataType::kI8: return 1;
    case DataType::kI16:
    case DataType::kU16:
    case DataType::kF16:
    case DataType::kBF16: return 2;
    case DataType::kI32:
    case DataType::kU32:
    case DataType::kF32: return 4;
    default: return 8;
  }
}

SafetensorsFile::SafetensorsFile(std::filesystem::path path) : path_(std::move(path)) {
  const int fd = ::open(path_.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) reject(path_, "cannot be opened");
  struct stat st {};
  if (::fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
    ::close(fd);
    reject(path_, "is not a readable regular file");
  }
  size_ = (std::size_t)st.st_size;
  if (size_ < 8) {
    ::close(fd);
    reject(path_, "is shorter than the 8-byte header length");
  }
  void* map = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (map == MAP_FAILED) reject(path_, "cannot be mapped");
  base_ = static_cast<const std::byte*>(map);
  try {
    std::uint64_t header = 0;
    for (int i = 7; i >= 0; --i) header = (header << 8) | std::to_integer<std::uint64_t>(base_[i]);
    if (header == 0 || header > kHeaderLimit || header > size_ - 8) reject(path_, "has an invalid header length");
    data_start_ = 8 + (std::size_t)header;
    json::Value doc;
    try {
      doc = json::parse(std::string_view(reinterpret_cast<const char*>(base_) + 8, (std::size_t)header));
    } catch (const json::ParseError& e) {
      reject(path_, std::string("header is not valid JSON: ") + e.what());
    }
    if (!doc.is_object()) reject(path_, "header is not a JSON object");
    const std::size_t data_bytes = size_ - data_start_;
    for (const auto& [name, value] : doc.object)
      if (name != "__metadata__") tensors_.push_back(record(path_, name, value, data_bytes));
    if (tensors_.empty()) reject(path_, "holds no tensors");
    // Byte ranges in file order must not overlap.
    std::vector<const TensorMetadata*> order;
    for (const TensorMetadata& t : tensors_) order.push_back(&t);
    std::sort(order.begin(), order.end(),
              [](const TensorMetadata* a, const TensorMetadata* b) { return a->data_offset < b->data_offset; });
    for (std::size_t i = 1; i < order.size(); ++i)
      if (order[i]->data_offset < order[i - 1]->data_offset + order[i - 1]->byte_length)
        reject(path_, "'" + order[i]->name + "' overlaps '" + order[i - 1]->name + "'");
    std::sort(tensors_.begin(), tensors_.end(),
              [](const TensorMetadata& a, const TensorMetadata& b) { return a.name < b.name; });
    for (std::size_t i = 1; i < tensors_.size(); ++i)
      if (tensors_[i].name == tensors_[i - 1].name) reject(path_, "names '" + tensors_[i].name + "' twice");
  } catch (...) {
    unmap();
    throw;
  }
}

SafetensorsFile::~SafetensorsFile() { unmap(); }

void SafetensorsFile::unmap() noexcept {
  if (base_) ::munmap(const_cast<std::byte*>(base_), size_);
  base_ = nullptr;
}

SafetensorsFile::SafetensorsFile(SafetensorsFile&& other) noexcept
    : path_(std::move(other.path_)),
      base_(std::exchange(other.base_, nullptr)),
      size_(other.size_),
      data_start_(other.data_start_),
      tensors_(std::move(other.tensors_)) {}

SafetensorsFile& SafetensorsFile::operator=(SafetensorsFile&& other) noexcept {
  if (this != &other) {
    unmap();
    path_ = std::move(other.path_);
    base_ = std::exchange(other.base_, nullptr);
    size_ = other.size_;
    data_start_ = other.data_start_;
    tensors_ = std::move(other.tensors_);
  }
  return *this;
}

const TensorMetadata& SafetensorsFile::tensor(std::string_view name) const {
  const auto it = std::lower_bound(tensors_.begin(), tensors_.end(), name,
                                   [](const TensorMetadata& t, std::string_view n) { return t.name < n; });
  if (it == tensors_.end() || it->name != name) reject(path_, "has no tensor '" + std::string(name) + "'");
  return *it;
}

std::span<const std::byte> SafetensorsFile::payload(const TensorMetadata& tensor) const {
  if (!base_) reject(path_, "is not mapped");
  return {base_ + data_start_ + tensor.data_offset, tensor.byte_length};
}

}  // namespace hllm_rocm::runtime
