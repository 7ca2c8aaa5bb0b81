// Safetensors checkpoint files (cpp/include/hllm/runtime/safetensors.hpp,
// cpp/src/safetensors.cpp): an 8-byte little-endian header length, a JSON header of
// tensor records {dtype, shape, data_offsets}, then the data section. Every record is
// checked (dtype, shape x element size == byte range, ranges inside the data section and
// not overlapping) before any payload is read. Malformed files are INCOMPATIBLE_WORKER.
#pragma once

#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <string>
#include <string_view>
#include <vector>

#include "runtime.hpp"

namespace hllm_rocm::runtime {

enum class DataType : std::uint8_t { kBool, kU8, kI8, kI16, kU16, kI32, kU32, kI64, kU64, kF16, kBF16, kF32, kF64 };
std::size_t data_type_bytes(DataType dtype) noexcept;

struct TensorMetadata {
  std::string name;
  DataType dtype;
  std::vector<std::size_t> shape;
  std::size_t data_offset;  // within the data section
  std::size_t byte_length;
};

class SafetensorsError : public Error {
 public:
  explicit SafetensorsError(const std::string& message) : Error(ErrorCode::kIncompatibleWorker, message) {}
};

class SafetensorsFile final {
 public:
  explicit SafetensorsFile(std::filesystem::path path);
  const std::filesystem::path& path() const noexcept { return path_; }
  std::size_t file_size() const noexcept { return file_size_; }
  std::size_t header_size() const noexcept { return header_size_; }  // prefix + JSON
  const std::vector<TensorMetadata>& tensors() const noexcept { return tensors_; }  // by name
  const TensorMetadata& tensor(std::string_view name) const;
  // Reads `length` bytes of a tensor's payload starting at byte `offset` of the tensor.
  void read(const TensorMetadata& tensor, std::size_t offset, void* out, std::size_t length) const;

 private:
  std::filesystem::path path_;
  std::size_t file_size_{0}, header_size_{0};
  std::vector<TensorMetadata> tensors_;
};

}  // namespace hllm_rocm::runtime
