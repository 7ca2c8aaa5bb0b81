// Safetensors checkpoint files, read through a read-only memory mapping. The format (an
// 8-byte little-endian header length, a JSON header of tensor records {dtype, shape,
// data_offsets}, then the data section) and its acceptance rules follow the reference
// reader (cpp/include/hllm/runtime/safetensors.hpp, cpp/src/safetensors.cpp): every record is
// checked before any payload is touched, and a file the reference rejects is rejected here
// (INCOMPATIBLE_WORKER). Payloads are exposed as views into the mapping, so the stage uploads
// them to the device without an intermediate host copy.
#pragma once

#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <span>
#include <string>
#include <string_view>
#include <vector>

#include "runtime.hpp"

namespace hllm_rocm::runtime {

// The Safetensors element types (the names of the format's "dtype" field).
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
  // Maps the file and validates its header; throws SafetensorsError.
  explicit SafetensorsFile(std::filesystem::path path);
  ~SafetensorsFile();
  SafetensorsFile(SafetensorsFile&& other) noexcept;
  SafetensorsFile& operator=(SafetensorsFile&& other) noexcept;
  SafetensorsFile(const SafetensorsFile&) = delete;
  SafetensorsFile& operator=(const SafetensorsFile&) = delete;

  const std::filesystem::path& path() const noexcept { return path_; }
  std::size_t file_size() const noexcept { return size_; }
  std::size_t header_size() const noexcept { return data_start_; }  // length prefix + JSON
  const std::vector<TensorMetadata>& tensors() const noexcept { return tensors_; }  // sorted by name
  const TensorMetadata& tensor(std::string_view name) const;
  // The tensor's bytes inside the mapping (valid while this object lives).
  std::span<const std::byte> payload(const TensorMetadata& tensor) const;

 private:
  void unmap() noexcept;
  std::filesystem::path path_;
  const std::byte* base_{nullptr};
  std::size_t size_{0}, data_start_{0};
  std::vector<TensorMetadata> tensors_;
};

}  // namespace hllm_rocm::runtime
