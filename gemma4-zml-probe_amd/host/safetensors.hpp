// safetensors.hpp -- read-only access to a .safetensors file (memory-mapped).
//
// Layout: 8-byte little-endian header length H, H bytes of JSON
//   { "<name>": {"dtype": "I32", "shape": [..], "data_offsets": [begin, end]}, ...,
//     "__metadata__": {...} }
// then the tensor bytes; offsets are relative to the end of the header.  This is
// the container the reference loads its packed checkpoints from
// (zml_runner/w4.zig:166-168, W4Model.load).  Nothing in the file is executed.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace w4 {

struct TensorInfo {
  std::string dtype;           // "I32", "BF16", "I64", "F32", ...
  std::vector<int64_t> shape;
  uint64_t begin = 0, end = 0;  // byte offsets into the data section
  size_t nbytes() const { return (size_t)(end - begin); }
  int64_t numel() const;
};

class SafeTensorsFile {
 public:
  SafeTensorsFile() = default;
  explicit SafeTensorsFile(const std::string& path);  // throws std::runtime_error
  ~SafeTensorsFile();
  SafeTensorsFile(const SafeTensorsFile&) = delete;
  SafeTensorsFile& operator=(const SafeTensorsFile&) = delete;
  SafeTensorsFile(SafeTensorsFile&& o) noexcept;
  SafeTensorsFile& operator=(SafeTensorsFile&& o) noexcept;

  bool has(const std::string& name) const { return tensors_.count(name) != 0; }
  const TensorInfo& info(const std::string& name) const;  // throws if absent
  const void* data(const std::string& name) const;        // host pointer into the mapping
  const std::map<std::string, TensorInfo>& tensors() const { return tensors_; }
  const std::map<std::string, std::string>& metadata() const { return metadata_; }
  const std::string& path() const { return path_; }

  // Parse a header (the JSON text) into tensors/metadata; data_size bounds the offsets.
  // Exposed for tests.  Throws std::runtime_error on malformed input.
  static void parse_header(const std::string& json, uint64_t data_size, std::map<std::string, TensorInfo>& tensors,
                           std::map<std::string, std::string>& metadata);

 private:
  std::string path_;
  void* map_ = nullptr;
  size_t map_size_ = 0;
  const uint8_t* data_ = nullptr;
  std::map<std::string, TensorInfo> tensors_;
  std::map<std::string, std::string> metadata_;
};

// Bytes per element of a safetensors dtype string (0 if unknown).
size_t dtype_size(const std::string& dtype);

}  // namespace w4
