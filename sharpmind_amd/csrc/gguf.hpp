// gguf.hpp — GGUF container parsing (host side).
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace smhip {

struct GgufTensor {
  std::string name;
  std::vector<int64_t> dims;  // ne[0] (innermost) first, as stored
  uint32_t type;              // ggml type id (0 F32, 1 F16, 8 Q8_0, 12 Q4_K, ...)
  uint64_t offset;            // relative to the data section
};

struct GgufFile {
  uint32_t version = 0;
  std::vector<GgufTensor> tensors;
  // integer-valued metadata (any integer type), by key; other values are skipped
  std::vector<std::pair<std::string, int64_t>> ints;
  std::vector<std::pair<std::string, std::string>> strings;
  uint64_t data_offset = 0;  // absolute file offset of the data section
  bool int_value(const std::string& key, int64_t* v) const;
  const std::string* string_value(const std::string& key) const;
  const GgufTensor* find(const std::string& name) const;
};

// Parses the header, metadata and tensor table of `path`; returns SMHIP_OK or an error code
// with the message set.
int gguf_parse(const std::string& path, GgufFile* out);
// Byte size of a tensor of ggml type `type` and the given dims (QuantizationOps.cs:15-72);
// -1 for types this build does not read.
int64_t gguf_tensor_bytes(uint32_t type, const std::vector<int64_t>& dims);

}  // namespace smhip
