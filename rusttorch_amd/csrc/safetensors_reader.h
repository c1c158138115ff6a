// Minimal safetensors reader (format: 8-byte little-endian header length,
// JSON header {name: {dtype, shape, data_offsets}}, raw data), following
// rusttorch-core/src/nn/safetensors.rs:94-151 (header and offset checks) and
// :232-348 (dtype decoding to f32; BF16 = bits << 16, :389-391).
#pragma once
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

namespace rtg {

struct StEntry {
  std::string dtype;
  std::vector<size_t> shape;
  size_t begin = 0, end = 0;  // offsets into the data section
};

// A safetensors file mapped read-only (unmapped on destruction).
struct StFile {
  const uint8_t* base = nullptr;
  size_t size = 0;
  size_t data_start = 0;
  std::map<std::string, StEntry> entries;
  StFile() = default;
  StFile(const StFile&) = delete;
  StFile& operator=(const StFile&) = delete;
  ~StFile();
};

// Returns "" on success or an error message in the reference's words.
std::string st_read_file(const std::string& path, StFile* out);
// First byte of an entry's data.
inline const uint8_t* st_data(const StFile& f, const StEntry& e) { return f.base + f.data_start + e.begin; }
// "" when the entry holds exactly numel * elem_bytes bytes, else the reference's error.
std::string st_check_size(const StEntry& e, size_t elem_bytes, const char* name);
// Decode entry to f32 (F32, F64, F16, BF16, I32, I64, U8, BOOL).
std::string st_decode_f32(const StFile& f, const StEntry& e, std::vector<float>* out);

}  // namespace rtg
