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

struct StFile {
  std::vector<uint8_t> bytes;  // whole file
  size_t data_start = 0;
  std::map<std::string, StEntry> entries;
};

// Returns "" on success or an error message in the reference's words.
std::string st_read_file(const std::string& path, StFile* out);
// Decode entry to f32 (F32, F64, F16, BF16, I32, I64, U8, BOOL).
std::string st_decode_f32(const StFile& f, const StEntry& e, std::vector<float>* out);

}  // namespace rtg
