// Minimal safetensors reader; see safetensors_reader.h.
#include "safetensors_reader.h"

#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace rtg {
namespace {

struct Json {
  const char* p;
  const char* e;
  std::string err;

  void ws() {
    while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool eat(char c) {
    ws();
    if (p < e && *p == c) {
      ++p;
      return true;
    }
    return false;
  }
  bool str(std::string* out) {
    ws();
    if (p >= e || *p != '"') return fail("expected string");
    ++p;
    out->clear();
    while (p < e && *p != '"') {
      if (*p == '\\') {
        ++p;
        if (p >= e) return fail("bad escape");
        char c = *p++;
        switch (c) {
          case 'n': out->push_back('\n'); break;
          case 't': out->push_back('\t'); break;
          case 'r': out->push_back('\r'); break;
          case 'b': out->push_back('\b'); break;
          case 'f': out->push_back('\f'); break;
          case 'u': {
            if (e - p < 4) return fail("bad unicode escape");
            unsigned v = 0;
            for (int i = 0; i < 4; ++i) {
              char h = *p++;
              v <<= 4;
              if (h >= '0' && h <= '9') v |= h - '0';
              else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
              else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
              else return fail("bad unicode escape");
            }
            if (v < 0x80) out->push_back((char)v);
            else if (v < 0x800) {
              out->push_back((char)(0xC0 | (v >> 6)));
              out->push_back((char)(0x80 | (v & 0x3F)));
            } else {
              out->push_back((char)(0xE0 | (v >> 12)));
              out->push_back((char)(0x80 | ((v >> 6) & 0x3F)));
              out->push_back((char)(0x80 | (v & 0x3F)));
            }
            break;
          }
          default: out->push_back(c);
        }
      } else {
        out->push_back(*p++);
      }
    }
    if (p >= e) return fail("unterminated string");
    ++p;
    return true;
  }
  bool num(size_t* out) {
    ws();
    if (p >= e || *p < '0' || *p > '9') return fail("expected unsigned integer");
    size_t v = 0;
    while (p < e && *p >= '0' && *p <= '9') v = v * 10 + (size_t)(*p++ - '0');
    *out = v;
    return true;
  }
  bool skip_value() {
    ws();
    if (p >= e) return fail("unexpected end");
    if (*p == '"') {
      std::string s;
      return str(&s);
    }
    if (*p == '{' || *p == '[') {
      char open = *p, close = open == '{' ? '}' : ']';
      ++p;
      if (eat(close)) return true;
      for (;;) {
        if (open == '{') {
          std::string k;
          if (!str(&k) || !eat(':')) return fail("bad object");
        }
        if (!skip_value()) return false;
        if (eat(',')) continue;
        if (eat(close)) return true;
        return fail("bad container");
      }
    }
    while (p < e && *p != ',' && *p != '}' && *p != ']') ++p;
    return true;
  }
  bool fail(const char* m) {
    if (err.empty()) err = m;
    return false;
  }
};

bool parse_entry(Json& j, StEntry* en) {
  if (!j.eat('{')) return j.fail("expected tensor object");
  if (j.eat('}')) return true;
  for (;;) {
    std::string k;
    if (!j.str(&k) || !j.eat(':')) return j.fail("bad tensor entry");
    if (k == "dtype") {
      if (!j.str(&en->dtype)) return false;
    } else if (k == "shape") {
      if (!j.eat('[')) return j.fail("bad shape");
      if (!j.eat(']')) {
        for (;;) {
          size_t v;
          if (!j.num(&v)) return false;
          en->shape.push_back(v);
          if (j.eat(',')) continue;
          if (j.eat(']')) break;
          return j.fail("bad shape");
        }
      }
    } else if (k == "data_offsets") {
      if (!j.eat('[') || !j.num(&en->begin) || !j.eat(',') || !j.num(&en->end) || !j.eat(']'))
        return j.fail("bad data_offsets");
    } else {
      if (!j.skip_value()) return false;
    }
    if (j.eat(',')) continue;
    if (j.eat('}')) return true;
    return j.fail("bad tensor entry");
  }
}

float f16_to_f32(uint16_t h) {
  uint32_t sign = (h >> 15) & 1, exp = (h >> 10) & 0x1f, frac = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (frac == 0) {
      bits = sign << 31;
    } else {
      int e = -1;
      do {
        ++e;
        frac <<= 1;
      } while ((frac & 0x400) == 0);
      frac &= 0x3ff;
      bits = (sign << 31) | ((uint32_t)(127 - 15 - e) << 23) | (frac << 13);
    }
  } else if (exp == 31) {
    bits = (sign << 31) | 0x7f800000u | (frac << 13);
  } else {
    bits = (sign << 31) | ((exp + 127 - 15) << 23) | (frac << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

}  // namespace

StFile::~StFile() {
  if (base) munmap(const_cast<uint8_t*>(base), size);
}

// The file is mapped read-only, not read: tensor bytes go from the page
// cache to the device (nn/safetensors.rs:94-151 reads it into memory).
std::string st_read_file(const std::string& path, StFile* out) {
  // std::io::Error's Display form, "<strerror> (os error N)"
  auto io_err = [](int e) { return std::string("I/O error: ") + strerror(e) + " (os error " + std::to_string(e) + ")"; };
  const int fd = open(path.c_str(), O_RDONLY);
  if (fd < 0) return io_err(errno);
  struct stat stt;
  if (fstat(fd, &stt) != 0) {
    const int e = errno;
    close(fd);
    return io_err(e);
  }
  const size_t fsize = (size_t)stt.st_size;
  if (fsize > 0) {
    void* m = mmap(nullptr, fsize, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      const int e = errno;
      close(fd);
      return io_err(e);
    }
    out->base = static_cast<const uint8_t*>(m);
    out->size = fsize;
  }
  close(fd);
  const uint8_t* d = out->base;
  // safetensors.rs:95-118
  if (fsize < 8) return "Invalid safetensors format: File too small — need at least 8 bytes for header size";
  uint64_t hs = 0;
  for (int i = 7; i >= 0; --i) hs = (hs << 8) | d[i];
  if (hs == 0) return "Invalid safetensors format: Header size is zero";
  if (hs > fsize - 8)
    return "Invalid safetensors format: Header size " + std::to_string(hs) + " exceeds file size " + std::to_string(fsize);
  out->data_start = 8 + (size_t)hs;
  Json j{reinterpret_cast<const char*>(d) + 8, reinterpret_cast<const char*>(d) + 8 + hs, {}};
  if (!j.eat('{')) return "Invalid safetensors format: header is not a JSON object";
  if (!j.eat('}')) {
    for (;;) {
      std::string name;
      if (!j.str(&name) || !j.eat(':')) return "Invalid safetensors format: " + j.err;
      if (name == "__metadata__") {
        if (!j.skip_value()) return "Invalid safetensors format: " + j.err;
      } else {
        StEntry en;
        if (!parse_entry(j, &en)) return "Invalid safetensors format: " + j.err;
        out->entries[name] = en;
      }
      if (j.eat(',')) continue;
      if (j.eat('}')) break;
      return "Invalid safetensors format: malformed header";
    }
  }
  const size_t data_len = fsize - out->data_start;
  for (auto& kv : out->entries) {
    const StEntry& en = kv.second;
    if (en.end > data_len || en.begin > en.end)
      return "Invalid safetensors format: Tensor '" + kv.first + "' data_offsets [" + std::to_string(en.begin) + ", " +
             std::to_string(en.end) + "] exceeds data buffer size " + std::to_string(data_len);
  }
  return "";
}

// Element count of e's shape; false when the product overflows.
static bool st_numel(const StEntry& e, size_t* n) {
  size_t c = 1;
  for (size_t s : e.shape)
    if (__builtin_mul_overflow(c, s, &c)) return false;
  *n = c;
  return true;
}

std::string st_check_size(const StEntry& e, size_t elem_bytes, const char* name) {
  const size_t len = e.end - e.begin;
  size_t n = 0, bytes = 0;
  if (!st_numel(e, &n) || __builtin_mul_overflow(n, elem_bytes, &bytes))
    return std::string("Invalid safetensors format: ") + name + " tensor: shape overflows, got " +
           std::to_string(len) + " bytes";
  if (len != bytes)
    return std::string("Invalid safetensors format: ") + name + " tensor: expected " + std::to_string(bytes) +
           " bytes, got " + std::to_string(len);
  return "";
}

std::string st_decode_f32(const StFile& f, const StEntry& e, std::vector<float>* out) {
  // the byte count is checked against the shape before anything is allocated
  size_t w = 0;
  const char* name = nullptr;
  if (e.dtype == "F32" || e.dtype == "I32") w = 4, name = e.dtype == "F32" ? "F32" : "I32";
  else if (e.dtype == "F64" || e.dtype == "I64") w = 8, name = e.dtype == "F64" ? "F64" : "I64";
  else if (e.dtype == "F16" || e.dtype == "BF16") w = 2, name = e.dtype == "F16" ? "F16" : "BF16";
  else if (e.dtype == "U8" || e.dtype == "BOOL") w = 1, name = "U8";
  else return "Unsupported dtype: " + e.dtype;
  const std::string err = st_check_size(e, w, name);
  if (!err.empty()) return err;
  const size_t n = (e.end - e.begin) / w;
  const uint8_t* raw = st_data(f, e);
  out->resize(n);
  if (e.dtype == "F32") {
    memcpy(out->data(), raw, n * 4);
  } else if (e.dtype == "F64") {
    for (size_t i = 0; i < n; ++i) {
      double v;
      memcpy(&v, raw + 8 * i, 8);
      (*out)[i] = (float)v;
    }
  } else if (e.dtype == "F16") {
    for (size_t i = 0; i < n; ++i) (*out)[i] = f16_to_f32((uint16_t)(raw[2 * i] | (raw[2 * i + 1] << 8)));
  } else if (e.dtype == "BF16") {
    for (size_t i = 0; i < n; ++i) {
      uint32_t b = (uint32_t)(raw[2 * i] | (raw[2 * i + 1] << 8)) << 16;
      memcpy(&(*out)[i], &b, 4);
    }
  } else if (e.dtype == "I32") {
    for (size_t i = 0; i < n; ++i) {
      int32_t v;
      memcpy(&v, raw + 4 * i, 4);
      (*out)[i] = (float)v;
    }
  } else if (e.dtype == "I64") {
    for (size_t i = 0; i < n; ++i) {
      int64_t v;
      memcpy(&v, raw + 8 * i, 8);
      (*out)[i] = (float)v;
    }
  } else {  // U8, BOOL
    for (size_t i = 0; i < n; ++i) (*out)[i] = (float)raw[i];
  }
  return "";
}

}  // namespace rtg
