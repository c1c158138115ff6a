// Byte-level BPE tokenizer (GPT-2 style) behind the C ABI: the behaviour of
// rusttorch-core/src/data/tokenizer.rs (BpeTokenizer), host-side text in and
// token ids out. Each function cites the reference lines it follows.
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <new>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/rtgpu.h"
#include "unicode_tables.h"

namespace {

// ---------------------------------------------------------------------------
// UTF-8
// ---------------------------------------------------------------------------

void put_utf8(std::string& s, uint32_t c) {
  if (c < 0x80) {
    s.push_back((char)c);
  } else if (c < 0x800) {
    s.push_back((char)(0xC0 | (c >> 6)));
    s.push_back((char)(0x80 | (c & 0x3F)));
  } else if (c < 0x10000) {
    s.push_back((char)(0xE0 | (c >> 12)));
    s.push_back((char)(0x80 | ((c >> 6) & 0x3F)));
    s.push_back((char)(0x80 | (c & 0x3F)));
  } else {
    s.push_back((char)(0xF0 | (c >> 18)));
    s.push_back((char)(0x80 | ((c >> 12) & 0x3F)));
    s.push_back((char)(0x80 | ((c >> 6) & 0x3F)));
    s.push_back((char)(0x80 | (c & 0x3F)));
  }
}

// Decode one scalar value at s[i] with the well-formedness rules of Unicode
// (Table 3-7). Returns its length, or the length of the maximal ill-formed
// subpart (>= 1) with *ok = false.
size_t utf8_step(const uint8_t* s, size_t n, size_t i, uint32_t* cp, bool* ok) {
  const uint8_t b0 = s[i];
  *ok = false;
  if (b0 < 0x80) {
    *cp = b0;
    *ok = true;
    return 1;
  }
  int len;
  uint8_t lo = 0x80, hi = 0xBF;
  if (b0 >= 0xC2 && b0 <= 0xDF) len = 2;
  else if (b0 >= 0xE0 && b0 <= 0xEF) {
    len = 3;
    if (b0 == 0xE0) lo = 0xA0;
    if (b0 == 0xED) hi = 0x9F;
  } else if (b0 >= 0xF0 && b0 <= 0xF4) {
    len = 4;
    if (b0 == 0xF0) lo = 0x90;
    if (b0 == 0xF4) hi = 0x8F;
  } else {
    return 1;  // C0, C1, F5..FF, or a stray continuation byte
  }
  uint32_t c = b0 & (len == 2 ? 0x1F : len == 3 ? 0x0F : 0x07);
  size_t k = 1;
  for (; k < (size_t)len; ++k) {
    if (i + k >= n) return k;
    const uint8_t b = s[i + k];
    if (b < (k == 1 ? lo : 0x80) || b > (k == 1 ? hi : 0xBF)) return k;
    c = (c << 6) | (b & 0x3F);
  }
  *cp = c;
  *ok = true;
  return k;
}

bool utf8_decode(const char* p, size_t n, std::vector<uint32_t>* out) {
  const uint8_t* s = reinterpret_cast<const uint8_t*>(p);
  out->clear();
  for (size_t i = 0; i < n;) {
    uint32_t c;
    bool ok;
    const size_t k = utf8_step(s, n, i, &c, &ok);
    if (!ok) return false;
    out->push_back(c);
    i += k;
  }
  return true;
}

// String::from_utf8_lossy: every maximal ill-formed subpart becomes one
// U+FFFD (decode, tokenizer.rs:129).
std::string utf8_lossy(const std::string& bytes) {
  const uint8_t* s = reinterpret_cast<const uint8_t*>(bytes.data());
  const size_t n = bytes.size();
  std::string out;
  out.reserve(n);
  for (size_t i = 0; i < n;) {
    uint32_t c;
    bool ok;
    const size_t k = utf8_step(s, n, i, &c, &ok);
    if (ok) out.append(bytes, i, k);
    else put_utf8(out, 0xFFFD);
    i += k;
  }
  return out;
}

// ---------------------------------------------------------------------------
// byte encoder (build_byte_encoder / is_printable_byte, tokenizer.rs:223-251)
// ---------------------------------------------------------------------------

bool printable_byte(unsigned b) { return (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255); }

struct ByteTable {
  uint32_t enc[256];
  std::unordered_map<uint32_t, uint8_t> dec;
  ByteTable() {
    uint32_t next = 256;  // non-printable bytes take U+0100, U+0101, ... in byte order
    for (unsigned b = 0; b < 256; ++b) {
      enc[b] = printable_byte(b) ? b : next++;
      dec[enc[b]] = (uint8_t)b;
    }
  }
};

const ByteTable& bytes_table() {
  static const ByteTable t;
  return t;
}

// ---------------------------------------------------------------------------
// pre-tokenizer (pre_tokenize / match_contraction, tokenizer.rs:260-353)
// ---------------------------------------------------------------------------

bool alpha(uint32_t c) { return rtg::unicode::is_alphabetic(c); }
bool space(uint32_t c) { return rtg::unicode::is_whitespace(c); }
bool digit(uint32_t c) { return c >= '0' && c <= '9'; }
// char::to_lowercase of c equals the ASCII letter l (lower case) only for the
// two ASCII cases of l: no other code point lowercases to s, t, m, d, r, e, v
// or l.
bool is_letter_ci(uint32_t c, char l) { return c == (uint32_t)l || c == (uint32_t)(l - 'a' + 'A'); }

// Length of the contraction starting at the apostrophe c[i], or 0.
size_t contraction(const std::vector<uint32_t>& c, size_t i) {
  const size_t rem = c.size() - i;
  if (rem >= 3) {
    const uint32_t a = c[i + 1], b = c[i + 2];
    if ((is_letter_ci(a, 'r') && is_letter_ci(b, 'e')) || (is_letter_ci(a, 'v') && is_letter_ci(b, 'e')) ||
        (is_letter_ci(a, 'l') && is_letter_ci(b, 'l')))
      return 3;
  }
  if (rem >= 2) {
    const uint32_t a = c[i + 1];
    if (is_letter_ci(a, 's') || is_letter_ci(a, 't') || is_letter_ci(a, 'm') || is_letter_ci(a, 'd')) return 2;
  }
  return 0;
}

// Words of the text as code point ranges [first, second).
std::vector<std::pair<size_t, size_t>> pre_tokenize(const std::vector<uint32_t>& c) {
  std::vector<std::pair<size_t, size_t>> w;
  const size_t n = c.size();
  size_t i = 0;
  while (i < n) {
    if (c[i] == '\'' && i + 1 < n) {
      if (const size_t k = contraction(c, i)) {
        w.emplace_back(i, i + k);
        i += k;
        continue;
      }
    }
    if (space(c[i])) {
      // a space takes the letters (or ASCII digits) that follow it
      if (c[i] == ' ' && i + 1 < n && (alpha(c[i + 1]) || digit(c[i + 1]))) {
        const bool letters = alpha(c[i + 1]);
        const size_t s = i++;
        while (i < n && (letters ? alpha(c[i]) : digit(c[i]))) ++i;
        w.emplace_back(s, i);
        continue;
      }
      w.emplace_back(i, i + 1);
      ++i;
      continue;
    }
    if (alpha(c[i]) || digit(c[i])) {
      const bool letters = alpha(c[i]);
      const size_t s = i;
      while (i < n && (letters ? alpha(c[i]) : digit(c[i]))) ++i;
      w.emplace_back(s, i);
      continue;
    }
    w.emplace_back(i, i + 1);  // any other character is a word of its own
    ++i;
  }
  return w;
}

// ---------------------------------------------------------------------------
// vocab.json / merges.txt parsers (tokenizer.rs:356-514)
// ---------------------------------------------------------------------------

// Rust's Debug form of Option<char> as the reference's messages print it.
std::string debug_opt_char(bool some, uint32_t c) {
  if (!some) return "None";
  std::string s = "Some('";
  switch (c) {
    case '\'': s += "\\'"; break;
    case '\\': s += "\\\\"; break;
    case '\n': s += "\\n"; break;
    case '\r': s += "\\r"; break;
    case '\t': s += "\\t"; break;
    case 0: s += "\\0"; break;
    default:
      if (c < 0x20 || c == 0x7F) {
        char buf[16];
        snprintf(buf, sizeof buf, "\\u{%x}", c);
        s += buf;
      } else {
        put_utf8(s, c);
      }
  }
  return s + "')";
}

struct Chars {  // a peekable iterator over code points
  const std::vector<uint32_t>& c;
  size_t i, end;
  bool peek(uint32_t* x) const {
    if (i >= end) return false;
    *x = c[i];
    return true;
  }
  bool next(uint32_t* x) {
    if (i >= end) return false;
    *x = c[i++];
    return true;
  }
  void skip_ws() {
    while (i < end && space(c[i])) ++i;
  }
};

// parse_json_string, tokenizer.rs:404-447
bool json_string(Chars& it, std::string* out, std::string* err) {
  uint32_t x = 0;
  bool got = it.next(&x);
  if (!got || x != '"') {
    *err = "Expected '\"', got " + debug_opt_char(got, x);
    return false;
  }
  out->clear();
  for (;;) {
    if (!it.next(&x)) {
      *err = "Unexpected end of string";
      return false;
    }
    if (x == '"') return true;
    if (x != '\\') {
      put_utf8(*out, x);
      continue;
    }
    if (!it.next(&x)) {
      *err = "Unexpected end of string";
      return false;
    }
    switch (x) {
      case '"': out->push_back('"'); break;
      case '\\': out->push_back('\\'); break;
      case '/': out->push_back('/'); break;
      case 'n': out->push_back('\n'); break;
      case 'r': out->push_back('\r'); break;
      case 't': out->push_back('\t'); break;
      case 'u': {
        std::string hex;  // up to 4 characters, as UTF-8
        for (int k = 0; k < 4 && it.next(&x); ++k) put_utf8(hex, x);
        if (hex.size() != 4) {
          *err = "Incomplete unicode escape";
          return false;
        }
        // u32::from_str_radix(hex, 16): an optional '+', then hex digits
        size_t p = hex[0] == '+' ? 1 : 0;
        bool valid = p < hex.size();
        uint32_t code = 0;
        for (; valid && p < hex.size(); ++p) {
          const char h = hex[p];
          int v = h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10 : h >= 'A' && h <= 'F' ? h - 'A' + 10 : -1;
          if (v < 0) valid = false;
          else code = code * 16 + (uint32_t)v;
        }
        if (!valid) {
          *err = "Invalid unicode escape: \\u" + hex;
          return false;
        }
        if (code >= 0xD800 && code <= 0xDFFF) {  // char::from_u32 refuses surrogates
          *err = "Invalid unicode code point: " + std::to_string(code);
          return false;
        }
        put_utf8(*out, code);
        break;
      }
      default:
        out->push_back('\\');
        put_utf8(*out, x);
    }
  }
}

// parse_json_int, tokenizer.rs:450-470
bool json_int(Chars& it, uint32_t* v, std::string* err) {
  std::string num;
  uint32_t x;
  if (it.peek(&x) && x == '-') {
    it.next(&x);
    num.push_back('-');
  }
  while (it.peek(&x) && x >= '0' && x <= '9') {
    it.next(&x);
    num.push_back((char)x);
  }
  // str::parse::<u32>: digits only (the '-' makes it fail), no overflow
  bool ok = !num.empty() && num[0] != '-';
  uint64_t acc = 0;
  for (size_t k = 0; ok && k < num.size(); ++k) {
    acc = acc * 10 + (uint64_t)(num[k] - '0');
    if (acc > 0xFFFFFFFFull) ok = false;
  }
  if (!ok) {
    *err = "Failed to parse integer: '" + num + "'";
    return false;
  }
  *v = (uint32_t)acc;
  return true;
}

// parse_vocab_json, tokenizer.rs:356-401. Entries in file order (a key that
// repeats keeps its last id).
bool parse_vocab(const std::string& json, std::vector<std::pair<std::string, uint32_t>>* out, std::string* err) {
  std::vector<uint32_t> c;
  if (!utf8_decode(json.data(), json.size(), &c)) {
    *err = "vocab.json is not valid UTF-8";
    return false;
  }
  size_t b = 0, e = c.size();  // str::trim
  while (b < e && space(c[b])) ++b;
  while (e > b && space(c[e - 1])) --e;
  if (e - b < 2 || c[b] != '{' || c[e - 1] != '}') {
    *err = "vocab.json must be a JSON object";
    return false;
  }
  Chars it{c, b + 1, e - 1};
  for (;;) {
    it.skip_ws();
    uint32_t x;
    if (!it.peek(&x)) break;
    std::string key;
    if (!json_string(it, &key, err)) return false;
    it.skip_ws();
    const bool got = it.next(&x);
    if (!got || x != ':') {
      *err = "Expected ':', got " + debug_opt_char(got, x);
      return false;
    }
    it.skip_ws();
    uint32_t v;
    if (!json_int(it, &v, err)) return false;
    out->emplace_back(std::move(key), v);
    it.skip_ws();
    if (it.peek(&x) && x == ',') it.next(&x);
  }
  return true;
}

struct PairHash {
  size_t operator()(const std::pair<std::string, std::string>& p) const {
    return std::hash<std::string>()(p.first) * 1000003u ^ std::hash<std::string>()(p.second);
  }
};
using Merges = std::unordered_map<std::pair<std::string, std::string>, size_t, PairHash>;

// parse_merges, tokenizer.rs:486-514: rank = line index (header and blank
// lines count), split at the first space.
void parse_merges(const std::string& txt, Merges* m) {
  size_t rank = 0, pos = 0;
  while (pos < txt.size()) {
    size_t nl = txt.find('\n', pos);
    const bool last = nl == std::string::npos;
    std::string line = txt.substr(pos, last ? std::string::npos : nl - pos);
    pos = last ? txt.size() : nl + 1;
    if (!last && !line.empty() && line.back() == '\r') line.pop_back();  // str::lines: "\r\n" ends a line too
    const size_t r = rank++;
    if ((!line.empty() && line[0] == '#') || line.compare(0, 7, "version") == 0) continue;
    std::vector<uint32_t> c;
    if (!utf8_decode(line.data(), line.size(), &c)) continue;
    size_t b = 0, e = c.size();  // str::trim
    while (b < e && space(c[b])) ++b;
    while (e > b && space(c[e - 1])) --e;
    if (b == e) continue;
    std::string t;
    for (size_t k = b; k < e; ++k) put_utf8(t, c[k]);
    const size_t sp = t.find(' ');
    if (sp == std::string::npos) continue;
    (*m)[{t.substr(0, sp), t.substr(sp + 1)}] = r;
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// BpeTokenizer (tokenizer.rs:26-220)
// ---------------------------------------------------------------------------

struct rtg_tokenizer {
  std::unordered_map<std::string, uint32_t> encoder;
  std::vector<std::string> decoder;
  Merges merges;

  // apply_bpe, tokenizer.rs:148-183: repeatedly merge the adjacent pair of
  // lowest rank (the leftmost one among equal ranks), one merge per pass.
  void apply_bpe(std::vector<std::string>& t) const {
    if (t.size() < 2) return;
    for (;;) {
      size_t best = SIZE_MAX, best_rank = SIZE_MAX;
      for (size_t i = 0; i + 1 < t.size(); ++i) {
        auto it = merges.find({t[i], t[i + 1]});
        if (it != merges.end() && (best == SIZE_MAX || it->second < best_rank)) {
          best = i;
          best_rank = it->second;
        }
      }
      if (best == SIZE_MAX) return;
      t[best] += t[best + 1];
      t.erase(t.begin() + (long)best + 1);
    }
  }

  // encode, tokenizer.rs:85-112
  bool encode(const char* text, size_t len, std::vector<uint32_t>* ids) const {
    std::vector<uint32_t> c;
    if (!utf8_decode(text, len, &c)) return false;
    const ByteTable& bt = bytes_table();
    for (const auto& w : pre_tokenize(c)) {
      std::string word;
      for (size_t k = w.first; k < w.second; ++k) put_utf8(word, c[k]);
      std::vector<std::string> toks;
      toks.reserve(word.size());
      for (unsigned char b : word) {
        std::string one;
        put_utf8(one, bt.enc[b]);
        toks.push_back(std::move(one));
      }
      apply_bpe(toks);
      for (const auto& tk : toks) {
        auto it = encoder.find(tk);
        if (it != encoder.end()) ids->push_back(it->second);  // unknown tokens are skipped
      }
    }
    return true;
  }

  // decode, tokenizer.rs:115-130
  std::string decode(const uint32_t* ids, size_t n) const {
    std::string s;
    for (size_t k = 0; k < n; ++k)
      if (ids[k] < decoder.size()) s += decoder[ids[k]];
    std::vector<uint32_t> c;
    utf8_decode(s.data(), s.size(), &c);  // tokens are valid UTF-8 strings
    const ByteTable& bt = bytes_table();
    std::string bytes;
    for (uint32_t x : c) {
      auto it = bt.dec.find(x);
      if (it != bt.dec.end()) bytes.push_back((char)it->second);
    }
    return utf8_lossy(bytes);
  }
};

namespace {

rtg_result ok_result() { return rtg_result{true, nullptr}; }
rtg_result err_result(const std::string& m) {
  char* p = static_cast<char*>(malloc(m.size() + 1));
  if (p) memcpy(p, m.c_str(), m.size() + 1);
  return rtg_result{false, p};
}

// from_strings, tokenizer.rs:55-82
rtg_result build_from_strings(const std::string& vocab, const std::string& merges, rtg_tokenizer** out) {
  std::vector<std::pair<std::string, uint32_t>> entries;
  std::string err;
  std::vector<uint32_t> c;  // both texts are &str in the reference: valid UTF-8
  if (!utf8_decode(merges.data(), merges.size(), &c)) return err_result("merges.txt is not valid UTF-8");
  if (!parse_vocab(vocab, &entries, &err)) return err_result(err);
  try {
    auto* t = new rtg_tokenizer();
    uint32_t max_id = 0;
    for (const auto& e : entries) {
      t->encoder[e.first] = e.second;
      max_id = e.second > max_id ? e.second : max_id;
    }
    t->decoder.assign((size_t)max_id + 1, std::string());
    for (const auto& kv : t->encoder) t->decoder[kv.second] = kv.first;
    parse_merges(merges, &t->merges);
    *out = t;
  } catch (const std::bad_alloc&) {
    return err_result("out of memory");
  }
  return ok_result();
}

// fs::read_to_string with the io::Error's Display text
bool read_file(const char* path, std::string* s, std::string* err) {
  auto io_err = [&](int e) {
    *err = std::string(strerror(e)) + " (os error " + std::to_string(e) + ")";
    return false;
  };
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return io_err(errno);
  char buf[1 << 16];
  for (;;) {
    const ssize_t r = read(fd, buf, sizeof buf);
    if (r < 0) {
      const int e = errno;
      close(fd);
      return io_err(e);
    }
    if (r == 0) break;
    s->append(buf, (size_t)r);
  }
  close(fd);
  std::vector<uint32_t> c;
  if (!utf8_decode(s->data(), s->size(), &c)) {
    *err = "stream did not contain valid UTF-8";
    return false;
  }
  return true;
}

}  // namespace

extern "C" {

rtg_result rtg_tokenizer_from_files(const char* vocab_json_path, const char* merges_txt_path, rtg_tokenizer** out) {
  if (!vocab_json_path || !merges_txt_path || !out) return err_result("null argument");
  std::string v, m, e;
  if (!read_file(vocab_json_path, &v, &e)) return err_result("Failed to read vocab.json: " + e);
  if (!read_file(merges_txt_path, &m, &e)) return err_result("Failed to read merges.txt: " + e);
  return build_from_strings(v, m, out);
}

rtg_result rtg_tokenizer_from_strings(const char* vocab_json, size_t vocab_len, const char* merges_txt,
                                      size_t merges_len, rtg_tokenizer** out) {
  if ((!vocab_json && vocab_len) || (!merges_txt && merges_len) || !out) return err_result("null argument");
  return build_from_strings(std::string(vocab_json ? vocab_json : "", vocab_len),
                            std::string(merges_txt ? merges_txt : "", merges_len), out);
}

rtg_result rtg_tokenizer_from_vocab_and_merges(const char* const* vocab, size_t n_vocab, const char* const* merge_a,
                                               const char* const* merge_b, size_t n_merges, rtg_tokenizer** out) {
  if ((!vocab && n_vocab) || ((!merge_a || !merge_b) && n_merges) || !out) return err_result("null argument");
  try {
    auto* t = new rtg_tokenizer();
    for (size_t i = 0; i < n_vocab; ++i) {  // from_vocab_and_merges, tokenizer.rs:186-219
      t->encoder[vocab[i]] = (uint32_t)i;
      t->decoder.emplace_back(vocab[i]);
    }
    for (size_t r = 0; r < n_merges; ++r) t->merges[{merge_a[r], merge_b[r]}] = r;
    *out = t;
  } catch (const std::bad_alloc&) {
    return err_result("out of memory");
  }
  return ok_result();
}

void rtg_tokenizer_destroy(rtg_tokenizer* t) { delete t; }

rtg_result rtg_tokenizer_encode(const rtg_tokenizer* t, const char* text, size_t len, uint32_t** ids, size_t* n) {
  if (!t || (!text && len) || !ids || !n) return err_result("null argument");
  std::vector<uint32_t> v;
  if (!t->encode(text ? text : "", len, &v)) return err_result("text is not valid UTF-8");
  *n = v.size();
  *ids = static_cast<uint32_t*>(malloc(v.size() * 4 + 4));
  if (!*ids) return err_result("out of memory");
  if (!v.empty()) memcpy(*ids, v.data(), v.size() * 4);
  return ok_result();
}

rtg_result rtg_tokenizer_decode(const rtg_tokenizer* t, const uint32_t* ids, size_t n, char** text, size_t* len) {
  if (!t || (!ids && n) || !text || !len) return err_result("null argument");
  const std::string s = t->decode(ids, n);
  *len = s.size();
  *text = static_cast<char*>(malloc(s.size() + 1));
  if (!*text) return err_result("out of memory");
  memcpy(*text, s.c_str(), s.size() + 1);
  return ok_result();
}

size_t rtg_tokenizer_vocab_size(const rtg_tokenizer* t) { return t ? t->encoder.size() : 0; }

bool rtg_tokenizer_token_to_id(const rtg_tokenizer* t, const char* token, size_t len, uint32_t* id) {
  if (!t || (!token && len)) return false;
  auto it = t->encoder.find(std::string(token ? token : "", len));
  if (it == t->encoder.end()) return false;
  if (id) *id = it->second;
  return true;
}

bool rtg_tokenizer_id_to_token(const rtg_tokenizer* t, uint32_t id, const char** token, size_t* len) {
  if (!t || id >= t->decoder.size()) return false;
  if (token) *token = t->decoder[id].data();
  if (len) *len = t->decoder[id].size();
  return true;
}

rtg_result rtg_tokenizer_pre_tokenize(const char* text, size_t len, size_t** spans, size_t* n_words) {
  if ((!text && len) || !spans || !n_words) return err_result("null argument");
  std::vector<uint32_t> c;
  if (!utf8_decode(text ? text : "", len, &c)) return err_result("text is not valid UTF-8");
  // code point index -> byte offset
  std::vector<size_t> off(c.size() + 1, 0);
  for (size_t k = 0; k < c.size(); ++k) off[k + 1] = off[k] + (c[k] < 0x80 ? 1 : c[k] < 0x800 ? 2 : c[k] < 0x10000 ? 3 : 4);
  const auto w = pre_tokenize(c);
  *n_words = w.size();
  *spans = static_cast<size_t*>(malloc(w.size() * 2 * sizeof(size_t) + sizeof(size_t)));
  if (!*spans) return err_result("out of memory");
  for (size_t k = 0; k < w.size(); ++k) {
    (*spans)[2 * k] = off[w[k].first];
    (*spans)[2 * k + 1] = off[w[k].second];
  }
  return ok_result();
}

void rtg_tokenizer_byte_encoder(uint32_t out[256]) {
  const ByteTable& bt = bytes_table();
  for (int b = 0; b < 256; ++b) out[b] = bt.enc[b];
}

void rtg_free_buffer(void* p) { free(p); }

}  // extern "C"
