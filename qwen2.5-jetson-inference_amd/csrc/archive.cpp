// QWENBIN1 archives on the host: reader, W8A16 / W16A16 exporter and the
// config.json loader (include/infer_archive.h).  The format is the
// reference's (src/archive.cpp:14-102, tools/export_model.py:25-29,
// 103-108, 202-396, src/model_config.cpp:15-46); the code is this
// repository's: a small JSON reader for the metadata subset, mmap for the
// payload, and a SHA-256 (FIPS 180-4) for the per-tensor digests the
// exporter records.
#include "infer_archive.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cfenv>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "status.hpp"

using namespace qlin;

namespace {

// ----------------------------------------------------------------- JSON --
// RFC 8259 JSON: objects, arrays, strings (UTF-8 checked, \uXXXX escapes
// and surrogate pairs decoded to UTF-8), numbers in the strict grammar
// (integers exact to 2^63), true, false, null; at most 64 levels deep.
struct Json {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  bool b = false;
  double num = 0.0;
  bool integral = false;
  long long integer = 0;
  std::string str;
  std::vector<Json> items;
  std::vector<std::pair<std::string, Json>> members;

  // The last member of that name: a repeated key overrides the earlier one,
  // as in nlohmann::json (which the reference parses with) and Python's json.
  const Json* get(const char* key) const {
    if (kind != kObject) return nullptr;
    for (auto m = members.rbegin(); m != members.rend(); ++m) {
      if (m->first == key) return &m->second;
    }
    return nullptr;
  }
};

class JsonParser {
 public:
  JsonParser(const char* begin, const char* end) : p_(begin), end_(end) {}

  bool parse(Json& out, std::string& error) {
    if (!value(out, 0)) {
      error = error_;
      return false;
    }
    ws();
    if (p_ != end_) {
      error = "trailing characters after the metadata";
      return false;
    }
    return true;
  }

 private:
  const char* p_;
  const char* end_;
  std::string error_;

  bool bad(const char* what) {
    error_ = what;
    return false;
  }
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* word) {
    const size_t n = std::strlen(word);
    if (static_cast<size_t>(end_ - p_) < n || std::memcmp(p_, word, n) != 0) return false;
    p_ += n;
    return true;
  }
  static void put_utf8(std::string& s, unsigned cp) {
    if (cp < 0x80) {
      s.push_back(static_cast<char>(cp));
    } else if (cp < 0x800) {
      s.push_back(static_cast<char>(0xC0 | (cp >> 6)));
      s.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
      s.push_back(static_cast<char>(0xE0 | (cp >> 12)));
      s.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
      s.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else {
      s.push_back(static_cast<char>(0xF0 | (cp >> 18)));
      s.push_back(static_cast<char>(0x80 | ((cp >> 12) & 0x3F)));
      s.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
      s.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    }
  }
  bool hex4(unsigned& v) {
    if (end_ - p_ < 4) return false;
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= static_cast<unsigned>(c - '0');
      else if (c >= 'a' && c <= 'f') v |= static_cast<unsigned>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= static_cast<unsigned>(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  // One RFC 3629 sequence whose lead byte `lead` (>= 0x80) was just read:
  // appended to s, or false for an ill-formed one (a stray continuation
  // byte, an overlong form, a surrogate, a code point past U+10FFFF or a cut
  // sequence).
  bool utf8_sequence(std::string& s, unsigned lead) {
    int more;
    unsigned lo = 0x80, hi = 0xBF;
    if (lead >= 0xC2 && lead <= 0xDF) {
      more = 1;
    } else if (lead >= 0xE0 && lead <= 0xEF) {
      more = 2;
      if (lead == 0xE0) lo = 0xA0;
      if (lead == 0xED) hi = 0x9F;
    } else if (lead >= 0xF0 && lead <= 0xF4) {
      more = 3;
      if (lead == 0xF0) lo = 0x90;
      if (lead == 0xF4) hi = 0x8F;
    } else {
      return false;
    }
    if (end_ - p_ < more) return false;
    s.push_back(static_cast<char>(lead));
    for (int i = 0; i < more; ++i) {
      const unsigned b = static_cast<unsigned char>(*p_++);
      if (b < (i == 0 ? lo : 0x80u) || b > (i == 0 ? hi : 0xBFu)) return false;
      s.push_back(static_cast<char>(b));
    }
    return true;
  }
  bool string(std::string& s) {
    if (p_ >= end_ || *p_ != '"') return bad("expected a string");
    ++p_;
    while (true) {
      if (p_ >= end_) return bad("unterminated string");
      const char c = *p_++;
      if (c == '"') return true;
      if (static_cast<unsigned char>(c) < 0x20) return bad("control character in a string");
      if (static_cast<unsigned char>(c) >= 0x80) {
        if (!utf8_sequence(s, static_cast<unsigned char>(c))) {
          return bad("ill-formed UTF-8 in a string");
        }
        continue;
      }
      if (c != '\\') {
        s.push_back(c);
        continue;
      }
      if (p_ >= end_) return bad("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': s.push_back('"'); break;
        case '\\': s.push_back('\\'); break;
        case '/': s.push_back('/'); break;
        case 'b': s.push_back('\b'); break;
        case 'f': s.push_back('\f'); break;
        case 'n': s.push_back('\n'); break;
        case 'r': s.push_back('\r'); break;
        case 't': s.push_back('\t'); break;
        case 'u': {
          unsigned cp;
          if (!hex4(cp)) return bad("bad \\u escape");
          if (cp >= 0xDC00 && cp < 0xE000) return bad("bad surrogate pair");
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            unsigned lo;
            if (!lit("\\u") || !hex4(lo) || lo < 0xDC00 || lo >= 0xE000) {
              return bad("bad surrogate pair");
            }
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(s, cp);
          break;
        }
        default: return bad("bad escape");
      }
    }
  }
  // -? (0 | [1-9][0-9]*) (. [0-9]+)? ([eE] [+-]? [0-9]+)?
  bool number(Json& out) {
    const char* start = p_;
    auto digits = [this] {
      const char* from = p_;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
      return p_ != from;
    };
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ < end_ && *p_ == '0') {
      ++p_;
    } else if (!digits()) {
      return bad("bad number");
    }
    bool frac = false;
    if (p_ < end_ && *p_ == '.') {
      ++p_;
      frac = true;
      if (!digits()) return bad("bad number");
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      ++p_;
      frac = true;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (!digits()) return bad("bad number");
    }
    const std::string text(start, p_);
    out.kind = Json::kNumber;
    out.num = std::strtod(text.c_str(), nullptr);
    if (!frac) {
      char* stop = nullptr;
      errno = 0;
      out.integer = std::strtoll(text.c_str(), &stop, 10);
      out.integral = errno == 0 && *stop == '\0';
    }
    return true;
  }
  bool value(Json& out, int depth) {
    if (depth > 64) return bad("metadata nested too deeply");
    ws();
    if (p_ >= end_) return bad("unexpected end of the metadata");
    const char c = *p_;
    if (c == '{') {
      ++p_;
      out.kind = Json::kObject;
      ws();
      if (p_ < end_ && *p_ == '}') {
        ++p_;
        return true;
      }
      while (true) {
        ws();
        std::string key;
        if (!string(key)) return false;
        ws();
        if (p_ >= end_ || *p_ != ':') return bad("expected ':'");
        ++p_;
        Json v;
        if (!value(v, depth + 1)) return false;
        out.members.emplace_back(std::move(key), std::move(v));
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          ++p_;
          return true;
        }
        return bad("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p_;
      out.kind = Json::kArray;
      ws();
      if (p_ < end_ && *p_ == ']') {
        ++p_;
        return true;
      }
      while (true) {
        Json v;
        if (!value(v, depth + 1)) return false;
        out.items.push_back(std::move(v));
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          ++p_;
          return true;
        }
        return bad("expected ',' or ']'");
      }
    }
    if (c == '"') {
      out.kind = Json::kString;
      return string(out.str);
    }
    if (lit("true")) {
      out.kind = Json::kBool;
      out.b = true;
      return true;
    }
    if (lit("false")) {
      out.kind = Json::kBool;
      return true;
    }
    if (lit("null")) {
      out.kind = Json::kNull;
      return true;
    }
    return number(out);
  }
};

// Python's json.dumps(ensure_ascii=False) string form, which the reference's
// exporter writes: short escapes for \b \f \n \r \t, \u00XX for the other
// control characters, UTF-8 kept as is.
void json_escape(std::string& out, const std::string& s) {
  out.push_back('"');
  for (const char ch : s) {
    const unsigned char c = static_cast<unsigned char>(ch);
    if (c == '"') {
      out += "\\\"";
    } else if (c == '\\') {
      out += "\\\\";
    } else if (c == '\b') {
      out += "\\b";
    } else if (c == '\f') {
      out += "\\f";
    } else if (c == '\n') {
      out += "\\n";
    } else if (c == '\r') {
      out += "\\r";
    } else if (c == '\t') {
      out += "\\t";
    } else if (c < 0x20) {
      char buf[8];
      std::snprintf(buf, sizeof buf, "\\u%04x", c);
      out += buf;
    } else {
      out.push_back(ch);
    }
  }
  out.push_back('"');
}

// -------------------------------------------------------------- SHA-256 --
// FIPS 180-4.  The round constants are the first 32 bits of the fractional
// parts of the cube roots of the first 64 primes; the initial hash those of
// the square roots of the first 8 primes.
class Sha256 {
 public:
  Sha256() { reset(); }
  void reset() {
    static const uint32_t init[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                     0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    std::memcpy(h_, init, sizeof h_);
    bytes_ = 0;
    fill_ = 0;
  }
  void update(const void* data, size_t n) {
    const auto* p = static_cast<const uint8_t*>(data);
    bytes_ += n;
    while (n > 0) {
      const size_t take = std::min(n, sizeof(buf_) - fill_);
      std::memcpy(buf_ + fill_, p, take);
      fill_ += take;
      p += take;
      n -= take;
      if (fill_ == sizeof(buf_)) {
        block(buf_);
        fill_ = 0;
      }
    }
  }
  std::string hex() {
    const uint64_t bits = bytes_ * 8;
    const uint8_t one = 0x80, zero = 0;
    update(&one, 1);
    while (fill_ != 56) update(&zero, 1);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = static_cast<uint8_t>(bits >> (56 - 8 * i));
    update(len, 8);
    static const char* digits = "0123456789abcdef";
    std::string out;
    for (int i = 0; i < 8; ++i)
      for (int j = 28; j >= 0; j -= 4) out.push_back(digits[(h_[i] >> j) & 15]);
    return out;
  }

 private:
  uint32_t h_[8];
  uint8_t buf_[64];
  uint64_t bytes_;
  size_t fill_;

  static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
  void block(const uint8_t* p) {
    static const uint32_t k[64] = {
        0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4,
        0xab1c5ed5, 0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe,
        0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f,
        0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7,
        0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc,
        0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85, 0xa2bfe8a1, 0xa81a664b,
        0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116,
        0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
        0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7,
        0xc67178f2};
    uint32_t w[64];
    for (int i = 0; i < 16; ++i) {
      w[i] = (uint32_t(p[4 * i]) << 24) | (uint32_t(p[4 * i + 1]) << 16) |
             (uint32_t(p[4 * i + 2]) << 8) | uint32_t(p[4 * i + 3]);
    }
    for (int i = 16; i < 64; ++i) {
      const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
      const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h_[0], b = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6],
             h = h_[7];
    for (int i = 0; i < 64; ++i) {
      const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) +
                          k[i] + w[i];
      const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
      h = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = b;
      b = a;
      a = t1 + t2;
    }
    h_[0] += a; h_[1] += b; h_[2] += c; h_[3] += d;
    h_[4] += e; h_[5] += f; h_[6] += g; h_[7] += h;
  }
};

// ------------------------------------------------------------- BF16 RNE --
// (bits + 0x7FFF + lsb) >> 16, NaN keeps its high half with the quiet bit
// (export_model.py:123-131).
uint16_t bf16_rne(float v) {
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  if ((bits & 0x7F800000u) == 0x7F800000u && (bits & 0x007FFFFFu) != 0u) {
    return static_cast<uint16_t>((bits >> 16) | 0x0040u);
  }
  bits += 0x7FFFu + ((bits >> 16) & 1u);
  return static_cast<uint16_t>(bits >> 16);
}
float bf16_value(uint16_t w) {
  const uint32_t bits = static_cast<uint32_t>(w) << 16;
  float v;
  std::memcpy(&v, &bits, 4);
  return v;
}

constexpr char kMagic[8] = {'Q', 'W', 'E', 'N', 'B', 'I', 'N', '1'};
constexpr uint64_t kDataOffset = 1024 * 1024;  // export_model.py:27
constexpr uint64_t kAlignment = 256;           // export_model.py:29

#pragma pack(push, 1)
struct FileHeader {  // struct.Struct("<8sIIQQ")
  char magic[8];
  uint32_t version;
  uint32_t json_size;
  uint64_t data_offset;
  uint64_t reserved;
};
#pragma pack(pop)
static_assert(sizeof(FileHeader) == 32, "packed header");

size_t dtype_size(int d) { return d == INFER_HIP_DTYPE_FLOAT32 ? 4 : d == INFER_HIP_DTYPE_BFLOAT16 ? 2 : 1; }

}  // namespace

struct infer_hip_archive {
  std::string path;
  void* mapping = nullptr;
  size_t mapped_bytes = 0;
  int fd = -1;
  uint64_t data_offset = 0;
  std::string precision;
  struct Rec {
    std::string name;
    std::vector<int64_t> shape;
    int dtype = INFER_HIP_DTYPE_FLOAT32;
    uint64_t offset = 0;
    uint64_t nbytes = 0;
    int group_size = 0;
    int axis = 1;
    std::string scale_tensor;
    std::string sha256;  // "" when the record has none
  };
  std::vector<Rec> records;
  std::unordered_map<std::string, int> index;

  ~infer_hip_archive() {
    if (mapping) munmap(mapping, mapped_bytes);
    if (fd >= 0) ::close(fd);
  }
};

namespace {

bool as_u64(const Json* j, uint64_t& v) {
  if (!j || j->kind != Json::kNumber || !j->integral || j->integer < 0) return false;
  v = static_cast<uint64_t>(j->integer);
  return true;
}
bool as_int(const Json* j, int& v) {
  if (!j || j->kind != Json::kNumber || !j->integral || j->integer < INT32_MIN ||
      j->integer > INT32_MAX) {
    return false;
  }
  v = static_cast<int>(j->integer);
  return true;
}

}  // namespace

extern "C" int infer_hip_archive_open(const char* path, infer_hip_archive** out) {
  if (!out) return fail(INFER_HIP_INVALID_ARGUMENT, "archive: null output pointer");
  *out = nullptr;
  if (!path) return fail(INFER_HIP_INVALID_ARGUMENT, "archive: null path");
  std::unique_ptr<infer_hip_archive> a(new (std::nothrow) infer_hip_archive());
  if (!a) return fail(INFER_HIP_RUNTIME_ERROR, "archive: out of host memory");
  a->path = path;
  a->fd = ::open(path, O_RDONLY);
  if (a->fd < 0) return fail(INFER_HIP_INVALID_ARGUMENT, "cannot open archive: %s", path);
  struct stat st {};
  if (fstat(a->fd, &st) != 0) return fail(INFER_HIP_RUNTIME_ERROR, "cannot stat archive");
  a->mapped_bytes = static_cast<size_t>(st.st_size);
  // An empty file cannot be mapped (the reference's first error for it).
  a->mapping = a->mapped_bytes
                   ? mmap(nullptr, a->mapped_bytes, PROT_READ, MAP_PRIVATE, a->fd, 0)
                   : MAP_FAILED;
  if (a->mapping == MAP_FAILED) {
    a->mapping = nullptr;
    return fail(INFER_HIP_INVALID_ARGUMENT, "cannot mmap archive");
  }
  (void)madvise(a->mapping, a->mapped_bytes, MADV_SEQUENTIAL);
  if (a->mapped_bytes < sizeof(FileHeader)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "archive is truncated");
  }
  FileHeader header;
  std::memcpy(&header, a->mapping, sizeof header);
  if (std::memcmp(header.magic, kMagic, 8) != 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "bad archive magic");
  }
  if (header.version != 1) return fail(INFER_HIP_INVALID_ARGUMENT, "unsupported archive version");
  if (sizeof(FileHeader) + static_cast<uint64_t>(header.json_size) > a->mapped_bytes) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "bad archive JSON size");
  }
  if (header.data_offset >= a->mapped_bytes) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "bad archive data offset");
  }
  a->data_offset = header.data_offset;
  const char* json = static_cast<const char*>(a->mapping) + sizeof(FileHeader);
  Json meta;
  std::string error;
  if (!JsonParser(json, json + header.json_size).parse(meta, error)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "archive metadata: %s", error.c_str());
  }
  if (const Json* p = meta.get("precision"); p && p->kind == Json::kString) a->precision = p->str;
  const Json* tensors = meta.get("tensors");
  if (!tensors || tensors->kind != Json::kArray) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "archive metadata: no tensors array");
  }
  for (const Json& item : tensors->items) {
    infer_hip_archive::Rec rec;
    const Json* name = item.get("name");
    if (!name || name->kind != Json::kString) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "archive metadata: tensor without a name");
    }
    rec.name = name->str;
    const Json* shape = item.get("shape");
    if (!shape || shape->kind != Json::kArray || shape->items.size() > INFER_HIP_ARCHIVE_MAX_DIMS) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "archive metadata: bad shape of %s",
                  rec.name.c_str());
    }
    // numel exactly: `huge` marks a product past 2^64 (then no nbytes
    // matches it); a zero extent makes it 0 whatever the others are.
    uint64_t numel = 1;
    bool huge = false;
    for (const Json& d : shape->items) {
      uint64_t v;
      if (!as_u64(&d, v)) {
        return fail(INFER_HIP_INVALID_ARGUMENT, "archive metadata: bad shape of %s",
                    rec.name.c_str());
      }
      rec.shape.push_back(static_cast<int64_t>(v));
      if (numel != 0 && v > UINT64_MAX / numel) huge = true;
      numel *= v;
    }
    for (const int64_t v : rec.shape) {
      if (v == 0) huge = false;
    }
    const Json* dtype = item.get("dtype");
    const std::string dt = dtype && dtype->kind == Json::kString ? dtype->str : "";
    if (dt == "float32") {
      rec.dtype = INFER_HIP_DTYPE_FLOAT32;
    } else if (dt == "bfloat16") {
      rec.dtype = INFER_HIP_DTYPE_BFLOAT16;
    } else if (dt == "int8") {
      rec.dtype = INFER_HIP_DTYPE_INT8;
    } else {
      return fail(INFER_HIP_INVALID_ARGUMENT, "unsupported archive dtype: %s", dt.c_str());
    }
    if (!as_u64(item.get("offset"), rec.offset) || !as_u64(item.get("nbytes"), rec.nbytes)) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "archive metadata: bad offset or nbytes of %s",
                  rec.name.c_str());
    }
    const uint64_t elem = dtype_size(rec.dtype);
    if (huge || numel > UINT64_MAX / elem || rec.nbytes != numel * elem) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "tensor size mismatch: %s", rec.name.c_str());
    }
    if (a->data_offset + rec.offset + rec.nbytes > a->mapped_bytes ||
        rec.offset > a->mapped_bytes || rec.nbytes > a->mapped_bytes) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "tensor lies outside archive: %s", rec.name.c_str());
    }
    if (const Json* h = item.get("sha256"); h && h->kind == Json::kString) rec.sha256 = h->str;
    if (const Json* q = item.get("quant")) {
      const Json* scale = q->get("scale_tensor");
      if (!as_int(q->get("group_size"), rec.group_size) || rec.group_size <= 0 || !scale ||
          scale->kind != Json::kString) {
        return fail(INFER_HIP_INVALID_ARGUMENT, "archive metadata: bad quant record of %s",
                    rec.name.c_str());
      }
      if (const Json* axis = q->get("axis"); axis && !as_int(axis, rec.axis)) {
        return fail(INFER_HIP_INVALID_ARGUMENT, "archive metadata: bad quant axis of %s",
                    rec.name.c_str());
      }
      rec.scale_tensor = scale->str;
    }
    if (!a->index.emplace(rec.name, static_cast<int>(a->records.size())).second) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "duplicate tensor: %s", rec.name.c_str());
    }
    a->records.push_back(std::move(rec));
  }
  *out = a.release();
  return ok();
}

// Leaves the last error as it is, so that a caller can close an archive on
// its error path without losing the message.
extern "C" int infer_hip_archive_close(infer_hip_archive* a) {
  delete a;
  return INFER_HIP_OK;
}

extern "C" int infer_hip_archive_tensor_count(const infer_hip_archive* a) {
  return a ? static_cast<int>(a->records.size()) : 0;
}

extern "C" int infer_hip_archive_record(const infer_hip_archive* a, int index,
                                        infer_hip_tensor_record* out) {
  if (!a || !out) return fail(INFER_HIP_INVALID_ARGUMENT, "archive: null argument");
  if (index < 0 || index >= static_cast<int>(a->records.size())) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "archive: no record %d", index);
  }
  const auto& r = a->records[index];
  std::memset(out, 0, sizeof *out);
  out->name = r.name.c_str();
  out->ndim = static_cast<int>(r.shape.size());
  for (size_t i = 0; i < r.shape.size(); ++i) out->shape[i] = r.shape[i];
  out->dtype = r.dtype;
  out->offset = r.offset;
  out->nbytes = r.nbytes;
  out->quant_group_size = r.group_size;
  out->quant_axis = r.group_size ? r.axis : 0;
  out->scale_tensor = r.group_size ? r.scale_tensor.c_str() : nullptr;
  out->sha256 = r.sha256.c_str();
  return ok();
}

// verify_archive (export_model.py:148-199): every offset a multiple of 256
// and every payload's SHA-256 equal to its record's.
extern "C" int infer_hip_archive_verify(const infer_hip_archive* a) {
  if (!a) return fail(INFER_HIP_INVALID_ARGUMENT, "archive: null archive");
  for (const auto& r : a->records) {
    if (r.offset % kAlignment != 0) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "unaligned tensor %s", r.name.c_str());
    }
    Sha256 sha;
    sha.update(static_cast<const char*>(a->mapping) + a->data_offset + r.offset, r.nbytes);
    if (sha.hex() != r.sha256) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "SHA-256 mismatch for %s", r.name.c_str());
    }
  }
  return ok();
}

extern "C" int infer_hip_archive_find(const infer_hip_archive* a, const char* name) {
  if (!a || !name) return -1;
  const auto it = a->index.find(name);
  return it == a->index.end() ? -1 : it->second;
}

extern "C" const void* infer_hip_archive_data(const infer_hip_archive* a, int index) {
  if (!a || index < 0 || index >= static_cast<int>(a->records.size())) return nullptr;
  return static_cast<const char*>(a->mapping) + a->data_offset + a->records[index].offset;
}

extern "C" uint64_t infer_hip_archive_data_offset(const infer_hip_archive* a) {
  return a ? a->data_offset : 0;
}

extern "C" size_t infer_hip_archive_mapped_bytes(const infer_hip_archive* a) {
  return a ? a->mapped_bytes : 0;
}

extern "C" const char* infer_hip_archive_precision(const infer_hip_archive* a) {
  return a ? a->precision.c_str() : "";
}

// --------------------------------------------------------------- export --

namespace {

struct Writer {
  FILE* f = nullptr;
  std::string json_tensors;
  int records = 0;
  bool ok = true;

  // Pad the payload so the next tensor starts at a multiple of 256 bytes
  // from the data offset (align_file, export_model.py:103-108).
  uint64_t align() {
    const long pos = std::ftell(f);
    const uint64_t rel = static_cast<uint64_t>(pos) - kDataOffset;
    const uint64_t pad = (kAlignment - rel % kAlignment) % kAlignment;
    static const char zeros[kAlignment] = {};
    if (pad && std::fwrite(zeros, 1, pad, f) != pad) ok = false;
    return rel + pad;
  }

  void tensor(const std::string& name, const std::vector<int64_t>& shape, const char* dtype,
              const void* data, uint64_t nbytes, const std::string& quant_json) {
    const uint64_t offset = align();
    if (nbytes && std::fwrite(data, 1, nbytes, f) != nbytes) ok = false;
    Sha256 sha;
    sha.update(data, nbytes);
    std::string rec = "{\"name\":";
    json_escape(rec, name);
    rec += ",\"shape\":[";
    for (size_t i = 0; i < shape.size(); ++i) {
      if (i) rec += ",";
      rec += std::to_string(shape[i]);
    }
    rec += "],\"dtype\":\"";
    rec += dtype;
    rec += "\",\"offset\":" + std::to_string(offset) + ",\"nbytes\":" + std::to_string(nbytes) +
           ",\"sha256\":\"" + sha.hex() + "\"";
    if (!quant_json.empty()) rec += ",\"quant\":" + quant_json;
    rec += "}";
    if (records++) json_tensors += ",";
    json_tensors += rec;
  }
};

bool should_quantize(const std::string& name, int ndim) {  // export_model.py:220-223
  return ndim == 2 && name != "model.embed_tokens.weight" && name != "lm_head.weight";
}

}  // namespace

extern "C" int infer_hip_archive_export(const char* path, const char* precision, int group_size,
                                        const infer_hip_export_tensor* tensors, int count,
                                        const char* source, infer_hip_export_report* report) {
  if (!path || !precision || (count > 0 && !tensors) || count < 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "export: null argument");
  }
  const std::string prec = precision;
  if (prec != "w8a16" && prec != "w16a16" && prec != "fp32") {
    return fail(INFER_HIP_INVALID_ARGUMENT, "export: unknown precision %s", precision);
  }
  if (prec == "w8a16" && group_size != 64) {  // export_model.py:274-275
    return fail(INFER_HIP_INVALID_ARGUMENT, "w8a16 currently requires group size 64");
  }
  for (int i = 0; i < count; ++i) {
    const infer_hip_export_tensor& t = tensors[i];
    if (!t.name || t.ndim < 0 || t.ndim > INFER_HIP_ARCHIVE_MAX_DIMS || (t.ndim > 0 && !t.shape)) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "export: bad tensor %d", i);
    }
    for (int d = 0; d < t.ndim; ++d) {
      if (t.shape[d] < 0) return fail(INFER_HIP_INVALID_ARGUMENT, "export: bad shape of %s", t.name);
    }
  }
  Writer w;
  w.f = std::fopen(path, "w+b");
  if (!w.f) return fail(INFER_HIP_INVALID_ARGUMENT, "export: cannot create %s", path);
  // Payload from the data offset on; the header and metadata are written last.
  if (std::fseek(w.f, static_cast<long>(kDataOffset), SEEK_SET) != 0) w.ok = false;
  infer_hip_export_report rep{};
  const int old_round = std::fegetround();
  std::fesetround(FE_TONEAREST);  // np.rint: round half to even
  for (int i = 0; i < count && w.ok; ++i) {
    const infer_hip_export_tensor& t = tensors[i];
    std::vector<int64_t> shape(t.shape, t.shape + t.ndim);
    uint64_t numel = 1;
    for (int64_t d : shape) numel *= static_cast<uint64_t>(d);
    if (numel > 0 && !t.data) {
      w.ok = false;
      break;
    }
    const std::string name = t.name;
    if (prec == "w8a16" && should_quantize(name, t.ndim)) {
      // quantize_groupwise (export_model.py:226-247) in float32 throughout.
      const int64_t rows = shape[0], cols = shape[1];
      const int64_t groups = (cols + group_size - 1) / group_size;
      std::vector<int8_t> q(static_cast<size_t>(rows * cols));
      std::vector<uint16_t> s(static_cast<size_t>(rows * groups));
      double max_err = 0.0, scale_err = 0.0;
      for (int64_t r = 0; r < rows; ++r) {
        const float* row = t.data + r * cols;
        for (int64_t g = 0; g < groups; ++g) {
          const int64_t b = g * group_size, e = std::min<int64_t>(cols, b + group_size);
          float m = 0.0f;
          for (int64_t c = b; c < e; ++c) m = std::max(m, std::fabs(row[c]));
          float scale = m / 127.0f;
          if (scale == 0.0f) scale = 1.0f;
          const uint16_t sw = bf16_rne(scale);
          s[static_cast<size_t>(r * groups + g)] = sw;
          const float stored = bf16_value(sw);
          scale_err = std::max(scale_err, static_cast<double>(std::fabs(scale - stored)));
          for (int64_t c = b; c < e; ++c) {
            float v = std::nearbyint(row[c] / scale);
            v = std::min(127.0f, std::max(-127.0f, v));
            const int8_t qv = static_cast<int8_t>(v);
            q[static_cast<size_t>(r * cols + c)] = qv;
            // reconstruction error against the stored (BF16) scale
            max_err = std::max(max_err, static_cast<double>(std::fabs(
                                            row[c] - static_cast<float>(qv) * stored)));
          }
        }
      }
      const std::string scale_name = name + ".scale";
      std::string quant = "{\"scheme\":\"symmetric_group_w8a16\",\"group_size\":" +
                          std::to_string(group_size) + ",\"axis\":1,\"scale_tensor\":";
      json_escape(quant, scale_name);
      quant += ",\"scale_dtype\":\"bfloat16\"}";
      w.tensor(name, shape, "int8", q.data(), q.size(), quant);
      w.tensor(scale_name, {rows, groups}, "bfloat16", s.data(), s.size() * 2, "");
      rep.quantized_count += 1;
      rep.int8_count += 1;
      rep.bfloat16_count += 1;
      rep.max_groupwise_abs_error = std::max(rep.max_groupwise_abs_error, max_err);
      rep.max_bfloat16_abs_error = std::max(rep.max_bfloat16_abs_error, scale_err);
    } else if (prec == "w16a16" || prec == "w8a16") {
      std::vector<uint16_t> b(static_cast<size_t>(numel));
      double max_err = 0.0;
      for (uint64_t k = 0; k < numel; ++k) {
        b[k] = bf16_rne(t.data[k]);
        const double err = std::fabs(static_cast<double>(t.data[k]) - bf16_value(b[k]));
        if (err == err) max_err = std::max(max_err, err);
      }
      w.tensor(name, shape, "bfloat16", b.data(), b.size() * 2, "");
      rep.bfloat16_count += 1;
      rep.max_bfloat16_abs_error = std::max(rep.max_bfloat16_abs_error, max_err);
    } else {
      w.tensor(name, shape, "float32", t.data, numel * 4, "");
      rep.float32_count += 1;
    }
  }
  std::fesetround(old_round);
  rep.tensor_count = w.records;
  // metadata (export_model.py:353-364), compact separators
  std::string meta = "{\"format\":\"QWENBIN1\",\"version\":1,\"source\":";
  json_escape(meta, source ? source : "");
  meta += ",\"precision\":\"" + prec + "\",\"group_size\":" +
          (prec == "w8a16" ? std::to_string(group_size) : std::string("null")) +
          ",\"tensors\":[" + w.json_tensors + "]}";
  if (w.ok && sizeof(FileHeader) + meta.size() > kDataOffset) {
    std::fclose(w.f);
    return fail(INFER_HIP_INVALID_ARGUMENT, "archive JSON exceeds reserved header region");
  }
  // A payload-free archive still spans the reserved region.
  if (w.ok) {
    std::fseek(w.f, 0, SEEK_END);
    if (static_cast<uint64_t>(std::ftell(w.f)) < kDataOffset) {
      if (std::fseek(w.f, static_cast<long>(kDataOffset) - 1, SEEK_SET) != 0 ||
          std::fputc(0, w.f) == EOF) {
        w.ok = false;
      }
    }
  }
  FileHeader header{};
  std::memcpy(header.magic, kMagic, 8);
  header.version = 1;
  header.json_size = static_cast<uint32_t>(meta.size());
  header.data_offset = kDataOffset;
  if (w.ok && (std::fseek(w.f, 0, SEEK_SET) != 0 ||
               std::fwrite(&header, sizeof header, 1, w.f) != 1 ||
               std::fwrite(meta.data(), 1, meta.size(), w.f) != meta.size())) {
    w.ok = false;
  }
  if (w.ok) {
    std::fseek(w.f, 0, SEEK_END);
    rep.bytes = static_cast<uint64_t>(std::ftell(w.f));
  }
  if (std::fclose(w.f) != 0) w.ok = false;
  if (!w.ok) return fail(INFER_HIP_RUNTIME_ERROR, "export: cannot write %s", path);
  if (report) *report = rep;
  return ok();
}

// ---------------------------------------------------------- config.json --

extern "C" int infer_hip_model_config_load(const char* path, infer_hip_model_config* config,
                                           int* max_position_embeddings) {
  if (!path || !config) return fail(INFER_HIP_INVALID_ARGUMENT, "config: null argument");
  FILE* f = std::fopen(path, "rb");
  if (!f) return fail(INFER_HIP_INVALID_ARGUMENT, "cannot open model config: %s", path);
  std::string text;
  char buf[4096];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, n);
  std::fclose(f);
  Json j;
  std::string error;
  if (!JsonParser(text.data(), text.data() + text.size()).parse(j, error)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model config: %s", error.c_str());
  }
  const Json* type = j.get("model_type");
  if (!type || type->kind != Json::kString || type->str != "qwen2") {
    return fail(INFER_HIP_INVALID_ARGUMENT, "only model_type=qwen2 is supported");
  }
  infer_hip_model_config c{};
  int max_pos = 0;
  if (!as_int(j.get("hidden_size"), c.hidden_size) ||
      !as_int(j.get("intermediate_size"), c.intermediate_size) ||
      !as_int(j.get("num_hidden_layers"), c.num_layers) ||
      !as_int(j.get("num_attention_heads"), c.num_heads) ||
      !as_int(j.get("num_key_value_heads"), c.num_kv_heads) ||
      !as_int(j.get("vocab_size"), c.vocab_size) ||
      !as_int(j.get("max_position_embeddings"), max_pos)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model config: missing or non-integer field");
  }
  // The optional fields (model_config.cpp:30-34): absent takes the default;
  // present with another JSON type (null included) is an error, as
  // nlohmann's value() raises for it.  bos_token_id and tie_word_embeddings
  // are checked and not kept (the reference keeps them but never reads them).
  c.eos_token_id = -1;
  if (const Json* e = j.get("eos_token_id"); e && !as_int(e, c.eos_token_id)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model config: bad eos_token_id");
  }
  int bos_token_id = -1;
  if (const Json* e = j.get("bos_token_id"); e && !as_int(e, bos_token_id)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model config: bad bos_token_id");
  }
  c.rms_norm_eps = 1e-6f;
  if (const Json* e = j.get("rms_norm_eps")) {
    if (e->kind != Json::kNumber) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "model config: bad rms_norm_eps");
    }
    c.rms_norm_eps = static_cast<float>(e->num);
  }
  c.rope_theta = 1e6f;
  if (const Json* e = j.get("rope_theta")) {
    if (e->kind != Json::kNumber) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "model config: bad rope_theta");
    }
    c.rope_theta = static_cast<float>(e->num);
  }
  if (const Json* e = j.get("tie_word_embeddings"); e && e->kind != Json::kBool) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model config: bad tie_word_embeddings");
  }
  // model_config.cpp:39-46
  if (c.hidden_size <= 0 || c.intermediate_size <= 0 || c.num_layers <= 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "invalid model dimensions");
  }
  if (c.num_heads <= 0 || c.num_kv_heads <= 0 || c.num_heads % c.num_kv_heads != 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "invalid GQA head counts");
  }
  if (c.hidden_size % c.num_heads != 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "invalid attention head dimension");
  }
  if (c.vocab_size <= 0) return fail(INFER_HIP_INVALID_ARGUMENT, "invalid vocabulary size");
  *config = c;
  if (max_position_embeddings) *max_position_embeddings = max_pos;
  return ok();
}
