// safetensors.cpp -- see safetensors.hpp.
#include "safetensors.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <stdexcept>

namespace w4 {

namespace {

[[noreturn]] void bad(const std::string& what) { throw std::runtime_error("safetensors: " + what); }

// Minimal JSON reader for the safetensors header: objects, arrays, strings,
// integers, and (inside __metadata__) string values.  Other JSON values are
// accepted and skipped where the format allows them.
class Json {
 public:
  explicit Json(const std::string& s) : s_(s) {}

  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
  }
  bool peek(char c) {
    ws();
    return i_ < s_.size() && s_[i_] == c;
  }
  void expect(char c) {
    ws();
    if (i_ >= s_.size() || s_[i_] != c) bad(std::string("expected '") + c + "' at offset " + std::to_string(i_));
    ++i_;
  }
  std::string str() {
    expect('"');
    std::string out;
    while (true) {
      if (i_ >= s_.size()) bad("unterminated string");
      const char c = s_[i_++];
      if (c == '"') break;
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      if (i_ >= s_.size()) bad("bad escape");
      const char e = s_[i_++];
      switch (e) {
        case '"': out.push_back('"'); break;
        case '\\': out.push_back('\\'); break;
        case '/': out.push_back('/'); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': {
          if (i_ + 4 > s_.size()) bad("bad \\u escape");
          const unsigned cp = (unsigned)std::stoul(s_.substr(i_, 4), nullptr, 16);
          i_ += 4;
          // UTF-8 encode (the BMP is enough for tensor names)
          if (cp < 0x80) out.push_back((char)cp);
          else if (cp < 0x800) { out.push_back((char)(0xC0 | (cp >> 6))); out.push_back((char)(0x80 | (cp & 0x3F))); }
          else {
            out.push_back((char)(0xE0 | (cp >> 12)));
            out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
          }
          break;
        }
        default: bad("bad escape");
      }
    }
    return out;
  }
  int64_t integer() {
    ws();
    size_t j = i_;
    if (j < s_.size() && s_[j] == '-') ++j;
    const size_t digits = j;
    while (j < s_.size() && s_[j] >= '0' && s_[j] <= '9') ++j;
    if (j == digits) bad("expected an integer at offset " + std::to_string(i_));
    if (j < s_.size() && (s_[j] == '.' || s_[j] == 'e' || s_[j] == 'E')) bad("non-integer number in header");
    const int64_t v = std::stoll(s_.substr(i_, j - i_));
    i_ = j;
    return v;
  }
  std::vector<int64_t> int_array() {
    std::vector<int64_t> v;
    expect('[');
    if (peek(']')) { ++i_; return v; }
    while (true) {
      v.push_back(integer());
      if (peek(',')) { ++i_; continue; }
      expect(']');
      return v;
    }
  }
  // Skip any JSON value (used for unknown fields).
  void skip() {
    ws();
    if (i_ >= s_.size()) bad("unexpected end");
    const char c = s_[i_];
    if (c == '"') { str(); return; }
    if (c == '{') {
      ++i_;
      if (peek('}')) { ++i_; return; }
      while (true) {
        str();
        expect(':');
        skip();
        if (peek(',')) { ++i_; continue; }
        expect('}');
        return;
      }
    }
    if (c == '[') {
      ++i_;
      if (peek(']')) { ++i_; return; }
      while (true) {
        skip();
        if (peek(',')) { ++i_; continue; }
        expect(']');
        return;
      }
    }
    // number / true / false / null
    size_t j = i_;
    while (j < s_.size() && s_[j] != ',' && s_[j] != '}' && s_[j] != ']' && s_[j] != ' ' && s_[j] != '\n') ++j;
    if (j == i_) bad("bad value at offset " + std::to_string(i_));
    i_ = j;
  }
  bool done() {
    ws();
    return i_ == s_.size();
  }

 private:
  const std::string& s_;
  size_t i_ = 0;
};

}  // namespace

int64_t TensorInfo::numel() const {
  // dims are checked non-negative and their product checked for overflow when the
  // header is parsed (numel_checked), so this product fits
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}

namespace {
// Product of the dims times the element size, or false when it overflows 63 bits
// (a crafted shape such as [2^62, 4] would otherwise wrap to a small byte count
// and pass the data_offsets check).
bool numel_checked(const std::vector<int64_t>& shape, size_t es, uint64_t* bytes) {
  int64_t n = 1;
  for (int64_t d : shape)
    if (__builtin_mul_overflow(n, d, &n)) return false;
  int64_t b;
  if (__builtin_mul_overflow(n, (int64_t)es, &b)) return false;
  *bytes = (uint64_t)b;
  return true;
}
}  // namespace

size_t dtype_size(const std::string& d) {
  if (d == "BOOL" || d == "U8" || d == "I8" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
  if (d == "I16" || d == "U16" || d == "F16" || d == "BF16") return 2;
  if (d == "I32" || d == "U32" || d == "F32") return 4;
  if (d == "I64" || d == "U64" || d == "F64") return 8;
  return 0;
}

void SafeTensorsFile::parse_header(const std::string& json, uint64_t data_size, std::map<std::string, TensorInfo>& tensors,
                                   std::map<std::string, std::string>& metadata) {
  Json p(json);
  p.expect('{');
  if (p.peek('}')) {
    p.expect('}');
    return;
  }
  while (true) {
    const std::string name = p.str();
    p.expect(':');
    if (name == "__metadata__") {
      p.expect('{');
      if (!p.peek('}')) {
        while (true) {
          const std::string k = p.str();
          p.expect(':');
          metadata[k] = p.str();
          if (p.peek(',')) { p.expect(','); continue; }
          break;
        }
      }
      p.expect('}');
    } else {
      TensorInfo t;
      bool has_dtype = false, has_shape = false, has_off = false;
      p.expect('{');
      while (true) {
        const std::string k = p.str();
        p.expect(':');
        if (k == "dtype") { t.dtype = p.str(); has_dtype = true; }
        else if (k == "shape") { t.shape = p.int_array(); has_shape = true; }
        else if (k == "data_offsets") {
          const auto off = p.int_array();
          if (off.size() != 2 || off[0] < 0 || off[1] < off[0]) bad(name + ": bad data_offsets");
          t.begin = (uint64_t)off[0];
          t.end = (uint64_t)off[1];
          has_off = true;
        } else {
          p.skip();
        }
        if (p.peek(',')) { p.expect(','); continue; }
        break;
      }
      p.expect('}');
      if (!has_dtype || !has_shape || !has_off) bad(name + ": missing dtype, shape or data_offsets");
      for (int64_t d : t.shape)
        if (d < 0) bad(name + ": negative dimension");
      const size_t es = dtype_size(t.dtype);
      if (es == 0) bad(name + ": unknown dtype " + t.dtype);
      uint64_t nbytes = 0;
      if (!numel_checked(t.shape, es, &nbytes)) bad(name + ": shape x dtype overflows 64 bits");
      if (nbytes != t.end - t.begin) bad(name + ": data_offsets do not match shape x dtype");
      if (t.end > data_size) bad(name + ": data_offsets past the end of the file");
      if (tensors.count(name)) bad(name + ": duplicate tensor name");
      tensors[name] = t;
    }
    if (p.peek(',')) { p.expect(','); continue; }
    break;
  }
  p.expect('}');
  if (!p.done()) bad("trailing bytes after the header");
}

SafeTensorsFile::SafeTensorsFile(const std::string& path) : path_(path) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) bad("cannot open " + path);
  struct stat st;
  if (fstat(fd, &st) != 0) { ::close(fd); bad("cannot stat " + path); }
  map_size_ = (size_t)st.st_size;
  if (map_size_ < 8) { ::close(fd); bad(path + ": shorter than the 8-byte header length"); }
  map_ = mmap(nullptr, map_size_, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (map_ == MAP_FAILED) { map_ = nullptr; bad("cannot map " + path); }
  const uint8_t* b = static_cast<const uint8_t*>(map_);
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | b[i];  // little endian
  if (hlen > map_size_ - 8) {
    munmap(map_, map_size_);
    map_ = nullptr;
    bad(path + ": header length past the end of the file");
  }
  data_ = b + 8 + hlen;
  try {
    parse_header(std::string(reinterpret_cast<const char*>(b + 8), (size_t)hlen), map_size_ - 8 - hlen, tensors_, metadata_);
  } catch (...) {
    munmap(map_, map_size_);
    map_ = nullptr;
    throw;
  }
}

SafeTensorsFile::~SafeTensorsFile() {
  if (map_) munmap(map_, map_size_);
  map_ = nullptr;
}

SafeTensorsFile::SafeTensorsFile(SafeTensorsFile&& o) noexcept { *this = std::move(o); }

SafeTensorsFile& SafeTensorsFile::operator=(SafeTensorsFile&& o) noexcept {
  if (this != &o) {
    if (map_) munmap(map_, map_size_);
    path_ = std::move(o.path_);
    map_ = o.map_;
    map_size_ = o.map_size_;
    data_ = o.data_;
    tensors_ = std::move(o.tensors_);
    metadata_ = std::move(o.metadata_);
    o.map_ = nullptr;
    o.data_ = nullptr;
    o.map_size_ = 0;
  }
  return *this;
}

const TensorInfo& SafeTensorsFile::info(const std::string& name) const {
  auto it = tensors_.find(name);
  if (it == tensors_.end()) bad(path_ + ": no tensor " + name);
  return it->second;
}

const void* SafeTensorsFile::data(const std::string& name) const { return data_ + info(name).begin; }

}  // namespace w4
