#include "safetensors.h"

#include "identity.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cstring>
#include <thread>
#include <utility>

namespace fe {
namespace {

// A reader for the safetensors JSON header: one object whose members are tensor entries
// {"dtype": "...", "shape": [...], "data_offsets": [a, b]} plus an optional "__metadata__" object.
// Strings are decoded with their escapes, so a name holding braces, quotes or the text of a dtype
// is read as what it is.  Values the loader does not use (metadata, unknown keys) are skipped.
class Json {
 public:
  explicit Json(const std::string& s) : s_(s) {}

  bool eat(char c) {
    ws();
    if (p_ < s_.size() && s_[p_] == c) {
      ++p_;
      return true;
    }
    return false;
  }
  bool peek(char c) {
    ws();
    return p_ < s_.size() && s_[p_] == c;
  }

  bool string(std::string& out) {
    out.clear();
    if (!eat('"')) return false;
    while (p_ < s_.size()) {
      const unsigned char c = static_cast<unsigned char>(s_[p_++]);
      if (c == '"') return true;
      if (c < 0x20) return false;
      if (c != '\\') {
        out.push_back(static_cast<char>(c));
        continue;
      }
      if (p_ >= s_.size()) return false;
      const char e = s_[p_++];
      switch (e) {
        case '"': case '\\': case '/': out.push_back(e); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': {
          std::uint32_t cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            std::uint32_t lo;
            if (p_ + 1 >= s_.size() || s_[p_] != '\\' || s_[p_ + 1] != 'u') return false;
            p_ += 2;
            if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            return false;
          }
          utf8(cp, out);
          break;
        }
        default: return false;
      }
    }
    return false;
  }

  // A non-negative integer (shape and offset entries).
  bool uint(std::uint64_t& v) {
    ws();
    v = 0;
    const std::size_t p0 = p_;
    while (p_ < s_.size() && s_[p_] >= '0' && s_[p_] <= '9') {
      const auto d = static_cast<std::uint64_t>(s_[p_++] - '0');
      if (v > (UINT64_MAX - d) / 10) return false;
      v = v * 10 + d;
    }
    return p_ > p0;
  }

  bool uint_list(std::vector<std::uint64_t>& out) {
    out.clear();
    if (!eat('[')) return false;
    if (eat(']')) return true;
    do {
      std::uint64_t v;
      if (!uint(v)) return false;
      out.push_back(v);
    } while (eat(','));
    return eat(']');
  }

  // Skips any JSON value.
  bool skip(int depth = 0) {
    if (depth > 64) return false;
    ws();
    if (p_ >= s_.size()) return false;
    const char c = s_[p_];
    std::string tmp;
    if (c == '"') return string(tmp);
    if (c == '{' || c == '[') {
      const char close = c == '{' ? '}' : ']';
      ++p_;
      if (eat(close)) return true;
      do {
        if (c == '{' && (!string(tmp) || !eat(':'))) return false;
        if (!skip(depth + 1)) return false;
      } while (eat(','));
      return eat(close);
    }
    const std::size_t p0 = p_;
    while (p_ < s_.size() && (std::isalnum(static_cast<unsigned char>(s_[p_])) ||
                              s_[p_] == '-' || s_[p_] == '+' || s_[p_] == '.'))
      ++p_;
    return p_ > p0;
  }

 private:
  void ws() {
    while (p_ < s_.size() &&
           (s_[p_] == ' ' || s_[p_] == '\n' || s_[p_] == '\t' || s_[p_] == '\r'))
      ++p_;
  }
  bool hex4(std::uint32_t& v) {
    v = 0;
    for (int i = 0; i < 4; ++i) {
      if (p_ >= s_.size()) return false;
      const char h = s_[p_++];
      v <<= 4;
      if (h >= '0' && h <= '9') v |= static_cast<std::uint32_t>(h - '0');
      else if (h >= 'a' && h <= 'f') v |= static_cast<std::uint32_t>(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') v |= static_cast<std::uint32_t>(h - 'A' + 10);
      else return false;
    }
    return true;
  }
  static void utf8(std::uint32_t cp, std::string& out) {
    if (cp < 0x80) {
      out.push_back(static_cast<char>(cp));
    } else if (cp < 0x800) {
      out.push_back(static_cast<char>(0xC0 | (cp >> 6)));
      out.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
      out.push_back(static_cast<char>(0xE0 | (cp >> 12)));
      out.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
      out.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else {
      out.push_back(static_cast<char>(0xF0 | (cp >> 18)));
      out.push_back(static_cast<char>(0x80 | ((cp >> 12) & 0x3F)));
      out.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
      out.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    }
  }

  const std::string& s_;
  std::size_t p_ = 0;
};

struct Entry {
  std::string dtype;
  std::vector<std::uint64_t> shape, offsets;
  bool has_shape = false, has_offsets = false;
};

// One tensor entry object; keys other than dtype, shape and data_offsets are skipped.
bool parse_entry(Json& j, Entry& e) {
  if (!j.eat('{')) return false;
  if (j.eat('}')) return true;
  std::string key;
  do {
    if (!j.string(key) || !j.eat(':')) return false;
    if (key == "dtype") {
      if (!j.string(e.dtype)) return false;
    } else if (key == "shape") {
      if (!j.uint_list(e.shape)) return false;
      e.has_shape = true;
    } else if (key == "data_offsets") {
      if (!j.uint_list(e.offsets)) return false;
      e.has_offsets = true;
    } else if (!j.skip()) {
      return false;
    }
  } while (j.eat(','));
  return j.eat('}');
}

}  // namespace

Checkpoint::~Checkpoint() {
  if (map_) munmap(map_, map_size_);
}

std::shared_ptr<const Checkpoint> Checkpoint::open(const char* path, std::string& error) {
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) {
    error = std::string("cannot open checkpoint: ") + path;
    return nullptr;
  }
  struct stat st {};
  if (fstat(fd, &st) != 0 || st.st_size < 8) {
    ::close(fd);
    error = "checkpoint file too small";
    return nullptr;
  }
  const std::size_t size = static_cast<std::size_t>(st.st_size);
  void* map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (map == MAP_FAILED) {
    error = "cannot map checkpoint";
    return nullptr;
  }
  std::shared_ptr<Checkpoint> ck(new Checkpoint());
  ck->map_ = map;
  ck->map_size_ = size;
  const auto* bytes = static_cast<const unsigned char*>(map);
  std::uint64_t header_len = 0;
  std::memcpy(&header_len, bytes, 8);  // little-endian host
  if (header_len > size - 8) {
    error = "invalid safetensors header length";
    return nullptr;
  }
  const std::string header(reinterpret_cast<const char*>(bytes + 8), header_len);
  const unsigned char* data = bytes + 8 + header_len;
  const std::uint64_t data_size = size - 8 - header_len;
  std::vector<std::pair<std::uint64_t, std::uint64_t>> spans;

  Json j(header);
  bool closed = false;
  if (j.eat('{')) {
    closed = j.eat('}');
    std::string name;
    while (!closed) {
      Entry ent;
      if (!j.string(name) || !j.eat(':')) break;
      if (name == "__metadata__") {
        if (!j.skip()) break;
      } else {
        if (!parse_entry(j, ent)) {
          error = "malformed tensor entry: " + name;
          return nullptr;
        }
        const bool f32 = ent.dtype == "F32";
        const bool bf16 = ent.dtype == "BF16";
        if (f32 || bf16) {
          if (!ent.has_shape || ent.shape.size() > 4 || !ent.has_offsets ||
              ent.offsets.size() != 2 || ent.offsets[1] < ent.offsets[0]) {
            error = "malformed tensor entry: " + name;
            return nullptr;
          }
          const std::vector<std::uint64_t>& offs = ent.offsets;
          const std::uint64_t len = offs[1] - offs[0];
          if (offs[0] > data_size || len > data_size - offs[0]) {
            error = "tensor storage out of bounds: " + name;
            return nullptr;
          }
          for (const auto& sp : spans)
            if (offs[0] < sp.second && sp.first < offs[1]) {
              error = "overlapping tensor storage: " + name;
              return nullptr;
            }
          spans.emplace_back(offs[0], offs[1]);
          TensorInfo t;
          t.name = name;
          t.bf16 = bf16;
          std::uint64_t elements = 1;
          for (std::uint64_t d : ent.shape) {
            if (d != 0 && elements > UINT64_MAX / d) {
              error = "tensor shape overflow";
              return nullptr;
            }
            elements *= d;
            t.shape.push_back(static_cast<std::size_t>(d));
          }
          const std::uint64_t esize = bf16 ? 2 : 4;
          if (elements > UINT64_MAX / esize || elements * esize != len) {
            error = "tensor byte length does not match shape: " + t.name;
            return nullptr;
          }
          t.data = data + offs[0];
          t.bytes = static_cast<std::size_t>(len);
          ck->weight_bytes_ += t.bytes;
          ck->tensors_.push_back(std::move(t));
        }
      }
      if (j.eat('}')) {
        closed = true;
        break;
      }
      if (!j.eat(',')) break;
    }
  }
  if (!closed || ck->tensors_.empty()) {
    error = "malformed safetensors header";
    return nullptr;
  }
  const unsigned hw = std::thread::hardware_concurrency();
  ck->digest_ = fingerprint_tensors(ck->tensors_, std::min(hw == 0 ? 1u : hw, 8u));
  ck->precision_ = checkpoint_precision(ck->tensors_);
  return ck;
}

const TensorInfo* Checkpoint::find(const std::string& name) const {
  for (const auto& t : tensors_)
    if (t.name == name) return &t;
  return nullptr;
}

}  // namespace fe
