#include "safetensors.h"

#include "identity.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <thread>
#include <utility>

namespace fe {
namespace {

// Parses "[a, b, ...]" starting at the first '[' at or after `pos`.
bool parse_list(const std::string& s, std::size_t pos, std::vector<std::uint64_t>& out) {
  out.clear();
  if (pos == std::string::npos) return false;
  pos = s.find('[', pos);
  if (pos == std::string::npos) return false;
  std::uint64_t v = 0;
  bool have = false;
  for (++pos; pos < s.size(); ++pos) {
    const char c = s[pos];
    if (c >= '0' && c <= '9') {
      if (v > (UINT64_MAX - 9) / 10) return false;
      v = v * 10 + static_cast<std::uint64_t>(c - '0');
      have = true;
    } else if (c == ',' || c == ']') {
      if (have) out.push_back(v);
      else if (c == ',') return false;
      v = 0;
      have = false;
      if (c == ']') return true;
    } else if (c != ' ' && c != '\n' && c != '\t' && c != '\r') {
      return false;
    }
  }
  return false;
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

  std::size_t p = header.find('{');
  if (p == std::string::npos) {
    error = "malformed safetensors header";
    return nullptr;
  }
  ++p;
  bool closed = false;
  while (p < header.size()) {
    while (p < header.size() && header[p] != '"' && header[p] != '}') ++p;
    if (p >= header.size()) break;
    if (header[p] == '}') {
      closed = true;
      break;
    }
    const std::size_t n0 = p + 1;
    const std::size_t n1 = header.find('"', n0);
    if (n1 == std::string::npos) break;
    std::string name = header.substr(n0, n1 - n0);
    const std::size_t ob = header.find('{', n1);
    if (ob == std::string::npos) break;
    int depth = 1;
    std::size_t e = ob + 1;
    for (; e < header.size() && depth > 0; ++e) depth += (header[e] == '{') - (header[e] == '}');
    if (depth != 0) break;
    const std::string obj = header.substr(ob, e - ob);
    p = e;
    if (name == "__metadata__") continue;
    const bool f32 = obj.find("\"F32\"") != std::string::npos;
    const bool bf16 = obj.find("\"BF16\"") != std::string::npos;
    if (!f32 && !bf16) continue;
    std::vector<std::uint64_t> shape, offs;
    if (!parse_list(obj, obj.find("\"shape\""), shape) || shape.size() > 4 ||
        !parse_list(obj, obj.find("\"data_offsets\""), offs) || offs.size() != 2 ||
        offs[1] < offs[0]) {
      error = "malformed tensor entry: " + name;
      return nullptr;
    }
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
    t.name = std::move(name);
    t.bf16 = bf16;
    std::uint64_t elements = 1;
    for (std::uint64_t s : shape) {
      if (s != 0 && elements > UINT64_MAX / s) {
        error = "tensor shape overflow";
        return nullptr;
      }
      elements *= s;
      t.shape.push_back(static_cast<std::size_t>(s));
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
