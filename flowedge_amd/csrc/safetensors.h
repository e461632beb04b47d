// Read-only safetensors view over an mmapped checkpoint (F32 / BF16 tensors).
//
// Contract follows the reference loader (src/core/loader/safetensors.cc:168-238, 365-482):
// little-endian u64 header length, JSON header of {name: {dtype, shape, data_offsets}},
// `__metadata__` skipped, tensors of other dtypes ignored, every tensor's byte length must equal
// prod(shape) * element size, spans must lie inside the data section and must not overlap.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace fe {

struct TensorInfo {
  std::string name;
  bool bf16 = false;
  std::vector<std::size_t> shape;
  const void* data = nullptr;
  std::size_t bytes = 0;

  std::size_t elements() const {
    std::size_t n = 1;
    for (std::size_t s : shape) n *= s;
    return n;
  }
};

class Checkpoint {
 public:
  // Returns nullptr and sets `error` on failure.
  static std::shared_ptr<const Checkpoint> open(const char* path, std::string& error);
  ~Checkpoint();
  Checkpoint(const Checkpoint&) = delete;
  Checkpoint& operator=(const Checkpoint&) = delete;

  const TensorInfo* find(const std::string& name) const;
  const std::vector<TensorInfo>& tensors() const { return tensors_; }
  std::size_t weight_bytes() const { return weight_bytes_; }
  // Model fingerprint and FE_PRECISION_* class, computed once at open.
  const std::array<std::uint8_t, 16>& digest() const { return digest_; }
  std::uint32_t precision() const { return precision_; }

 private:
  Checkpoint() = default;
  void* map_ = nullptr;
  std::size_t map_size_ = 0;
  std::vector<TensorInfo> tensors_;
  std::size_t weight_bytes_ = 0;
  std::array<std::uint8_t, 16> digest_{};
  std::uint32_t precision_ = 0;
};

}  // namespace fe
