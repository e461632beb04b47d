#include "identity.h"

#include <algorithm>
#include <atomic>
#include <cstring>
#include <thread>

namespace fe {
namespace {

// xxHash64 primes (xxHash specification, "XXH64 algorithm description").
constexpr std::uint64_t P1 = 0x9E3779B185EBCA87ull;
constexpr std::uint64_t P2 = 0xC2B2AE3D27D4EB4Full;
constexpr std::uint64_t P3 = 0x165667B19E3779F9ull;
constexpr std::uint64_t P4 = 0x85EBCA77C2B2AE63ull;
constexpr std::uint64_t P5 = 0x27D4EB2F165667C5ull;

inline std::uint64_t rotl(std::uint64_t v, int r) { return (v << r) | (v >> (64 - r)); }

inline std::uint64_t load64(const unsigned char* p) {
  std::uint64_t v;
  std::memcpy(&v, p, 8);  // little-endian host (x86-64)
  return v;
}

inline std::uint32_t load32(const unsigned char* p) {
  std::uint32_t v;
  std::memcpy(&v, p, 4);
  return v;
}

inline std::uint64_t xround(std::uint64_t acc, std::uint64_t lane) {
  return rotl(acc + lane * P2, 31) * P1;
}

inline std::uint64_t mix_final(std::uint64_t h) {
  h = (h ^ (h >> 33)) * P2;
  h = (h ^ (h >> 29)) * P3;
  return h ^ (h >> 32);
}

// One 64-bit value folded into a running fingerprint lane (model_identity.cc:98-102); the same
// step as XXH64's 8-byte tail.
inline std::uint64_t fold(std::uint64_t acc, std::uint64_t value) {
  return rotl(acc ^ xround(0, value), 27) * P1 + P4;
}

Digest to_digest(std::uint64_t lo, std::uint64_t hi) {
  Digest d{};
  for (int i = 0; i < 8; ++i) {
    d[i] = static_cast<std::uint8_t>(lo >> (8 * i));
    d[8 + i] = static_cast<std::uint8_t>(hi >> (8 * i));
  }
  return d;
}

}  // namespace

std::uint64_t xxh64(const void* data, std::size_t len, std::uint64_t seed) {
  const auto* p = static_cast<const unsigned char*>(data);
  const unsigned char* const end = p + len;
  std::uint64_t h;
  if (len >= 32) {
    std::uint64_t a = seed + P1 + P2, b = seed + P2, c = seed, d = seed - P1;
    const unsigned char* const last = end - 32;
    do {
      a = xround(a, load64(p));
      b = xround(b, load64(p + 8));
      c = xround(c, load64(p + 16));
      d = xround(d, load64(p + 24));
      p += 32;
    } while (p <= last);
    h = rotl(a, 1) + rotl(b, 7) + rotl(c, 12) + rotl(d, 18);
    for (std::uint64_t v : {a, b, c, d}) h = (h ^ xround(0, v)) * P1 + P4;
  } else {
    h = seed + P5;
  }
  h += static_cast<std::uint64_t>(len);
  for (; p + 8 <= end; p += 8) h = rotl(h ^ xround(0, load64(p)), 27) * P1 + P4;
  if (p + 4 <= end) {
    h = rotl(h ^ (static_cast<std::uint64_t>(load32(p)) * P1), 23) * P2 + P3;
    p += 4;
  }
  for (; p < end; ++p) h = rotl(h ^ (static_cast<std::uint64_t>(*p) * P5), 11) * P1;
  return mix_final(h);
}

Digest fingerprint_tensors(const std::vector<TensorInfo>& tensors, unsigned threads) {
  // Content hashes are independent per tensor; only their combination is ordered.
  const std::size_t n = tensors.size();
  std::vector<std::uint64_t> content(n);
  std::atomic<std::size_t> next{0};
  auto work = [&]() {
    for (std::size_t i = next.fetch_add(1); i < n; i = next.fetch_add(1))
      content[i] = xxh64(tensors[i].data, tensors[i].bytes, P5);
  };
  const unsigned workers = std::max(1u, std::min<unsigned>(threads, static_cast<unsigned>(n)));
  std::vector<std::thread> pool;
  for (unsigned w = 1; w < workers; ++w) pool.emplace_back(work);
  work();
  for (auto& t : pool) t.join();

  // model_identity.cc:124-148.  Names longer than 127 bytes are cut as the reference's
  // TensorView name buffer cuts them (loader/safetensors.h:32, safetensors.cc:474-476).
  std::uint64_t first = fold(0x243f6a8885a308d3ull, n);
  std::uint64_t second = fold(0x13198a2e03707344ull, n);
  for (std::size_t i = 0; i < n; ++i) {
    const TensorInfo& t = tensors[i];
    const std::size_t name_len = std::min<std::size_t>(t.name.size(), 127);
    const std::uint64_t name_hash = xxh64(t.name.data(), name_len, P3);
    first = fold(first, name_hash);
    second = fold(second, rotl(name_hash, 17));
    const std::uint64_t format =
        (t.bf16 ? 1ull : 0ull) | (static_cast<std::uint64_t>(t.shape.size()) << 8);
    first = fold(first, format);
    second = fold(second, format ^ static_cast<std::uint64_t>(t.bytes));
    for (std::size_t s : t.shape) {
      first = fold(first, s);
      second = fold(second, rotl(static_cast<std::uint64_t>(s), 23));
    }
    first = fold(first, content[i]);
    second = fold(second, rotl(content[i], 31) ^ static_cast<std::uint64_t>(t.bytes));
  }
  return to_digest(mix_final(first), mix_final(second));
}

std::uint32_t checkpoint_precision(const std::vector<TensorInfo>& tensors) {
  bool f32 = false, bf16 = false;
  for (const TensorInfo& t : tensors) (t.bf16 ? bf16 : f32) = true;
  // FE_PRECISION_{MIXED=3, BF16=2, F32=1, UNKNOWN=0} (protocol/contracts.h:29-35).
  return f32 && bf16 ? 3u : bf16 ? 2u : f32 ? 1u : 0u;
}

}  // namespace fe
