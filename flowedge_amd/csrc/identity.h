// Model identity of a checkpoint: the 16-byte fingerprint and the precision class that the
// reference reports in fe_model_metadata and checks in versioned flow requests
// (src/core/protocol/model_identity.cc:104-165, engine_runtime.cc:159-161).
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <vector>

#include "safetensors.h"

namespace fe {

using Digest = std::array<std::uint8_t, 16>;

// XXH64 of `len` bytes (the published xxHash64 algorithm; the reference's hash64,
// model_identity.cc:54-101, is this function).
std::uint64_t xxh64(const void* data, std::size_t len, std::uint64_t seed);

// Fingerprint over the tensors in checkpoint order: name, dtype/rank, shape and content of each
// (model_identity.cc:124-148).  Content hashes run on up to `threads` host threads.
Digest fingerprint_tensors(const std::vector<TensorInfo>& tensors, unsigned threads);

// FE_PRECISION_* class of the checkpoint's tensors (model_identity.cc:150-165).
std::uint32_t checkpoint_precision(const std::vector<TensorInfo>& tensors);

}  // namespace fe
