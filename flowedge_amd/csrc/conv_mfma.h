// Shared pieces of the batched (matrix-core) convolution kernels: the implicit-GEMM argument
// block, the input index of a tap, and the BF16-MFMA launcher (conv_mfma_bf16.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace fe::hip::mm {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kMmThreads = 256;

// Column tiles: 64 output channels x 128 columns, or 64 x 64 when the larger column tile would
// leave CUs without a workgroup.
enum MmTile : int { kTile64x128 = 0, kTile64x64 = 1, kTile64x32 = 2 };

__host__ __device__ constexpr int lout_for(int mode, int lin) {
  return mode == kConvSame ? lin : (mode == kConvDown ? lin / 2 : 2 * lin);
}

struct MmArgs {
  const void* w;
  const float* bias;
  float* y;
  std::int64_t ys;
  const float* src;
  std::int64_t src_stride;
  int split;
  const float* plain;
  std::int64_t plain_stride;
  int oc, ic, batch;
  int mtiles, ntiles;
  int ksplit;   // workgroups sharing one output tile's K range (1: no split)
  float* part;  // ksplit > 1, ypart == 0: partial tiles [ksplit][mtiles * ntiles][64 * NT]
  // ksplit > 1, ypart > 0: split ks writes its partial sum in the output layout at
  // y + ks * ypart (bias in split 0), and the consumer adds the partials.
  std::int64_t ypart;
  // Byte sizes of the weight tensor and the batch of `src` / `plain` (buffer ranges of the BF16
  // kernels; each below 2 GiB).
  unsigned wbytes, srcbytes, plainbytes;
  // Column order of a tile: 0 = (sample, position); 1 = output parity first (ConvTranspose
  // tiles: the first half holds the even positions of its samples, the second half the odd
  // ones).
  int par;
};

// Sample and output position of tile column `col` (NT columns, lout positions per sample).
__host__ __device__ inline void col_pos(int col, int nt, int lout, int par, int& bl, int& t) {
  if (par) {
    const int half = nt / 2, p = col >= half ? 1 : 0, c2 = col - p * half;
    bl = c2 / (lout / 2);
    t = 2 * (c2 - bl * (lout / 2)) + p;
  } else {
    bl = col / lout;
    t = col - bl * lout;
  }
}

// Input index read by output t through tap k, or -1 in the padding (t known only at run time).
template <int MODE, int K, int LIN>
__device__ __forceinline__ int src_at(int t, int k) {
  if constexpr (MODE == kConvSame) {
    const int j = t + k - K / 2;
    return (j >= 0 && j < LIN) ? j : -1;
  } else if constexpr (MODE == kConvDown) {
    const int j = 2 * t + k - 1;
    return (j >= 0 && j < LIN) ? j : -1;
  } else {
    const int num = t + 1 - k;  // ConvTranspose: output t = 2 * j + k - 1
    if (num < 0 || (num & 1)) return -1;
    const int j = num >> 1;
    return j < LIN ? j : -1;
  }
}

// BF16 matrix-core path: each MFMA contracts kKCB input channels of one tap; a K step stages
// kKCB channels (F32 weights, split while staged) or 2 kKCB (BF16 weights).
constexpr int kKCB = 32;
inline int mm_bf16_step(const ConvOp& op) { return op.bf16 ? 2 * kKCB : kKCB; }

// True when the BF16 kernels cover this convolution's shape (input channels and the concat
// split in multiples of the K step).
bool mm_bf16_ok(const ConvOp& op, int split);

// Launches the BF16 implicit GEMM for `a` (tiles and split as the F32 path plans them): two BF16
// terms of the input against BF16 weights, or three products of split input and split F32
// weights.
hipError_t launch_mm_bf16(const ConvOp& op, int tile, const MmArgs& a, hipStream_t s);

}  // namespace fe::hip::mm
