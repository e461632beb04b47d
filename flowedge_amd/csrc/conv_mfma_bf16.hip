// Batched convolution on the BF16 matrix cores (gfx950 v_mfma_f32_16x16x32_bf16).  Same implicit
// GEMM and tiling as the F32 path (conv_mfma.hip):
//     Y[oc][(b, t)] = bias[oc] + sum_{k, ic} W[oc][k][ic] * X[b][ic][src(t, k)]
// but each MFMA contracts 32 input channels of one tap, and the fp32 input is split into two
// BF16 terms, X = Xh + Xl (Xh = bf16(X), Xl = bf16(X - Xh)), so that
//     W X = W Xh + W Xl      (two MFMAs per tile, fp32 accumulation)
// keeps about 16 significant bits of every input value instead of BF16's 8.  BF16 weights are
// exact in this form; what remains is the rounding of Xl (about 2^-17 relative per product).
// F32 weights are split the same way while they are staged (W = Wh + Wl) and contracted as
//     W X ~ Wh Xh + Wh Xl + Wl Xh      (three MFMAs; the dropped Wl Xl is about 2^-16 relative)
// so HBM still carries the F32 weights once.
//
// Lane layouts (checked on gfx950): a lane holds A[l % 16][8 (l / 16) .. +7] and
// B[8 (l / 16) .. +7][l % 16] as eight BF16 values, and receives D[4 (l / 16) + e][l % 16].
// In LDS a weight row stores the 32 channels of each tap contiguously and an input row (one
// sample position) its 32 channels, so every operand is one 16-byte read.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "conv_mfma.h"

namespace fe::hip::mm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kPadB = 8;  // LDS row padding (BF16 values)

template <int MODE, int K, int LIN, int MT, int NT, bool WF32>
struct BShape {
  static constexpr int LOUT = lout_for(MODE, LIN);
  static constexpr int SB = NT / LOUT;            // samples per column tile
  static constexpr int WROW = K * kKCB + kPadB;   // LDS BF16 values per weight row
  static constexpr int XROW = kKCB + kPadB;       // LDS BF16 values per (sample, position) row
  static constexpr int ZERO = SB * LIN;           // index of the zero row
  static constexpr int XROWS = SB * LIN + 1;
  static constexpr int WVALS = MT * WROW;
  static constexpr int XVALS = XROWS * XROW;
  // 16-byte weight units per lane per step: 8 BF16 values, or 4 F32 values.
  static constexpr int UW = MT * K * (kKCB / (WF32 ? 4 : 8)) / kMmThreads;
  static constexpr int WARR = WF32 ? 2 : 1;  // weight arrays in LDS (hi, lo)
  static constexpr int XELEMS = SB * kKCB * LIN;               // input floats per step
  static constexpr int XV = LIN >= 4 ? 4 : 1;
  static constexpr int XUNITS = XELEMS / XV;
  static constexpr int UX = (XUNITS + kMmThreads - 1) / kMmThreads;
  static constexpr int WM = MT / 2, WN = NT / 2;
  static constexpr int TI = WM / 16, TJ = WN / 16;
  static constexpr std::size_t LDS_BYTES = (2 * WARR * WVALS + 4 * XVALS) * 2;
  static_assert(MT * K * (kKCB / (WF32 ? 4 : 8)) % kMmThreads == 0, "weight units per lane");
  static_assert(NT % LOUT == 0 && XELEMS % XV == 0, "column tile");
  static_assert(WROW % 8 == 0 && XROW % 8 == 0, "16-byte LDS rows");
};

__device__ __forceinline__ unsigned short bf16_bits(float v) {
  return __builtin_bit_cast(unsigned short, static_cast<__bf16>(v));
}

// Splits v into (hi, lo) BF16 bit patterns with v ~ hi + lo.
__device__ __forceinline__ void split_bf16(float v, unsigned short& hi, unsigned short& lo) {
  const __bf16 h = static_cast<__bf16>(v);
  hi = __builtin_bit_cast(unsigned short, h);
  lo = bf16_bits(v - static_cast<float>(h));
}

template <int MODE, int K, int LIN, int MT, int NT, bool WF32>
__global__ __launch_bounds__(kMmThreads) void conv_mfma_bf16_kernel(MmArgs a) {
  using S = BShape<MODE, K, LIN, MT, NT, WF32>;
  extern __shared__ uint4 lds_b[];
  unsigned short* Ws = reinterpret_cast<unsigned short*>(lds_b);  // [2][WVALS] (hi)
  unsigned short* Wl = Ws + 2 * S::WVALS;                          // [2][WVALS] (lo, F32 weights)
  unsigned short* Xh = Ws + 2 * S::WARR * S::WVALS;                // [2][XVALS]
  unsigned short* Xl = Xh + 2 * S::XVALS;                          // [2][XVALS]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int id = blockIdx.x;
  const int tiles = a.mtiles * a.ntiles;
  const int total = tiles * a.ksplit;
  if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
  const int ks = id / tiles;
  const int tile = id - ks * tiles;
  const int mt = tile / a.ntiles, nt = tile - mt * a.ntiles;
  const int m0 = mt * MT;
  const int b0 = nt * S::SB;
  const int nall = a.ic / kKCB;
  const int s0 = ks * nall / a.ksplit, s1 = (ks + 1) * nall / a.ksplit;

  // Zero rows of both input buffers (never overwritten).
  if (tid < 2 * kKCB) {
    const int buf = tid / kKCB, c = tid % kKCB;
    Xh[buf * S::XVALS + S::ZERO * S::XROW + c] = 0;
    Xl[buf * S::XVALS + S::ZERO * S::XROW + c] = 0;
  }

  constexpr int QPT = kKCB / (WF32 ? 4 : 8);  // 16-byte units per (row, tap)
  constexpr int QW = WF32 ? 4 : 8;             // weights per unit
  uint4 wreg[S::UW];
  float4 xreg[S::XV == 4 ? S::UX : 1];
  float xs1[S::XV == 1 ? S::UX : 1];
  auto load_step = [&](int step) {
    const int ic0 = step * kKCB;
#pragma unroll
    for (int r = 0; r < S::UW; ++r) {
      const int u = tid + r * kMmThreads;
      const int m = u / (K * QPT), rem = u - m * (K * QPT);
      const int k = rem / QPT, q = rem - k * QPT;
      const int oc = m0 + m;
      const std::int64_t idx = (static_cast<std::int64_t>(oc) * K + k) * a.ic + ic0 + QW * q;
      wreg[r] = uint4{0u, 0u, 0u, 0u};
      if (oc < a.oc) {
        if constexpr (WF32)
          wreg[r] = *reinterpret_cast<const uint4*>(static_cast<const float*>(a.w) + idx);
        else
          wreg[r] = *reinterpret_cast<const uint4*>(static_cast<const unsigned short*>(a.w) + idx);
      }
    }
#pragma unroll
    for (int r = 0; r < S::UX; ++r) {
      const int u = tid + r * kMmThreads;
      if constexpr (S::XV == 4) {
        const int bl = u / (kKCB * LIN / 4), v = u - bl * (kKCB * LIN / 4);
        const int ch = v / (LIN / 4), t4 = (v - ch * (LIN / 4)) * 4;
        const int b = b0 + bl, c = ic0 + ch;
        float4 val = float4{0.0f, 0.0f, 0.0f, 0.0f};
        if (u < S::XUNITS && b < a.batch) {
          const float* p = c < a.split ? a.src + b * a.src_stride + static_cast<std::int64_t>(c) * LIN
                                       : a.plain + b * a.plain_stride +
                                             static_cast<std::int64_t>(c - a.split) * LIN;
          val = *reinterpret_cast<const float4*>(p + t4);
        }
        xreg[r] = val;
      } else {
        const int bl = u / (kKCB * LIN), v = u - bl * (kKCB * LIN);
        const int ch = v / LIN, t = v - ch * LIN;
        const int b = b0 + bl, c = ic0 + ch;
        float val = 0.0f;
        if (u < S::XUNITS && b < a.batch)
          val = c < a.split ? a.src[b * a.src_stride + static_cast<std::int64_t>(c) * LIN + t]
                            : a.plain[b * a.plain_stride + static_cast<std::int64_t>(c - a.split) * LIN + t];
        xs1[r] = val;
      }
    }
  };
  auto store_step = [&](int buf) {
    unsigned short* W = Ws + buf * S::WVALS;
    unsigned short* H = Xh + buf * S::XVALS;
    unsigned short* L = Xl + buf * S::XVALS;
#pragma unroll
    for (int r = 0; r < S::UW; ++r) {
      const int u = tid + r * kMmThreads;
      const int m = u / (K * QPT), rem = u - m * (K * QPT);
      const int k = rem / QPT, q = rem - k * QPT;
      const int off = m * S::WROW + k * kKCB + QW * q;
      if constexpr (WF32) {
        const float4 v = __builtin_bit_cast(float4, wreg[r]);
        unsigned short h[4], l[4];
        split_bf16(v.x, h[0], l[0]);
        split_bf16(v.y, h[1], l[1]);
        split_bf16(v.z, h[2], l[2]);
        split_bf16(v.w, h[3], l[3]);
        *reinterpret_cast<uint2*>(W + off) =
            uint2{h[0] | (static_cast<unsigned>(h[1]) << 16), h[2] | (static_cast<unsigned>(h[3]) << 16)};
        *reinterpret_cast<uint2*>(Wl + buf * S::WVALS + off) =
            uint2{l[0] | (static_cast<unsigned>(l[1]) << 16), l[2] | (static_cast<unsigned>(l[3]) << 16)};
      } else {
        *reinterpret_cast<uint4*>(W + off) = wreg[r];
      }
    }
#pragma unroll
    for (int r = 0; r < S::UX; ++r) {
      const int u = tid + r * kMmThreads;
      if (u >= S::XUNITS) continue;
      if constexpr (S::XV == 4) {
        const int bl = u / (kKCB * LIN / 4), v = u - bl * (kKCB * LIN / 4);
        const int ch = v / (LIN / 4), t4 = (v - ch * (LIN / 4)) * 4;
        const int row = (bl * LIN + t4) * S::XROW + ch;
        const float vals[4] = {xreg[r].x, xreg[r].y, xreg[r].z, xreg[r].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) split_bf16(vals[e], H[row + e * S::XROW], L[row + e * S::XROW]);
      } else {
        const int bl = u / (kKCB * LIN), v = u - bl * (kKCB * LIN);
        const int ch = v / LIN, t = v - ch * LIN;
        const int row = (bl * LIN + t) * S::XROW + ch;
        split_bf16(xs1[r], H[row], L[row]);
      }
    }
  };

  // Per-lane input row of every (column tile j, tap k): fixed for the whole K loop.
  const int wr = wave >> 1, wc = wave & 1;
  const int kq = lane >> 4, l16 = lane & 15;
  int xrow[S::TJ][K];
#pragma unroll
  for (int j = 0; j < S::TJ; ++j) {
    const int col = wc * S::WN + 16 * j + l16;
    const int bl = col / S::LOUT, t = col - bl * S::LOUT;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int ti = src_at<MODE, K, LIN>(t, k);
      xrow[j][k] = (ti >= 0 ? bl * LIN + ti : S::ZERO) * S::XROW + 8 * kq;
    }
  }
  const int arow = (wr * S::WM + l16) * S::WROW + 8 * kq;

  floatx4 acc[S::TI][S::TJ];
#pragma unroll
  for (int i = 0; i < S::TI; ++i)
#pragma unroll
    for (int j = 0; j < S::TJ; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  load_step(s0);
  store_step(0);
  __syncthreads();
  for (int step = s0; step < s1; ++step) {
    const int buf = (step - s0) & 1;
    if (step + 1 < s1) load_step(step + 1);
    const unsigned short* W = Ws + buf * S::WVALS;
    const unsigned short* WL = Wl + buf * S::WVALS;
    const unsigned short* H = Xh + buf * S::XVALS;
    const unsigned short* L = Xl + buf * S::XVALS;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      bf16x8 av[S::TI], al[WF32 ? S::TI : 1], bh[S::TJ], bl[S::TJ];
#pragma unroll
      for (int i = 0; i < S::TI; ++i) {
        av[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(
                                               W + arow + i * 16 * S::WROW + k * kKCB));
        if constexpr (WF32)
          al[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(
                                                 WL + arow + i * 16 * S::WROW + k * kKCB));
      }
#pragma unroll
      for (int j = 0; j < S::TJ; ++j) {
        bh[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(H + xrow[j][k]));
        bl[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(L + xrow[j][k]));
      }
#pragma unroll
      for (int i = 0; i < S::TI; ++i)
#pragma unroll
        for (int j = 0; j < S::TJ; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i], bh[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i], bl[j], acc[i][j], 0, 0, 0);
          if constexpr (WF32)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], bh[j], acc[i][j], 0, 0, 0);
        }
    }
    if (step + 1 < s1) store_step(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds rows 4 * (lane / 16) + e of each 16x16 tile, column lane % 16.
  if (a.ksplit > 1) {
    float* P = a.part + (static_cast<std::int64_t>(ks) * tiles + tile) * (MT * NT);
#pragma unroll
    for (int i = 0; i < S::TI; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int j = 0; j < S::TJ; ++j)
          P[(wr * S::WM + 16 * i + 4 * kq + e) * NT + wc * S::WN + 16 * j + l16] = acc[i][j][e];
    return;
  }
#pragma unroll
  for (int i = 0; i < S::TI; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int oc = m0 + wr * S::WM + 16 * i + 4 * kq + e;
      if (oc >= a.oc) continue;
      const float bias = a.bias[oc];
#pragma unroll
      for (int j = 0; j < S::TJ; ++j) {
        const int col = wc * S::WN + 16 * j + l16;
        const int bl2 = col / S::LOUT, t = col - bl2 * S::LOUT;
        const int b = b0 + bl2;
        if (b < a.batch)
          a.y[b * a.ys + static_cast<std::int64_t>(oc) * S::LOUT + t] = acc[i][j][e] + bias;
      }
    }
}

template <int MODE, int K, int LIN, int MT, int NT, bool WF32>
hipError_t launch(const MmArgs& a, hipStream_t s) {
  using S = BShape<MODE, K, LIN, MT, NT, WF32>;
  auto fn = conv_mfma_bf16_kernel<MODE, K, LIN, MT, NT, WF32>;
  static bool raised = false;
  if (!raised && S::LDS_BYTES > 48 * 1024) {
    const hipError_t st = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                              hipFuncAttributeMaxDynamicSharedMemorySize,
                                              static_cast<int>(S::LDS_BYTES));
    if (st != hipSuccess) return st;
    raised = true;
  }
  hipLaunchKernelGGL(fn, dim3(a.mtiles * a.ntiles * a.ksplit), dim3(kMmThreads), S::LDS_BYTES, s,
                     a);
  return hipGetLastError();
}

template <int MODE, int K, int LIN>
hipError_t by_tile(int tile, bool wf32, const MmArgs& a, hipStream_t s) {
  if (wf32)
    return tile == kTile64x128 ? launch<MODE, K, LIN, 64, 128, true>(a, s)
                               : launch<MODE, K, LIN, 64, 64, true>(a, s);
  return tile == kTile64x128 ? launch<MODE, K, LIN, 64, 128, false>(a, s)
                             : launch<MODE, K, LIN, 64, 64, false>(a, s);
}

template <int MODE, int K>
hipError_t by_lin(int lin, int tile, bool wf32, const MmArgs& a, hipStream_t s) {
  switch (lin) {
    case 1:
      if constexpr (MODE != kConvDown) return by_tile<MODE, K, 1>(tile, wf32, a, s);
      break;
    case 2: return by_tile<MODE, K, 2>(tile, wf32, a, s);
    case 4: return by_tile<MODE, K, 4>(tile, wf32, a, s);
    case 8: return by_tile<MODE, K, 8>(tile, wf32, a, s);
    case 16:
      if constexpr (MODE != kConvTranspose) return by_tile<MODE, K, 16>(tile, wf32, a, s);
      break;
    default: break;
  }
  return hipErrorInvalidValue;
}

}  // namespace

bool mm_bf16_ok(const ConvOp& op, int split) {
  if (op.ic % kKCB != 0 || split % kKCB != 0 || split <= 0 || split > op.ic) return false;
  if (op.lin != 1 && op.lin != 2 && op.lin != 4 && op.lin != 8 && op.lin != 16) return false;
  if (op.lout != lout_for(op.mode, op.lin)) return false;
  if (op.mode == kConvSame) return op.k == 1 || op.k == 3 || op.k == 5;
  if (op.mode == kConvDown) return op.k == 3 && op.lin >= 2;
  return op.mode == kConvTranspose && op.k == 4 && op.lin <= 8;
}

hipError_t launch_mm_bf16(const ConvOp& op, int tile, const MmArgs& a, hipStream_t s) {
  const bool wf32 = !op.bf16;
  if (op.mode == kConvSame) {
    switch (op.k) {
      case 1: return by_lin<kConvSame, 1>(op.lin, tile, wf32, a, s);
      case 3: return by_lin<kConvSame, 3>(op.lin, tile, wf32, a, s);
      case 5: return by_lin<kConvSame, 5>(op.lin, tile, wf32, a, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (op.mode == kConvDown && op.k == 3) return by_lin<kConvDown, 3>(op.lin, tile, wf32, a, s);
  if (op.mode == kConvTranspose && op.k == 4)
    return by_lin<kConvTranspose, 4>(op.lin, tile, wf32, a, s);
  return hipErrorInvalidValue;
}

}  // namespace fe::hip::mm
