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
// In LDS a weight row stores the KS channels of each tap contiguously and an input row (one
// sample position) its KS channels, so every operand is one 16-byte read.  A K step stages KS =
// 64 channels with BF16 weights (two contractions per tap; one weight buffer, refilled after a
// barrier, so that two 79 KB workgroups fit a CU) and 32 with F32 weights (double-buffered):
// half the steps, and so half the per-step staging chains, of 32-channel steps at BF16
// (bimanual B=16 4.87 -> 4.72 ms).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "conv_mfma.h"

namespace fe::hip::mm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kPadB = 8;  // LDS row padding (BF16 values)

// Workgroup shape per column tile: 64 x 128 and 64 x 64 blocks take eight wavefronts (two per
// SIMD, so one wavefront's LDS reads and staging overlap another's MFMAs) in a 2 x 4 grid of
// 32 x 32 or 32 x 16 tiles (bimanual B=64 6.34 -> 6.15 ms against four wavefronts on 64 x 64);
// 64 x 32 blocks take four in a 2 x 2 grid.
__host__ __device__ constexpr int threads_for(int nt) { return nt >= 64 ? 512 : 256; }
constexpr int kWaveRows = 2;

template <int MODE, int K, int LIN, int MT, int NT, bool WF32>
struct BShape {
  static constexpr int kBThreads = threads_for(NT);
  static constexpr int kWaveCols = kBThreads / 64 / kWaveRows;
  static constexpr int LOUT = lout_for(MODE, LIN);
  static constexpr int SB = NT / LOUT;            // samples per column tile
  static constexpr int KS = WF32 ? kKCB : 2 * kKCB;  // input channels per K step (mm_bf16_step)
  static constexpr int SUB = KS / kKCB;              // MFMA contractions per tap and step
  static constexpr bool W1 = !WF32;                  // one weight buffer in LDS
  static constexpr int WBUF = W1 ? 1 : 2;
  static constexpr int WROW = K * KS + kPadB;   // LDS BF16 values per weight row
  static constexpr int XROW = KS + kPadB;       // LDS BF16 values per (sample, position) row
  static constexpr int ZERO = SB * LIN;           // index of the zero row
  static constexpr int XROWS = SB * LIN + 1;
  static constexpr int WVALS = MT * WROW;
  static constexpr int XVALS = XROWS * XROW;
  // 16-byte weight units per lane per step: 8 BF16 values, or 4 F32 values.
  static constexpr int WUNITS = MT * K * (KS / (WF32 ? 4 : 8));  // weight units per step
  static constexpr int UW = (WUNITS + kBThreads - 1) / kBThreads;
  static constexpr int WARR = WF32 ? 2 : 1;  // weight arrays in LDS (hi, lo)
  // Input units: CPU channels x PPU positions of one sample, read as contiguous 16-byte vectors
  // of its [channel][position] block (LIN = 1: 4 channels; 2: 2 channels x 2 positions; >= 4:
  // 2 channels x 4 positions, two vectors).
  static constexpr int CPU = LIN == 1 ? 4 : 2;
  static constexpr int PPU = LIN >= 4 ? 4 : LIN;
  static constexpr int XVEC = LIN >= 4 ? 2 : 1;     // 16-byte loads per unit
  static constexpr int UPS = (KS / CPU) * (LIN / PPU);  // units per sample and step
  static constexpr int XUNITS = SB * UPS;
  static constexpr int WM = MT / kWaveRows, WN = NT / kWaveCols;
  static constexpr int TI = WM / 16, TJ = WN / 16;
  static constexpr std::size_t LDS_BYTES = (WBUF * WARR * WVALS + 4 * XVALS) * 2;
  static_assert(WM % 16 == 0 && WN % 16 == 0, "wavefront tiles of 16 x 16 MFMA blocks");
  static_assert(NT % LOUT == 0, "column tile");
  static constexpr int UXN = (XUNITS + kBThreads - 1) / kBThreads;  // input units per lane
  static_assert(WROW % 8 == 0 && XROW % 8 == 0, "16-byte LDS rows");
};

constexpr unsigned kOutOfRange = 0x80000000u;
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, kRsrcWord3);
}

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
__global__ __launch_bounds__(threads_for(NT)) void conv_mfma_bf16_kernel(MmArgs a) {
  using S = BShape<MODE, K, LIN, MT, NT, WF32>;
  constexpr int kBThreads = S::kBThreads, kWaveCols = S::kWaveCols;
  extern __shared__ uint4 lds_b[];
  unsigned short* Ws = reinterpret_cast<unsigned short*>(lds_b);  // [2][WVALS] (hi)
  unsigned short* Wl = Ws + S::WBUF * S::WVALS;                    // [2][WVALS] (lo, F32 weights)
  unsigned short* Xh = Ws + S::WBUF * S::WARR * S::WVALS;          // [2][XVALS]
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
  const int nall = a.ic / S::KS;
  const int s0 = ks * nall / a.ksplit, s1 = (ks + 1) * nall / a.ksplit;

  // The bias of the tile's rows (first K slice only), read before the first K step's loads
  // and kept in LDS for the epilogue.
  __shared__ float bias_t[MT];
  float bias_r = 0.0f;
  if (tid < MT && ks == 0 && m0 + tid < a.oc) bias_r = a.bias[m0 + tid];

  // Zero rows of both input buffers (never overwritten).
  if (tid < 2 * S::KS) {
    const int buf = tid / S::KS, c = tid % S::KS;
    Xh[buf * S::XVALS + S::ZERO * S::XROW + c] = 0;
    Xl[buf * S::XVALS + S::ZERO * S::XROW + c] = 0;
  }

  // Staging.  Every global read is a buffer load whose per-lane byte offset is fixed for the
  // whole K loop (computed once below); a wave-uniform scalar offset walks the K steps, and lanes
  // with nothing to read get an out-of-range offset, which returns zeros without a branch.
  constexpr int QPT = S::KS / (WF32 ? 4 : 8);  // 16-byte weight units per (row, tap)
  constexpr int QW = WF32 ? 4 : 8;             // weights per unit
  constexpr unsigned ES = WF32 ? 4u : 2u;      // weight element size
  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(a.w, a.wbytes);
  unsigned wvoff[S::UW];
  int wlds[S::UW];
#pragma unroll
  for (int r = 0; r < S::UW; ++r) {
    const int uu = tid + r * kBThreads;
    const bool act = uu < S::WUNITS;
    const int u = act ? uu : 0;
    const int m = u / (K * QPT), rem = u - m * (K * QPT);
    const int k = rem / QPT, q = rem - k * QPT;
    const int oc = m0 + m;
    wvoff[r] = act && oc < a.oc ? static_cast<unsigned>((oc * K + k) * a.ic + QW * q) * ES
                                : kOutOfRange;
    wlds[r] = act ? m * S::WROW + k * S::KS + QW * q : -1;
  }
  // Input units (see BShape): consecutive lanes read consecutive 16-byte pieces of a sample's
  // 32-channel block, and each unit is stored as PPU rows (positions) of CPU BF16 channels per
  // term.
  int xlds[S::UXN];
  unsigned xvs[S::UXN], xvp[S::UXN];
#pragma unroll
  for (int n = 0; n < S::UXN; ++n) {
    const int uu = tid + n * kBThreads;
    const bool act = uu < S::XUNITS;
    const int u = act ? uu : 0;
    const int bl = u / S::UPS, v = u - bl * S::UPS;
    const int tq = v % (LIN / S::PPU), cg = v / (LIN / S::PPU);
    const int c = cg * S::CPU, t0 = tq * S::PPU;
    const int b = b0 + bl;
    xlds[n] = act ? (bl * LIN + t0) * S::XROW + c : -1;
    xvs[n] = kOutOfRange;
    xvp[n] = kOutOfRange;
    if (act && b < a.batch) {
      xvs[n] = static_cast<unsigned>((b * a.src_stride + c * LIN + t0) * 4);
      if (a.plain != nullptr)
        xvp[n] = static_cast<unsigned>((b * a.plain_stride + c * LIN + t0) * 4);
    }
  }
  const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(a.src, a.srcbytes);
  const __amdgpu_buffer_rsrc_t prs = buffer_rsrc(a.plain != nullptr ? a.plain : a.src,
                                                 a.plain != nullptr ? a.plainbytes : a.srcbytes);
  // One K step's staged data in registers.
  struct Regs {
    uint4 w[S::UW];
    float4 x[S::UXN][S::XVEC];
  };
  auto load_step = [&](int step, Regs& R) {
    const int ic0 = step * S::KS;
    const unsigned ws = static_cast<unsigned>(ic0) * ES;
#pragma unroll
    for (int r = 0; r < S::UW; ++r)
      R.w[r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wrs, wvoff[r], ws, 0));
    const bool from_src = ic0 < a.split;
    const __amdgpu_buffer_rsrc_t xrs = from_src ? srs : prs;
    const unsigned xs0 = static_cast<unsigned>((from_src ? ic0 : ic0 - a.split) * LIN * 4);
#pragma unroll
    for (int n = 0; n < S::UXN; ++n) {
      const unsigned xv = from_src ? xvs[n] : xvp[n];
#pragma unroll
      for (int j = 0; j < S::XVEC; ++j)
        R.x[n][j] = __builtin_bit_cast(
            float4, __builtin_amdgcn_raw_buffer_load_b128(
                        xrs, xv, xs0 + static_cast<unsigned>(j * LIN * 4), 0));
    }
  };
  auto store_step = [&](int buf, const Regs& R) {
    unsigned short* W = Ws + (S::W1 ? 0 : buf * S::WVALS);
#pragma unroll
    for (int r = 0; r < S::UW; ++r) {
      if (S::WUNITS % kBThreads != 0 && wlds[r] < 0) continue;
      if constexpr (WF32) {
        const float4 v = __builtin_bit_cast(float4, R.w[r]);
        unsigned short h[4], l[4];
        split_bf16(v.x, h[0], l[0]);
        split_bf16(v.y, h[1], l[1]);
        split_bf16(v.z, h[2], l[2]);
        split_bf16(v.w, h[3], l[3]);
        *reinterpret_cast<uint2*>(W + wlds[r]) =
            uint2{h[0] | (static_cast<unsigned>(h[1]) << 16), h[2] | (static_cast<unsigned>(h[3]) << 16)};
        *reinterpret_cast<uint2*>(Wl + buf * S::WVALS + wlds[r]) =
            uint2{l[0] | (static_cast<unsigned>(l[1]) << 16), l[2] | (static_cast<unsigned>(l[3]) << 16)};
      } else {
        *reinterpret_cast<uint4*>(W + wlds[r]) = R.w[r];
      }
    }
#pragma unroll
    for (int n = 0; n < S::UXN; ++n) {
      if (S::XUNITS % kBThreads != 0 && xlds[n] < 0) continue;
      unsigned short* H = Xh + buf * S::XVALS + xlds[n];
      unsigned short* L = Xl + buf * S::XVALS + xlds[n];
      // Value of channel c (0 .. CPU-1) at position p (0 .. PPU-1) of the unit.
      auto val = [&](int c, int p) {
        const float4& v = R.x[n][LIN >= 4 ? c : 0];
        const int e = LIN >= 4 ? p : c * LIN + p;
        return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
      };
#pragma unroll
      for (int p = 0; p < S::PPU; ++p) {
        unsigned short hb[S::CPU], lb[S::CPU];
#pragma unroll
        for (int c = 0; c < S::CPU; ++c) split_bf16(val(c, p), hb[c], lb[c]);
        if constexpr (S::CPU == 4) {
          *reinterpret_cast<uint2*>(H + p * S::XROW) =
              uint2{hb[0] | (static_cast<unsigned>(hb[1]) << 16),
                    hb[2] | (static_cast<unsigned>(hb[3]) << 16)};
          *reinterpret_cast<uint2*>(L + p * S::XROW) =
              uint2{lb[0] | (static_cast<unsigned>(lb[1]) << 16),
                    lb[2] | (static_cast<unsigned>(lb[3]) << 16)};
        } else {
          *reinterpret_cast<unsigned*>(H + p * S::XROW) =
              hb[0] | (static_cast<unsigned>(hb[1]) << 16);
          *reinterpret_cast<unsigned*>(L + p * S::XROW) =
              lb[0] | (static_cast<unsigned>(lb[1]) << 16);
        }
      }
    }
  };

  // Per-lane input row of every (column tile j, tap k): fixed for the whole K loop.  With
  // ConvTranspose the columns are in parity order (even output positions in the first half of
  // the tile), so each wavefront's columns have one output parity, which taps of the other
  // parity never reach.
  constexpr int PAR = MODE == kConvTranspose ? 1 : 0;
  const int wr = wave / kWaveCols, wc = wave % kWaveCols;
  const int par = 2 * wc / kWaveCols;  // output parity of this wavefront's columns (PAR)
  const int kq = lane >> 4, l16 = lane & 15;
  int xrow[S::TJ][K];
#pragma unroll
  for (int j = 0; j < S::TJ; ++j) {
    const int col = wc * S::WN + 16 * j + l16;
    int bl, t;
    col_pos(col, NT, S::LOUT, PAR, bl, t);
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

  auto compute = [&](int buf) {
    const unsigned short* W = Ws + (S::W1 ? 0 : buf * S::WVALS);
    const unsigned short* WL = Wl + buf * S::WVALS;
    const unsigned short* H = Xh + buf * S::XVALS;
    const unsigned short* L = Xl + buf * S::XVALS;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      // Output t takes tap k when t + 1 - k is even.
      if constexpr (PAR) {
        if (((k + par + 1) & 1) != 0) continue;
      }
#pragma unroll
      for (int kc = 0; kc < S::SUB; ++kc) {
        bf16x8 av[S::TI], al[WF32 ? S::TI : 1], bh[S::TJ], bl[S::TJ];
        const int wo = k * S::KS + kc * kKCB;
#pragma unroll
        for (int i = 0; i < S::TI; ++i) {
          av[i] = __builtin_bit_cast(
              bf16x8, *reinterpret_cast<const uint4*>(W + arow + i * 16 * S::WROW + wo));
          if constexpr (WF32)
            al[i] = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const uint4*>(WL + arow + i * 16 * S::WROW + wo));
        }
#pragma unroll
        for (int j = 0; j < S::TJ; ++j) {
          const int xo = xrow[j][k] + kc * kKCB;
          bh[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(H + xo));
          bl[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(L + xo));
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
    }
  };

  // K loop: the next step's loads are in flight while the matrix cores work on the current one.
  // (Three steps in flight, in rotating register sets, measured slower at B=64: 21.9 against
  // 20.8 us for the 2048<-2048 L2 layer.)
  Regs rn;
  load_step(s0, rn);
  if (tid < MT) bias_t[tid] = bias_r;
  store_step(0, rn);
  __syncthreads();
  for (int step = s0; step < s1; ++step) {
    const int buf = (step - s0) & 1;
    if (step + 1 < s1) load_step(step + 1, rn);
    compute(buf);
    if (step + 1 < s1) {
      if constexpr (S::W1) __syncthreads();  // the one weight buffer is read by every wavefront
      store_step(buf ^ 1, rn);
    }
    __syncthreads();
  }

  // Epilogue: lane holds rows 4 * (lane / 16) + e of each 16x16 tile, column lane % 16.
  if (a.ksplit > 1 && a.ypart == 0) {
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
  // Output layout: the tile goes through LDS as [sample, position][channel], so that each
  // sample's MT x LOUT block (contiguous in y) is written by consecutive lanes.
  constexpr int TROW = MT + 1;
  static_assert(static_cast<std::size_t>(NT) * TROW * 4 <= S::LDS_BYTES, "epilogue tile in LDS");
  float* T = reinterpret_cast<float*>(lds_b);
  __syncthreads();  // the last K step's LDS reads are done
#pragma unroll
  for (int j = 0; j < S::TJ; ++j) {
    const int col = wc * S::WN + 16 * j + l16;
    int bl2, t;
    col_pos(col, NT, S::LOUT, PAR, bl2, t);
    float* tr = T + (bl2 * S::LOUT + t) * TROW + wr * S::WM + 4 * kq;
#pragma unroll
    for (int i = 0; i < S::TI; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) tr[16 * i + e] = acc[i][j][e];
  }
  __syncthreads();
  float* yk = a.y + ks * a.ypart;
  for (int idx = tid; idx < NT * MT; idx += kBThreads) {
    const int bl2 = idx / (MT * S::LOUT);
    const int rem = idx - bl2 * (MT * S::LOUT);
    const int row = rem / S::LOUT, t = rem - row * S::LOUT;
    const int b = b0 + bl2, oc = m0 + row;
    if (b < a.batch && oc < a.oc)
      yk[b * a.ys + static_cast<std::int64_t>(oc) * S::LOUT + t] =
          T[(bl2 * S::LOUT + t) * TROW + row] + bias_t[row];
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
  hipLaunchKernelGGL(fn, dim3(a.mtiles * a.ntiles * a.ksplit), dim3(S::kBThreads), S::LDS_BYTES, s,
                     a);
  return hipGetLastError();
}

template <int MODE, int K, int LIN>
hipError_t by_tile(int tile, bool wf32, const MmArgs& a, hipStream_t s) {
  if (wf32)
    return tile == kTile64x128 ? launch<MODE, K, LIN, 64, 128, true>(a, s)
                               : launch<MODE, K, LIN, 64, 64, true>(a, s);
  if (tile == kTile64x32) return launch<MODE, K, LIN, 64, 32, false>(a, s);
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
  const int ks = mm_bf16_step(op);
  if (op.ic % ks != 0 || split % ks != 0 || split <= 0 || split > op.ic) return false;
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
