// Batched convolution on the matrix cores (gfx950 v_mfma_f32_16x16x4f32), for sampling calls with
// many samples.  Each convolution is an implicit GEMM
//     Y[oc][(b, t)] = bias[oc] + sum_{k, ic} W[oc][k][ic] * X[b][ic][src(t, k)]
// with A = the repacked weights [OC][K][IC] (row-major [OC][K*IC]) and B = the input gathered per
// tap (src(t, k) as conv1d / ConvTranspose1d define it, zero outside the input).  The GroupNorm +
// Mish (+ FiLM) (+ residual) prologue runs first as its own per-sample kernel (norm_act), whose
// output the GEMM reads as a plain tensor.
//
// GEMM tiling: a 256-lane workgroup owns 64 output channels x NT columns (samples x output
// positions, NT = 128, or 64 when 128 would leave CUs without a workgroup); its four wavefronts
// each own 32 x (NT/2).  The K loop walks 16 input channels at a time (all taps), double-buffered
// in LDS: the next step's weights and inputs are loaded into registers while the matrix cores
// work on the current one.  Within a 16-channel step a lane
// feeds the MFMA k-slot (lane / 16) with channels 4 * (lane / 16) + s over four MFMAs s, so
// every operand read is one 16-byte LDS load.  Output positions whose input index falls in the
// padding read a zero row.  Workgroups that share a weight tile are placed on the same XCD
// (dispatch is round-robin over the 8 XCDs), so the tile is fetched into one L2.
//
// Reference semantics: conv1d diffusion_ops.cc:82-163, conv_transpose1d :165-268,
// group_norm :270-350, film :352-377.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "conv_mfma.h"
#include "device_common.h"
#include "kernels.h"

namespace fe::hip {
namespace {

using namespace dev;

using namespace mm;

constexpr int kKC = 16;   // input channels per K step
constexpr int kPad = 4;   // LDS row padding (floats)

__host__ __device__ constexpr int mm_threads(int nt, int ks) {
  return nt >= 128 || (nt >= 64 && ks > kKC) ? 512 : kMmThreads;
}

// KS: input channels per K step, kKC (narrow inputs, double-buffered weights) or 2 kKC (one
// weight buffer, refilled after a barrier: half the per-step staging chains).
template <int MODE, int K, int LIN, int MT, int NT, int KS = kKC>
struct MmShape {
  static constexpr int LOUT = lout_for(MODE, LIN);
  static constexpr int SB = NT / LOUT;           // samples per column tile
  // One weight buffer in LDS (two workgroups per CU) for 32-channel steps on 64 x 64 and
  // 64 x 32 tiles; 64 x 128 tiles (one eight-wavefront workgroup per CU at the batches that
  // choose them) keep two and skip the refill barrier: pusht B=256 54.3 -> 53.9 ms.
  static constexpr bool W1 = KS > kKC && NT < 128;
  static constexpr int WBUF = W1 ? 1 : 2;
  static constexpr int WROW = K * KS + kPad;     // LDS floats per weight row
  static constexpr int XROW = KS + kPad;         // LDS floats per (sample, position) row
  static constexpr int ZERO = SB * LIN;          // index of the zero row
  static constexpr int XROWS = SB * LIN + 1;
  static constexpr int WFLOATS = MT * WROW;
  static constexpr int XFLOATS = XROWS * XROW;
  // 64 x 128 and (32-channel steps) 64 x 64 tiles take eight wavefronts, two per SIMD, so one
  // wavefront's LDS reads overlap another's MFMAs (a 2 x 4 grid of 32 x 32 or 32 x 16 tiles);
  // 64 x 32 and narrow 64 x 64 tiles four in a 2 x 2 grid.
  static constexpr int THREADS = mm_threads(NT, KS);
  static constexpr int WAVE_COLS = THREADS / 64 / 2;
  static constexpr int UW = MT * K * (KS / 4) / THREADS;  // weight float4 per lane per step
  static constexpr int XELEMS = SB * KS * LIN;               // input floats per step
  static constexpr int XV = LIN >= 4 ? 4 : 1;          // vector width of input loads
  static constexpr int XUNITS = XELEMS / XV;
  static constexpr int UX = (XUNITS + THREADS - 1) / THREADS;
  static constexpr int WM = MT / 2, WN = NT / WAVE_COLS;
  static constexpr int TI = WM / 16, TJ = WN / 16;
  static_assert(MT * K * (KS / 4) % THREADS == 0, "weight units per lane");
  static constexpr std::size_t LDS_FLOATS = WBUF * WFLOATS + 2 * XFLOATS;
  static_assert(NT % LOUT == 0 && XELEMS % XV == 0, "column tile");
};

template <bool BF16>
__device__ __forceinline__ float4 load_w4(const void* base, std::int64_t idx) {
  if constexpr (BF16) {
    const uint2 raw = *reinterpret_cast<const uint2*>(static_cast<const unsigned short*>(base) + idx);
    return float4{__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                  __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u)};
  } else {
    return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
  }
}

template <int MODE, int K, int LIN, bool BF16, int MT, int NT, bool NARROW>
__global__ __launch_bounds__(mm_threads(NT, NARROW ? kKC : 2 * kKC))
void conv_mfma_kernel(MmArgs a) {
  using S = MmShape<MODE, K, LIN, MT, NT, NARROW ? kKC : 2 * kKC>;
  constexpr int KS = NARROW ? kKC : 2 * kKC;
  extern __shared__ float4 lds4[];
  float* Ws = reinterpret_cast<float*>(lds4);  // [WBUF][WFLOATS]
  float* Xs = Ws + S::WBUF * S::WFLOATS;       // [2][XFLOATS]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // Tile index, grouped so that the workgroups on one XCD share weight tiles; with a split K
  // loop, workgroup (ks, tile) covers K steps [ks * n / ksplit, (ks + 1) * n / ksplit).
  int id = blockIdx.x;
  const int tiles = a.mtiles * a.ntiles;
  const int total = tiles * a.ksplit;
  if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
  const int ks = id / tiles;
  const int tile = id - ks * tiles;
  const int mt = tile / a.ntiles, nt = tile - mt * a.ntiles;
  const int m0 = mt * MT;
  const int b0 = nt * S::SB;
  const int nall = (a.ic + KS - 1) / KS;
  const int s0 = ks * nall / a.ksplit, s1 = (ks + 1) * nall / a.ksplit;

  // The bias of the tile's rows (first K slice only), read before the first K step's loads
  // and kept in LDS for the epilogue.
  __shared__ float bias_t[MT];
  float bias_r = 0.0f;
  if (tid < MT && ks == 0 && m0 + tid < a.oc) bias_r = a.bias[m0 + tid];

  // Zero rows of both input buffers (never overwritten).
  if (tid < 2 * KS) Xs[(tid / KS) * S::XFLOATS + S::ZERO * S::XROW + (tid % KS)] = 0.0f;

  float4 wreg[S::UW];
  float4 xreg[S::UX > 0 ? S::UX : 1];
  float xs1[S::XV == 1 ? S::UX : 1];
  auto load_step = [&](int step) {
    const int ic0 = step * KS;
#pragma unroll
    for (int r = 0; r < S::UW; ++r) {
      const int u = tid + r * S::THREADS;
      const int m = u / (K * (KS / 4)), rem = u - m * (K * (KS / 4));
      const int k = rem / (KS / 4), q = rem % (KS / 4);
      const int oc = m0 + m;
      if constexpr (NARROW) {
        // Channel counts that are not a multiple of 16: element-wise guarded loads.
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = ic0 + 4 * q + e;
          const std::int64_t idx = (static_cast<std::int64_t>(oc) * K + k) * a.ic + c;
          v[e] = 0.0f;
          if (oc < a.oc && c < a.ic)
            v[e] = BF16 ? __uint_as_float(static_cast<unsigned>(
                              static_cast<const unsigned short*>(a.w)[idx]) << 16)
                        : static_cast<const float*>(a.w)[idx];
        }
        wreg[r] = float4{v[0], v[1], v[2], v[3]};
      } else {
        wreg[r] = oc < a.oc ? load_w4<BF16>(a.w, (static_cast<std::int64_t>(oc) * K + k) * a.ic + ic0 + 4 * q)
                            : float4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
#pragma unroll
    for (int r = 0; r < S::UX; ++r) {
      const int u = tid + r * S::THREADS;
      if constexpr (S::XV == 4) {
        const int bl = u / (KS / 4 * LIN), v = u - bl * (KS / 4 * LIN);
        const int ch = v / (LIN / 4), t4 = (v - ch * (LIN / 4)) * 4;
        const int b = b0 + bl, c = ic0 + ch;
        float4 val = float4{0.0f, 0.0f, 0.0f, 0.0f};
        if (u < S::XUNITS && b < a.batch && (!NARROW || c < a.ic)) {
          const float* p = c < a.split ? a.src + b * a.src_stride + static_cast<std::int64_t>(c) * LIN
                                       : a.plain + b * a.plain_stride +
                                             static_cast<std::int64_t>(c - a.split) * LIN;
          val = *reinterpret_cast<const float4*>(p + t4);
        }
        xreg[r] = val;
      } else {
        const int bl = u / (KS * LIN), v = u - bl * (KS * LIN);
        const int ch = v / LIN, t = v - ch * LIN;
        const int b = b0 + bl, c = ic0 + ch;
        float val = 0.0f;
        if (u < S::XUNITS && b < a.batch && (!NARROW || c < a.ic))
          val = c < a.split ? a.src[b * a.src_stride + static_cast<std::int64_t>(c) * LIN + t]
                            : a.plain[b * a.plain_stride + static_cast<std::int64_t>(c - a.split) * LIN + t];
        xs1[r] = val;
      }
    }
  };
  auto store_step = [&](int buf) {
    float* W = Ws + (S::W1 ? 0 : buf * S::WFLOATS);
    float* X = Xs + buf * S::XFLOATS;
#pragma unroll
    for (int r = 0; r < S::UW; ++r) {
      const int u = tid + r * S::THREADS;
      const int m = u / (K * (KS / 4)), rem = u - m * (K * (KS / 4));
      const int k = rem / (KS / 4), q = rem % (KS / 4);
      *reinterpret_cast<float4*>(W + m * S::WROW + k * KS + 4 * q) = wreg[r];
    }
#pragma unroll
    for (int r = 0; r < S::UX; ++r) {
      const int u = tid + r * S::THREADS;
      if (u >= S::XUNITS) continue;
      if constexpr (S::XV == 4) {
        const int bl = u / (KS / 4 * LIN), v = u - bl * (KS / 4 * LIN);
        const int ch = v / (LIN / 4), t4 = (v - ch * (LIN / 4)) * 4;
        float* row = X + (bl * LIN + t4) * S::XROW + ch;
        row[0] = xreg[r].x;
        row[S::XROW] = xreg[r].y;
        row[2 * S::XROW] = xreg[r].z;
        row[3 * S::XROW] = xreg[r].w;
      } else {
        const int bl = u / (KS * LIN), v = u - bl * (KS * LIN);
        const int ch = v / LIN, t = v - ch * LIN;
        X[(bl * LIN + t) * S::XROW + ch] = xs1[r];
      }
    }
  };

  // Per-lane input row of every (column tile j, tap k): fixed for the whole K loop.  With
  // ConvTranspose the columns are in parity order, so wavefront column half wc holds output
  // positions of parity wc only, which taps of the other parity never reach.
  constexpr int PAR = MODE == kConvTranspose ? 1 : 0;
  const int wr = wave / S::WAVE_COLS, wc = wave % S::WAVE_COLS;
  const int par = 2 * wc / S::WAVE_COLS;  // output parity of this wavefront's columns (PAR)
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
      xrow[j][k] = (ti >= 0 ? bl * LIN + ti : S::ZERO) * S::XROW + 4 * kq;
    }
  }
  const int arow = (wr * S::WM + l16) * S::WROW + 4 * kq;

  floatx4 acc[S::TI][S::TJ];
#pragma unroll
  for (int i = 0; i < S::TI; ++i)
#pragma unroll
    for (int j = 0; j < S::TJ; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  load_step(s0);
  if (tid < MT) bias_t[tid] = bias_r;
  store_step(0);
  __syncthreads();
  for (int step = s0; step < s1; ++step) {
    const int buf = (step - s0) & 1;
    if (step + 1 < s1) load_step(step + 1);
    const float* W = Ws + (S::W1 ? 0 : buf * S::WFLOATS);
    const float* X = Xs + buf * S::XFLOATS;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      // Output t takes tap k when t + 1 - k is even: parity par takes the taps k = par + 1 mod 2.
      if constexpr (PAR) {
        if (((k + par + 1) & 1) != 0) continue;
      }
#pragma unroll
      for (int kc = 0; kc < KS / kKC; ++kc) {
        float4 av[S::TI], bv[S::TJ];
#pragma unroll
        for (int i = 0; i < S::TI; ++i)
          av[i] = *reinterpret_cast<const float4*>(W + arow + i * 16 * S::WROW + k * KS +
                                                   kc * kKC);
#pragma unroll
        for (int j = 0; j < S::TJ; ++j)
          bv[j] = *reinterpret_cast<const float4*>(X + xrow[j][k] + kc * kKC);
#pragma unroll
        for (int i = 0; i < S::TI; ++i)
#pragma unroll
          for (int j = 0; j < S::TJ; ++j) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i].x, bv[j].x, acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i].y, bv[j].y, acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i].z, bv[j].z, acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i].w, bv[j].w, acc[i][j], 0, 0, 0);
          }
      }
    }
    if (step + 1 < s1) {
      if constexpr (S::W1) __syncthreads();  // the one weight buffer is read by every wavefront
      store_step(buf ^ 1);
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
  // Output layout: when the tile fits the staging LDS it goes through it as [sample, position]
  // [channel], so that each sample's MT x LOUT block (contiguous in y) is written by
  // consecutive lanes.
  constexpr int TROW = MT + 1;
  if constexpr (NT * TROW <= S::LDS_FLOATS) {
    float* T = reinterpret_cast<float*>(lds4);
    __syncthreads();  // the last K step's LDS reads are done
#pragma unroll
    for (int j = 0; j < S::TJ; ++j) {
      const int col = wc * S::WN + 16 * j + l16;
      int bl, t;
      col_pos(col, NT, S::LOUT, PAR, bl, t);
      float* tr = T + (bl * S::LOUT + t) * TROW + wr * S::WM + 4 * kq;
#pragma unroll
      for (int i = 0; i < S::TI; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) tr[16 * i + e] = acc[i][j][e];
    }
    __syncthreads();
    float* yk = a.y + ks * a.ypart;
    for (int idx = tid; idx < NT * MT; idx += S::THREADS) {
      const int bl = idx / (MT * S::LOUT);
      const int rem = idx - bl * (MT * S::LOUT);
      const int row = rem / S::LOUT, t = rem - row * S::LOUT;
      const int b = b0 + bl, oc = m0 + row;
      if (b < a.batch && oc < a.oc)
        yk[b * a.ys + static_cast<std::int64_t>(oc) * S::LOUT + t] =
            T[(bl * S::LOUT + t) * TROW + row] + bias_t[row];
    }
  } else {
#pragma unroll
    for (int i = 0; i < S::TI; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int oc = m0 + wr * S::WM + 16 * i + 4 * kq + e;
        if (oc >= a.oc) continue;
        const float bias = bias_t[wr * S::WM + 16 * i + 4 * kq + e];
#pragma unroll
        for (int j = 0; j < S::TJ; ++j) {
          const int col = wc * S::WN + 16 * j + l16;
          int bl, t;
          col_pos(col, NT, S::LOUT, PAR, bl, t);
          const int b = b0 + bl;
          if (b < a.batch)
            a.y[ks * a.ypart + b * a.ys + static_cast<std::int64_t>(oc) * S::LOUT + t] =
                acc[i][j][e] + bias;
        }
      }
  }
}

// Sums the ksplit partial tiles of a split-K convolution in a fixed order and adds the bias.
__global__ __launch_bounds__(kMmThreads) void splitk_reduce_kernel(MmArgs a, int nt_cols, int lout) {
  const int tiles = a.mtiles * a.ntiles;
  const int per = 64 * nt_cols;
  const std::int64_t e = static_cast<std::int64_t>(blockIdx.x) * kMmThreads + threadIdx.x;
  if (e >= static_cast<std::int64_t>(tiles) * per) return;
  const int tile = static_cast<int>(e / per), local = static_cast<int>(e - static_cast<std::int64_t>(tile) * per);
  float sum = 0.0f;
  for (int ks = 0; ks < a.ksplit; ++ks)
    sum += a.part[(static_cast<std::int64_t>(ks) * tiles + tile) * per + local];
  const int mt = tile / a.ntiles, nt = tile - mt * a.ntiles;
  const int r = local / nt_cols, c = local - r * nt_cols;
  const int oc = mt * 64 + r;
  int bl, t;
  col_pos(c, nt_cols, lout, a.par, bl, t);
  const int b = nt * (nt_cols / lout) + bl;
  if (oc < a.oc && b < a.batch)
    a.y[b * a.ys + static_cast<std::int64_t>(oc) * lout + t] = sum + a.bias[oc];
}

// ---------------------------------------------------------------------------------------------
// Per-sample prologue: dst = mish(GN(src)) [* scale + shift] [+ res] for the `split` channels.
// ---------------------------------------------------------------------------------------------
constexpr int kNaThreads = 512;
constexpr int kNaMaxFloats = 8192;

template <int LIN>
__global__ __launch_bounds__(kNaThreads) void norm_act_kernel(ConvInput in, float* dst,
                                                              std::int64_t dst_stride) {
  constexpr int QN = kNaMaxFloats / 4 / kNaThreads;
  __shared__ double ps[kNaMaxFloats / 4], pq[kNaMaxFloats / 4];
  __shared__ float gmean[32], ginv[32];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int nqn = in.split * LIN / 4;
  const int npg = in.split / in.groups * LIN / 4;
  const float* src = in.src + b * in.src_stride;
  const float* ft = in.film_time != nullptr ? in.film_time + in.film_off : nullptr;
  const float* fc = in.film_time != nullptr ? in.film_cond + b * in.film_cond_stride + in.film_off : nullptr;
  // LIN >= 4: one channel per 16-byte group, whose affine and FiLM coefficients are read with the
  // values, before the statistics, so that their latency is not added after them.
  constexpr bool PRE = LIN >= 4;
  float ga[QN], be[QN], t0[QN], c0[QN], t1[QN], c1[QN];
  if constexpr (PRE) {
#pragma unroll
    for (int m = 0; m < QN; ++m) {
      const int q = tid + m * kNaThreads;
      const int c = q < nqn ? 4 * q / LIN : 0;
      ga[m] = in.gamma[c];
      be[m] = in.beta[c];
      t0[m] = ft != nullptr ? ft[c] : 0.0f;
      c0[m] = ft != nullptr ? fc[c] : 0.0f;
      t1[m] = ft != nullptr ? ft[in.split + c] : 0.0f;
      c1[m] = ft != nullptr ? fc[in.split + c] : 0.0f;
    }
  }
  float4 x[QN], r[QN];
#pragma unroll
  for (int m = 0; m < QN; ++m) {
    const int q = tid + m * kNaThreads;
    x[m] = float4{0.0f, 0.0f, 0.0f, 0.0f};
    r[m] = float4{0.0f, 0.0f, 0.0f, 0.0f};
    if (q < nqn) {
      x[m] = *reinterpret_cast<const float4*>(src + 4 * q);
      if (in.res != nullptr) r[m] = *reinterpret_cast<const float4*>(in.res + b * in.res_stride + 4 * q);
    }
  }
#pragma unroll
  for (int m = 0; m < QN; ++m) {
    const int q = tid + m * kNaThreads;
    if (q < nqn) {
      const double d0 = x[m].x, d1 = x[m].y, d2 = x[m].z, d3 = x[m].w;
      ps[q] = (d0 + d1) + (d2 + d3);
      pq[q] = (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
    }
  }
  __syncthreads();
  // Sixteen lanes per group (all 32 groups in one pass), a 16-lane row reduction (DPP), and the
  // row's first lane finishes the mean and 1/std.
  {
    const int g = tid >> 4, sub = tid & 15;
    double s = 0.0, sq = 0.0;
    if (g < in.groups) {
      for (int i = sub; i < npg; i += 16) {
        s += ps[g * npg + i];
        sq += pq[g * npg + i];
      }
    }
    s = row_sum(s);
    sq = row_sum(sq);
    if (sub == 0 && g < in.groups) {
      const double n = 4.0 * npg;
      const double mean = s / n;
      const double var = fmax(0.0, sq / n - mean * mean);
      gmean[g] = static_cast<float>(mean);
      ginv[g] = static_cast<float>(1.0 / sqrt(var + 1e-5));
    }
  }
  __syncthreads();
#pragma unroll
  for (int m = 0; m < QN; ++m) {
    const int q = tid + m * kNaThreads;
    if (q >= nqn) continue;
    const int g = q / npg;
    const float mean = gmean[g], inv = ginv[g];
    float v[4] = {x[m].x, x[m].y, x[m].z, x[m].w};
    const float rr[4] = {r[m].x, r[m].y, r[m].z, r[m].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float val;
      if constexpr (PRE) {
        val = mish_fast(fmaf(v[i] - mean, inv * ga[m], be[m]));
        if (ft != nullptr) val = fmaf(t0[m] + c0[m], val, t1[m] + c1[m]);
      } else {
        const int c = (4 * q + i) / LIN;
        val = mish_fast(fmaf(v[i] - mean, inv * in.gamma[c], in.beta[c]));
        if (ft != nullptr) val = fmaf(ft[c] + fc[c], val, ft[in.split + c] + fc[in.split + c]);
      }
      v[i] = val + rr[i];
    }
    *reinterpret_cast<float4*>(dst + b * dst_stride + 4 * q) = float4{v[0], v[1], v[2], v[3]};
  }
}

template <int MODE, int K, int LIN, bool BF16, int MT, int NT, bool NARROW>
hipError_t launch_mm(const MmArgs& a, hipStream_t s) {
  using S = MmShape<MODE, K, LIN, MT, NT, NARROW ? kKC : 2 * kKC>;
  const std::size_t smem = S::LDS_FLOATS * sizeof(float);
  auto fn = conv_mfma_kernel<MODE, K, LIN, BF16, MT, NT, NARROW>;
  static bool raised = false;
  if (!raised && smem > 48 * 1024) {
    const hipError_t st = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                              hipFuncAttributeMaxDynamicSharedMemorySize,
                                              static_cast<int>(smem));
    if (st != hipSuccess) return st;
    raised = true;
  }
  hipLaunchKernelGGL(fn, dim3(a.mtiles * a.ntiles * a.ksplit), dim3(S::THREADS), smem, s, a);
  return hipGetLastError();
}

template <int MODE, int K, int LIN, bool BF16>
hipError_t by_tile(int tile, bool narrow, const MmArgs& a, hipStream_t s) {
  if (narrow) {
    if constexpr (MODE == kConvSame) return launch_mm<MODE, K, LIN, BF16, 64, 64, true>(a, s);
    return hipErrorInvalidValue;
  }
  if (tile == kTile64x32) return launch_mm<MODE, K, LIN, BF16, 64, 32, false>(a, s);
  return tile == kTile64x128 ? launch_mm<MODE, K, LIN, BF16, 64, 128, false>(a, s)
                             : launch_mm<MODE, K, LIN, BF16, 64, 64, false>(a, s);
}

template <int MODE, int K, bool BF16>
hipError_t by_lin_mm(int lin, int tile, bool narrow, const MmArgs& a, hipStream_t s) {
  switch (lin) {
    case 1:
      if constexpr (MODE != kConvDown) return by_tile<MODE, K, 1, BF16>(tile, narrow, a, s);
      break;
    case 2: return by_tile<MODE, K, 2, BF16>(tile, narrow, a, s);
    case 4: return by_tile<MODE, K, 4, BF16>(tile, narrow, a, s);
    case 8: return by_tile<MODE, K, 8, BF16>(tile, narrow, a, s);
    case 16:
      if constexpr (MODE != kConvTranspose) return by_tile<MODE, K, 16, BF16>(tile, narrow, a, s);
      break;
    default: break;
  }
  return hipErrorInvalidValue;
}

template <bool BF16>
hipError_t by_kernel_mm(const ConvOp& op, int tile, bool narrow, const MmArgs& a, hipStream_t s) {
  if (op.mode == kConvSame) {
    switch (op.k) {
      case 1: return by_lin_mm<kConvSame, 1, BF16>(op.lin, tile, narrow, a, s);
      case 3: return by_lin_mm<kConvSame, 3, BF16>(op.lin, tile, narrow, a, s);
      case 5: return by_lin_mm<kConvSame, 5, BF16>(op.lin, tile, narrow, a, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (op.mode == kConvDown && op.k == 3) return by_lin_mm<kConvDown, 3, BF16>(op.lin, tile, narrow, a, s);
  if (op.mode == kConvTranspose && op.k == 4)
    return by_lin_mm<kConvTranspose, 4, BF16>(op.lin, tile, narrow, a, s);
  return hipErrorInvalidValue;
}

bool lin_mm_ok(int mode, int lin) {
  if (lin != 1 && lin != 2 && lin != 4 && lin != 8 && lin != 16) return false;
  if (mode == kConvDown && lin < 2) return false;
  if (mode == kConvTranspose && lin > 8) return false;
  return true;
}

}  // namespace

bool conv_mfma_supported(const ConvOp& op, int split) {
  if (!lin_mm_ok(op.mode, op.lin) || op.lout != lout_for(op.mode, op.lin)) return false;
  if (split > op.ic || split <= 0 || op.oc <= 0 || op.ic <= 0) return false;
  if (op.ic % (2 * kKC) != 0) {
    // Narrow inputs (the first convolution reads action_dim channels; widths that are not
    // 32-channel multiples): one plain source, 16-channel steps with guarded loads.
    return split == op.ic && op.mode == kConvSame && (op.k == 1 || op.k == 3 || op.k == 5);
  }
  if (split % kKC != 0) return false;
  if (op.mode == kConvSame) return op.k == 1 || op.k == 3 || op.k == 5;
  if (op.mode == kConvDown) return op.k == 3;
  return op.mode == kConvTranspose && op.k == 4;
}

namespace {

// Tile shape, kernel choice and K split of one matrix-core convolution.  With max_parts >= 2 a
// split K writes up to max_parts partial sums in the output layout (no workspace, no
// reduction pass); otherwise partial tiles go to a workspace of workspace_floats.
struct MmPlan {
  int tile = kTile64x128;
  int nt_cols = 128;
  bool narrow = false, use_bf16 = false;
  int mtiles = 0, ntiles = 0, ksplit = 1;
  bool in_output = false;
  std::uint64_t wb = 0, sb = 0, pb = 0;
};

// Tuning overrides, read once: FLOWEDGE_MM_TILE=32|64|128 forces the column tile (64 x 32,
// 64 x 64 or 64 x 128 blocks; narrow inputs always take 64 x 64),
// FLOWEDGE_MM_WGS the workgroup count the K split aims at (default 512, two per CU).
struct MmTuning {
  int tile = 0;
  int target = 512;
};
const MmTuning& mm_tuning() {
  static const MmTuning t = [] {
    MmTuning m;
    if (const char* v = std::getenv("FLOWEDGE_MM_TILE")) m.tile = std::atoi(v);
    if (const char* v = std::getenv("FLOWEDGE_MM_WGS")) m.target = std::max(1, std::atoi(v));
    return m;
  }();
  return t;
}

MmPlan mm_plan(const ConvOp& op, int split, std::int64_t src_stride, const float* plain,
               std::int64_t plain_stride, int batch, std::size_t workspace_floats, bool bf16_mma,
               bool f32_split, int max_parts) {
  const MmTuning& tune = mm_tuning();
  MmPlan p;
  p.narrow = op.ic % (2 * kKC) != 0;
  p.mtiles = (op.oc + 63) / 64;
  p.ntiles = (batch + 128 / op.lout - 1) / (128 / op.lout);
  const bool small = tune.tile == 64 || (tune.tile != 128 && p.mtiles * p.ntiles < 256);
  if (p.narrow || small) {
    p.tile = kTile64x64;
    p.ntiles = (batch + 64 / op.lout - 1) / (64 / op.lout);
  }
  p.nt_cols = p.tile == kTile64x128 ? 128 : 64;
  // The BF16 kernels address weights and inputs through 32-bit buffer offsets.
  p.wb = static_cast<std::uint64_t>(op.oc) * op.k * op.ic * (op.bf16 ? 2 : 4);
  p.sb = static_cast<std::uint64_t>(batch) * src_stride * 4;
  p.pb = plain != nullptr ? static_cast<std::uint64_t>(batch) * plain_stride * 4 : 0;
  const bool ranges_fit = p.wb < (1ull << 31) && p.sb < (1ull << 31) && p.pb < (1ull << 31);
  p.use_bf16 = (op.bf16 ? bf16_mma : f32_split) && ranges_fit && mm_bf16_ok(op, split);
  // Fewer than 64 tiles of 64 x 64: 64 x 32 blocks, so that the split K loop runs on twice the
  // workgroups (two per CU, whose K steps overlap), and a batch that fills under 64 columns
  // leaves none of them empty.  (Not for F32 weights on the BF16 matrix cores, which have no
  // 64 x 32 instance.)
  if (!(p.use_bf16 && !op.bf16) && p.tile == kTile64x64 && !p.narrow &&
      (tune.tile == 32 || (tune.tile == 0 && p.mtiles * p.ntiles < 64))) {
    p.tile = kTile64x32;
    p.nt_cols = 32;
    p.ntiles = (batch + 32 / op.lout - 1) / (32 / op.lout);
  }
  const int tiles = p.mtiles * p.ntiles;
  const int fks = p.narrow ? kKC : 2 * kKC;  // F32 kernel's K step
  const int nsteps = p.use_bf16 ? op.ic / mm_bf16_step(op) : (op.ic + fks - 1) / fks;
  // Split the K loop when the output tiles alone leave CUs idle (small batches): aim at two
  // workgroups per CU, so that two K steps of weights stream per CU at a time.
  if (tiles < tune.target / 2) {
    int ks = (tune.target + tiles - 1) / tiles;
    if (ks > nsteps) ks = nsteps;
    if (max_parts >= 2) {
      if (ks > max_parts) ks = max_parts;
      if (ks > 1) {
        p.ksplit = ks;
        p.in_output = true;
      }
    } else if (ks > 1 &&
               static_cast<std::size_t>(ks) * tiles * 64 * p.nt_cols <= workspace_floats) {
      p.ksplit = ks;
    }
  }
  return p;
}

}  // namespace

int conv_mfma_parts(const ConvOp& op, int split, std::int64_t src_stride, const float* plain,
                    std::int64_t plain_stride, int batch, bool bf16_mma, bool f32_split,
                    int max_parts) {
  if (!conv_mfma_supported(op, split) || batch <= 0 || max_parts < 2) return 1;
  return mm_plan(op, split, src_stride, plain, plain_stride, batch, 0, bf16_mma, f32_split,
                 max_parts)
      .ksplit;
}

int conv_mfma_ksplit(const ConvOp& op, int split, std::int64_t src_stride, const float* plain,
                     std::int64_t plain_stride, int batch, std::size_t workspace_floats,
                     bool bf16_mma, bool f32_split, int max_parts) {
  if (!conv_mfma_supported(op, split) || batch <= 0) return 1;
  return mm_plan(op, split, src_stride, plain, plain_stride, batch, workspace_floats, bf16_mma,
                 f32_split, max_parts)
      .ksplit;
}

hipError_t conv_mfma(const ConvOp& op, const float* src, std::int64_t src_stride, int split,
                     const float* plain, std::int64_t plain_stride, View y, int batch,
                     float* workspace, std::size_t workspace_floats, bool bf16_mma,
                     bool f32_split, hipStream_t stream, int max_parts) {
  if (!conv_mfma_supported(op, split) || batch <= 0) return hipErrorInvalidValue;
  if (split < op.ic && plain == nullptr) return hipErrorInvalidValue;
  const MmPlan p = mm_plan(op, split, src_stride, plain, plain_stride, batch,
                           workspace != nullptr ? workspace_floats : 0, bf16_mma, f32_split,
                           max_parts);
  if (p.in_output && y.part <= 0) return hipErrorInvalidValue;
  MmArgs a{};
  a.w = op.w;
  a.bias = op.b;
  a.y = y.p;
  a.ys = y.stride;
  a.src = src;
  a.src_stride = src_stride;
  a.split = split;
  a.plain = plain;
  a.plain_stride = plain_stride;
  a.oc = op.oc;
  a.ic = op.ic;
  a.batch = batch;
  a.mtiles = p.mtiles;
  a.ntiles = p.ntiles;
  // The kernels order ConvTranspose tile columns by output parity (the split-K reduction reads
  // the partial tiles in the same order).
  a.par = op.mode == kConvTranspose ? 1 : 0;
  a.wbytes = static_cast<unsigned>(p.wb);
  a.srcbytes = static_cast<unsigned>(p.sb);
  a.plainbytes = static_cast<unsigned>(p.pb);
  a.ksplit = p.ksplit;
  if (p.ksplit > 1) {
    if (p.in_output)
      a.ypart = y.part;
    else
      a.part = workspace;
  }
  const hipError_t st = p.use_bf16 ? launch_mm_bf16(op, p.tile, a, stream)
                        : op.bf16  ? by_kernel_mm<true>(op, p.tile, p.narrow, a, stream)
                                   : by_kernel_mm<false>(op, p.tile, p.narrow, a, stream);
  if (st != hipSuccess || a.ksplit == 1 || p.in_output) return st;
  const std::int64_t elems = static_cast<std::int64_t>(p.mtiles * p.ntiles) * 64 * p.nt_cols;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(static_cast<unsigned>((elems + kMmThreads - 1) / kMmThreads)),
                     dim3(kMmThreads), 0, stream, a, p.nt_cols, op.lout);
  return hipGetLastError();
}

hipError_t norm_act(const ConvInput& in, int lin, float* dst, std::int64_t dst_stride, int batch,
                    hipStream_t stream) {
  if (!in.norm || batch <= 0 || in.groups <= 0 || in.split % in.groups != 0)
    return hipErrorInvalidValue;
  // Below 256 samples the one-workgroup-per-sample kernel leaves CUs idle; the general form
  // spreads each sample over one workgroup per group (measured equal at 256).  Inputs made of
  // partial sums run on the general form too.
  if (batch < 256 || in.parts > 1 || in.res_parts > 1 || in.groups > 32 || (in.split / in.groups * lin) % 4 != 0 ||
      static_cast<std::int64_t>(in.split) * lin > kNaMaxFloats)
    return norm_act_general(in, lin, dst, dst_stride, batch, stream);
  switch (lin) {
    case 1: hipLaunchKernelGGL(norm_act_kernel<1>, dim3(batch), dim3(kNaThreads), 0, stream, in, dst, dst_stride); break;
    case 2: hipLaunchKernelGGL(norm_act_kernel<2>, dim3(batch), dim3(kNaThreads), 0, stream, in, dst, dst_stride); break;
    case 4: hipLaunchKernelGGL(norm_act_kernel<4>, dim3(batch), dim3(kNaThreads), 0, stream, in, dst, dst_stride); break;
    case 8: hipLaunchKernelGGL(norm_act_kernel<8>, dim3(batch), dim3(kNaThreads), 0, stream, in, dst, dst_stride); break;
    case 16: hipLaunchKernelGGL(norm_act_kernel<16>, dim3(batch), dim3(kNaThreads), 0, stream, in, dst, dst_stride); break;
    default: return norm_act_general(in, lin, dst, dst_stride, batch, stream);
  }
  return hipGetLastError();
}

}  // namespace fe::hip
