// Fused weight-streaming convolution for the Diffusion Policy U-Net on gfx950 (device template).
//
// One launch computes a Conv1d (kernel 3/5 "same", the K=3 stride-2 conv of Downsample1d, or the
// K=4 stride-2 ConvTranspose1d of Upsample1d) of one sample per grid row, optionally together with
// the ResidualBlock's 1x1 projection of the same input (as an extra tap with its own outputs).
// Weights are stored [OC][K][IC] (repacked at load), so the lanes of a row group stream
// consecutive 16-byte vectors of one (oc, tap) row.
//
// Work split: 512-lane workgroups, at most one per CU (two wavefronts per SIMD, so up to 256
// VGPRs per lane hold the weights in flight).  A workgroup
//   1. requests its share of the input (raw producer output, residual, GroupNorm/FiLM parameters)
//      into registers,
//   2. then requests every weight vector of its first row tile (up to 128 floats per lane), so the
//      input arrives first and the weights keep streaming during the prologue,
//   3. computes the GroupNorm statistics of the sample (fp64 partials, var = E[x^2] - mean^2 as
//      group_norm, diffusion_ops.cc:270-350), applies GN + Mish (+ FiLM) (+ residual), writes its
//      share of the result out for ops that read it again ("materialises" it), and stages the
//      whole input in LDS, channel-swizzled so row-group reads are bank-conflict free,
//   4. walks its row tiles: as each input chunk's products are accumulated, the registers that
//      held its weights are refilled with the next tile's, then partial sums are folded with a
//      wavefront reduce-scatter (and across wavefronts through LDS when a row spans several).
// Barriers inside the kernel order LDS only; weight loads stay in flight across them.
//
// Reference semantics: conv1d diffusion_ops.cc:82-163, conv_transpose1d :165-268, film :352-377,
// ResidualBlock diffusion.cc:724-773.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

namespace fe::hip::conv {

using namespace dev;

constexpr int kThreads = 512;
constexpr int kMaxStageFloats = 16384;  // staged input per sample: channels * positions (64 KB)
constexpr int kMaxNormFloats = 8192;    // of which normalised (GroupNorm prologue)
constexpr int kMaxGroups = 32;
constexpr int kWeightRegs = 128;        // weight floats in flight per lane
constexpr int kMaxBlocks = 256;         // one workgroup per CU

// Input prologue kinds (the only ones the U-Net produces).
enum Prologue : int {
  kProPlain = 0,  // raw tensor(s)
  kProFilm = 1,   // FiLM(mish(GN(src)))            (ResidualBlock conv2 input)
  kProResid = 2,  // mish(GN(src)) + res, then plain (ResidualBlock output, maybe with a skip)
};

__host__ __device__ constexpr int lout_of(int mode, int lin) {
  return mode == kConvSame ? lin : (mode == kConvDown ? lin / 2 : 2 * lin);
}

// Input chunks (VEC channels each) a lane handles per row: bounded by the weight registers (fewer
// at LIN >= 8, where the chunk's input vectors take more), by what the largest staged input needs
// at 64 lanes per row, and by 8.
__host__ __device__ constexpr int chunk_budget(int k, int lin, bool res, int vec) {
  const int taps = k + (res ? 1 : 0);
  const int regs = lin >= 16 ? kWeightRegs - 64 : (lin >= 8 ? kWeightRegs - 32 : kWeightRegs);
  const int by_regs = regs / (taps * vec);
  const int by_size = (kMaxStageFloats / (lin * vec) + 63) / 64;
  const int n = by_regs < by_size ? by_regs : by_size;
  return n < 8 ? n : 8;
}

// Weight floats per lane requested before the input prologue.
constexpr int kEarlyFloats = 64;
__host__ __device__ constexpr int early_chunks(int taps) {
  return kEarlyFloats / (taps * 4) > 0 ? kEarlyFloats / (taps * 4) : 1;
}

struct Args {
  const void* w;       // [oc][K][ic]
  const float* bias;   // [oc]
  float* y;            // [B][oc][lout]
  std::int64_t ys;
  const void* rw;      // fused 1x1 projection [oc][ic] (RES)
  const float* rbias;
  float* yr;
  std::int64_t yrs;
  int bf16, rbf16;
  unsigned wbytes, rwbytes;  // weight tensor sizes (buffer range; < 2 GiB)
  int oc, ic;
  int tiles;   // row tiles of kThreads / tpr rows
  int blocks;  // workgroups (grid.x); workgroup g takes tiles g, g + blocks, ...
  int tpr;     // lanes per row
  int nch;     // chunks per lane (<= chunk_budget)
  // Input-channel slices (sliced kernel only): grid.x = blocks * slices; workgroup x takes slice
  // x % slices and, within it, tiles x / slices, + blocks, ... of `tiles`; it stages channels
  // [slice * ics, +ics) and writes the partial sum of that slice to y + slice * ypart (bias in
  // slice 0 only).
  int slices = 1;
  int ics = 0;
  std::int64_t ypart = 0, yrpart = 0;
  ConvInput in;
};

// Per-launch replacements of two input pointers (the persistent tick kernel runs one step table
// for every evaluation): the FiLM time row of the evaluation and a per-workgroup input.
struct Override {
  const float* src = nullptr;        // replaces in.src when set
  const float* film_time = nullptr;  // replaces in.film_time when set
};

// Workgroup barrier that orders LDS accesses only: global loads in flight are not waited for.
__device__ __forceinline__ void lds_barrier() { __barrier(__CLK_LOCAL_MEM_FENCE); }

// Input index read by output t through tap k, or -1 when it falls in the zero padding.
template <int MODE, int K, int LIN>
__device__ __forceinline__ constexpr int src_index(int t, int k) {
  if constexpr (MODE == kConvSame) {
    const int j = t + k - K / 2;
    return (j >= 0 && j < LIN) ? j : -1;
  } else if constexpr (MODE == kConvDown) {
    const int j = 2 * t + k - 1;
    return (j >= 0 && j < LIN) ? j : -1;
  } else {
    // ConvTranspose: output ot = 2 * it + k - 1.
    const int num = t + 1 - k;
    if (num < 0 || (num & 1)) return -1;
    const int j = num / 2;
    return j < LIN ? j : -1;
  }
}

template <int VEC>
__device__ __forceinline__ void load_w(const void* base, int bf16, std::int64_t idx, float* out) {
  if (bf16) {
    const unsigned short* p = static_cast<const unsigned short*>(base) + idx;
    if constexpr (VEC == 4) {
      const uint2 raw = *reinterpret_cast<const uint2*>(p);
      out[0] = __uint_as_float(raw.x << 16);
      out[1] = __uint_as_float(raw.x & 0xffff0000u);
      out[2] = __uint_as_float(raw.y << 16);
      out[3] = __uint_as_float(raw.y & 0xffff0000u);
    } else {
      out[0] = bf16_to_f32(*p);
    }
  } else {
    const float* p = static_cast<const float*>(base) + idx;
    if constexpr (VEC == 4) {
      const float4 v = *reinterpret_cast<const float4*>(p);
      out[0] = v.x;
      out[1] = v.y;
      out[2] = v.z;
      out[3] = v.w;
    } else {
      out[0] = *p;
    }
  }
}

// Weight vectors are read with buffer loads: an inactive lane or chunk gets an out-of-range offset,
// which returns zeros without touching memory, so every load is issued unconditionally (no
// branches around them, and the waits the compiler places for the prologue's reads leave the
// weight loads in flight).
constexpr unsigned kOutOfRange = 0x80000000u;
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, kRsrcWord3);
}

// voff: byte offset of the row/chunk (or kOutOfRange); soff: wave-uniform byte offset of the tap.
// Weights are read once per U-Net evaluation (about 1 GB for the pusht-size model, more than the
// 256 MB MALL holds), so they are loaded non-temporal (cache policy nt): they then stop evicting
// the activations the next layers read from L2 and MALL (B=1 DDIM-10 tick 3.49 -> 3.15 ms).
constexpr int kWeightPolicy = 2;  // nt

template <bool BF16>
__device__ __forceinline__ void load_vec4(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff,
                                          float* out) {
  if constexpr (BF16) {
    const auto t = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kWeightPolicy);
    const uint2 raw = __builtin_bit_cast(uint2, t);
    out[0] = __uint_as_float(raw.x << 16);
    out[1] = __uint_as_float(raw.x & 0xffff0000u);
    out[2] = __uint_as_float(raw.y << 16);
    out[3] = __uint_as_float(raw.y & 0xffff0000u);
  } else {
    const auto t = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kWeightPolicy);
    const float4 v = __builtin_bit_cast(float4, t);
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
  }
}

// Weights of one input chunk (all taps, then the projection tap) of one row.
// `c0`: first input channel of the workgroup's slice (0 unsliced).
template <int K, int VEC, bool RES, bool BF16>
__device__ __forceinline__ void load_chunk(const Args& a, __amdgpu_buffer_rsrc_t wr,
                                           __amdgpu_buffer_rsrc_t rr, int row, int cv, bool valid,
                                           float (&w)[K + (RES ? 1 : 0)][VEC], int c0 = 0) {
  if constexpr (VEC == 4) {
    constexpr unsigned es = BF16 ? 2u : 4u;
    const unsigned voff =
        valid ? static_cast<unsigned>(row * K * a.ic + c0 + cv * 4) * es : kOutOfRange;
#pragma unroll
    for (int k = 0; k < K; ++k)
      load_vec4<BF16>(wr, voff, static_cast<unsigned>(k * a.ic) * es, w[k]);
    if constexpr (RES) {
      const unsigned roff =
          valid ? static_cast<unsigned>(row * a.ic + c0 + cv * 4) * es : kOutOfRange;
      load_vec4<BF16>(rr, roff, 0u, w[K]);
    }
  } else {
    // Narrow inputs (first convolution only): plain loads, bf16 decided at run time.
    if (valid) {
#pragma unroll
      for (int k = 0; k < K; ++k)
        load_w<1>(a.w, a.bf16, (static_cast<std::int64_t>(row) * K + k) * a.ic + cv, w[k]);
      if constexpr (RES) load_w<1>(a.rw, a.rbf16, static_cast<std::int64_t>(row) * a.ic + cv, w[K]);
    } else {
#pragma unroll
      for (int k = 0; k < K + (RES ? 1 : 0); ++k) w[k][0] = 0.0f;
    }
  }
}

// LDS layout of the staged input: channel c = 4 cv + v, position t lives at
//   (v * NPB + t / P) * (nv * P + kSwzPad) + cv * P + t % P,   P = min(LIN, 4), NPB = LIN / P,
// so for fixed (v, t / P) the lanes of a row group (consecutive cv) read consecutive P-float
// vectors.  The staging writes run the other way (consecutive lanes hold consecutive positions,
// then channels, i.e. consecutive planes v * NPB + t / P); the pad of 4 floats per plane moves
// each plane to the next 16-byte bank group so those writes are free of bank conflicts too.
constexpr int kSwzPad = 4;
template <int LIN>
struct Swz {
  static constexpr int P = LIN >= 4 ? 4 : LIN;
  static constexpr int NPB = LIN / P;
  __device__ static __forceinline__ int at(int c, int t, int nv) {
    return ((c & 3) * NPB + t / P) * (nv * P + kSwzPad) + (c >> 2) * P + t % P;
  }
};

template <int LIN, int PRO>
struct StageRegs {
  static constexpr int QMAX = (kMaxStageFloats / 4 + kThreads - 1) / kThreads;
  static constexpr int QN = PRO == kProPlain ? 1 : (kMaxNormFloats / 4 + kThreads - 1) / kThreads;
  static constexpr int QP = LIN >= 4 ? QN : 1;  // per-chunk parameters (one channel per chunk)
  float4 x[QMAX];
  float4 r[PRO == kProResid ? QN : 1];
  float gam[QP], bet[QP];
  float ts[PRO == kProFilm ? QP : 1], cs[PRO == kProFilm ? QP : 1];
  float tb[PRO == kProFilm ? QP : 1], cb[PRO == kProFilm ? QP : 1];
};

// The per-channel prologue parameters of chunk q (GroupNorm affine, FiLM time and condition rows;
// one channel per chunk at LIN >= 4): tensors no step of a tick writes.
template <int LIN, int PRO>
__device__ __forceinline__ void stage_chunk_params(const Args& a, int b, StageRegs<LIN, PRO>& s,
                                                   Override ov, int m, int q) {
  if constexpr (PRO != kProPlain && LIN >= 4) {
    const ConvInput& in = a.in;
    const int c = 4 * q / LIN;
    s.gam[m] = in.gamma[c];
    s.bet[m] = in.beta[c];
    if constexpr (PRO == kProFilm) {
      const float* ft = (ov.film_time != nullptr ? ov.film_time : in.film_time) + in.film_off;
      const float* fc = in.film_cond + b * in.film_cond_stride + in.film_off;
      s.ts[m] = ft[c];
      s.cs[m] = fc[c];
      s.tb[m] = ft[in.split + c];
      s.cb[m] = fc[in.split + c];
    }
  }
}

// The tick kernel's early half of step 1: the parameters, requested before it waits for the
// producers of the input.
template <int LIN, int PRO>
__device__ __forceinline__ void stage_params(const Args& a, int b, StageRegs<LIN, PRO>& s,
                                             Override ov) {
  using S = StageRegs<LIN, PRO>;
  if constexpr (PRO != kProPlain && LIN >= 4) {
    const int nqn = a.in.split * LIN / 4;
#pragma unroll
    for (int m = 0; m < S::QN; ++m) {
      const int q = threadIdx.x + m * kThreads;
      if (q < nqn) stage_chunk_params<LIN, PRO>(a, b, s, ov, m, q);
    }
  }
}

// Step 1: every global read of the prologue, issued before any weight load.  Lane `tid` takes the
// float4 chunks q = tid + m * kThreads of the flat [C][L] input; chunks q < nqn come from `src`.
// CHAIN (persistent tick kernel): activations written by other workgroups of the same launch are
// read device-coherently, and the parameters were requested by stage_params.
template <int LIN, int PRO, bool CHAIN>
__device__ __forceinline__ void stage_issue(const Args& a, int b, StageRegs<LIN, PRO>& s,
                                            Override ov) {
  using S = StageRegs<LIN, PRO>;
  const ConvInput& in = a.in;
  const int nq = a.ic * LIN / 4;
  const int nqn = in.split * LIN / 4;
  const int tid = threadIdx.x;
  const float* src = (ov.src != nullptr ? ov.src : in.src) + b * in.src_stride;
  const float* plain = in.plain != nullptr ? in.plain + b * in.plain_stride : src;
#pragma unroll
  for (int m = 0; m < S::QMAX; ++m) {
    const int q = tid + m * kThreads;
    s.x[m] = float4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (CHAIN) {
      if (q < nq) s.x[m] = ld4_dev(q < nqn ? src + 4 * q : plain + 4 * (q - nqn));
    } else if (q < nq) {
      const float* p = q < nqn ? src + 4 * q : plain + 4 * (q - nqn);
      s.x[m] = *reinterpret_cast<const float4*>(p);
    }
  }
  if constexpr (PRO != kProPlain) {
#pragma unroll
    for (int m = 0; m < S::QN; ++m) {
      const int q = tid + m * kThreads;
      if (q < nqn) {
        if constexpr (PRO == kProResid) {
          if constexpr (CHAIN)
            s.r[m] = ld4_dev(in.res + b * in.res_stride + 4 * q);
          else
            s.r[m] = *reinterpret_cast<const float4*>(in.res + b * in.res_stride + 4 * q);
        }
        if constexpr (!CHAIN) stage_chunk_params<LIN, PRO>(a, b, s, ov, m, q);
      }
    }
  }
}

template <int LIN>
__device__ __forceinline__ void write_chunk(float* xs, int nv, int q, float4 v) {
  const int e = 4 * q;
  if constexpr (LIN >= 4) {
    *reinterpret_cast<float4*>(xs + Swz<LIN>::at(e / LIN, e % LIN, nv)) = v;
  } else if constexpr (LIN == 2) {
    *reinterpret_cast<float2*>(xs + Swz<2>::at(e / 2, 0, nv)) = float2{v.x, v.y};
    *reinterpret_cast<float2*>(xs + Swz<2>::at(e / 2 + 1, 0, nv)) = float2{v.z, v.w};
  } else {
    xs[Swz<1>::at(e, 0, nv)] = v.x;
    xs[Swz<1>::at(e + 1, 0, nv)] = v.y;
    xs[Swz<1>::at(e + 2, 0, nv)] = v.z;
    xs[Swz<1>::at(e + 3, 0, nv)] = v.w;
  }
}

// Steps 3: statistics, transform, materialisation and LDS staging.  Called by every lane.
template <int LIN, int PRO, bool CHAIN>
__device__ __forceinline__ void stage_finish(const Args& a, int b, int wg, StageRegs<LIN, PRO>& s,
                                             float* xs, float* gmean, float* ginv, Override ov) {
  using S = StageRegs<LIN, PRO>;
  const ConvInput& in = a.in;
  const int nq = a.ic * LIN / 4;
  const int nv = a.ic / 4;
  const int tid = threadIdx.x;
  if constexpr (PRO != kProPlain) {
    const int nqn = in.split * LIN / 4;
    const int npg = in.split / in.groups * LIN / 4;  // chunks per group
    // fp64 partial sums, aliased over xs (written only after the next two barriers).
    double* ps = reinterpret_cast<double*>(xs);
    // Mean and 1/std of group g from its sums over n = 4 npg values.
    auto finish = [&](int g, double sum, double sq) {
      const double n = 4.0 * npg;
      const double mean = sum / n;
      const double var = fmax(0.0, sq / n - mean * mean);
      gmean[g] = static_cast<float>(mean);
      ginv[g] = static_cast<float>(1.0 / sqrt(var + 1e-5));
    };
    int gq[S::QN];  // group of chunk tid + m * kThreads
    // One fp64 partial pair per chunk; sixteen lanes per group, all kMaxGroups groups in one
    // pass, each lane summing every 16th partial of its group before a 16-lane row reduction
    // (DPP), and the row's first lane finishes the group.
    double* pq = ps + nqn;
#pragma unroll
    for (int m = 0; m < S::QN; ++m) {
      const int q = tid + m * kThreads;
      gq[m] = q / npg;
      if (q < nqn) {
        const double d0 = s.x[m].x, d1 = s.x[m].y, d2 = s.x[m].z, d3 = s.x[m].w;
        ps[q] = (d0 + d1) + (d2 + d3);
        pq[q] = (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
      }
    }
    lds_barrier();
    static_assert(kThreads / 16 >= kMaxGroups, "one 16-lane row per group");
    {
      const int g = tid >> 4, sub = tid & 15;
      double sum = 0.0, sq = 0.0;
      if (g < in.groups) {
        for (int i = sub; i < npg; i += 16) {
          sum += ps[g * npg + i];
          sq += pq[g * npg + i];
        }
      }
      sum = row_sum(sum);
      sq = row_sum(sq);
      if (sub == 0 && g < in.groups) finish(g, sum, sq);
    }
    lds_barrier();  // statistics visible; the partials are no longer read
    const float* ft =
        PRO == kProFilm
            ? (ov.film_time != nullptr ? ov.film_time : in.film_time) + in.film_off
            : nullptr;
    const float* fc = PRO == kProFilm ? in.film_cond + b * in.film_cond_stride + in.film_off : nullptr;
    // Workgroup wg materialises the chunks q with q % blocks == wg; r tracks q % blocks.
    int r = in.mat != nullptr ? tid % a.blocks : 0;
    const int rstep = in.mat != nullptr ? kThreads % a.blocks : 0;
#pragma unroll
    for (int m = 0; m < S::QN; ++m) {
      const int q = tid + m * kThreads;
      if (q < nqn) {
        const int g = gq[m];
        const float mean = gmean[g], inv = ginv[g];
        float v[4] = {s.x[m].x, s.x[m].y, s.x[m].z, s.x[m].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float gm, bt, sc = 0.0f, sh = 0.0f;
          if constexpr (LIN >= 4) {
            gm = s.gam[m];
            bt = s.bet[m];
            if constexpr (PRO == kProFilm) {
              sc = s.ts[m] + s.cs[m];
              sh = s.tb[m] + s.cb[m];
            }
          } else {
            const int c = (4 * q + i) / LIN;
            gm = in.gamma[c];
            bt = in.beta[c];
            if constexpr (PRO == kProFilm) {
              sc = ft[c] + fc[c];
              sh = ft[in.split + c] + fc[in.split + c];
            }
          }
          float val = mish_fast(fmaf(v[i] - mean, inv * gm, bt));
          if constexpr (PRO == kProFilm) val = fmaf(sc, val, sh);
          v[i] = val;
        }
        if constexpr (PRO == kProResid) {
          v[0] += s.r[m].x;
          v[1] += s.r[m].y;
          v[2] += s.r[m].z;
          v[3] += s.r[m].w;
        }
        s.x[m] = float4{v[0], v[1], v[2], v[3]};
        if (in.mat != nullptr && r == wg) {
          if constexpr (CHAIN)
            st4_dev(in.mat + b * in.mat_stride + 4 * q, s.x[m]);
          else
            *reinterpret_cast<float4*>(in.mat + b * in.mat_stride + 4 * q) = s.x[m];
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < S::QMAX; ++m) {
    const int q = tid + m * kThreads;
    if (q < nq) write_chunk<LIN>(xs, nv, q, s.x[m]);
  }
  lds_barrier();
}

// ---- Sliced prologue: the workgroup's slice of the input, one 16-byte chunk per lane ----
//
// Slice `sl` covers channels [c0, c0 + ics), c0 = sl * ics, wholly inside the normalised part
// [0, split) or wholly inside the plain part (the planner aligns slices with `split` and with the
// GroupNorm groups), so every statistic the slice needs is a sum over its own chunks.
template <int LIN, int PRO>
struct SliceRegs {
  static constexpr int NPC = LIN >= 4 ? 1 : 4 / LIN;  // channels per chunk
  float4 x;
  float4 r;
  float gam[NPC], bet[NPC];
  float ts[PRO == kProFilm ? NPC : 1], cs[PRO == kProFilm ? NPC : 1];
  float tb[PRO == kProFilm ? NPC : 1], cb[PRO == kProFilm ? NPC : 1];
};

// Sum of the partials p < n of a sliced producer's output at p (consecutive partials `stride`
// floats apart), added in order p = 0, 1, ...; every load is issued before the first add.
__device__ __forceinline__ float4 load_parts(const float* p, int n, std::int64_t stride) {
  float4 v[kMaxSlices];
#pragma unroll
  for (int j = 0; j < kMaxSlices; ++j)
    if (j < n) v[j] = *reinterpret_cast<const float4*>(p + j * stride);
  float4 s = v[0];
#pragma unroll
  for (int j = 1; j < kMaxSlices; ++j)
    if (j < n) s = float4{s.x + v[j].x, s.y + v[j].y, s.z + v[j].z, s.w + v[j].w};
  return s;
}

template <int LIN, int PRO>
__device__ __forceinline__ void slice_issue(const Args& a, int b, int sl, SliceRegs<LIN, PRO>& s) {
  using S = SliceRegs<LIN, PRO>;
  const ConvInput& in = a.in;
  const int c0 = sl * a.ics;
  const int nq = a.ics * LIN / 4;
  const int q = threadIdx.x;
  s.x = float4{0.0f, 0.0f, 0.0f, 0.0f};
  s.r = s.x;
  if (q >= nq) return;
  const std::int64_t e = static_cast<std::int64_t>(c0) * LIN + 4 * q;
  if (c0 >= in.split) {
    s.x = *reinterpret_cast<const float4*>(in.plain + b * in.plain_stride + e -
                                           static_cast<std::int64_t>(in.split) * LIN);
    return;
  }
  s.x = load_parts(in.src + b * in.src_stride + e, in.parts, in.part_stride);
  if constexpr (PRO == kProResid)
    s.r = load_parts(in.res + b * in.res_stride + e, in.res_parts, in.res_part_stride);
  if constexpr (PRO != kProPlain) {
    const float* ft = PRO == kProFilm ? in.film_time + in.film_off : nullptr;
    const float* fc = PRO == kProFilm ? in.film_cond + b * in.film_cond_stride + in.film_off : nullptr;
#pragma unroll
    for (int i = 0; i < S::NPC; ++i) {
      const int c = c0 + (4 * q) / LIN + i;
      s.gam[i] = in.gamma[c];
      s.bet[i] = in.beta[c];
      if constexpr (PRO == kProFilm) {
        s.ts[i] = ft[c];
        s.cs[i] = fc[c];
        s.tb[i] = ft[in.split + c];
        s.cb[i] = fc[in.split + c];
      }
    }
  }
}

// Statistics of the slice's groups, transform, materialisation (workgroup wt of `a.blocks` of
// the slice writes chunks q with q % blocks == wt) and LDS staging.  `wsum` holds
// 2 * kMaxGroups doubles (sums, then sums of squares).
template <int LIN, int PRO>
__device__ __forceinline__ void slice_finish(const Args& a, int b, int sl, int wt,
                                             SliceRegs<LIN, PRO>& s, float* xs, double* wsum) {
  using S = SliceRegs<LIN, PRO>;
  const ConvInput& in = a.in;
  const int c0 = sl * a.ics;
  const int nq = a.ics * LIN / 4;
  const int nv = a.ics / 4;
  const int q = threadIdx.x;
  const int lane = q & (kWave - 1);
  if (PRO != kProPlain && c0 < in.split) {
    const int npg = in.split / in.groups * LIN / 4;  // chunks per group
    double sum = 0.0, sq = 0.0;
    if (q < nq) {
      const double d0 = s.x.x, d1 = s.x.y, d2 = s.x.z, d3 = s.x.w;
      sum = (d0 + d1) + (d2 + d3);
      sq = (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
    }
    double gsum = 0.0, gsq = 0.0;
    if (npg % kWave == 0) {
      // Each wavefront lies in one group: wavefront sums, then the group's wavefronts in order.
      sum = wave_sum(sum);
      sq = wave_sum(sq);
      if (lane == 0) {
        wsum[q / kWave] = sum;
        wsum[kMaxGroups + q / kWave] = sq;
      }
      lds_barrier();
      if (q < nq) {
        const int w0 = q / npg * (npg / kWave);
        for (int i = 0; i < npg / kWave; ++i) {
          gsum += wsum[w0 + i];
          gsq += wsum[kMaxGroups + w0 + i];
        }
      }
    } else {
      // Small groups: per-chunk partials in LDS (aliased over xs, written again only after the
      // next barrier), then one 16-lane row per group.
      double* ps = reinterpret_cast<double*>(xs);
      double* pq = ps + nq;
      if (q < nq) {
        ps[q] = sum;
        pq[q] = sq;
      }
      lds_barrier();
      const int g = q >> 4, sub = q & 15;
      const int ng = nq / npg;
      double rs = 0.0, rq = 0.0;
      if (g < ng)
        for (int i = sub; i < npg; i += 16) {
          rs += ps[g * npg + i];
          rq += pq[g * npg + i];
        }
      rs = row_sum(rs);
      rq = row_sum(rq);
      if (sub == 0 && g < ng) {
        wsum[g] = rs;
        wsum[kMaxGroups + g] = rq;
      }
      lds_barrier();
      if (q < nq) {
        gsum = wsum[q / npg];
        gsq = wsum[kMaxGroups + q / npg];
      }
    }
    if (q < nq) {
      const double n = 4.0 * npg;
      const double mean = gsum / n;
      const double var = fmax(0.0, gsq / n - mean * mean);
      const float fmean = static_cast<float>(mean);
      const float inv = static_cast<float>(1.0 / sqrt(var + 1e-5));
      float v[4] = {s.x.x, s.x.y, s.x.z, s.x.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = LIN >= 4 ? 0 : i / LIN;  // channel of element i within the chunk
        float val = mish_fast(fmaf(v[i] - fmean, inv * s.gam[k], s.bet[k]));
        if constexpr (PRO == kProFilm) val = fmaf(s.ts[k] + s.cs[k], val, s.tb[k] + s.cb[k]);
        v[i] = val;
      }
      if constexpr (PRO == kProResid) {
        v[0] += s.r.x;
        v[1] += s.r.y;
        v[2] += s.r.z;
        v[3] += s.r.w;
      }
      s.x = float4{v[0], v[1], v[2], v[3]};
      if (in.mat != nullptr && q % a.blocks == wt)
        *reinterpret_cast<float4*>(in.mat + b * in.mat_stride + static_cast<std::int64_t>(c0) * LIN +
                                   4 * q) = s.x;
    }
  }
  if (q < nq) write_chunk<LIN>(xs, nv, q, s.x);
  lds_barrier();
}

// The wait of a stand-alone launch: the stream order has already made the input visible.
struct NoWait {
  __device__ bool operator()() const { return true; }
};

// One fused convolution by workgroup `wg` (of a.blocks) for sample `b`.  In CHAIN mode (a step of
// the persistent tick kernel) it starts with `wait()` (a workgroup-uniform call that returns once
// the producers of the input have finished, false if the launch is being abandoned), and the
// input and all outputs use device-coherent accesses.
// Weight chunks per lane the registers allow (as chunk_budget, without the staging bound).
__host__ __device__ constexpr int reg_chunks(int k, int lin, bool res) {
  const int regs = lin >= 16 ? kWeightRegs - 64 : (lin >= 8 ? kWeightRegs - 32 : kWeightRegs);
  const int n = regs / ((k + (res ? 1 : 0)) * 4);
  return n < 8 ? n : 8;
}

// Lanes per row of the sliced kernel: 16, 32 or 64 (an instance parameter, chosen per
// convolution by the planner), at least the reduced values per row.
__host__ __device__ constexpr bool slice_tpr_ok(int mode, int lin, bool res, int tpr) {
  return (res ? 2 : 1) * lout_of(mode, lin) <= tpr;
}

// SL (sliced kernel, stand-alone launches only): workgroup wg takes input-channel slice
// wg % a.slices and row tiles wg / a.slices, + a.blocks, ...; rows are STPR lanes wide and
// reduced within their lane segment.
template <int MODE, int K, int LIN, int VEC, int PRO, bool RES, bool BF16, int NC,
          bool CHAIN = false, typename Wait = NoWait, bool SL = false, int STPR = 64>
__device__ __forceinline__ bool conv_body(const Args& a, int wg, int b, float* xs, float* gmean,
                                          float* ginv, float* red, const Wait& wait = Wait{},
                                          Override ov = Override{}) {
  constexpr int LOUT = lout_of(MODE, LIN);
  constexpr int TAPS = K + (RES ? 1 : 0);
  constexpr int NCH = NC;  // chunk slots per lane: the plan's chunk count, or the budget
  constexpr int V = RES ? 2 * LOUT : LOUT;
  static_assert(!SL || (VEC == 4 && !CHAIN && V <= STPR && STPR <= kWave),
                "sliced: 16-byte chunks, stand-alone launches, one reduced value per lane");
  const int tid = threadIdx.x;
  const int tpr = SL ? STPR : a.tpr;
  const int rpt = kThreads / tpr;  // rows per tile
  const int gid = tid / tpr;
  const int lg = tid - gid * tpr;
  const int sl = SL ? wg % a.slices : 0;   // input-channel slice
  const int c0 = SL ? sl * a.ics : 0;      // its first channel
  const int nv = SL ? a.ics / 4 : a.ic / VEC;
  const int lane = tid & (kWave - 1);
  if constexpr (SL) wg /= a.slices;        // workgroup index within the slice

  const __amdgpu_buffer_rsrc_t wr = buffer_of(a.w, a.wbytes);
  const __amdgpu_buffer_rsrc_t rr = buffer_of(RES ? a.rw : a.w, RES ? a.rwbytes : a.wbytes);
  std::conditional_t<SL, SliceRegs<LIN, PRO>, StageRegs<LIN, PRO>> st;
  if constexpr (CHAIN) {
    // The input is produced by other workgroups of this launch: wait for them first (a wait
    // issued behind weight loads would only complete once those arrive).  The parameters do not
    // depend on them and are requested before.
    if constexpr (VEC == 4) stage_params<LIN, PRO>(a, b, st, ov);
    if (!wait()) return false;
  }
  if constexpr (SL) {
    slice_issue<LIN, PRO>(a, b, sl, st);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
  } else if constexpr (VEC == 4) {
    stage_issue<LIN, PRO, CHAIN>(a, b, st, ov);
    // Every wavefront's prologue reads are issued before any wavefront's weight loads: a CU's
    // vector memory path returns data in order, so an input read queued behind weight misses
    // would only arrive with them.
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    // In the tick kernel every CU reaches this point at the same moment, so the CUs' first
    // weight requests (tens of MB) would reach the memory channels together with the input
    // reads and delay them by their whole transfer: the input is waited for first.
    if constexpr (CHAIN) wait_vmem();
  }
  __builtin_amdgcn_sched_barrier(0);
  // The first tile's weights: EARLY chunks go out before the prologue (enough to keep HBM busy
  // while it runs, without stalling the wavefront on a long run of issues), the rest after it.
  constexpr int EARLY = VEC == 4 ? early_chunks(TAPS) : NCH;
  int tile = wg;
  float w[NCH][TAPS][VEC];
  const int row0 = tile * rpt + gid;
#pragma unroll
  for (int j = 0; j < (EARLY < NCH ? EARLY : NCH); ++j) {
    const int cv = lg + j * tpr;
    load_chunk<K, VEC, RES, BF16>(a, wr, rr, row0, cv, j < a.nch && cv < nv && row0 < a.oc, w[j],
                                  c0);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (SL)
    slice_finish<LIN, PRO>(a, b, sl, wg, st, xs, reinterpret_cast<double*>(red));
  else if constexpr (VEC == 4)
    stage_finish<LIN, PRO, CHAIN>(a, b, wg, st, xs, gmean, ginv, ov);
#pragma unroll
  for (int j = EARLY; j < NCH; ++j) {
    const int cv = lg + j * tpr;
    load_chunk<K, VEC, RES, BF16>(a, wr, rr, row0, cv, j < a.nch && cv < nv && row0 < a.oc, w[j],
                                  c0);
  }

  const int waves = SL ? 1 : a.tpr / kWave;
  const int wig = lg / kWave;
  const float* xsrc = (ov.src != nullptr ? ov.src : a.in.src) + b * a.in.src_stride;
  int parity = 0;
  // One row tile; `refill` (true for every tile but the workgroup's last) streams the next tile's
  // weights into each chunk's registers once its products are accumulated.  The last tile is a
  // separate instance, so it issues no refill loads at all.
  auto do_tile = [&](int tile, auto refill) {
    const int row = tile * rpt + gid;
    const int nrow = (tile + a.blocks) * rpt + gid;
    // The row's biases (added by slice 0 only), read before the products so that their latency
    // hides behind them instead of delaying the output stores.
    const bool brow = row < a.oc && (!SL || sl == 0);
    const float bv = brow ? a.bias[row] : 0.0f;
    float rbv = 0.0f;
    if constexpr (RES) rbv = brow ? a.rbias[row] : 0.0f;
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int cv = lg + j * tpr;
      const bool on = j < a.nch && cv < nv;
      if (on) {
        float xr[VEC][LIN];
        if constexpr (VEC == 4) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            constexpr int P = Swz<LIN>::P;
#pragma unroll
            for (int t = 0; t < LIN; t += P) {
              const float* p = xs + Swz<LIN>::at(4 * cv + v, t, nv);
              if constexpr (P == 4) {
                const float4 f = *reinterpret_cast<const float4*>(p);
                xr[v][t] = f.x;
                xr[v][t + 1] = f.y;
                xr[v][t + 2] = f.z;
                xr[v][t + 3] = f.w;
              } else if constexpr (P == 2) {
                const float2 f = *reinterpret_cast<const float2*>(p);
                xr[v][t] = f.x;
                xr[v][t + 1] = f.y;
              } else {
                xr[v][t] = *p;
              }
            }
          }
        } else {
          // Narrow inputs (channel count not a multiple of 4, raw tensors only) are read directly.
          const float* p = cv < a.in.split
                               ? xsrc + static_cast<std::int64_t>(cv) * LIN
                               : a.in.plain + b * a.in.plain_stride +
                                     static_cast<std::int64_t>(cv - a.in.split) * LIN;
#pragma unroll
          for (int t = 0; t < LIN; ++t) xr[0][t] = CHAIN ? ld_dev(p + t) : p[t];
        }
#pragma unroll
        for (int t = 0; t < LOUT; ++t)
#pragma unroll
          for (int k = 0; k < K; ++k) {
            const int jj = src_index<MODE, K, LIN>(t, k);
            if (jj >= 0) {
#pragma unroll
              for (int v = 0; v < VEC; ++v) acc[t] = fmaf(w[j][k][v], xr[v][jj], acc[t]);
            }
          }
        if constexpr (RES) {
#pragma unroll
          for (int t = 0; t < LOUT; ++t)
#pragma unroll
            for (int v = 0; v < VEC; ++v)
              acc[LOUT + t] = fmaf(w[j][K][v], xr[v][t], acc[LOUT + t]);
        }
      }
      // Refill this chunk's registers with the next tile's weights.
      if constexpr (decltype(refill)::value)
        load_chunk<K, VEC, RES, BF16>(a, wr, rr, nrow, cv, j < a.nch && cv < nv && nrow < a.oc,
                                      w[j], c0);
    }

    auto put = [&](float* p, float v) {
      if constexpr (CHAIN) st_dev(p, v);
      else *p = v;
    };
    if constexpr (SL) {
      // Rows of STPR lanes: reduce within the segment; slice sl writes its partial sum.
      rs_step<V, STPR / 2>(acc, lane);
      const int off = rs_offset_seg<V, STPR>(lane);
      if (rs_writer_seg<V, STPR>(lane) && row < a.oc) {
        if (!RES || off < LOUT)
          put(a.y + b * a.ys + sl * a.ypart + static_cast<std::int64_t>(row) * LOUT + off,
              sl == 0 ? acc[0] + bv : acc[0]);
        else
          put(a.yr + b * a.yrs + sl * a.yrpart + static_cast<std::int64_t>(row) * LOUT + off - LOUT,
              sl == 0 ? acc[0] + rbv : acc[0]);
      }
      return;
    }
    rs_step<V, 32>(acc, lane);
    const int off = rs_offset<V>(lane);
    if (waves == 1) {
      if (rs_writer<V>(lane) && row < a.oc) {
        if (!RES || off < LOUT)
          put(a.y + b * a.ys + static_cast<std::int64_t>(row) * LOUT + off, acc[0] + bv);
        else
          put(a.yr + b * a.yrs + static_cast<std::int64_t>(row) * LOUT + off - LOUT,
              acc[0] + rbv);
      }
      return;
    }
    // Several wavefronts per row: combine through LDS.  red holds two alternating buffers of
    // [row group][wavefront in group][V], so one barrier per tile suffices.
    float* gred = red + parity * (kThreads / kWave) * V + gid * waves * V;
    parity ^= 1;
    if (rs_writer<V>(lane)) gred[wig * V + off] = acc[0];
    lds_barrier();
    if (lg < V && row < a.oc) {
      float sum = 0.0f;
      for (int wv = 0; wv < waves; ++wv) sum += gred[wv * V + lg];
      if (!RES || lg < LOUT)
        put(a.y + b * a.ys + static_cast<std::int64_t>(row) * LOUT + lg, sum + bv);
      else
        put(a.yr + b * a.yrs + static_cast<std::int64_t>(row) * LOUT + lg - LOUT,
            sum + rbv);
    }
  };
  for (; tile + a.blocks < a.tiles; tile += a.blocks) do_tile(tile, std::true_type{});
  do_tile(tile, std::false_type{});
  return true;
}

template <int MODE, int K, int LIN, int VEC, int PRO, bool RES, int NC>
__global__ __launch_bounds__(kThreads) void conv_kernel(Args a) {
  constexpr int V = RES ? 2 * lout_of(MODE, LIN) : lout_of(MODE, LIN);
  static_assert(V <= kWave, "one reduced value per lane");
  extern __shared__ float4 xs4[];
  __shared__ float gmean[kMaxGroups], ginv[kMaxGroups];
  __shared__ float red[2 * (kThreads / kWave) * V];
  float* xs = reinterpret_cast<float*>(xs4);
  const int wg = blockIdx.x, b = blockIdx.y;
  if constexpr (VEC == 4) {
    if (a.bf16)
      conv_body<MODE, K, LIN, VEC, PRO, RES, true, NC>(a, wg, b, xs, gmean, ginv, red);
    else
      conv_body<MODE, K, LIN, VEC, PRO, RES, false, NC>(a, wg, b, xs, gmean, ginv, red);
  } else {
    conv_body<MODE, K, LIN, VEC, PRO, RES, false, NC>(a, wg, b, xs, gmean, ginv, red);
  }
}

// The sliced kernel: rows of TPR lanes over the workgroup's input-channel slice.
template <int MODE, int K, int LIN, int PRO, bool RES, int NC, int TPR>
__global__ __launch_bounds__(kThreads) void conv_slice_kernel(Args a) {
  extern __shared__ float4 xs4[];
  __shared__ double wsum[2 * kMaxGroups];
  float* xs = reinterpret_cast<float*>(xs4);
  float* red = reinterpret_cast<float*>(wsum);
  const int wg = blockIdx.x, b = blockIdx.y;
  if (a.bf16)
    conv_body<MODE, K, LIN, 4, PRO, RES, true, NC, false, NoWait, true, TPR>(a, wg, b, xs, nullptr,
                                                                             nullptr, red);
  else
    conv_body<MODE, K, LIN, 4, PRO, RES, false, NC, false, NoWait, true, TPR>(a, wg, b, xs,
                                                                              nullptr, nullptr, red);
}

// Chunk slots per lane of the sliced kernel at TPR lanes per row: bounded by the weight
// registers and by a slice of kSliceFloats staged floats.
__host__ __device__ constexpr int slice_budget(int k, int lin, bool res, int tpr) {
  const int by_regs = reg_chunks(k, lin, res);
  const int by_size = (kSliceFloats / (lin * 4) + tpr - 1) / tpr;
  return by_regs < by_size ? by_regs : by_size;
}

inline std::size_t stage_bytes(int ic, int lin, int vec) {
  if (vec != 4) return 0;
  const int planes = 4 * (lin >= 4 ? lin / 4 : 1);
  return (static_cast<std::size_t>(ic) * lin + planes * kSwzPad) * sizeof(float);
}
constexpr std::size_t kMaxStageBytes = (kMaxStageFloats + 16 * kSwzPad) * sizeof(float);

template <int MODE, int K, int LIN, int VEC, int PRO, bool RES, int NC, bool SL = false,
          int TPR = 64>
hipError_t launch_nc(const Args& a, int batch, hipStream_t s) {
  if constexpr (SL) {
    hipLaunchKernelGGL((conv_slice_kernel<MODE, K, LIN, PRO, RES, NC, TPR>),
                       dim3(a.blocks * a.slices, batch), dim3(kThreads),
                       stage_bytes(a.ics, LIN, 4), s, a);
    return hipGetLastError();
  }
  const std::size_t smem = stage_bytes(a.ic, LIN, VEC);
  auto fn = conv_kernel<MODE, K, LIN, VEC, PRO, RES, NC>;
  if (smem > 48 * 1024) {  // opt in to more than 48 KB of dynamic LDS (up to 160 KB per CU)
    static bool raised = false;
    if (!raised) {
      const hipError_t st = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                                static_cast<int>(kMaxStageBytes));
      if (st != hipSuccess) return st;
      raised = true;
    }
  }
  hipLaunchKernelGGL(fn, dim3(a.blocks, batch), dim3(kThreads), smem, s, a);
  return hipGetLastError();
}

// Chunk slots per lane: the plan's count when it is 1, 2 or 4 (the common plans), otherwise the
// register budget.  Slots beyond the plan's count still issue their (out-of-range, traffic-free)
// loads, since the loads are branch-free, so exact counts save memory-pipeline issue slots.
template <int MODE, int K, int LIN, int VEC, int PRO, bool RES, bool SL = false, int TPR = 64>
hipError_t launch(const Args& a, int batch, hipStream_t s) {
  if constexpr (SL && !slice_tpr_ok(MODE, LIN, RES, TPR)) {
    return hipErrorInvalidValue;
  } else {
    constexpr int B = SL ? slice_budget(K, LIN, RES, TPR) : chunk_budget(K, LIN, RES, VEC);
    if (a.nch == 1) return launch_nc<MODE, K, LIN, VEC, PRO, RES, 1, SL, TPR>(a, batch, s);
    if constexpr (B > 2)
      if (a.nch == 2) return launch_nc<MODE, K, LIN, VEC, PRO, RES, 2, SL, TPR>(a, batch, s);
    if constexpr (B > 4)
      if (a.nch == 4) return launch_nc<MODE, K, LIN, VEC, PRO, RES, 4, SL, TPR>(a, batch, s);
    return launch_nc<MODE, K, LIN, VEC, PRO, RES, B, SL, TPR>(a, batch, s);
  }
}

template <int MODE, int K, int LIN, int VEC, bool SL = false, int TPR = 64>
hipError_t by_prologue(int pro, bool res, const Args& a, int batch, hipStream_t s) {
  if constexpr (VEC == 1) {
    if (pro == kProPlain && MODE == kConvSame)
      return res ? launch<MODE, K, LIN, 1, kProPlain, true>(a, batch, s)
                 : launch<MODE, K, LIN, 1, kProPlain, false>(a, batch, s);
  } else if constexpr (MODE == kConvSame) {
    switch (pro) {
      case kProPlain:
        return res ? launch<MODE, K, LIN, 4, kProPlain, true, SL, TPR>(a, batch, s)
                   : launch<MODE, K, LIN, 4, kProPlain, false, SL, TPR>(a, batch, s);
      case kProFilm:
        if (!res) return launch<MODE, K, LIN, 4, kProFilm, false, SL, TPR>(a, batch, s);
        break;
      case kProResid:
        return res ? launch<MODE, K, LIN, 4, kProResid, true, SL, TPR>(a, batch, s)
                   : launch<MODE, K, LIN, 4, kProResid, false, SL, TPR>(a, batch, s);
      default:
        break;
    }
  } else {
    if (!res && pro == kProPlain)
      return launch<MODE, K, LIN, 4, kProPlain, false, SL, TPR>(a, batch, s);
    if (!res && pro == kProResid)
      return launch<MODE, K, LIN, 4, kProResid, false, SL, TPR>(a, batch, s);
  }
  return hipErrorInvalidValue;
}

template <int MODE, int K, int VEC>
hipError_t by_lin(int lin, int pro, bool res, const Args& a, int batch, hipStream_t s) {
  switch (lin) {
    case 1:
      if constexpr (MODE != kConvDown) return by_prologue<MODE, K, 1, VEC>(pro, res, a, batch, s);
      break;
    case 2: return by_prologue<MODE, K, 2, VEC>(pro, res, a, batch, s);
    case 4: return by_prologue<MODE, K, 4, VEC>(pro, res, a, batch, s);
    case 8: return by_prologue<MODE, K, 8, VEC>(pro, res, a, batch, s);
    case 16: return by_prologue<MODE, K, 16, VEC>(pro, res, a, batch, s);
    default: break;
  }
  return hipErrorInvalidValue;
}

// Sliced instances at TPR lanes per row for the lengths LINS (a.tpr selected the TPR).
template <int MODE, int K, int TPR, int... LINS>
hipError_t slice_lins(int lin, int pro, bool res, const Args& a, int batch, hipStream_t s) {
  hipError_t st = hipErrorInvalidValue;
  (void)((lin == LINS ? (st = by_prologue<MODE, K, LINS, 4, true, TPR>(pro, res, a, batch, s),
                         true)
                      : false) ||
         ...);
  return st;
}

// Host: the plan and arguments conv_fused launches with (false when it has no kernel for them);
// `vec` and `pro` receive the instance's vector width and prologue kind.
bool fused_args(const ConvOp& op, const ConvOp* res1x1, const ConvInput& in, View y, View yr,
                int batch, Args& a, int& vec, int& pro);

// Chunk slots of the kernel instance a plan with `nch` chunks per lane runs on (launch()).
constexpr int instance_nc(int k, int lin, bool res, int vec, int nch) {
  const int b = chunk_budget(k, lin, res, vec);
  return nch == 1 ? 1 : (nch == 2 && b > 2 ? 2 : (nch == 4 && b > 4 ? 4 : b));
}

// Launchers, one translation unit each (they instantiate the kernel for every length/prologue).
hipError_t launch_same5(int lin, int vec, int pro, bool res, const Args& a, int batch,
                        hipStream_t s);
hipError_t launch_same3(int lin, int vec, int pro, bool res, const Args& a, int batch,
                        hipStream_t s);
hipError_t launch_resample(int mode, int lin, int pro, const Args& a, int batch, hipStream_t s);
// The sliced kernel's instances (conv_slice*.hip): true when one exists for the shape; a.tpr
// selects the lanes per row (16, 32 or 64).
bool slice_instance(int mode, int k, int lin, bool res);
hipError_t launch_slice(int mode, int k, int lin, int pro, bool res, const Args& a, int batch,
                        hipStream_t s);

}  // namespace fe::hip::conv
