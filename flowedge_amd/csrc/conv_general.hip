// General-shape convolution and GroupNorm prologue on gfx950.  The specialised kernels cover the
// common U-Net shapes (kernel 3 / 5, power-of-two lengths up to 16, widths in multiples of 4 or
// 16); these cover everything else the checkpoint format admits: any odd kernel size, any horizon
// divisible by the down factor, any width divisible by the group count
// (diffusion.cc:391-427 validation; conv semantics diffusion_ops.cc:82-268, GroupNorm
// diffusion_ops.cc:270-350, FiLM diffusion_ops.cc:352-377).
//
// conv_general is an implicit GEMM on the FP32 vector ALUs.  A workgroup of 256 lanes owns a tile
// of 64 output channels x NT output columns (column = sample * lout + position) and walks the
// reduction one tap x 16 input channels at a time: the weight slice [64][16] and the gathered
// input slice [16][NT] go through LDS, and each lane accumulates 4 channels x NT/16 columns.
// When the tiles alone leave CUs idle the reduction is split over workgroups, whose partial tiles
// a second kernel sums in a fixed order (results do not depend on the launch shape's timing).
//
// norm_act_general is the prologue with one workgroup per (sample, group): fp64 statistics over
// the group, then GroupNorm, Mish, FiLM and the residual in one pass.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "device_common.h"
#include "kernels.h"

namespace fe::hip {
namespace {

using namespace dev;

constexpr int kGenThreads = 256;
constexpr int kGenMT = 64;  // output channels per tile
constexpr int kGenKC = 16;  // input channels per reduction step

struct GenArgs {
  const void* w;  // [oc][k][ic]
  int bf16;
  const float* bias;
  float* y;
  std::int64_t ys;
  const float* src;
  std::int64_t src_stride;
  int split;
  const float* plain;
  std::int64_t plain_stride;
  int mode, k, ic, oc, lin, lout, batch;
  int mtiles, ntiles;
  int steps;        // reduction steps: ceil(ic / kGenKC) * k
  int ksplit, per;  // workgroups per tile, steps per workgroup
  float* part;      // ksplit > 1: partial tiles [ksplit][mtiles * ntiles][kGenMT * NT]
};

// Input position read by output t through tap k, or -1 in the padding.
__device__ __forceinline__ int gen_src(int mode, int K, int lin, int t, int k) {
  int j;
  if (mode == kConvSame) {
    j = t + k - K / 2;
  } else if (mode == kConvDown) {
    j = 2 * t + k - 1;
  } else {
    const int num = t + 1 - k;  // ConvTranspose: output t = 2 * j + k - 1
    if (num < 0 || (num & 1)) return -1;
    j = num >> 1;
  }
  return (j >= 0 && j < lin) ? j : -1;
}

template <int NT>
__global__ __launch_bounds__(kGenThreads) void conv_general_kernel(GenArgs a) {
  constexpr int CPT = NT / 16;                 // columns per lane
  constexpr int XR = kGenKC * NT / kGenThreads;  // staged input values per lane
  constexpr int WR = kGenKC * kGenMT / kGenThreads;
  __shared__ float ws[kGenKC][kGenMT + 1];
  __shared__ float xs[kGenKC][NT];
  const int tiles = a.mtiles * a.ntiles;
  const int tile = blockIdx.x % tiles;
  const int kp = blockIdx.x / tiles;
  const int mt = tile % a.mtiles, nt = tile / a.mtiles;
  const int o0 = mt * kGenMT, n0 = nt * NT;
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;  // compute: columns tx + 16 j, channels ty + 16 i

  // The one column this lane stages (NT divides the workgroup size).
  const int scol = tid % NT;
  const int srow = tid / NT;  // first staged channel row; rows srow + (256 / NT) r
  const int sn = n0 + scol;
  const int sb = sn / a.lout, st = sn % a.lout;
  const bool scol_ok = sb < a.batch;

  float acc[4][CPT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < CPT; ++j) acc[i][j] = 0.0f;

  const int s_begin = kp * a.per;
  const int s_end = min(a.steps, s_begin + a.per);
  const float* wf = static_cast<const float*>(a.w);
  const unsigned short* wh = static_cast<const unsigned short*>(a.w);
  for (int s = s_begin; s < s_end; ++s) {
    const int c0 = (s / a.k) * kGenKC, kk = s % a.k;
    float wv[WR], xv[XR];
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      const int idx = tid + r * kGenThreads;
      const int o = o0 + idx / kGenKC, c = c0 + idx % kGenKC;
      float v = 0.0f;
      if (o < a.oc && c < a.ic) {
        const std::int64_t off = (static_cast<std::int64_t>(o) * a.k + kk) * a.ic + c;
        v = a.bf16 ? bf16_to_f32(wh[off]) : wf[off];
      }
      wv[r] = v;
    }
    const int j = scol_ok ? gen_src(a.mode, a.k, a.lin, st, kk) : -1;
#pragma unroll
    for (int r = 0; r < XR; ++r) {
      const int c = c0 + srow + r * (kGenThreads / NT);
      float v = 0.0f;
      if (j >= 0 && c < a.ic) {
        v = c < a.split ? a.src[sb * a.src_stride + static_cast<std::int64_t>(c) * a.lin + j]
                        : a.plain[sb * a.plain_stride +
                                  static_cast<std::int64_t>(c - a.split) * a.lin + j];
      }
      xv[r] = v;
    }
    __syncthreads();  // the previous step's reads of ws / xs are done
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      const int idx = tid + r * kGenThreads;
      ws[idx % kGenKC][idx / kGenKC] = wv[r];
    }
#pragma unroll
    for (int r = 0; r < XR; ++r) xs[srow + r * (kGenThreads / NT)][scol] = xv[r];
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kGenKC; ++c) {
      float w4[4], x4[CPT];
#pragma unroll
      for (int i = 0; i < 4; ++i) w4[i] = ws[c][ty + 16 * i];
#pragma unroll
      for (int jj = 0; jj < CPT; ++jj) x4[jj] = xs[c][tx + 16 * jj];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < CPT; ++jj) acc[i][jj] = fmaf(w4[i], x4[jj], acc[i][jj]);
    }
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ol = ty + 16 * i;
#pragma unroll
    for (int jj = 0; jj < CPT; ++jj) {
      const int cl = tx + 16 * jj;
      if (a.ksplit > 1) {
        a.part[(static_cast<std::int64_t>(kp) * tiles + tile) * (kGenMT * NT) + ol * NT + cl] =
            acc[i][jj];
      } else {
        const int o = o0 + ol, n = n0 + cl;
        const int b = n / a.lout, t = n % a.lout;
        if (o < a.oc && b < a.batch)
          a.y[b * a.ys + static_cast<std::int64_t>(o) * a.lout + t] = acc[i][jj] + a.bias[o];
      }
    }
  }
}

// y = bias + the ksplit partial tiles, summed in split order.
template <int NT>
__global__ __launch_bounds__(kGenThreads) void conv_general_reduce_kernel(GenArgs a) {
  const int tiles = a.mtiles * a.ntiles;
  const std::int64_t e = static_cast<std::int64_t>(blockIdx.x) * kGenThreads + threadIdx.x;
  if (e >= static_cast<std::int64_t>(tiles) * kGenMT * NT) return;
  const int tile = static_cast<int>(e / (kGenMT * NT));
  const int within = static_cast<int>(e % (kGenMT * NT));
  const int mt = tile % a.mtiles, nt = tile / a.mtiles;
  const int o = mt * kGenMT + within / NT, n = nt * NT + within % NT;
  const int b = n / a.lout, t = n % a.lout;
  if (o >= a.oc || b >= a.batch) return;
  float s = 0.0f;
  for (int p = 0; p < a.ksplit; ++p)
    s += a.part[(static_cast<std::int64_t>(p) * tiles + tile) * (kGenMT * NT) + within];
  a.y[b * a.ys + static_cast<std::int64_t>(o) * a.lout + t] = s + a.bias[o];
}

template <int NT>
hipError_t launch_general(GenArgs a, float* workspace, std::size_t workspace_floats,
                          hipStream_t stream) {
  a.ntiles = static_cast<int>((static_cast<std::int64_t>(a.batch) * a.lout + NT - 1) / NT);
  const int tiles = a.mtiles * a.ntiles;
  a.ksplit = 1;
  a.per = a.steps;
  if (tiles < 256 && workspace != nullptr && a.steps > 1) {
    int ks = (512 + tiles - 1) / tiles;
    if (ks > a.steps) ks = a.steps;
    const int per = (a.steps + ks - 1) / ks;
    ks = (a.steps + per - 1) / per;
    const std::size_t need = static_cast<std::size_t>(ks) * tiles * kGenMT * NT;
    if (ks > 1 && need <= workspace_floats) {
      a.ksplit = ks;
      a.per = per;
      a.part = workspace;
    }
  }
  hipLaunchKernelGGL(conv_general_kernel<NT>, dim3(static_cast<unsigned>(tiles * a.ksplit)),
                     dim3(kGenThreads), 0, stream, a);
  if (a.ksplit == 1) return hipGetLastError();
  const std::int64_t elems = static_cast<std::int64_t>(tiles) * kGenMT * NT;
  hipLaunchKernelGGL(conv_general_reduce_kernel<NT>,
                     dim3(static_cast<unsigned>((elems + kGenThreads - 1) / kGenThreads)),
                     dim3(kGenThreads), 0, stream, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Prologue: dst = mish(GN(src)) [* scale + shift] [+ res], one workgroup per (sample, group).
// ---------------------------------------------------------------------------------------------
constexpr int kNgThreads = 256;

// Sum of the `parts` partials of one element (`stride` floats apart), added in order; every
// load is issued before the first add.
__device__ __forceinline__ float part_sum(const float* p, int parts, std::int64_t stride) {
  float v[kMaxSlices];
#pragma unroll
  for (int j = 0; j < kMaxSlices; ++j) v[j] = j < parts ? p[j * stride] : 0.0f;
  float s = v[0];
#pragma unroll
  for (int j = 1; j < kMaxSlices; ++j)
    if (j < parts) s += v[j];
  return s;
}

constexpr int kNgRegs = 8;  // region values kept in registers between the two passes
constexpr int kNaThreads = 512;  // lanes of the per-(sample, group) GroupNorm pass

__global__ __launch_bounds__(kNaThreads) void norm_act_general_kernel(ConvInput in, int lin,
                                                                      float* dst,
                                                                      std::int64_t dst_stride) {
  __shared__ double rs[kNaThreads / kWave], rq[kNaThreads / kWave];
  const int b = blockIdx.x / in.groups, g = blockIdx.x % in.groups;
  const int cpg = in.split / in.groups;
  const int n = cpg * lin;
  const std::int64_t base = static_cast<std::int64_t>(g) * n;
  const float* src = in.src + b * in.src_stride + base;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  // Sources made of partial sums (a split K loop's outputs) are added while read; the first
  // kNgRegs values per lane stay in registers for the second pass.
  float v[kNgRegs];
  double s = 0.0, q = 0.0;
#pragma unroll
  for (int r = 0; r < kNgRegs; ++r) {
    const int i = tid + r * kNaThreads;
    v[r] = i < n ? part_sum(src + i, in.parts, in.part_stride) : 0.0f;
    const double d = static_cast<double>(v[r]);
    s += d;
    q += d * d;
  }
  for (int i = tid + kNgRegs * kNaThreads; i < n; i += kNaThreads) {
    const double d = static_cast<double>(part_sum(src + i, in.parts, in.part_stride));
    s += d;
    q += d * d;
  }
  s = wave_sum(s);
  q = wave_sum(q);
  if (lane == 0) {
    rs[wave] = s;
    rq[wave] = q;
  }
  __syncthreads();
  s = 0.0;
  q = 0.0;
  for (int w = 0; w < kNaThreads / kWave; ++w) {
    s += rs[w];
    q += rq[w];
  }
  const double cnt = static_cast<double>(n);
  const double mean = s / cnt;
  const double var = fmax(0.0, q / cnt - mean * mean);
  const float meanf = static_cast<float>(mean);
  const float inv = static_cast<float>(1.0 / sqrt(var + 1e-5));
  const float* ft = in.film_time != nullptr ? in.film_time + in.film_off : nullptr;
  const float* fc =
      in.film_time != nullptr ? in.film_cond + b * in.film_cond_stride + in.film_off : nullptr;
  float* out = dst + b * dst_stride + base;
  const float* res = in.res != nullptr ? in.res + b * in.res_stride + base : nullptr;
  auto put = [&](int i, float x) {
    const int c = g * cpg + i / lin;
    float val = mish_fast(fmaf(x - meanf, inv * in.gamma[c], in.beta[c]));
    if (ft != nullptr) val = fmaf(ft[c] + fc[c], val, ft[in.split + c] + fc[in.split + c]);
    if (res != nullptr) val += part_sum(res + i, in.res_parts, in.res_part_stride);
    out[i] = val;
  };
#pragma unroll
  for (int r = 0; r < kNgRegs; ++r) {
    const int i = tid + r * kNaThreads;
    if (i < n) put(i, v[r]);
  }
  for (int i = tid + kNgRegs * kNaThreads; i < n; i += kNaThreads)
    put(i, part_sum(src + i, in.parts, in.part_stride));
}

// norm_act_general_kernel for groups of at most R * kNaThreads values (R per lane): every load
// of the pass (the input's partial sums, the affine and FiLM coefficients of each value's
// channel and the residual's partial sums) is issued before the statistics, so the pass costs
// one memory round trip instead of two.  Same sums in the same order: bit-identical results.
template <int R>
__global__ __launch_bounds__(kNaThreads) void norm_act_small_kernel(ConvInput in, int lin,
                                                                    float* dst,
                                                                    std::int64_t dst_stride) {
  __shared__ double rs[kNaThreads / kWave], rq[kNaThreads / kWave];
  const int b = blockIdx.x / in.groups, g = blockIdx.x % in.groups;
  const int cpg = in.split / in.groups;
  const int n = cpg * lin;
  const std::int64_t base = static_cast<std::int64_t>(g) * n;
  const float* src = in.src + b * in.src_stride + base;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  const bool film = in.film_time != nullptr;
  const float* ft = film ? in.film_time + in.film_off : in.gamma;
  const float* fc = film ? in.film_cond + b * in.film_cond_stride + in.film_off : in.gamma;
  const int fo = film ? in.split : 0;
  const float* res = in.res != nullptr ? in.res + b * in.res_stride + base : nullptr;
  float v[R], ga[R], be[R], t0[R], c0[R], t1[R], c1[R], rv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid + r * kNaThreads;
    const bool act = i < n;
    const int c = g * cpg + (act ? i / lin : 0);
    v[r] = act ? part_sum(src + i, in.parts, in.part_stride) : 0.0f;
    ga[r] = in.gamma[c];
    be[r] = in.beta[c];
    t0[r] = ft[c];
    c0[r] = fc[c];
    t1[r] = ft[fo + c];
    c1[r] = fc[fo + c];
    rv[r] = act && res != nullptr ? part_sum(res + i, in.res_parts, in.res_part_stride) : 0.0f;
  }
  double s = 0.0, q = 0.0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const double d = static_cast<double>(v[r]);
    s += d;
    q += d * d;
  }
  s = wave_sum(s);
  q = wave_sum(q);
  if (lane == 0) {
    rs[wave] = s;
    rq[wave] = q;
  }
  __syncthreads();
  s = 0.0;
  q = 0.0;
  for (int w = 0; w < kNaThreads / kWave; ++w) {
    s += rs[w];
    q += rq[w];
  }
  const double cnt = static_cast<double>(n);
  const double mean = s / cnt;
  const double var = fmax(0.0, q / cnt - mean * mean);
  const float meanf = static_cast<float>(mean);
  const float inv = static_cast<float>(1.0 / sqrt(var + 1e-5));
  float* out = dst + b * dst_stride + base;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid + r * kNaThreads;
    if (i >= n) continue;
    float val = mish_fast(fmaf(v[r] - meanf, inv * ga[r], be[r]));
    if (film) val = fmaf(t0[r] + c0[r], val, t1[r] + c1[r]);
    if (res != nullptr) val += rv[r];
    out[i] = val;
  }
}

// dst[b][i] = sum over p of src[b][p][i], added in order.
__global__ __launch_bounds__(kNgThreads) void sum_parts_kernel(const float* src,
                                                               std::int64_t src_stride, int parts,
                                                               std::int64_t part_stride,
                                                               std::int64_t n, float* dst,
                                                               std::int64_t dst_stride) {
  const int b = blockIdx.y;
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * kNgThreads + threadIdx.x; i < n;
       i += static_cast<std::int64_t>(gridDim.x) * kNgThreads)
    dst[b * dst_stride + i] = part_sum(src + b * src_stride + i, parts, part_stride);
}

}  // namespace

hipError_t conv_general(const ConvOp& op, const float* src, std::int64_t src_stride, int split,
                        const float* plain, std::int64_t plain_stride, View y, int batch,
                        float* workspace, std::size_t workspace_floats, hipStream_t stream) {
  if (batch <= 0 || op.ic <= 0 || op.oc <= 0 || op.lin <= 0 || split <= 0 || split > op.ic)
    return hipErrorInvalidValue;
  if (op.mode == kConvSame) {
    if (op.k <= 0 || op.k % 2 == 0 || op.lout != op.lin) return hipErrorInvalidValue;
  } else if (op.mode == kConvDown) {
    if (op.k != 3 || op.lout != op.lin / 2) return hipErrorInvalidValue;
  } else if (op.mode == kConvTranspose) {
    if (op.k != 4 || op.lout != 2 * op.lin) return hipErrorInvalidValue;
  } else {
    return hipErrorInvalidValue;
  }
  if (split < op.ic && plain == nullptr) return hipErrorInvalidValue;
  const std::int64_t steps = static_cast<std::int64_t>((op.ic + kGenKC - 1) / kGenKC) * op.k;
  if (steps > 0x7fffffff) return hipErrorInvalidValue;
  GenArgs a{};
  a.w = op.w;
  a.bf16 = op.bf16 ? 1 : 0;
  a.bias = op.b;
  a.y = y.p;
  a.ys = y.stride;
  a.src = src;
  a.src_stride = src_stride;
  a.split = split;
  a.plain = plain;
  a.plain_stride = plain_stride;
  a.mode = op.mode;
  a.k = op.k;
  a.ic = op.ic;
  a.oc = op.oc;
  a.lin = op.lin;
  a.lout = op.lout;
  a.batch = batch;
  a.mtiles = (op.oc + kGenMT - 1) / kGenMT;
  a.steps = static_cast<int>(steps);
  const std::int64_t cols = static_cast<std::int64_t>(batch) * op.lout;
  if (cols <= 16) return launch_general<16>(a, workspace, workspace_floats, stream);
  if (cols <= 32) return launch_general<32>(a, workspace, workspace_floats, stream);
  return launch_general<64>(a, workspace, workspace_floats, stream);
}

hipError_t sum_parts(const float* src, std::int64_t src_stride, int parts,
                     std::int64_t part_stride, std::int64_t n, float* dst,
                     std::int64_t dst_stride, int batch, hipStream_t stream) {
  if (batch <= 0 || batch > 65535 || parts < 1 || n <= 0) return hipErrorInvalidValue;
  const std::int64_t blocks = std::min<std::int64_t>((n + kNgThreads - 1) / kNgThreads, 64);
  hipLaunchKernelGGL(sum_parts_kernel, dim3(static_cast<unsigned>(blocks), batch),
                     dim3(kNgThreads), 0, stream, src, src_stride, parts, part_stride, n, dst,
                     dst_stride);
  return hipGetLastError();
}

hipError_t norm_act_general(const ConvInput& in, int lin, float* dst, std::int64_t dst_stride,
                            int batch, hipStream_t stream) {
  if (!in.norm || batch <= 0 || lin <= 0 || in.groups <= 0 || in.split <= 0 ||
      in.split % in.groups != 0)
    return hipErrorInvalidValue;
  const std::int64_t blocks = static_cast<std::int64_t>(batch) * in.groups;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(blocks));
  const std::int64_t n = static_cast<std::int64_t>(in.split / in.groups) * lin;
  if (n <= kNaThreads)
    hipLaunchKernelGGL(norm_act_small_kernel<1>, grid, dim3(kNaThreads), 0, stream, in, lin, dst,
                       dst_stride);
  else if (n <= 2 * kNaThreads)
    hipLaunchKernelGGL(norm_act_small_kernel<2>, grid, dim3(kNaThreads), 0, stream, in, lin, dst,
                       dst_stride);
  else if (n <= 4 * kNaThreads)
    hipLaunchKernelGGL(norm_act_small_kernel<4>, grid, dim3(kNaThreads), 0, stream, in, lin, dst,
                       dst_stride);
  else
    hipLaunchKernelGGL(norm_act_general_kernel, grid, dim3(kNaThreads), 0, stream, in, lin, dst,
                       dst_stride);
  return hipGetLastError();
}

}  // namespace fe::hip
