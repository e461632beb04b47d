// Observation encoder kernels on gfx950: the Diffusion Policy RGB encoder (resnet18 trunk with
// GroupNorm, spatial-softmax keypoints, linear + ReLU) that turns camera images into the image
// part of the head's condition.  Semantics: LeRobot's DiffusionRgbEncoder as the reference's
// observation path runs it (integrations/lerobot/src/flowedge_lerobot/observation.py:152-216).
//
// enc_conv_kernel is an implicit GEMM on the FP32 vector ALUs: a workgroup of 256 lanes owns 64
// output channels x NT output columns (column = image * H * W + y * W + x) and walks the reduction
// one tap x 16 input channels at a time through LDS (weights repacked [O][tap][C] at load).  When
// the output tiles leave CUs idle, the reduction is split over workgroups and each writes its
// partial sum into its own copy of the output ([n][parts][C][H][W]); the GroupNorm pass that
// consumes the convolution adds the partials in order.  The convolutions carry no bias.
//
// enc_norm_kernel finishes a convolution: one workgroup per (image, group) sums the partials,
// takes fp64 statistics over the group, and applies GroupNorm with ReLU, plus the stem's 3x3
// stride-2 max pool, or a BasicBlock's residual (the block input, or GroupNorm of the 1x1
// projection, whose statistics it takes too).
//
// enc_head_kernel: per image, the keypoint 1x1 conv, a softmax over positions, the expected
// (x, y) on the [-1, 1] grid, and the output linear layer with ReLU.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.h"
#include "encoder.h"

namespace fe::hip::enc {
namespace {

using namespace dev;

constexpr int kThreads = 256;
constexpr int kMT = 64;  // output channels per tile
constexpr int kKC = 16;  // input channels per reduction step

template <int NT>
__global__ __launch_bounds__(kThreads) void enc_conv_kernel(ConvArgs a) {
  constexpr int CPT = NT / 16;               // columns per lane
  constexpr int XR = kKC * NT / kThreads;    // staged input values per lane
  constexpr int WR = kKC * kMT / kThreads;   // staged weights per lane
  __shared__ float ws[kKC][kMT + 1];
  __shared__ float xs[kKC][NT];
  const int tiles = a.mtiles * a.ntiles;
  const int tile = blockIdx.x % tiles;
  const int kp = blockIdx.x / tiles;
  const int mt = tile % a.mtiles, nt = tile / a.mtiles;
  const int o0 = mt * kMT, n0 = nt * NT;
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;  // compute: columns tx + 16 j, channels ty + 16 i
  const int taps = a.kh * a.kw;
  const int hw = a.hout * a.wout;

  // The one output column this lane stages (NT divides the workgroup size).
  const int scol = tid % NT;
  const int srow = tid / NT;  // first staged channel row; rows srow + (256 / NT) r
  const int sn = n0 + scol;
  const int simg = sn / hw, spix = sn - simg * hw;
  const int soy = spix / a.wout, sox = spix - soy * a.wout;
  const bool scol_ok = simg < a.n;

  float acc[4][CPT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < CPT; ++j) acc[i][j] = 0.0f;

  const int s_begin = kp * a.per;
  const int s_end = min(a.steps, s_begin + a.per);
  for (int s = s_begin; s < s_end; ++s) {
    const int c0 = (s / taps) * kKC, tap = s % taps;
    const int ky = tap / a.kw, kx = tap - ky * a.kw;
    float wv[WR], xv[XR];
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      const int idx = tid + r * kThreads;
      const int o = o0 + idx / kKC, c = c0 + idx % kKC;
      wv[r] = (o < a.cout && c < a.cin)
                  ? a.w[(static_cast<std::int64_t>(o) * taps + tap) * a.cin + c]
                  : 0.0f;
    }
    // Input position of this lane's column through tap (ky, kx), in the (cropped) view.
    const int iy = soy * a.stride - a.pad + ky, ix = sox * a.stride - a.pad + kx;
    const bool in = scol_ok && iy >= 0 && iy < a.vh && ix >= 0 && ix < a.vw;
    const float* xp = a.x + simg * a.xs + static_cast<std::int64_t>(iy + a.top) * a.xw + ix + a.left;
#pragma unroll
    for (int r = 0; r < XR; ++r) {
      const int c = c0 + srow + r * (kThreads / NT);
      xv[r] = (in && c < a.cin) ? xp[static_cast<std::int64_t>(c) * a.xplane] : 0.0f;
    }
    __syncthreads();  // the previous step's reads of ws / xs are done
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      const int idx = tid + r * kThreads;
      ws[idx % kKC][idx / kKC] = wv[r];
    }
#pragma unroll
    for (int r = 0; r < XR; ++r) xs[srow + r * (kThreads / NT)][scol] = xv[r];
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kKC; ++c) {
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

  float* y = a.y + kp * a.ypart;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int o = o0 + ty + 16 * i;
#pragma unroll
    for (int jj = 0; jj < CPT; ++jj) {
      const int n = n0 + tx + 16 * jj;
      const int img = n / hw, pix = n - img * hw;
      if (o < a.cout && img < a.n)
        y[img * a.ys + static_cast<std::int64_t>(o) * hw + pix] = acc[i][jj];
    }
  }
}

// Sum of the partials of one element (every load issued before the first add).
__device__ __forceinline__ float parts_at(const float* p, int parts, std::int64_t stride) {
  float v[kMaxParts];
#pragma unroll
  for (int j = 0; j < kMaxParts; ++j) v[j] = j < parts ? p[j * stride] : 0.0f;
  float s = v[0];
#pragma unroll
  for (int j = 1; j < kMaxParts; ++j)
    if (j < parts) s += v[j];
  return s;
}

// fp64 (sum, sum of squares) of a workgroup, returned to every lane.
__device__ __forceinline__ void block_stats(double& s, double& q, double* red) {
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  s = wave_sum(s);
  q = wave_sum(q);
  __syncthreads();  // earlier readers of red are done
  if (lane == 0) {
    red[wave] = s;
    red[kThreads / kWave + wave] = q;
  }
  __syncthreads();
  s = 0.0;
  q = 0.0;
  for (int w = 0; w < kThreads / kWave; ++w) {
    s += red[w];
    q += red[kThreads / kWave + w];
  }
}

__global__ __launch_bounds__(kThreads) void enc_norm_kernel(NormArgs a) {
  __shared__ double red[2 * kThreads / kWave];
  const int img = blockIdx.x / a.groups, g = blockIdx.x % a.groups;
  const int cpg = a.c / a.groups;
  const int hw = a.h * a.w;
  const int n = cpg * hw;
  const std::int64_t base = static_cast<std::int64_t>(g) * n;
  float* h = a.src + img * a.src_stride + base;
  const int tid = threadIdx.x;
  // Pass 1: the partials' sum, written back over the first partial, and its statistics.
  double s = 0.0, q = 0.0;
  for (int i = tid; i < n; i += kThreads) {
    const float v = parts_at(h + i, a.parts, a.part_stride);
    h[i] = v;
    s += v;
    q += static_cast<double>(v) * v;
  }
  block_stats(s, q, red);
  const double mean = s / n;
  const float meanf = static_cast<float>(mean);
  const float inv = static_cast<float>(1.0 / sqrt(fmax(0.0, q / n - mean * mean) + 1e-5));
  // The residual's own GroupNorm (projection path of a block).
  float rmean = 0.0f, rinv = 0.0f;
  float* r = a.res != nullptr ? a.res + img * a.res_stride + base : nullptr;
  if (a.mode == kNormEndGn) {
    s = 0.0;
    q = 0.0;
    for (int i = tid; i < n; i += kThreads) {
      const float v = parts_at(r + i, a.res_parts, a.res_part_stride);
      r[i] = v;
      s += v;
      q += static_cast<double>(v) * v;
    }
    block_stats(s, q, red);
    const double m = s / n;
    rmean = static_cast<float>(m);
    rinv = static_cast<float>(1.0 / sqrt(fmax(0.0, q / n - m * m) + 1e-5));
  }
  float* out = a.dst + img * a.dst_stride;
  if (a.mode == kNormStemPool) {
    // relu(GN(h)) then the 3x3 stride-2 max pool (padding 1) of each channel of the group.
    __syncthreads();  // pass 1 wrote h for the whole group
    const int ph = (a.h + 1) / 2, pw = (a.w + 1) / 2;
    const int m = cpg * ph * pw;
    for (int i = tid; i < m; i += kThreads) {
      const int cl = i / (ph * pw), p = i - cl * (ph * pw);
      const int py = p / pw, px = p - py * pw;
      const int c = g * cpg + cl;
      const float sc = inv * a.gamma[c], sh = a.beta[c];
      const float* hc = h + static_cast<std::int64_t>(cl) * hw;
      float best = 0.0f;  // relu output >= 0, and every window holds an input position
      for (int dy = -1; dy <= 1; ++dy) {
        const int yy = 2 * py + dy;
        if (yy < 0 || yy >= a.h) continue;
        for (int dx = -1; dx <= 1; ++dx) {
          const int xx = 2 * px + dx;
          if (xx < 0 || xx >= a.w) continue;
          best = fmaxf(best, fmaf(hc[yy * a.w + xx] - meanf, sc, sh));
        }
      }
      out[static_cast<std::int64_t>(c) * ph * pw + p] = best;
    }
    return;
  }
  out += base;
  const float* xres = a.mode == kNormEndPlain ? a.res + img * a.res_stride + base : nullptr;
  for (int i = tid; i < n; i += kThreads) {
    const int c = g * cpg + i / hw;
    float v = fmaf(h[i] - meanf, inv * a.gamma[c], a.beta[c]);
    if (a.mode == kNormEndPlain) v += xres[i];
    if (a.mode == kNormEndGn) v += fmaf(r[i] - rmean, rinv * a.rgamma[c], a.rbeta[c]);
    out[i] = fmaxf(v, 0.0f);
  }
}

__global__ __launch_bounds__(kThreads) void enc_head_kernel(HeadArgs a) {
  extern __shared__ float smem[];
  float* xs = smem;                        // [c][hw]
  float* att = xs + a.c * a.hw;            // [k][hw]
  float* kp = att + a.k * a.hw;            // [2k]
  const int img = blockIdx.x;
  const int tid = threadIdx.x;
  const float* x = a.x + img * a.x_stride;
  for (int i = tid; i < a.c * a.hw; i += kThreads) xs[i] = x[i];
  __syncthreads();
  // Keypoint logits: a 1x1 conv of the feature maps.
  for (int i = tid; i < a.k * a.hw; i += kThreads) {
    const int kk = i / a.hw, p = i - kk * a.hw;
    float v = a.nets_b[kk];
    const float* wr = a.nets_w + static_cast<std::int64_t>(kk) * a.c;
    for (int c = 0; c < a.c; ++c) v = fmaf(wr[c], xs[c * a.hw + p], v);
    att[i] = v;
  }
  __syncthreads();
  // Softmax over the positions of each keypoint map and the expected grid position.
  for (int kk = tid; kk < a.k; kk += kThreads) {
    float* row = att + kk * a.hw;
    float mx = row[0];
    for (int p = 1; p < a.hw; ++p) mx = fmaxf(mx, row[p]);
    float sum = 0.0f;
    for (int p = 0; p < a.hw; ++p) {
      const float e = expf(row[p] - mx);
      row[p] = e;
      sum += e;
    }
    float ex = 0.0f, ey = 0.0f;
    for (int p = 0; p < a.hw; ++p) {
      ex = fmaf(row[p], a.grid[2 * p], ex);
      ey = fmaf(row[p], a.grid[2 * p + 1], ey);
    }
    kp[2 * kk] = ex / sum;
    kp[2 * kk + 1] = ey / sum;
  }
  __syncthreads();
  const int f = 2 * a.k;
  for (int j = tid; j < a.fout; j += kThreads) {
    float v = a.out_b[j];
    const float* wr = a.out_w + static_cast<std::int64_t>(j) * f;
    for (int i = 0; i < f; ++i) v = fmaf(wr[i], kp[i], v);
    a.y[img * a.y_stride + a.y_offset + j] = fmaxf(v, 0.0f);
  }
}

}  // namespace

int conv_parts(const ConvArgs& shape) {
  ConvArgs a = shape;
  plan_conv(a);
  return a.ksplit;
}

void plan_conv(ConvArgs& a) {
  const std::int64_t cols = static_cast<std::int64_t>(a.n) * a.hout * a.wout;
  a.nt = cols <= 16 ? 16 : (cols <= 32 ? 32 : 64);
  a.mtiles = (a.cout + kMT - 1) / kMT;
  a.ntiles = static_cast<int>((cols + a.nt - 1) / a.nt);
  a.steps = ((a.cin + kKC - 1) / kKC) * a.kh * a.kw;
  const int tiles = a.mtiles * a.ntiles;
  a.ksplit = 1;
  a.per = a.steps;
  if (tiles < 256 && a.steps > 1) {
    int ks = (512 + tiles - 1) / tiles;
    if (ks > kMaxParts) ks = kMaxParts;
    if (ks > a.steps) ks = a.steps;
    a.per = (a.steps + ks - 1) / ks;
    a.ksplit = (a.steps + a.per - 1) / a.per;
  }
}

hipError_t conv(const ConvArgs& a, hipStream_t stream) {
  if (a.n <= 0 || a.cin <= 0 || a.cout <= 0 || a.ksplit < 1 || a.ksplit > kMaxParts ||
      (a.ksplit > 1 && a.ypart <= 0))
    return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(a.mtiles * a.ntiles * a.ksplit));
  switch (a.nt) {
    case 16: hipLaunchKernelGGL(enc_conv_kernel<16>, grid, dim3(kThreads), 0, stream, a); break;
    case 32: hipLaunchKernelGGL(enc_conv_kernel<32>, grid, dim3(kThreads), 0, stream, a); break;
    case 64: hipLaunchKernelGGL(enc_conv_kernel<64>, grid, dim3(kThreads), 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t norm(const NormArgs& a, hipStream_t stream) {
  if (a.n <= 0 || a.groups <= 0 || a.c % a.groups != 0 || a.parts < 1 || a.parts > kMaxParts ||
      a.res_parts < 1 || a.res_parts > kMaxParts)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(enc_norm_kernel, dim3(static_cast<unsigned>(a.n * a.groups)), dim3(kThreads),
                     0, stream, a);
  return hipGetLastError();
}

std::size_t head_lds_bytes(int c, int hw, int k) {
  return (static_cast<std::size_t>(c) * hw + static_cast<std::size_t>(k) * hw + 2 * k) *
         sizeof(float);
}

hipError_t head(const HeadArgs& a, hipStream_t stream) {
  const std::size_t lds = head_lds_bytes(a.c, a.hw, a.k);
  if (a.n <= 0 || lds > kMaxHeadLds) return hipErrorInvalidValue;
  static bool raised = false;
  if (!raised && lds > 48 * 1024) {
    const hipError_t st = hipFuncSetAttribute(reinterpret_cast<const void*>(enc_head_kernel),
                                              hipFuncAttributeMaxDynamicSharedMemorySize,
                                              static_cast<int>(kMaxHeadLds));
    if (st != hipSuccess) return st;
    raised = true;
  }
  hipLaunchKernelGGL(enc_head_kernel, dim3(static_cast<unsigned>(a.n)), dim3(kThreads), lds,
                     stream, a);
  return hipGetLastError();
}

}  // namespace fe::hip::enc
