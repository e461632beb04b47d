// Observation encoder kernels on gfx950: the Diffusion Policy RGB encoder (resnet18 trunk with
// GroupNorm, spatial-softmax keypoints, linear + ReLU) that turns camera images into the image
// part of the head's condition.  Semantics: LeRobot's DiffusionRgbEncoder as the reference's
// observation path runs it (integrations/lerobot/src/flowedge_lerobot/observation.py:152-216).
//
// enc_conv_kernel is an implicit GEMM on the FP32 vector ALUs: a workgroup of 256 lanes owns 64
// output channels x NT output columns (column = image * H * W + y * W + x) and walks the reduction
// index (tap * C + input channel) 16 at a time through LDS, with the loads of kPre steps in
// flight together.  The weights are repacked step-major at load ([step][O][16], zero past the
// end), so one step of a workgroup reads 4 KB of contiguous weights, and the 3-channel stem
// takes 10 steps rather than 49.  When the output tiles leave CUs idle, the
// reduction is split over workgroups and each writes its partial sum into its own copy of the
// output ([parts][n][C][H][W]); the GroupNorm pass that consumes the convolution adds the
// partials in order.  The convolutions carry no bias.
//
// The GroupNorm pass finishes a convolution.  Groups of at most kFusedMax values (every block
// of the trunk) take one launch, enc_norm_fused_kernel: a workgroup per (image, group) holds the
// group in registers, adds the partials, takes fp64 statistics and writes GroupNorm + ReLU with
// the BasicBlock's residual (the block input, or GroupNorm of the 1x1 projection).  The stem's
// larger groups take two: enc_stats_kernel, a workgroup per chunk of each (image, group), adds
// the partials (writing the sum over the first) and stores the chunk's fp64 sums;
// enc_apply_kernel, a lane per output value, combines its group's chunk sums in order and
// applies GroupNorm, ReLU and the 3x3 stride-2 max pool (the two-launch path takes the other
// modes too).
//
// The head: enc_keypoint_kernel, a wavefront per (image, keypoint), takes the keypoint 1x1 conv,
// the softmax over positions and the expected (x, y) on the [-1, 1] grid; enc_linear_kernel, a
// workgroup per image, the output linear layer with ReLU.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.h"
#include "encoder.h"

namespace fe::hip::enc {
namespace {

using namespace dev;

constexpr int kThreads = 256;
constexpr int kMT = 64;  // output channels per tile
constexpr int kKC = kReduceChunk;  // reduction indices per step
constexpr int kPre = 6;  // reduction steps whose loads are in flight together

template <int NT>
__global__ __launch_bounds__(kThreads) void enc_conv_kernel(ConvArgs a) {
  constexpr int CPT = NT / 16;               // columns per lane
  constexpr int XR = kKC * NT / kThreads;    // staged input values per lane
  constexpr int WR = kKC * kMT / kThreads;   // staged weights per lane
  __shared__ float ws[kKC][kMT + 1];
  __shared__ float xs[kKC][NT];
  const int tiles = a.mtiles * a.ntiles;
  const int kdim = a.kh * a.kw * a.cin;     // reduction length
  const bool tapwise = a.cin % kKC == 0;    // every step within one tap
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
  // Loads of the next kPre reduction steps are all issued before the first of them is staged,
  // so a workgroup waits about one memory latency per kPre steps.
  for (int s0 = s_begin; s0 < s_end; s0 += kPre) {
    float wv[kPre][WR], xv[kPre][XR];
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      const int s = s0 + u;
      const bool on = s < s_end;
      const float* wp = a.w + (static_cast<std::int64_t>(s) * a.cout + o0) * kKC;
#pragma unroll
      for (int r = 0; r < WR; ++r) {
        const int idx = tid + r * kThreads;
        wv[u][r] = (on && o0 + idx / kKC < a.cout) ? wp[idx] : 0.0f;
      }
      // Reduction index k0 + row: tap (k0 + row) / C, channel (k0 + row) % C; the input
      // position of this lane's column through that tap, in the (cropped) view.
      const int k0 = s * kKC;
      const int tap0 = tapwise ? k0 / a.cin : 0;
#pragma unroll
      for (int r = 0; r < XR; ++r) {
        const int row = srow + r * (kThreads / NT);
        const int kk = k0 + row;
        const int tap = tapwise ? tap0 : kk / a.cin;
        const int c = kk - tap * a.cin;
        const int ky = tap / a.kw, kx = tap - ky * a.kw;
        const int iy = soy * a.stride - a.pad + ky, ix = sox * a.stride - a.pad + kx;
        const bool in = on && scol_ok && kk < kdim && iy >= 0 && iy < a.vh && ix >= 0 &&
                        ix < a.vw;
        xv[u][r] = in ? a.x[simg * a.xs + static_cast<std::int64_t>(c) * a.xplane +
                            static_cast<std::int64_t>(iy + a.top) * a.xw + ix + a.left]
                      : 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      if (s0 + u >= s_end) break;
      __syncthreads();  // the previous step's reads of ws / xs are done
#pragma unroll
      for (int r = 0; r < WR; ++r) {
        const int idx = tid + r * kThreads;
        ws[idx % kKC][idx / kKC] = wv[u][r];
      }
#pragma unroll
      for (int r = 0; r < XR; ++r) xs[srow + r * (kThreads / NT)][scol] = xv[u][r];
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

constexpr int kStatR = 4;                     // values per lane of the statistics pass
constexpr int kChunk = kThreads * kStatR;     // group elements per statistics workgroup
constexpr int kNormThreads = 512;             // lanes of the one-launch GroupNorm
constexpr int kFusedMax = kNormThreads * 16;  // largest group it takes
constexpr int kHeadPos = 9;   // keypoint-map positions per wavefront pass of the head
constexpr int kHeadLanes = 4; // lanes per output feature of the head's linear layer

// The R values lane threadIdx.x owns of an n-element run (elements threadIdx.x + r * T), each
// the sum of `parts` partials `stride` apart, added in partial order; 32 loads in flight.
template <int R, int T>
__device__ __forceinline__ void load_group(const float* p, int parts, std::int64_t stride, int n,
                                           float (&v)[R]) {
  constexpr int PB = R >= 32 ? 1 : 32 / R;  // partials per batch
#pragma unroll
  for (int r = 0; r < R; ++r) v[r] = 0.0f;
  for (int j0 = 0; j0 < parts; j0 += PB) {
    float t[R][PB];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = threadIdx.x + r * T;
#pragma unroll
      for (int q = 0; q < PB; ++q)
        t[r][q] = (i < n && j0 + q < parts) ? p[(j0 + q) * stride + i] : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < PB; ++q)
        if (j0 + q < parts) v[r] += t[r][q];
  }
}

// fp64 (sum, sum of squares) of a workgroup of T lanes, returned to every lane.
template <int T>
__device__ __forceinline__ void block_stats(double& s, double& q, double* red) {
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  s = wave_sum(s);
  q = wave_sum(q);
  __syncthreads();  // earlier readers of red are done
  if (lane == 0) {
    red[wave] = s;
    red[T / kWave + wave] = q;
  }
  __syncthreads();
  s = 0.0;
  q = 0.0;
  for (int w = 0; w < T / kWave; ++w) {
    s += red[w];
    q += red[T / kWave + w];
  }
}

// Mean and 1 / std from fp64 sums over n values (eps 1e-5).
__device__ __forceinline__ void mean_inv(double s, double q, int n, float& mean, float& inv) {
  const double m = s / n;
  mean = static_cast<float>(m);
  inv = static_cast<float>(1.0 / sqrt(fmax(0.0, q / n - m * m) + 1e-5));
}

// Statistics pass: workgroup (image, group, chunk) adds the partials of kChunk elements of the
// group (writing the sum over the first partial) and stores their fp64 (sum, sum of squares);
// with a projection residual, the same for it.
__global__ __launch_bounds__(kThreads) void enc_stats_kernel(NormArgs a, int chunks) {
  __shared__ double red[2 * kThreads / kWave];
  const int ch = blockIdx.x % chunks;
  const int ig = blockIdx.x / chunks;
  const int img = ig / a.groups, g = ig % a.groups;
  const int n = a.c / a.groups * a.h * a.w;
  const std::int64_t base = static_cast<std::int64_t>(g) * n;
  const int i0 = ch * kChunk, len = min(n - i0, kChunk);
  const int tid = threadIdx.x;
  double* out = a.stats + (static_cast<std::int64_t>(ig) * chunks + ch) * 4;
  for (int t = 0; t < (a.mode == kNormEndGn ? 2 : 1); ++t) {
    float* p = (t == 0 ? a.src + img * a.src_stride : a.res + img * a.res_stride) + base + i0;
    const int parts = t == 0 ? a.parts : a.res_parts;
    const std::int64_t stride = t == 0 ? a.part_stride : a.res_part_stride;
    float v[kStatR];
    load_group<kStatR, kThreads>(p, parts, stride, len, v);
    double s = 0.0, q = 0.0;
#pragma unroll
    for (int r = 0; r < kStatR; ++r) {
      const int i = tid + r * kThreads;
      if (i < len) {
        p[i] = v[r];
        s += v[r];
        q += static_cast<double>(v[r]) * v[r];
      }
    }
    block_stats<kThreads>(s, q, red);
    if (tid == 0) {
      out[2 * t] = s;
      out[2 * t + 1] = q;
    }
  }
}

// Mean and 1 / std of (image, group) ig from its chunk statistics (slot t: 0 src, 1 residual).
__device__ __forceinline__ void group_stats(const NormArgs& a, int chunks, int ig, int t, int n,
                                            float& mean, float& inv) {
  const double* st = a.stats + static_cast<std::int64_t>(ig) * chunks * 4;
  double s = 0.0, q = 0.0;
  for (int c = 0; c < chunks; ++c) {
    s += st[4 * c + 2 * t];
    q += st[4 * c + 2 * t + 1];
  }
  mean_inv(s, q, n, mean, inv);
}

// Apply pass, one lane per output value: GN + ReLU, with the stem's max pool or a residual.
__global__ __launch_bounds__(kThreads) void enc_apply_kernel(NormArgs a, int chunks) {
  const int cpg = a.c / a.groups;
  const int hw = a.h * a.w;
  const int n = cpg * hw;
  const bool pool = a.mode == kNormStemPool;
  const int ph = (a.h + 1) / 2, pw = (a.w + 1) / 2;
  const int per_img = pool ? a.c * ph * pw : a.c * hw;
  const std::int64_t e = static_cast<std::int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= static_cast<std::int64_t>(a.n) * per_img) return;
  const int img = static_cast<int>(e / per_img);
  const int j = static_cast<int>(e - static_cast<std::int64_t>(img) * per_img);
  const int c = j / (pool ? ph * pw : hw);
  const int g = c / cpg;
  const int ig = img * a.groups + g;
  float mean, inv;
  group_stats(a, chunks, ig, 0, n, mean, inv);
  const float sc = inv * a.gamma[c], sh = a.beta[c];
  const float* h = a.src + img * a.src_stride + static_cast<std::int64_t>(c) * hw;
  float* out = a.dst + img * a.dst_stride;
  if (pool) {
    // relu(GN(h)) then the 3x3 stride-2 max pool (padding 1).
    const int p = j - c * ph * pw;
    const int py = p / pw, px = p - py * pw;
    float best = 0.0f;  // relu output >= 0, and every window holds an input position
    for (int dy = -1; dy <= 1; ++dy) {
      const int yy = 2 * py + dy;
      if (yy < 0 || yy >= a.h) continue;
      for (int dx = -1; dx <= 1; ++dx) {
        const int xx = 2 * px + dx;
        if (xx < 0 || xx >= a.w) continue;
        best = fmaxf(best, fmaf(h[yy * a.w + xx] - mean, sc, sh));
      }
    }
    out[j] = best;
    return;
  }
  const int p = j - c * hw;
  float v = fmaf(h[p] - mean, sc, sh);
  if (a.mode == kNormEndPlain) v += a.res[img * a.res_stride + j];
  if (a.mode == kNormEndGn) {
    float rm, ri;
    group_stats(a, chunks, ig, 1, n, rm, ri);
    v += fmaf(a.res[img * a.res_stride + j] - rm, ri * a.rgamma[c], a.rbeta[c]);
  }
  out[j] = fmaxf(v, 0.0f);
}

// One-launch GroupNorm for groups of at most kFusedMax values (every mode but the stem's): a
// workgroup per (image, group) holds the group's values (partials added) in registers, takes its
// fp64 statistics (and the projection residual's), and writes the normalized result.
template <int R>
__global__ __launch_bounds__(kNormThreads) void enc_norm_fused_kernel(NormArgs a) {
  __shared__ double red[2 * kNormThreads / kWave];
  const int ig = blockIdx.x;
  const int img = ig / a.groups, g = ig % a.groups;
  const int hw = a.h * a.w;
  const int cpg = a.c / a.groups;
  const int n = cpg * hw;
  const std::int64_t base = static_cast<std::int64_t>(g) * n;
  const int tid = threadIdx.x;
  float v[R], rv[R];
  load_group<R, kNormThreads>(a.src + img * a.src_stride + base, a.parts, a.part_stride, n, v);
  if (a.mode == kNormEndGn) {
    load_group<R, kNormThreads>(a.res + img * a.res_stride + base, a.res_parts,
                                a.res_part_stride, n, rv);
  } else if (a.mode == kNormEndPlain) {
    const float* rp = a.res + img * a.res_stride + base;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = tid + r * kNormThreads;
      rv[r] = i < n ? rp[i] : 0.0f;
    }
  }
  // The affine coefficients of each value's channel are read with the values, before the
  // statistics, so that their latency is not added after them.
  float ga[R], be[R], rga[R], rbe[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid + r * kNormThreads;
    const int c = g * cpg + (i < n ? i / hw : 0);
    ga[r] = a.gamma[c];
    be[r] = a.beta[c];
    rga[r] = a.mode == kNormEndGn ? a.rgamma[c] : 0.0f;
    rbe[r] = a.mode == kNormEndGn ? a.rbeta[c] : 0.0f;
  }
  double s = 0.0, q = 0.0;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (tid + r * kNormThreads < n) {
      s += v[r];
      q += static_cast<double>(v[r]) * v[r];
    }
  block_stats<kNormThreads>(s, q, red);
  float mean, inv;
  mean_inv(s, q, n, mean, inv);
  float rmean = 0.0f, rinv = 0.0f;
  if (a.mode == kNormEndGn) {
    s = 0.0;
    q = 0.0;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (tid + r * kNormThreads < n) {
        s += rv[r];
        q += static_cast<double>(rv[r]) * rv[r];
      }
    block_stats<kNormThreads>(s, q, red);
    mean_inv(s, q, n, rmean, rinv);
  }
  float* out = a.dst + img * a.dst_stride + base;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid + r * kNormThreads;
    if (i >= n) continue;
    float o = fmaf(v[r] - mean, inv * ga[r], be[r]);
    if (a.mode == kNormEndPlain) o += rv[r];
    if (a.mode == kNormEndGn) o += fmaf(rv[r] - rmean, rinv * rga[r], rbe[r]);
    out[i] = fmaxf(o, 0.0f);
  }
}

// Keypoint pass, a wavefront per (image, keypoint): the 1x1 conv logit of every position (lanes
// over the channels, kHeadPos positions per pass, fp64 wavefront sums), the softmax over the
// positions and the expected (x, y) on the grid, written to kp[image][2 * keypoint + {0, 1}].
__global__ __launch_bounds__(kWave) void enc_keypoint_kernel(HeadArgs a) {
  __shared__ float att[kMaxHeadPos];
  const int img = blockIdx.x / a.k, kk = blockIdx.x % a.k;
  const int lane = threadIdx.x;
  const float* x = a.x + img * a.x_stride;
  const float* wr = a.nets_w + static_cast<std::int64_t>(kk) * a.c;
  const float bias = a.nets_b[kk];
  for (int p0 = 0; p0 < a.hw; p0 += kHeadPos) {
    float acc[kHeadPos];
#pragma unroll
    for (int q = 0; q < kHeadPos; ++q) acc[q] = 0.0f;
#pragma unroll 8
    for (int c = lane; c < a.c; c += kWave) {
      const float wc = wr[c];
      const float* xc = x + static_cast<std::int64_t>(c) * a.hw + p0;
#pragma unroll
      for (int q = 0; q < kHeadPos; ++q)
        if (p0 + q < a.hw) acc[q] = fmaf(wc, xc[q], acc[q]);
    }
#pragma unroll
    for (int q = 0; q < kHeadPos; ++q) {
      const double sum = wave_sum(static_cast<double>(acc[q]));
      if (lane == 0 && p0 + q < a.hw) att[p0 + q] = static_cast<float>(sum) + bias;
    }
  }
  __syncthreads();
  float mx = -INFINITY;
  for (int p = lane; p < a.hw; p += kWave) mx = fmaxf(mx, att[p]);
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, kWave));
  double se = 0.0, sx = 0.0, sy = 0.0;
  for (int p = lane; p < a.hw; p += kWave) {
    const double ev = expf(att[p] - mx);
    se += ev;
    sx += ev * a.grid[2 * p];
    sy += ev * a.grid[2 * p + 1];
  }
  se = wave_sum(se);
  sx = wave_sum(sx);
  sy = wave_sum(sy);
  if (lane == 0) {
    float* kp = a.kp + static_cast<std::int64_t>(img) * 2 * a.k + 2 * kk;
    kp[0] = static_cast<float>(sx / se);
    kp[1] = static_cast<float>(sy / se);
  }
}

// Output pass, a workgroup per image: y = relu(out_w kp + out_b), kHeadLanes lanes per output
// feature (each over every kHeadLanes-th input), summed across the lane group.
__global__ __launch_bounds__(kThreads) void enc_linear_kernel(HeadArgs a) {
  __shared__ float kp[kMaxHeadInputs];
  const int img = blockIdx.x;
  const int tid = threadIdx.x;
  const int f = 2 * a.k;
  for (int i = tid; i < f; i += kThreads) kp[i] = a.kp[static_cast<std::int64_t>(img) * f + i];
  __syncthreads();
  const int sub = tid % kHeadLanes;
  for (int j0 = 0; j0 < a.fout; j0 += kThreads / kHeadLanes) {
    const int j = j0 + tid / kHeadLanes;
    float v = 0.0f;
    if (j < a.fout) {
      const float* wr = a.out_w + static_cast<std::int64_t>(j) * f;
#pragma unroll 4
      for (int i = sub; i < f; i += kHeadLanes) v = fmaf(wr[i], kp[i], v);
    }
#pragma unroll
    for (int m = 1; m < kHeadLanes; m <<= 1) v += __shfl_xor(v, m, kWave);
    if (j < a.fout && sub == 0)
      a.y[img * a.y_stride + a.y_offset + j] = fmaxf(v + a.out_b[j], 0.0f);
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
  a.steps = (a.kh * a.kw * a.cin + kKC - 1) / kKC;
  const int tiles = a.mtiles * a.ntiles;
  a.ksplit = 1;
  a.per = a.steps;
  if (tiles < 256 && a.steps > 1) {
    int ks = (512 + tiles - 1) / tiles;
    const int cap = static_cast<std::int64_t>(a.n) * a.cout * a.hout * a.wout <= kSmallOutput
                        ? kMaxParts
                        : kMaxPartsLarge;
    if (ks > cap) ks = cap;
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

int norm_chunks(const NormArgs& a) {
  const int n = a.c / a.groups * a.h * a.w;
  return (n + kChunk - 1) / kChunk;
}

hipError_t norm(const NormArgs& a, hipStream_t stream) {
  if (a.n <= 0 || a.groups <= 0 || a.c % a.groups != 0 || a.parts < 1 || a.parts > kMaxParts ||
      a.res_parts < 1 || a.res_parts > kMaxParts || a.stats == nullptr)
    return hipErrorInvalidValue;
  const int gsize = a.c / a.groups * a.h * a.w;
  if (a.mode != kNormStemPool && gsize <= kFusedMax) {
    const dim3 grid(static_cast<unsigned>(a.n * a.groups)), block(kNormThreads);
    if (gsize <= kNormThreads)
      hipLaunchKernelGGL(enc_norm_fused_kernel<1>, grid, block, 0, stream, a);
    else if (gsize <= 2 * kNormThreads)
      hipLaunchKernelGGL(enc_norm_fused_kernel<2>, grid, block, 0, stream, a);
    else if (gsize <= 4 * kNormThreads)
      hipLaunchKernelGGL(enc_norm_fused_kernel<4>, grid, block, 0, stream, a);
    else if (gsize <= 8 * kNormThreads)
      hipLaunchKernelGGL(enc_norm_fused_kernel<8>, grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL(enc_norm_fused_kernel<16>, grid, block, 0, stream, a);
    return hipGetLastError();
  }
  const int chunks = norm_chunks(a);
  hipLaunchKernelGGL(enc_stats_kernel, dim3(static_cast<unsigned>(a.n * a.groups * chunks)),
                     dim3(kThreads), 0, stream, a, chunks);
  const bool pool = a.mode == kNormStemPool;
  const std::int64_t per_img = pool ? static_cast<std::int64_t>(a.c) * ((a.h + 1) / 2) *
                                          ((a.w + 1) / 2)
                                    : static_cast<std::int64_t>(a.c) * a.h * a.w;
  const std::int64_t total = per_img * a.n;
  hipLaunchKernelGGL(enc_apply_kernel, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, a, chunks);
  return hipGetLastError();
}

hipError_t head(const HeadArgs& a, hipStream_t stream) {
  if (a.n <= 0 || a.k <= 0 || a.hw <= 0 || a.hw > kMaxHeadPos || 2 * a.k > kMaxHeadInputs ||
      a.kp == nullptr)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(enc_keypoint_kernel, dim3(static_cast<unsigned>(a.n * a.k)), dim3(kWave), 0,
                     stream, a);
  hipLaunchKernelGGL(enc_linear_kernel, dim3(static_cast<unsigned>(a.n)), dim3(kThreads), 0,
                     stream, a);
  return hipGetLastError();
}

}  // namespace fe::hip::enc
