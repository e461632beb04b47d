// HIP kernels for the Diffusion Policy U-Net on gfx950 (CDNA4).
//
// Batch-1 convolutions are weight-streaming GEMVs: each weight element is read once from HBM and
// multiplied against the L_out input positions it touches.  Weights are repacked at load to
// [OC][K][IC] so a 64-lane wavefront reads 64 consecutive 16-byte vectors of one (oc, tap) row;
// each lane keeps the four input channels it owns resident in registers for all taps and rows,
// and a wavefront reduce-scatter (halving exchange over lane bits) folds the per-lane partial
// sums so each lane ends holding a distinct finished output.
//
// Reference semantics: conv1d diffusion_ops.cc:82-163, conv_transpose1d :165-268, group_norm
// :270-350, film :352-377, timestep embedding :379-396, mish kernels_cuda.cu:126-133, DDIM/DDPM
// diffusion.cc:995-1024, flow updates span_ops.h:27-52, unnormalize diffusion.cc:1027-1033.
#include "kernels.h"

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fe::hip {
namespace {

constexpr int kBlock = 256;
constexpr int kWave = 64;

// mish(v) = v * tanh(log1p(e^v)).  With e = e^v, tanh(log(1 + e)) = ((1+e)^2 - 1) / ((1+e)^2 + 1)
// = n / (n + 2), n = e (e + 2): one exponential, no cancellation for v << 0.  For v > 20 the
// factor rounds to 1 in fp32.
__device__ __forceinline__ float mish_f(float v) {
  if (v > 20.0f) return v;
  const float e = expf(v);
  const float n = e * (e + 2.0f);
  return v * (n / (n + 2.0f));
}

__device__ __forceinline__ float bf16_to_f32(unsigned short bits) {
  return __uint_as_float(static_cast<unsigned>(bits) << 16);
}

// ---------------------------------------------------------------------------------------------
// Wavefront reduce-scatter.  On entry every lane holds N partial sums v[0..N); on exit lane l
// holds max(N/64, 1) finished sums (over all 64 lanes) of the original indices
// [rs_offset<N>(l), +max(N/64,1)).  Each halving step exchanges half of the remaining values
// with the partner lane (l ^ mask); once one value remains, plain butterfly steps finish it.
// ---------------------------------------------------------------------------------------------
template <int N, int MASK>
__device__ __forceinline__ void rs_step(float* v, int lane) {
  if constexpr (MASK > 0) {
    if constexpr (N >= 2) {
      const bool upper = (lane & MASK) != 0;
#pragma unroll
      for (int i = 0; i < N / 2; ++i) {
        const float send = upper ? v[i] : v[i + N / 2];
        const float keep = upper ? v[i + N / 2] : v[i];
        v[i] = keep + __shfl_xor(send, MASK, kWave);
      }
      rs_step<N / 2, MASK / 2>(v, lane);
    } else {
      v[0] += __shfl_xor(v[0], MASK, kWave);
      rs_step<1, MASK / 2>(v, lane);
    }
  }
}

template <int N>
__device__ __forceinline__ int rs_offset(int lane) {
  int off = 0, n = N;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    if (n >= 2) {
      if (lane & m) off += n / 2;
      n /= 2;
    }
  }
  return off;
}

// Lanes that hold a distinct result after rs_step (the butterfly bits must be zero).
template <int N>
__device__ __forceinline__ bool rs_writer(int lane) {
  if constexpr (N >= kWave) {
    return true;
  } else {
    return (lane & (kWave / N - 1)) == 0;
  }
}

// ---------------------------------------------------------------------------------------------
// Convolution (weight-streaming GEMV form).
// ---------------------------------------------------------------------------------------------
struct ConvArgs {
  const void* w;
  const float* bias;
  const float* x;
  float* y;
  std::int64_t xs, ys;
  int ic, oc;
  int tpr;  // lanes per row group: 64, 128 or 256
};

template <int MODE, int LIN>
struct ConvShape {
  static constexpr int lout = MODE == kConvSame ? LIN : (MODE == kConvDown ? LIN / 2 : 2 * LIN);
};

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

template <int VEC, bool BF16>
__device__ __forceinline__ void load_w(const void* base, std::int64_t idx, float* out) {
  if constexpr (BF16) {
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

template <int MODE, int K, int LIN, int VEC, int R, bool BF16>
__global__ __launch_bounds__(kBlock) void conv_kernel(ConvArgs a) {
  constexpr int LOUT = ConvShape<MODE, LIN>::lout;
  constexpr int V = R * LOUT;
  __shared__ float red[4 * V];

  const int tid = threadIdx.x;
  const int groups = kBlock / a.tpr;
  const int gid = tid / a.tpr;
  const int lg = tid - gid * a.tpr;
  const int row0 = (blockIdx.x * groups + gid) * R;
  const int b = blockIdx.y;
  const float* x = a.x + b * a.xs;
  const int nv = a.ic / VEC;

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;

  for (int cv = lg; cv < nv; cv += a.tpr) {
    float xr[VEC][LIN];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const float* row = x + static_cast<std::int64_t>(cv * VEC + v) * LIN;
      if constexpr (LIN % 4 == 0) {
#pragma unroll
        for (int j = 0; j < LIN; j += 4) {
          const float4 q = *reinterpret_cast<const float4*>(row + j);
          xr[v][j] = q.x;
          xr[v][j + 1] = q.y;
          xr[v][j + 2] = q.z;
          xr[v][j + 3] = q.w;
        }
      } else {
#pragma unroll
        for (int j = 0; j < LIN; ++j) xr[v][j] = row[j];
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int oc = row0 + r;
      if (oc < a.oc) {
        float wv[K][VEC];
#pragma unroll
        for (int k = 0; k < K; ++k)
          load_w<VEC, BF16>(a.w, (static_cast<std::int64_t>(oc) * K + k) * a.ic + cv * VEC,
                            wv[k]);
#pragma unroll
        for (int t = 0; t < LOUT; ++t) {
#pragma unroll
          for (int k = 0; k < K; ++k) {
            const int j = src_index<MODE, K, LIN>(t, k);
            if (j >= 0) {
#pragma unroll
              for (int v = 0; v < VEC; ++v) acc[r * LOUT + t] = fmaf(wv[k][v], xr[v][j], acc[r * LOUT + t]);
            }
          }
        }
      }
    }
  }

  const int lane = tid & (kWave - 1);
  rs_step<V, 32>(acc, lane);
  constexpr int NF = V >= kWave ? V / kWave : 1;
  const int off = rs_offset<V>(lane);
  const int waves = a.tpr / kWave;
  const int wig = lg / kWave;  // wave index inside the row group
  if (waves == 1) {
    if (rs_writer<V>(lane)) {
#pragma unroll
      for (int i = 0; i < NF; ++i) {
        const int idx = off + i;
        const int oc = row0 + idx / LOUT;
        if (oc < a.oc)
          a.y[b * a.ys + static_cast<std::int64_t>(oc) * LOUT + (idx % LOUT)] = acc[i] + a.bias[oc];
      }
    }
    return;
  }
  // Several waves per row group: combine through LDS.  red holds [wave-in-group][V] for each
  // group; a block has at most 4 waves in total, so 4 * V floats suffice.
  float* gred = red + gid * waves * V;
  if (rs_writer<V>(lane)) {
#pragma unroll
    for (int i = 0; i < NF; ++i) gred[wig * V + off + i] = acc[i];
  }
  __syncthreads();
  for (int idx = lg; idx < V; idx += a.tpr) {
    float s = 0.0f;
    for (int w = 0; w < waves; ++w) s += gred[w * V + idx];
    const int oc = row0 + idx / LOUT;
    if (oc < a.oc)
      a.y[b * a.ys + static_cast<std::int64_t>(oc) * LOUT + (idx % LOUT)] = s + a.bias[oc];
  }
}

constexpr int kRows = 2;

template <int MODE, int K, int LIN, int VEC, bool BF16>
hipError_t launch_conv_t(const ConvArgs& a, int batch, hipStream_t s) {
  const int groups = kBlock / a.tpr;
  const int rows_per_block = groups * kRows;
  const dim3 grid((a.oc + rows_per_block - 1) / rows_per_block, batch);
  hipLaunchKernelGGL((conv_kernel<MODE, K, LIN, VEC, kRows, BF16>), grid, dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

template <int MODE, int K, int VEC, bool BF16>
hipError_t dispatch_lin(const ConvArgs& a, int lin, int batch, hipStream_t s) {
  switch (lin) {
    case 1:
      if constexpr (MODE != kConvDown) return launch_conv_t<MODE, K, 1, VEC, BF16>(a, batch, s);
      break;
    case 2: return launch_conv_t<MODE, K, 2, VEC, BF16>(a, batch, s);
    case 4: return launch_conv_t<MODE, K, 4, VEC, BF16>(a, batch, s);
    case 8: return launch_conv_t<MODE, K, 8, VEC, BF16>(a, batch, s);
    case 16: return launch_conv_t<MODE, K, 16, VEC, BF16>(a, batch, s);
    case 32:
      if constexpr (MODE != kConvTranspose) return launch_conv_t<MODE, K, 32, VEC, BF16>(a, batch, s);
      break;
    default: break;
  }
  return hipErrorInvalidValue;
}

template <int VEC, bool BF16>
hipError_t dispatch_mode(const ConvOp& op, const ConvArgs& a, int batch, hipStream_t s) {
  if (op.mode == kConvSame) {
    switch (op.k) {
      case 1: return dispatch_lin<kConvSame, 1, VEC, BF16>(a, op.lin, batch, s);
      case 3: return dispatch_lin<kConvSame, 3, VEC, BF16>(a, op.lin, batch, s);
      case 5: return dispatch_lin<kConvSame, 5, VEC, BF16>(a, op.lin, batch, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (op.mode == kConvDown && op.k == 3) return dispatch_lin<kConvDown, 3, VEC, BF16>(a, op.lin, batch, s);
  if (op.mode == kConvTranspose && op.k == 4)
    return dispatch_lin<kConvTranspose, 4, VEC, BF16>(a, op.lin, batch, s);
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------------------
// GroupNorm + Mish + FiLM + residual.  One block per (group, sample); statistics in fp64 with
// var = E[x^2] - mean^2 clamped at 0, eps 1e-5 (group_norm, diffusion_ops.cc:270-350).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ double block_sum(double v, double* sh) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) sh[w] = v;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < kBlock / kWave; ++i) s += sh[i];
  return s;
}

__global__ __launch_bounds__(kBlock) void norm_act_kernel(NormActOp op, const float* x,
                                                          std::int64_t xs, float* y,
                                                          std::int64_t ys) {
  __shared__ double sh[kBlock / kWave];
  const int g = blockIdx.x, b = blockIdx.y;
  const int cpg = op.c / op.groups;
  const int count = cpg * op.len;
  const std::int64_t base = static_cast<std::int64_t>(g) * count;
  const float* xb = x + b * xs + base;
  double sum = 0.0, sq = 0.0;
  for (int i = threadIdx.x; i < count; i += kBlock) {
    const double v = static_cast<double>(xb[i]);
    sum += v;
    sq += v * v;
  }
  sum = block_sum(sum, sh);
  sq = block_sum(sq, sh);
  const double mean = sum / static_cast<double>(count);
  const double var = fmax(0.0, sq / static_cast<double>(count) - mean * mean);
  const float inv = static_cast<float>(1.0 / sqrt(var + 1e-5));
  const float mean_f = static_cast<float>(mean);
  float* yb = y + b * ys + base;
  const float* rb = op.res ? op.res + b * op.res_stride + base : nullptr;
  for (int i = threadIdx.x; i < count; i += kBlock) {
    const int c = g * cpg + i / op.len;
    float v = fmaf(xb[i] - mean_f, inv * op.gamma[c], op.beta[c]);
    v = mish_f(v);
    if (op.film_time) {
      const float* fc = op.film_cond + b * op.film_cond_stride + op.film_off;
      const float* ft = op.film_time + op.film_off;
      const float scale = ft[c] + fc[c];
      const float shift = ft[op.c + c] + fc[op.c + c];
      v = fmaf(scale, v, shift);
    }
    if (rb) v += rb[i];
    yb[i] = v;
  }
}

// ---------------------------------------------------------------------------------------------
// Time MLP: m = mish(te2(mish(te1(emb(t)) + b1)) + b2), one block per timestep.
// ---------------------------------------------------------------------------------------------
__device__ float nfe_time(const TimeSpec& ts, int n) {
  if (ts.mode == kTimesSingle) return ts.t0;
  if (ts.mode == kTimesDiffusion) return static_cast<float>((ts.steps - 1 - n) * ts.ratio);
  const int stages = ts.method == 2 ? 4 : (ts.method == 1 ? 2 : 1);
  const int s = n / stages, j = n % stages;
  const float dt = 1.0f / static_cast<float>(ts.steps);
  const float t = static_cast<float>(s) * dt;
  if (j == 0) return t;
  if (ts.method == 1) return t + dt;
  const float half_dt = 0.5f * dt;
  return j == 3 ? t + dt : t + half_dt;
}

__global__ __launch_bounds__(kBlock) void time_mlp_kernel(TimeSpec ts, const float* w1,
                                                          const float* b1, const float* w2,
                                                          const float* b2, int tdim, float* m) {
  extern __shared__ float smem[];
  float* emb = smem;            // [tdim]
  float* hid = smem + tdim;     // [4 tdim]
  const float t = nfe_time(ts, blockIdx.x);
  const int half = tdim / 2;
  if (half == 1) {
    if (threadIdx.x == 0) {
      emb[0] = sinf(t);
      emb[1] = cosf(t);
    }
  } else {
    const float factor = logf(10000.0f) / static_cast<float>(half - 1);
    for (int i = threadIdx.x; i < half; i += kBlock) {
      const float freq = expf(-factor * static_cast<float>(i));
      const float phase = t * freq;
      emb[i] = sinf(phase);
      emb[half + i] = cosf(phase);
    }
  }
  __syncthreads();
  const int hdim = 4 * tdim;
  for (int j = threadIdx.x; j < hdim; j += kBlock) {
    const float* wr = w1 + static_cast<std::int64_t>(j) * tdim;
    float s = 0.0f;
    for (int k = 0; k < tdim; ++k) s = fmaf(wr[k], emb[k], s);
    hid[j] = mish_f(s + b1[j]);
  }
  __syncthreads();
  for (int j = threadIdx.x; j < tdim; j += kBlock) {
    const float* wr = w2 + static_cast<std::int64_t>(j) * hdim;
    float s = 0.0f;
    for (int k = 0; k < hdim; ++k) s = fmaf(wr[k], hid[k], s);
    m[static_cast<std::int64_t>(blockIdx.x) * tdim + j] = mish_f(s + b2[j]);
  }
}

// out[n][f] = bias[f] + sum_k wt[k][f] * act(in[n][k]); eight rows of n per block, k in chunks.
constexpr int kFilmRows = 8;
constexpr int kFilmChunk = 256;

__global__ __launch_bounds__(kBlock) void film_gemm_kernel(const float* in, std::int64_t in_stride,
                                                           int n, int kdim, const float* wt,
                                                           const float* bias, int fdim, int mish_in,
                                                           float* out, std::int64_t out_stride) {
  __shared__ float act[kFilmRows][kFilmChunk];
  const int f = blockIdx.x * kBlock + threadIdx.x;
  const int n0 = blockIdx.y * kFilmRows;
  float acc[kFilmRows];
#pragma unroll
  for (int r = 0; r < kFilmRows; ++r) acc[r] = 0.0f;
  for (int k0 = 0; k0 < kdim; k0 += kFilmChunk) {
    const int kc = min(kFilmChunk, kdim - k0);
    __syncthreads();
    for (int i = threadIdx.x; i < kFilmRows * kFilmChunk; i += kBlock) {
      const int r = i / kFilmChunk, k = i % kFilmChunk;
      float v = 0.0f;
      if (n0 + r < n && k < kc) {
        v = in[(n0 + r) * in_stride + k0 + k];
        if (mish_in) v = mish_f(v);
      }
      act[r][k] = v;
    }
    __syncthreads();
    if (f < fdim) {
      for (int k = 0; k < kc; ++k) {
        const float w = wt[static_cast<std::int64_t>(k0 + k) * fdim + f];
#pragma unroll
        for (int r = 0; r < kFilmRows; ++r) acc[r] = fmaf(w, act[r][k], acc[r]);
      }
    }
  }
  if (f < fdim) {
    const float bb = bias ? bias[f] : 0.0f;
#pragma unroll
    for (int r = 0; r < kFilmRows; ++r)
      if (n0 + r < n) out[(n0 + r) * out_stride + f] = acc[r] + bb;
  }
}

// ---------------------------------------------------------------------------------------------
// Sampler kernels.
// ---------------------------------------------------------------------------------------------
__global__ void begin_kernel(const float* noise, float* x, float* xin, int h, int a) {
  const int b = blockIdx.x;
  for (int i = threadIdx.x; i < h * a; i += blockDim.x) {
    const int t = i / a, c = i % a;
    const float v = noise[static_cast<std::int64_t>(b) * h * a + i];
    x[static_cast<std::int64_t>(b) * h * a + c * h + t] = v;
    if (xin != x) xin[static_cast<std::int64_t>(b) * h * a + c * h + t] = v;
  }
}

// splitmix64 (diffusion.cc:214-221): call i of the stream seeded `seed` mixes seed + (i+2)*GAMMA.
__device__ __forceinline__ float stream_uniform(std::uint64_t seed, std::uint64_t call) {
  std::uint64_t z = seed + (call + 2ull) * 0x9e3779b97f4a7c15ULL;
  z = (z ^ (z >> 30u)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27u)) * 0x94d049bb133111ebULL;
  z ^= z >> 31u;
  return static_cast<float>((z >> 40u) + 1u) / 16777217.0f;
}

// Value `n` of the reference's Box-Muller stream (pairs: cos first, then sin).
__device__ __forceinline__ float stream_gaussian(std::uint64_t seed, std::uint64_t n) {
  const std::uint64_t pair = n >> 1;
  const float first = fmaxf(stream_uniform(seed, 2 * pair), 1.17549435e-38f);
  const float second = stream_uniform(seed, 2 * pair + 1);
  const float radius = sqrtf(-2.0f * logf(first));
  const float angle = 6.28318530717958647692f * second;
  return (n & 1) ? radius * sinf(angle) : radius * cosf(angle);
}

__global__ __launch_bounds__(kBlock) void update_kernel(UpdateOp op) {
  const int b = blockIdx.x;
  const int H = op.horizon, A = op.action_dim;
  const std::int64_t sample = static_cast<std::int64_t>(b) * A * H;
  const float* hb = op.h + static_cast<std::int64_t>(b) * op.c0 * H;
  for (int i = threadIdx.x; i < A * H; i += kBlock) {
    const int a = i / H, t = i % H;  // state layout [A][H]
    const float* wr = op.wo + static_cast<std::int64_t>(a) * op.c0;
    float e = 0.0f;
    for (int c = 0; c < op.c0; ++c) e = fmaf(wr[c], hb[c * H + t], e);
    e += op.bo[a];
    const std::int64_t si = sample + i;
    switch (op.kind) {
      case kUpdateDenoise:
        op.out[sample + static_cast<std::int64_t>(t) * A + a] = e;
        break;
      case kUpdateDDIM: {
        float x0 = (op.x[si] - op.sqrt_bt * e) / op.sqrt_at;
        if (op.clip) x0 = fminf(fmaxf(x0, -op.clip_range), op.clip_range);
        const float nx = op.sqrt_ap * x0 + op.sqrt_1map * e;
        op.x[si] = nx;
        if (op.xin != op.x) op.xin[si] = nx;
        break;
      }
      case kUpdateDDPM: {
        float x0 = (op.x[si] - op.sqrt_bt * e) / op.sqrt_at;
        if (op.clip) x0 = fminf(fmaxf(x0, -op.clip_range), op.clip_range);
        float nx = op.coef_x0 * x0 + op.coef_x * op.x[si];
        if (op.add_noise)
          nx += op.sigma *
                stream_gaussian(*op.seed, op.noise_offset + static_cast<std::uint64_t>(t) * A + a);
        op.x[si] = nx;
        if (op.xin != op.x) op.xin[si] = nx;
        break;
      }
      case kUpdateEuler: {
        const float nx = op.x[si] + op.dt * e;
        op.x[si] = nx;
        op.xin[si] = nx;
        break;
      }
      case kUpdateStage: {
        const std::int64_t plane = static_cast<std::int64_t>(gridDim.x) * A * H;
        op.kbuf[op.slot * plane + si] = e;
        op.xin[si] = op.x[si] + op.dt * e;
        break;
      }
      case kUpdateHeun: {
        const float k1 = op.kbuf[si];
        const float nx = op.x[si] + 0.5f * op.dt * (k1 + e);
        op.x[si] = nx;
        op.xin[si] = nx;
        break;
      }
      case kUpdateRK4: {
        const std::int64_t plane = static_cast<std::int64_t>(gridDim.x) * A * H;
        const float k1 = op.kbuf[si], k2 = op.kbuf[plane + si], k3 = op.kbuf[2 * plane + si];
        const float nx = op.x[si] + (op.dt / 6.0f) * (k1 + 2.0f * k2 + 2.0f * k3 + e);
        op.x[si] = nx;
        op.xin[si] = nx;
        break;
      }
      default:
        break;
    }
  }
}

__global__ void finish_kernel(const float* x, const float* amin, const float* amax, float* action,
                              int h, int a) {
  const int b = blockIdx.x;
  for (int i = threadIdx.x; i < h * a; i += blockDim.x) {
    const int t = i / a, c = i % a;
    const float v = x[static_cast<std::int64_t>(b) * h * a + c * h + t];
    action[static_cast<std::int64_t>(b) * h * a + i] =
        amin ? (v + 1.0f) * 0.5f * (amax[c] - amin[c]) + amin[c] : v;
  }
}

}  // namespace

hipError_t conv(const ConvOp& op, const float* x, std::int64_t x_stride, View y, int batch,
                hipStream_t stream) {
  ConvArgs a{};
  a.w = op.w;
  a.bias = op.b;
  a.x = x;
  a.y = y.p;
  a.xs = x_stride;
  a.ys = y.stride;
  a.ic = op.ic;
  a.oc = op.oc;
  const bool vec4 = op.ic % 4 == 0;
  const int nv = vec4 ? op.ic / 4 : op.ic;
  a.tpr = nv >= 256 ? 256 : (nv >= 128 ? 128 : 64);
  if (vec4) return op.bf16 ? dispatch_mode<4, true>(op, a, batch, stream)
                           : dispatch_mode<4, false>(op, a, batch, stream);
  return op.bf16 ? dispatch_mode<1, true>(op, a, batch, stream)
                 : dispatch_mode<1, false>(op, a, batch, stream);
}

hipError_t norm_act(const NormActOp& op, const float* x, std::int64_t x_stride, View y, int batch,
                    hipStream_t stream) {
  hipLaunchKernelGGL(norm_act_kernel, dim3(op.groups, batch), dim3(kBlock), 0, stream, op, x,
                     x_stride, y.p, y.stride);
  return hipGetLastError();
}

hipError_t time_mlp(const TimeSpec& times, int count, const float* w1, const float* b1,
                    const float* w2, const float* b2, int tdim, float* m, hipStream_t stream) {
  const size_t smem = static_cast<size_t>(5 * tdim) * sizeof(float);
  hipLaunchKernelGGL(time_mlp_kernel, dim3(count), dim3(kBlock), smem, stream, times, w1, b1, w2,
                     b2, tdim, m);
  return hipGetLastError();
}

hipError_t film_gemm(const float* in, std::int64_t in_stride, int n, int kdim, const float* wt,
                     const float* bias, int fdim, bool mish_in, float* out,
                     std::int64_t out_stride, hipStream_t stream) {
  const dim3 grid((fdim + kBlock - 1) / kBlock, (n + kFilmRows - 1) / kFilmRows);
  hipLaunchKernelGGL(film_gemm_kernel, grid, dim3(kBlock), 0, stream, in, in_stride, n, kdim, wt,
                     bias, fdim, mish_in ? 1 : 0, out, out_stride);
  return hipGetLastError();
}

hipError_t begin_sample(const float* noise, float* x, float* xin, int batch, int horizon,
                        int action_dim, hipStream_t stream) {
  hipLaunchKernelGGL(begin_kernel, dim3(batch), dim3(kBlock), 0, stream, noise, x, xin, horizon,
                     action_dim);
  return hipGetLastError();
}

hipError_t update(const UpdateOp& op, int batch, hipStream_t stream) {
  hipLaunchKernelGGL(update_kernel, dim3(batch), dim3(kBlock), 0, stream, op);
  return hipGetLastError();
}

hipError_t finish_sample(const float* x, const float* amin, const float* amax, float* action,
                         int batch, int horizon, int action_dim, hipStream_t stream) {
  hipLaunchKernelGGL(finish_kernel, dim3(batch), dim3(kBlock), 0, stream, x, amin, amax, action,
                     horizon, action_dim);
  return hipGetLastError();
}

}  // namespace fe::hip
