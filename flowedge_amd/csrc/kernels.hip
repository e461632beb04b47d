// Small kernels of the Diffusion Policy sampler on gfx950: timestep MLP, FiLM projections, sampler
// begin/finish, and the final GroupNorm + Mish + 1x1 conv with the DDIM / DDPM / flow-ODE update
// fused into its epilogue.
//
// Reference semantics: timestep embedding diffusion_ops.cc:379-396, time MLP and FiLM input
// diffusion.cc:810-820, FiLM modulation :747-752, final conv block :895-913, DDIM/DDPM
// :995-1024, unnormalize :1027-1033, flow updates span_ops.h:27-52 / flow.cc:291-318.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.h"
#include "kernels.h"
#include "update_body.h"

namespace fe::hip {
namespace {

using namespace dev;

// ---------------------------------------------------------------------------------------------
// Time MLP: m = mish(te2(mish(te1(emb(t)) + b1)) + b2), one block per U-Net evaluation.
// ---------------------------------------------------------------------------------------------
__device__ float nfe_time(const TimeSpec& ts, int n) {
  if (ts.mode == kTimesSingle) return ts.t0;
  if (ts.mode == kTimesIndex) return static_cast<float>(n);
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
  float* emb = smem;         // [tdim]
  float* hid = smem + tdim;  // [4 tdim]
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

// ---------------------------------------------------------------------------------------------
// FiLM projection: out[n][f] = bias[f] + sum_k wt[k][f] * act(in[n][k]).  A block covers 64
// consecutive f (one per lane) and 8 rows of n; its four wavefronts split k and combine in LDS.
// ---------------------------------------------------------------------------------------------
constexpr int kFilmRows = 8;
constexpr int kFilmChunk = 256;

__global__ __launch_bounds__(kBlock) void film_gemm_kernel(const float* in, std::int64_t in_stride,
                                                           int n, int kdim, const float* wt,
                                                           const float* bias, int fdim,
                                                           int mish_in, float* out,
                                                           std::int64_t out_stride) {
  __shared__ float act[kFilmRows][kFilmChunk];
  __shared__ float part[kBlock / kWave][kFilmRows][kWave];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const int f = blockIdx.x * kWave + lane;
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
      // Eight weight loads in flight per lane ahead of their products (the same k order as the
      // one-at-a-time tail, so the sums are unchanged).
      constexpr int kStep = kBlock / kWave;
      const float* wp = wt + static_cast<std::int64_t>(k0) * fdim + f;
      int k = wave;
      for (; k + 7 * kStep < kc; k += 8 * kStep) {
        float w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = wp[static_cast<std::int64_t>(k + j * kStep) * fdim];
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int r = 0; r < kFilmRows; ++r) acc[r] = fmaf(w[j], act[r][k + j * kStep], acc[r]);
      }
      for (; k < kc; k += kStep) {
        const float w = wp[static_cast<std::int64_t>(k) * fdim];
#pragma unroll
        for (int r = 0; r < kFilmRows; ++r) acc[r] = fmaf(w, act[r][k], acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kFilmRows; ++r) part[wave][r][lane] = acc[r];
  __syncthreads();
  for (int i = threadIdx.x; i < kFilmRows * kWave; i += kBlock) {
    const int r = i / kWave, l = i % kWave;
    const int ff = blockIdx.x * kWave + l;
    if (n0 + r < n && ff < fdim) {
      float s = 0.0f;
      for (int w = 0; w < kBlock / kWave; ++w) s += part[w][r][l];
      out[(n0 + r) * out_stride + ff] = s + (bias ? bias[ff] : 0.0f);
    }
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

// Final GroupNorm + Mish + 1x1 conv + sampler update, one workgroup per sample (update_body.h).
template <int H, int CPL>
__global__ __launch_bounds__(upd::kUpdThreads) void update_kernel(UpdateOp op) {
  __shared__ upd::UpdateSmem<H> sm;
  upd::update_body<H, false, CPL>(op, blockIdx.x, gridDim.x, sm);
}

// update_kernel<H, 1> split over the groups of a 512-channel final width in 8 groups of 64: one
// wavefront per (sample, group), so the final convolution's partial sums are read by eight CUs
// instead of one.  Wavefront g does what wavefront g of update_kernel does (its group's
// statistics, GroupNorm + Mish, and the 1x1 conv's partial sums over the group's 64 channels,
// reduced in the same order) and stores them device-coherently in op.epart; the sample's last
// wavefront to arrive (op.done counts arrivals; that wavefront resets it) adds the eight partials
// in group order, as update_kernel adds its wavefronts' partials, and runs the sampler update.
// Results are bit-identical to update_kernel's.
constexpr int kSplitGroups = 8;
constexpr int kSplitChannels = kSplitGroups * kWave;
// Up to this batch (128 wavefronts): pusht B=1 tick 2.716 -> 2.683 ms; at 64 samples the
// one-workgroup form is ahead (bimanual B=64 5.45 against 5.48 ms).
constexpr int kSplitMaxBatch = 16;

template <int H>
__global__ __launch_bounds__(kWave) void update_split_kernel(UpdateOp op) {
  constexpr int AG = H >= kWave ? 1 : kWave / H;  // actions per reduction pass
  constexpr int V = AG * H;
  constexpr int PM = upd::kMaxUpdateParts;
  const int b = blockIdx.x / kSplitGroups, g = blockIdx.x % kSplitGroups;
  const int lane = threadIdx.x;
  const int A = op.action_dim, C = kSplitChannels;
  const int c = g * kWave + lane;
  const std::int64_t sample = static_cast<std::int64_t>(b) * A * H;
  const float* p = op.h + b * (op.hstride != 0 ? op.hstride : static_cast<std::int64_t>(C) * H) +
                   static_cast<std::int64_t>(c) * H;
  float w0[AG];
#pragma unroll
  for (int aa = 0; aa < AG; ++aa)
    w0[aa] = aa < A ? op.wo[static_cast<std::int64_t>(aa) * C + c] : 0.0f;
  const float gam = op.gamma[c], bet = op.beta[c];
  float pv[PM][H];
#pragma unroll
  for (int j = 0; j < PM; ++j) {
    const float* pj = p + j * op.hpart;
    const bool on = j < op.hparts;
    if constexpr (H >= 4) {
#pragma unroll
      for (int t = 0; t < H; t += 4) {
        const float4 v = on ? *reinterpret_cast<const float4*>(pj + t) : float4{0, 0, 0, 0};
        pv[j][t] = v.x;
        pv[j][t + 1] = v.y;
        pv[j][t + 2] = v.z;
        pv[j][t + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int t = 0; t < H; ++t) pv[j][t] = on ? pj[t] : 0.0f;
    }
  }
  float hv[H];
  double s = 0.0, q = 0.0;
#pragma unroll
  for (int t = 0; t < H; ++t) {
    float v = pv[0][t];
#pragma unroll
    for (int j = 1; j < PM; ++j)
      if (j < op.hparts) v += pv[j][t];
    hv[t] = v;
    const double d = static_cast<double>(v);
    s += d;
    q += d * d;
  }
  double gs = 0.0, gq = 0.0;
  gs += s;
  gq += q;
  gs = wave_sum(gs);
  gq = wave_sum(gq);
  const double n = static_cast<double>(kWave) * H;
  const double mean = gs / n;
  const double var = fmax(0.0, gq / n - mean * mean);
  const float meanf = static_cast<float>(mean);
  const float inv = static_cast<float>(1.0 / sqrt(var + 1e-5));
  const float scale = inv * gam;
#pragma unroll
  for (int t = 0; t < H; ++t) hv[t] = mish_fast(fmaf(hv[t] - meanf, scale, bet));
  float* ep = op.epart + (static_cast<std::int64_t>(b) * kSplitGroups + g) * A * H;
  for (int a0 = 0; a0 < A; a0 += AG) {
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.0f;
#pragma unroll
    for (int aa = 0; aa < AG; ++aa) {
      const int a = a0 + aa;
      const float w = a0 == 0 ? w0[aa]
                              : (a < A ? op.wo[static_cast<std::int64_t>(a) * C + c] : 0.0f);
#pragma unroll
      for (int t = 0; t < H; ++t) acc[aa * H + t] = fmaf(w, hv[t], acc[aa * H + t]);
    }
    rs_step<V, 32>(acc, lane);
    const int off = rs_offset<V>(lane);
    if (rs_writer<V>(lane) && a0 * H + off < A * H) st_dev(ep + a0 * H + off, acc[0]);
  }
  // Publish once the partials have reached the device's coherence point.
  wait_vmem();
  unsigned before = 0;
  if (lane == 0)
    before = __hip_atomic_fetch_add(global_ptr(op.done + b), 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
  before = __builtin_amdgcn_readfirstlane(before);
  if (before != kSplitGroups - 1) return;
  if (lane == 0) st_dev(op.done + b, 0u);
  const float* e0 = op.epart + static_cast<std::int64_t>(b) * kSplitGroups * A * H;
  for (int i = lane; i < A * H; i += kWave) {
    float e = 0.0f;
#pragma unroll
    for (int gg = 0; gg < kSplitGroups; ++gg) e += ld_dev(e0 + gg * A * H + i);
    const int a = i / H, t = i % H;
    const float xv = op.kind != kUpdateDenoise ? op.x[sample + i] : 0.0f;
    upd::apply_update<false>(op, sample, gridDim.x / kSplitGroups, a, t, A, H, e + op.bo[a], xv);
  }
}

// Shapes outside update_kernel's instances: one wavefront per output value eps[a][t] (lanes
// stride the c0 channels), the group statistics first (fp64, one wavefront per group).
constexpr int kUpdGenThreads = 256;
constexpr int kMaxUpdGenGroups = 64;

__global__ __launch_bounds__(kUpdGenThreads) void update_general_kernel(UpdateOp op) {
  __shared__ float gmean[kMaxUpdGenGroups], ginv[kMaxUpdGenGroups];
  const int b = blockIdx.x;
  const int A = op.action_dim, C = op.c0, H = op.horizon;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  constexpr int kWaves = kUpdGenThreads / kWave;
  const float* hb = op.h + b * (op.hstride != 0 ? op.hstride : static_cast<std::int64_t>(C) * H);
  const int cpg = C / op.groups;
  const int n = cpg * H;
  for (int g = wave; g < op.groups; g += kWaves) {
    double s = 0.0, q = 0.0;
    for (int i = lane; i < n; i += kWave) {
      const double d = static_cast<double>(hb[static_cast<std::int64_t>(g) * n + i]);
      s += d;
      q += d * d;
    }
    s = wave_sum(s);
    q = wave_sum(q);
    if (lane == 0) {
      const double cnt = static_cast<double>(n);
      const double mean = s / cnt;
      const double var = fmax(0.0, q / cnt - mean * mean);
      gmean[g] = static_cast<float>(mean);
      ginv[g] = static_cast<float>(1.0 / sqrt(var + 1e-5));
    }
  }
  __syncthreads();
  const std::int64_t sample = static_cast<std::int64_t>(b) * A * H;
  for (int o = wave; o < A * H; o += kWaves) {
    const int a = o / H, t = o % H;
    const float* wr = op.wo + static_cast<std::int64_t>(a) * C;
    float p = 0.0f;
    for (int c = lane; c < C; c += kWave) {
      const int g = c / cpg;
      const float v = mish_fast(
          fmaf(hb[static_cast<std::int64_t>(c) * H + t] - gmean[g], ginv[g] * op.gamma[c], op.beta[c]));
      p = fmaf(wr[c], v, p);
    }
#pragma unroll
    for (int m = kWave / 2; m >= 1; m >>= 1) p += __shfl_xor(p, m, kWave);
    if (lane == 0) {
      const float xv = op.kind != kUpdateDenoise ? op.x[sample + o] : 0.0f;
      upd::apply_update<false>(op, sample, gridDim.x, a, t, A, H, p + op.bo[a], xv);
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

hipError_t time_mlp(const TimeSpec& times, int count, const float* w1, const float* b1,
                    const float* w2, const float* b2, int tdim, float* m, hipStream_t stream) {
  const size_t smem = static_cast<size_t>(5 * tdim) * sizeof(float);
  if (tdim <= 0 || smem > kMaxTimeMlpLds) return hipErrorInvalidValue;
  static bool raised = false;
  if (!raised && smem > 64 * 1024) {
    const hipError_t st = hipFuncSetAttribute(reinterpret_cast<const void*>(time_mlp_kernel),
                                              hipFuncAttributeMaxDynamicSharedMemorySize,
                                              static_cast<int>(kMaxTimeMlpLds));
    if (st != hipSuccess) return st;
    raised = true;
  }
  hipLaunchKernelGGL(time_mlp_kernel, dim3(count), dim3(kBlock), smem, stream, times, w1, b1, w2,
                     b2, tdim, m);
  return hipGetLastError();
}

hipError_t film_gemm(const float* in, std::int64_t in_stride, int n, int kdim, const float* wt,
                     const float* bias, int fdim, bool mish_in, float* out,
                     std::int64_t out_stride, hipStream_t stream) {
  const dim3 grid((fdim + kWave - 1) / kWave, (n + kFilmRows - 1) / kFilmRows);
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

namespace {
bool update_fused_ok(int c0, int groups, int horizon, int action_dim) {
  return c0 <= upd::kUpdThreads * upd::kMaxUpdateChannelsPerLane && groups <= upd::kMaxUpdateGroups &&
         action_dim <= upd::kMaxActions &&
         (horizon == 1 || horizon == 2 || horizon == 4 || horizon == 8 || horizon == 16);
}
}  // namespace

int update_max_parts(int c0) {
  return c0 <= upd::kUpdThreads ? upd::kMaxUpdateParts : upd::kMaxUpdateParts / 2;
}

bool update_fused(int c0, int groups, int horizon, int action_dim) {
  return update_fused_ok(c0, groups, horizon, action_dim);
}

hipError_t update(const UpdateOp& op, int batch, hipStream_t stream) {
  if (batch <= 0 || op.c0 <= 0 || op.groups <= 0 || op.groups > kMaxUpdGenGroups ||
      op.c0 % op.groups != 0 || op.action_dim <= 0 || op.horizon <= 0)
    return hipErrorInvalidValue;
  // Partial sums of h (sliced final convolution) only on the fused kernel, up to its maximum.
  if (op.hparts < 1 || op.hparts > update_max_parts(op.c0) ||
      (op.hparts > 1 && !update_fused_ok(op.c0, op.groups, op.horizon, op.action_dim)))
    return hipErrorInvalidValue;
  if (!update_fused_ok(op.c0, op.groups, op.horizon, op.action_dim)) {
    hipLaunchKernelGGL(update_general_kernel, dim3(batch), dim3(kUpdGenThreads), 0, stream, op);
    return hipGetLastError();
  }
  if (op.done != nullptr && op.epart != nullptr && op.c0 == kSplitChannels &&
      op.groups == kSplitGroups && op.horizon <= kWave && batch <= kSplitMaxBatch) {
    const dim3 grid(static_cast<unsigned>(batch * kSplitGroups));
    switch (op.horizon) {
      case 1: hipLaunchKernelGGL(update_split_kernel<1>, grid, dim3(kWave), 0, stream, op); break;
      case 2: hipLaunchKernelGGL(update_split_kernel<2>, grid, dim3(kWave), 0, stream, op); break;
      case 4: hipLaunchKernelGGL(update_split_kernel<4>, grid, dim3(kWave), 0, stream, op); break;
      case 8: hipLaunchKernelGGL(update_split_kernel<8>, grid, dim3(kWave), 0, stream, op); break;
      default: hipLaunchKernelGGL(update_split_kernel<16>, grid, dim3(kWave), 0, stream, op); break;
    }
    return hipGetLastError();
  }
  if (op.c0 <= upd::kUpdThreads) {
    switch (op.horizon) {
      case 1: hipLaunchKernelGGL((update_kernel<1, 1>), dim3(batch), dim3(upd::kUpdThreads), 0, stream, op); break;
      case 2: hipLaunchKernelGGL((update_kernel<2, 1>), dim3(batch), dim3(upd::kUpdThreads), 0, stream, op); break;
      case 4: hipLaunchKernelGGL((update_kernel<4, 1>), dim3(batch), dim3(upd::kUpdThreads), 0, stream, op); break;
      case 8: hipLaunchKernelGGL((update_kernel<8, 1>), dim3(batch), dim3(upd::kUpdThreads), 0, stream, op); break;
      default: hipLaunchKernelGGL((update_kernel<16, 1>), dim3(batch), dim3(upd::kUpdThreads), 0, stream, op); break;
    }
    return hipGetLastError();
  }
  switch (op.horizon) {
    case 1: hipLaunchKernelGGL((update_kernel<1, 2>), dim3(batch), dim3(upd::kUpdThreads), 0, stream, op); break;
    case 2: hipLaunchKernelGGL((update_kernel<2, 2>), dim3(batch), dim3(upd::kUpdThreads), 0, stream, op); break;
    case 4: hipLaunchKernelGGL((update_kernel<4, 2>), dim3(batch), dim3(upd::kUpdThreads), 0, stream, op); break;
    case 8: hipLaunchKernelGGL((update_kernel<8, 2>), dim3(batch), dim3(upd::kUpdThreads), 0, stream, op); break;
    default: hipLaunchKernelGGL((update_kernel<16, 2>), dim3(batch), dim3(upd::kUpdThreads), 0, stream, op); break;
  }
  return hipGetLastError();
}

hipError_t finish_sample(const float* x, const float* amin, const float* amax, float* action,
                         int batch, int horizon, int action_dim, hipStream_t stream) {
  hipLaunchKernelGGL(finish_kernel, dim3(batch), dim3(kBlock), 0, stream, x, amin, amax, action,
                     horizon, action_dim);
  return hipGetLastError();
}

}  // namespace fe::hip
