// The final GroupNorm + Mish + 1x1 conv with the sampler update (DDIM / DDPM / flow-ODE) of one
// sample, shared by the stand-alone update kernel and the persistent tick kernel.
//
// Reference semantics: final conv block diffusion.cc:895-913, DDIM/DDPM :995-1024, the seeded
// Gaussian stream :193-231, flow updates span_ops.h:27-52 / flow.cc:291-318.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.h"
#include "kernels.h"

namespace fe::hip::upd {

using namespace dev;

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

// The sampler update of state value (a, t) (state layout [A][H]) from the U-Net output e and
// the current state xv (diffusion.cc:995-1024, flow.cc:291-318); `batch` samples per plane of
// the flow stage buffers.  CHAIN: the state is exchanged device-coherently.
template <bool CHAIN>
__device__ __forceinline__ void apply_update(const UpdateOp& op, std::int64_t sample, int batch,
                                             int a, int t, int A, int H, float e, float xv,
                                             float* state = nullptr) {
  const std::int64_t si = sample + static_cast<std::int64_t>(a) * H + t;
  // CHAIN: the workgroup's slot (x, xin, k0 .. k3) replaces the op's state buffers.
  float* const x = CHAIN ? state : op.x;
  float* const xin = CHAIN ? state + A * H : op.xin;
  float* const kbuf = CHAIN ? state + 2 * A * H : op.kbuf;
  auto put = [](float* p, float v) {
    if constexpr (CHAIN) st_dev(p, v);
    else *p = v;
  };
  auto get = [](const float* p) {
    if constexpr (CHAIN) return ld_dev(p);
    else return *p;
  };
  switch (op.kind) {
    case kUpdateDenoise:
      put(op.out + sample + static_cast<std::int64_t>(t) * A + a, e);
      break;
    case kUpdateDDIM: {
      float x0 = (xv - op.sqrt_bt * e) / op.sqrt_at;
      if (op.clip) x0 = fminf(fmaxf(x0, -op.clip_range), op.clip_range);
      const float nx = op.sqrt_ap * x0 + op.sqrt_1map * e;
      put(x + si, nx);
      if (xin != x) put(xin + si, nx);
      break;
    }
    case kUpdateDDPM: {
      float x0 = (xv - op.sqrt_bt * e) / op.sqrt_at;
      if (op.clip) x0 = fminf(fmaxf(x0, -op.clip_range), op.clip_range);
      float nx = op.coef_x0 * x0 + op.coef_x * xv;
      if (op.add_noise)
        nx += op.sigma *
              stream_gaussian(*op.seed, op.noise_offset + static_cast<std::uint64_t>(t) * A + a);
      put(x + si, nx);
      if (xin != x) put(xin + si, nx);
      break;
    }
    case kUpdateEuler: {
      const float nx = xv + op.dt * e;
      put(x + si, nx);
      put(xin + si, nx);
      break;
    }
    case kUpdateStage: {
      const std::int64_t plane = static_cast<std::int64_t>(batch) * A * H;
      put(kbuf + op.slot * plane + si, e);
      put(xin + si, xv + op.dt * e);
      break;
    }
    case kUpdateHeun: {
      const float k1 = get(kbuf + si);
      const float nx = xv + 0.5f * op.dt * (k1 + e);
      put(x + si, nx);
      put(xin + si, nx);
      break;
    }
    case kUpdateRK4: {
      const std::int64_t plane = static_cast<std::int64_t>(batch) * A * H;
      const float k1 = get(kbuf + si), k2 = get(kbuf + plane + si),
                  k3 = get(kbuf + 2 * plane + si);
      const float nx = xv + (op.dt / 6.0f) * (k1 + 2.0f * k2 + 2.0f * k3 + e);
      put(x + si, nx);
      put(xin + si, nx);
      break;
    }
    default:
      break;
  }
}

constexpr int kUpdThreads = 512;
constexpr int kMaxUpdateChannelsPerLane = 2;  // c0 <= 1024
// Partial sums of a sliced final convolution the update adds: 8 channel-rows of loads per lane
// (kMaxUpdateParts / CPL partials at CPL channels per lane).
constexpr int kMaxUpdateParts = 8;
constexpr int kMaxUpdateGroups = 32;
constexpr int kMaxActions = 64;

template <int H>
struct UpdateSmem {
  static constexpr int AG = H >= kWave ? 1 : kWave / H;  // actions per reduction pass
  static constexpr int V = AG * H;
  double ps[kUpdThreads * kMaxUpdateChannelsPerLane];
  double pq[kUpdThreads * kMaxUpdateChannelsPerLane];
  float gmean[kMaxUpdateGroups], ginv[kMaxUpdateGroups];
  float red[kUpdThreads / kWave][V];
  float eps[kMaxActions][H];
};

// Sample b of `batch`, by one 512-lane workgroup.  Lane l owns channels l and l + 512 (H
// positions each, loaded as 16-byte vectors); the workgroup reduces the GroupNorm statistics
// (fp64), applies GN + Mish, and forms the 1x1 conv's partial sums for up to 64 / H actions at a
// time, folded by one wavefront reduce-scatter and one LDS pass per action group.  The update
// then runs on the A*H state values.  CHAIN: the final conv output and the state were written by
// other workgroups of the same launch and are read device-coherently.
// `state` (CHAIN): the workgroup's own state slot, x, xin and the four flow stages (`values`
// floats each), used instead of op.x / op.xin / op.kbuf.
// CPL: channels per lane (c0 <= 512 * CPL).
template <int H, bool CHAIN, int CPL = kMaxUpdateChannelsPerLane>
__device__ __forceinline__ void update_body(const UpdateOp& op, int b, int batch,
                                            UpdateSmem<H>& sm, float* state = nullptr) {
  static_assert(CPL >= 1 && CPL <= kMaxUpdateChannelsPerLane, "channels per lane");
  constexpr int PM = kMaxUpdateParts / CPL;  // partials summed
  constexpr int AG = UpdateSmem<H>::AG;
  constexpr int V = UpdateSmem<H>::V;
  double* ps = sm.ps;
  double* pq = sm.pq;
  float* gmean = sm.gmean;
  float* ginv = sm.ginv;
  auto& red = sm.red;
  auto& eps = sm.eps;
  const int A = op.action_dim, C = op.c0;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  const std::int64_t sample = static_cast<std::int64_t>(b) * A * H;
  const float* hb = op.h + b * (op.hstride != 0 ? op.hstride : static_cast<std::int64_t>(C) * H);

  // Reads that do not depend on the statistics are issued first, so their latency overlaps the
  // reduction: the output conv's weights for the first action group and the sampler state.
  constexpr int XPL = (kMaxActions * H + kUpdThreads - 1) / kUpdThreads;  // state values per lane
  float w0[AG][CPL];
#pragma unroll
  for (int aa = 0; aa < AG; ++aa)
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = tid + i * kUpdThreads;
      w0[aa][i] = c < C && aa < A ? op.wo[static_cast<std::int64_t>(aa) * C + c] : 0.0f;
    }
  float xs[XPL];
#pragma unroll
  for (int r = 0; r < XPL; ++r) {
    const int i = tid + r * kUpdThreads;
    xs[r] = 0.0f;
    if (op.kind != kUpdateDenoise && i < A * H)
      xs[r] = CHAIN ? ld_dev(state + i) : op.x[sample + i];
  }

  float hv[CPL][H];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = tid + i * kUpdThreads;
    const float* p = hb + static_cast<std::int64_t>(c) * H;
    if constexpr (CHAIN) {
      if constexpr (H >= 4) {
#pragma unroll
        for (int t = 0; t < H; t += 4) {
          const float4 v = c < C ? ld4_dev(p + t) : float4{0, 0, 0, 0};
          hv[i][t] = v.x;
          hv[i][t + 1] = v.y;
          hv[i][t + 2] = v.z;
          hv[i][t + 3] = v.w;
        }
      } else {
#pragma unroll
        for (int t = 0; t < H; ++t) hv[i][t] = c < C ? ld_dev(p + t) : 0.0f;
      }
    } else {
      // Sum of the op.hparts partials, in order, with every load issued before the first add.
      float pv[PM][H];
#pragma unroll
      for (int j = 0; j < PM; ++j) {
        const float* pj = p + j * op.hpart;
        const bool on = c < C && j < op.hparts;
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
#pragma unroll
      for (int t = 0; t < H; ++t) {
        float v = pv[0][t];
#pragma unroll
        for (int j = 1; j < PM; ++j)
          if (j < op.hparts) v += pv[j][t];
        hv[i][t] = v;
      }
    }
    double s = 0.0, q = 0.0;
#pragma unroll
    for (int t = 0; t < H; ++t) {
      const double d = static_cast<double>(hv[i][t]);
      s += d;
      q += d * d;
    }
    if (c < C) {
      ps[c] = s;
      pq[c] = q;
    }
  }
  __syncthreads();
  const int cpg = C / op.groups;
  for (int g = wave; g < op.groups; g += kUpdThreads / kWave) {
    double s = 0.0, q = 0.0;
    for (int i = lane; i < cpg; i += kWave) {
      s += ps[g * cpg + i];
      q += pq[g * cpg + i];
    }
    s = wave_sum(s);
    q = wave_sum(q);
    if (lane == 0) {
      const double n = static_cast<double>(cpg) * H;
      const double mean = s / n;
      const double var = fmax(0.0, q / n - mean * mean);
      gmean[g] = static_cast<float>(mean);
      ginv[g] = static_cast<float>(1.0 / sqrt(var + 1e-5));
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = tid + i * kUpdThreads;
    if (c < C) {
      const int g = c / cpg;
      const float scale = ginv[g] * op.gamma[c];
      const float shift = op.beta[c];
      const float mean = gmean[g];
#pragma unroll
      for (int t = 0; t < H; ++t) hv[i][t] = mish_fast(fmaf(hv[i][t] - mean, scale, shift));
    }
  }
  for (int a0 = 0; a0 < A; a0 += AG) {
    float p[V];
#pragma unroll
    for (int v = 0; v < V; ++v) p[v] = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = tid + i * kUpdThreads;
      if (c < C) {
#pragma unroll
        for (int aa = 0; aa < AG; ++aa) {
          const int a = a0 + aa;
          const float w = a0 == 0 ? w0[aa][i]
                                  : (a < A ? op.wo[static_cast<std::int64_t>(a) * C + c] : 0.0f);
#pragma unroll
          for (int t = 0; t < H; ++t) p[aa * H + t] = fmaf(w, hv[i][t], p[aa * H + t]);
        }
      }
    }
    rs_step<V, 32>(p, lane);
    const int off = rs_offset<V>(lane);
    if (rs_writer<V>(lane)) red[wave][off] = p[0];
    __syncthreads();
    if (tid < V) {
      float s = 0.0f;
      for (int w = 0; w < kUpdThreads / kWave; ++w) s += red[w][tid];
      const int a = a0 + tid / H;
      if (a < A) eps[a][tid % H] = s + op.bo[a];
    }
    __syncthreads();
  }

#pragma unroll
  for (int r = 0; r < XPL; ++r) {
    const int i = tid + r * kUpdThreads;
    if (i >= A * H) break;
    apply_update<CHAIN>(op, sample, batch, i / H, i % H, A, H, eps[i / H][i % H], xs[r], state);
  }
}


}  // namespace fe::hip::upd
