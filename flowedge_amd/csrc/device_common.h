// Device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace fe::hip::dev {

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

// Same identity with the hardware exp2 (v_exp_f32) and reciprocal (v_rcp_f32), each about 1 ULP:
// the prologue form, where every workgroup transforms a whole activation tensor.  Branch-free
// (the exponent is clamped and the large-v case selected), so a wavefront never splits on it.
__device__ __forceinline__ float mish_fast(float v) {
  const float e = __builtin_amdgcn_exp2f(fminf(v, 20.0f) * 1.44269504088896341f);
  const float n = e * (e + 2.0f);
  const float m = v * n * __builtin_amdgcn_rcpf(n + 2.0f);
  return v > 20.0f ? v : m;
}

__device__ __forceinline__ float bf16_to_f32(unsigned short bits) {
  return __uint_as_float(static_cast<unsigned>(bits) << 16);
}

// Device-coherent accesses for data that workgroups of one running kernel hand to each other
// (the persistent tick kernel): relaxed agent-scope atomics, which gfx950 performs as loads and
// stores with the sc1 (device scope) cache policy, read and write at the device's coherence
// point, so no XCD's L2 or CU's L1 serves a stale copy and no whole-cache write-back or
// invalidation is needed.
// Global (address space 1) views of generic pointers, so the accesses compile to global_*
// instructions rather than flat ones (which would also hold the LDS wait counter).
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* global_ptr(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(global_ptr(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(global_ptr(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_dev(const unsigned* p) {
  return __hip_atomic_load(global_ptr(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(unsigned* p, unsigned v) {
  __hip_atomic_store(global_ptr(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16-byte accesses as two 8-byte device-scope atomics (per-lane addresses, 8-byte aligned).
__device__ __forceinline__ float4 ld4_dev(const float* p) {
  const auto* q = global_ptr(reinterpret_cast<const unsigned long long*>(p));
  const unsigned long long lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return float4{__uint_as_float(static_cast<unsigned>(lo)),
                __uint_as_float(static_cast<unsigned>(lo >> 32)),
                __uint_as_float(static_cast<unsigned>(hi)),
                __uint_as_float(static_cast<unsigned>(hi >> 32))};
}
__device__ __forceinline__ void st4_dev(float* p, float4 v) {
  auto* q = global_ptr(reinterpret_cast<unsigned long long*>(p));
  const unsigned long long lo = static_cast<unsigned long long>(__float_as_uint(v.x)) |
                                (static_cast<unsigned long long>(__float_as_uint(v.y)) << 32);
  const unsigned long long hi = static_cast<unsigned long long>(__float_as_uint(v.z)) |
                                (static_cast<unsigned long long>(__float_as_uint(v.w)) << 32);
  __hip_atomic_store(q, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(q + 1, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until every earlier vector memory access of this wavefront has completed (stores
// acknowledged by the device-coherent level).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// The value `v` of this lane's exchange partner for bit MASK, through VALU cross-lane moves: DPP
// quad_perm (lane ^ 1, lane ^ 2), DPP row_ror 8 (lane ^ 8 within a 16-lane row) and the gfx950
// permlane16 / permlane32 swaps (lane ^ 16, lane ^ 32).  For MASK 4 the partner is lane ^ 7 within
// its 8-lane group (DPP row_half_mirror): it flips bit 2 and keeps the higher bits, which is all
// the reductions below need.
template <int MASK>
__device__ __forceinline__ float partner(float v, int lane) {
  const unsigned u = __float_as_uint(v);
  unsigned r;
  if constexpr (MASK == 1) {
    r = __builtin_amdgcn_update_dpp(0u, u, 0xb1, 0xf, 0xf, false);
  } else if constexpr (MASK == 2) {
    r = __builtin_amdgcn_update_dpp(0u, u, 0x4e, 0xf, 0xf, false);
  } else if constexpr (MASK == 4) {
    r = __builtin_amdgcn_update_dpp(0u, u, 0x141, 0xf, 0xf, false);
  } else if constexpr (MASK == 8) {
    r = __builtin_amdgcn_update_dpp(0u, u, 0x128, 0xf, 0xf, false);
  } else if constexpr (MASK == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    r = (lane & 16) ? p[0] : p[1];
  } else {
    static_assert(MASK == 32, "exchange bits 1 to 32");
    const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    r = (lane & 32) ? p[0] : p[1];
  }
  return __uint_as_float(r);
}

// Wavefront reduce-scatter.  On entry every lane holds N partial sums v[0..N); on exit lane l
// holds max(N/64, 1) finished sums (over all 64 lanes) of the original indices
// [rs_offset<N>(l), +max(N/64,1)).  Each halving step exchanges half of the remaining values with
// the partner lane (see partner: it differs in the step's bit, shares the higher ones); once one
// value remains, plain butterfly steps finish it.
template <int N, int MASK>
__device__ __forceinline__ void rs_step(float* v, int lane) {
  if constexpr (MASK > 0) {
    if constexpr (N >= 2) {
      const bool upper = (lane & MASK) != 0;
#pragma unroll
      for (int i = 0; i < N / 2; ++i) {
        const float send = upper ? v[i] : v[i + N / 2];
        const float keep = upper ? v[i + N / 2] : v[i];
        v[i] = keep + partner<MASK>(send, lane);
      }
      rs_step<N / 2, MASK / 2>(v, lane);
    } else {
      v[0] += partner<MASK>(v[0], lane);
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

// The same for a reduce-scatter confined to SEG-lane segments (rs_step<N, SEG / 2>, N <= SEG):
// the index of the finished sum a lane holds, and whether the lane is its segment's writer of it.
template <int N, int SEG>
__device__ __forceinline__ int rs_offset_seg(int lane) {
  int off = 0, n = N;
#pragma unroll
  for (int m = SEG / 2; m >= 1; m >>= 1) {
    if (n >= 2) {
      if (lane & m) off += n / 2;
      n /= 2;
    }
  }
  return off;
}
template <int N, int SEG>
__device__ __forceinline__ bool rs_writer_seg(int lane) {
  if constexpr (N >= SEG) {
    return true;
  } else {
    return (lane & (SEG / N - 1)) == 0;
  }
}

// v + (v of lane l ^ 1), (l ^ 2), rotations by 4 and 8 within each 16-lane row, through DPP
// moves of the two 32-bit halves (no LDS round trip).
template <int CTRL>
__device__ __forceinline__ double dpp_add(double v) {
  const long long bits = __builtin_bit_cast(long long, v);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(bits), CTRL, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(bits >> 32), CTRL, 0xf, 0xf, false);
  const long long moved = (static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo);
  return v + __builtin_bit_cast(double, moved);
}

__device__ __forceinline__ double lane_value(double v, int lane) {
  const long long bits = __builtin_bit_cast(long long, v);
  const int lo = __builtin_amdgcn_readlane(static_cast<int>(bits), lane);
  const int hi = __builtin_amdgcn_readlane(static_cast<int>(bits >> 32), lane);
  return __builtin_bit_cast(double, (static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo));
}

// Sum over each 16-lane row, returned to every lane of the row: DPP quad_perm xor 1, xor 2, then
// row_ror 4 and row_ror 8.
__device__ __forceinline__ double row_sum(double v) {
  v = dpp_add<0xb1>(v);
  v = dpp_add<0x4e>(v);
  v = dpp_add<0x124>(v);
  return dpp_add<0x128>(v);
}

// Sum over the 64 lanes of a wavefront, returned to every lane: the four row sums, read out.
__device__ __forceinline__ double wave_sum(double v) {
  v = row_sum(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

}  // namespace fe::hip::dev
