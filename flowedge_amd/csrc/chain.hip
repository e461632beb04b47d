// Persistent tick kernel: a whole B=1 sampling tick (every convolution of every U-Net evaluation
// plus the sampler updates) in one launch of one workgroup per CU.
//
// Why: at batch 1 each convolution streams its weights once, and a dependent kernel launch costs
// ~2-3.5 us of dead time on this GPU (teardown, dispatch, ramp) in which no weight moves.  Here
// the next step's workgroups request their first weights *before* they wait for the previous
// step, so the weight stream continues across layer boundaries.
//
// Hand-off: a step's outputs are written with device-scope (sc1) stores; each workgroup then
// waits for its stores to complete (vmcnt(0)), meets its other wavefronts at a barrier and
// publishes the number of steps it has finished in its own 256-byte counter.  A consumer's 256
// lanes each poll one counter (sc1 loads) until every workgroup has finished the previous step,
// then read the input with sc1 loads.  No whole-L2 write-back or invalidation is involved, and
// workgroups only ever wait for earlier steps, so the wait always ends while all workgroups are
// resident; a bounded poll count guards against a workgroup that never started (another
// process on the GPU): the tick is then abandoned and reported through `abort`.
//
// The convolution body is conv_kernel.h's (CHAIN mode); the update is update_body.h's, computed by
// every workgroup into its own state slot.  Reference semantics as there: diffusion.cc:724-1035,
// diffusion_ops.cc:82-377, flow.cc:291-318.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

#include "conv_kernel.h"
#include "kernels.h"
#include "update_body.h"

namespace fe::hip {
namespace chain {

using namespace conv;

struct Step {
  Args a;
  int variant;  // index into the variant table
  int film;     // FiLM time rows of the evaluation
  int state;    // input from the workgroup's state slot
};

// The fused-convolution instances the tick kernel carries: (MODE, K, LIN, VEC, PRO, RES, NC) of
// every convolution of the F32 U-Nets with horizon 16 (LeRobot pusht-size and its flow head, and
// the 64/128/256-wide test model).
#define FE_CHAIN_VARIANTS(X)      \
  X(0, 5, 16, 1, 0, true, 1)      \
  X(0, 5, 16, 4, 0, false, 1)     \
  X(0, 5, 16, 4, 1, false, 1)     \
  X(0, 5, 16, 4, 2, false, 1)     \
  X(1, 3, 16, 4, 2, false, 1)     \
  X(0, 5, 8, 4, 0, true, 1)       \
  X(0, 5, 8, 4, 0, true, 2)       \
  X(0, 5, 8, 4, 1, false, 1)      \
  X(0, 5, 8, 4, 1, false, 2)      \
  X(0, 5, 8, 4, 2, false, 1)      \
  X(0, 5, 8, 4, 2, false, 2)      \
  X(1, 3, 8, 4, 2, false, 1)      \
  X(1, 3, 8, 4, 2, false, 2)      \
  X(2, 4, 8, 4, 2, false, 1)      \
  X(0, 5, 4, 4, 0, true, 1)       \
  X(0, 5, 4, 4, 0, true, 4)       \
  X(0, 5, 4, 4, 1, false, 1)      \
  X(0, 5, 4, 4, 1, false, 2)      \
  X(0, 5, 4, 4, 1, false, 4)      \
  X(0, 5, 4, 4, 2, false, 1)      \
  X(0, 5, 4, 4, 2, false, 2)      \
  X(0, 5, 4, 4, 2, false, 4)      \
  X(0, 5, 4, 4, 2, true, 1)       \
  X(0, 5, 4, 4, 2, true, 4)       \
  X(2, 4, 4, 4, 2, false, 1)      \
  X(2, 4, 4, 4, 2, false, 2)

struct Key {
  int mode, k, lin, vec, pro;
  bool res;
  int nc;
};
#define FE_CHAIN_KEY(MODE, K, LIN, VEC, PRO, RES, NC) Key{MODE, K, LIN, VEC, PRO, RES, NC},
constexpr Key kKeys[] = {FE_CHAIN_VARIANTS(FE_CHAIN_KEY)};
#undef FE_CHAIN_KEY
constexpr int kVariants = sizeof(kKeys) / sizeof(kKeys[0]);

// The hand-off words of a tick, copied out of the kernel argument (a generic reference to the
// argument itself would place a copy of it in private memory).
struct Sync {
  unsigned* flags;
  unsigned* abort;
  long long spin_limit;
};

// Waits until every workgroup has finished `target` steps (false if the tick is abandoned).
// Called by all lanes of the workgroup.
__device__ bool wait_all(Sync y, unsigned target, int* s_abort) {
  const int tid = threadIdx.x;
  if (tid < kChainGrid) {
    const unsigned* f = y.flags + tid * kChainFlagStride;
    long long polls = 0;
    while (ld_dev(f) < target) {
      if ((++polls & 63) == 0 && (polls > y.spin_limit || ld_dev(y.abort) != 0)) {
        st_dev(y.abort, 1u);
        *s_abort = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
  return *s_abort == 0;
}

// Publishes that this workgroup has finished `done` steps, once all its stores have completed.
__device__ void signal(Sync y, unsigned done) {
  wait_vmem();
  __syncthreads();
  if (threadIdx.x == 0) st_dev(y.flags + blockIdx.x * kChainFlagStride, done);
}

struct ChainWait {
  Sync y;
  unsigned target;
  int* s_abort;
  bool on;
  __device__ bool operator()() const { return on ? wait_all(y, target, s_abort) : true; }
};

__device__ __forceinline__ bool run_step(const Step& st, int wg, float* xs, float* gmean,
                                         float* ginv, float* red, const ChainWait& wait,
                                         Override ov) {
  switch (st.variant) {
#define FE_CHAIN_CASE(MODE, K, LIN, VEC, PRO, RES, NC)                                          \
  case __COUNTER__ - kBase:                                                                     \
    return conv_body<MODE, K, LIN, VEC, PRO, RES, false, NC, true>(st.a, wg, 0, xs, gmean, ginv, \
                                                                   red, wait, ov);
    enum { kBase = __COUNTER__ + 1 };
    FE_CHAIN_VARIANTS(FE_CHAIN_CASE)
#undef FE_CHAIN_CASE
    default:
      return false;
  }
}

// Read-only views of the step and evaluation tables (constant address space): the compiler then
// knows the kernel's own stores cannot change them, so their fields stay in scalar registers or
// the scalar cache across the stores of a step.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(4))) T* constant_ptr(const void* p) {
  return (const __attribute__((address_space(4))) T*)p;
}

template <int H>
__global__ __launch_bounds__(kThreads) void tick_kernel(ChainTick t) {
  __shared__ float4 xs4[(kMaxStageBytes + 15) / 16];
  __shared__ float gmean[kMaxGroups], ginv[kMaxGroups];
  __shared__ float red[2 * (kThreads / kWave) * kWave];
  __shared__ int s_abort;
  static_assert(sizeof(upd::UpdateSmem<H>) <= sizeof(xs4), "update aliases the staging buffer");
  float* xs = reinterpret_cast<float*>(xs4);
  auto& usm = *reinterpret_cast<upd::UpdateSmem<H>*>(xs4);
  const int wg = blockIdx.x, tid = threadIdx.x;
  if (tid == 0) s_abort = 0;
  const Sync y{t.flags, t.abort, t.spin_limit};
  const auto* steps = constant_ptr<Step>(t.steps);
  const auto* evals = constant_ptr<ChainEval>(t.evals);
  float* sx = t.slots + static_cast<std::int64_t>(wg) * t.slot_floats;
  float* sxin = sx + t.values;
  for (int i = tid; i < t.values; i += kThreads) {
    st_dev(sx + i, t.x0[i]);
    st_dev(sxin + i, t.xin0[i]);
  }
  wait_vmem();
  __syncthreads();
  unsigned done = 0;  // steps this workgroup has finished
  for (int e = 0; e < t.nevals; ++e) {
    const ChainEval& ev = *(const ChainEval*)(evals + e);
    for (int s = 0; s < t.nsteps; ++s) {
      const Step& st = *(const Step*)(steps + s);
      Override ov;
      ov.film_time = st.film ? ev.film_row : nullptr;
      ov.src = st.state ? sxin : nullptr;
      // The first convolution of an evaluation reads only this workgroup's slot.
      const ChainWait wait{y, done, &s_abort, s != 0};
      if (wg < st.a.blocks && !run_step(st, wg, xs, gmean, ginv, red, wait, ov)) return;
      signal(y, ++done);
    }
    // Every workgroup: wait for the final convolution, then update its own copy of the state.
    if (!wait_all(y, done, &s_abort)) return;
    upd::update_body<H, true>(ev.upd, 0, 1, usm, sx);
    wait_vmem();
    __syncthreads();
  }
  if (wg == 0)
    for (int i = tid; i < t.values; i += kThreads) t.x_out[i] = ld_dev(sx + i);
}

__global__ void reset_kernel(unsigned* flags, unsigned* abort) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < kChainGrid) flags[i * kChainFlagStride] = 0;
  if (i == 0) *abort = 0;
}

}  // namespace chain

std::size_t chain_step_bytes() { return sizeof(chain::Step); }

bool chain_supported_horizon(int horizon) { return horizon == 16; }

bool chain_build(const ChainConv* convs, int n, void* steps, const char** why) {
  using namespace chain;
  if (n <= 0 || n > kMaxChainSteps) {
    *why = "step count";
    return false;
  }
  auto* out = static_cast<Step*>(steps);
  for (int i = 0; i < n; ++i) {
    const ChainConv& c = convs[i];
    Step st;
    std::memset(&st, 0, sizeof st);
    int vec = 4, pro = 0;
    if (!conv::fused_args(c.op, c.has_res ? &c.res : nullptr, c.in, c.y, c.yr, 1, st.a, vec,
                          pro)) {
      *why = "a convolution has no fused batch-1 plan";
      return false;
    }
    if (st.a.bf16 || (c.has_res && st.a.rbf16)) {
      *why = "BF16 convolution weights";
      return false;
    }
    if (st.a.blocks > kChainGrid) {
      *why = "a plan wider than the grid";
      return false;
    }
    const Key key{c.op.mode, c.op.k, c.op.lin, vec, pro, c.has_res,
                  conv::instance_nc(c.op.k, c.op.lin, c.has_res, vec, st.a.nch)};
    st.variant = -1;
    for (int v = 0; v < kVariants; ++v)
      if (kKeys[v].mode == key.mode && kKeys[v].k == key.k && kKeys[v].lin == key.lin &&
          kKeys[v].vec == key.vec && kKeys[v].pro == key.pro && kKeys[v].res == key.res &&
          kKeys[v].nc == key.nc)
        st.variant = v;
    if (st.variant < 0) {
      *why = "a convolution shape outside the tick kernel's variants";
      return false;
    }
    st.film = c.film ? 1 : 0;
    st.state = c.state ? 1 : 0;
    out[i] = st;
  }
  return true;
}

hipError_t chain_tick(const ChainTick& t, hipStream_t stream) {
  if (!chain_supported_horizon(t.horizon) || t.nsteps <= 0 || t.nsteps > kMaxChainSteps ||
      t.nevals <= 0 || t.values <= 0 || t.values > upd::kMaxActions * t.horizon)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(chain::reset_kernel, dim3(1), dim3(kChainGrid), 0, stream, t.flags, t.abort);
  hipError_t st = hipGetLastError();
  if (st != hipSuccess) return st;
  hipLaunchKernelGGL(chain::tick_kernel<16>, dim3(kChainGrid), dim3(conv::kThreads), 0, stream, t);
  return hipGetLastError();
}

}  // namespace fe::hip
