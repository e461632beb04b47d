// Device operations for the Diffusion Policy U-Net on gfx950 (internal C++ API).
//
// This is the layer the host runtime calls to enqueue work; it plays the role the reference's
// `fe::cuda_ops` plays for its CUDA resident (src/core/kernels/cuda/kernels_cuda_api.h:8-120),
// but every op here works on device-resident buffers, takes a batch dimension and is
// enqueue-only (no allocation, no synchronisation), so a whole tick can be captured in one
// hipGraph.
//
// Activation layout: [B][C][L] fp32 with channel stride L; a view may use a larger sample stride
// (skip tensors live in the second half of an up-stage concat buffer).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace fe::hip {

// Convolution kinds on the path.
enum ConvMode : int {
  kConvSame = 0,       // stride 1, padding K/2 (K odd): residual convs, final conv, 1x1 convs
  kConvDown = 1,       // stride 2, padding 1, K = 3: Downsample1d
  kConvTranspose = 2,  // ConvTranspose1d stride 2, padding 1, K = 4: Upsample1d
};

struct ConvOp {
  const void* w = nullptr;  // [OC][K][IC], fp32 or bf16 bit patterns
  const float* b = nullptr; // [OC]
  bool bf16 = false;
  int mode = kConvSame;
  int k = 1;
  int ic = 0, oc = 0;
  int lin = 0, lout = 0;
};

struct View {
  float* p = nullptr;
  std::int64_t stride = 0;  // floats between samples
  std::int64_t part = 0;    // floats between the partial sums of a sliced convolution's output
};

// Input-channel slices: a fused convolution may split its input channels into up to
// kMaxSlices slices (whole GroupNorm groups each), one slice per workgroup, and then writes one
// partial sum per slice ([B][S][oc][lout] at View::part spacing, bias in partial 0); the consumer
// adds the partials in slice order while it reads them.
constexpr int kMaxSlices = 8;
// Staged floats of one slice (channels * positions): one 16-byte chunk per lane.
constexpr int kSliceFloats = 2048;

// Input of a fused convolution.  Channels [0, split) come from `src` (a raw producer output,
// bias included) through the optional prologue
//     v = mish(GroupNorm(src))           (statistics over all `split` channels of the sample)
//     v = scale[c] * v + shift[c]        (FiLM, when film_time != null)
//     v += res[c]                        (residual, when res != null)
// and are written to `mat` (when non-null) so later ops can read them as a plain tensor;
// channels [split, ic) are read unchanged from `plain`.  Without `norm`, src channels are read
// unchanged too.
struct ConvInput {
  const float* src = nullptr;
  std::int64_t src_stride = 0;
  int split = 0;
  bool norm = false;
  const float* gamma = nullptr;
  const float* beta = nullptr;
  int groups = 1;
  const float* film_time = nullptr;
  const float* film_cond = nullptr;
  std::int64_t film_cond_stride = 0;
  int film_off = 0;
  const float* res = nullptr;
  std::int64_t res_stride = 0;
  float* mat = nullptr;
  std::int64_t mat_stride = 0;
  const float* plain = nullptr;
  std::int64_t plain_stride = 0;
  // `src` and `res` as sums of partials (outputs of sliced convolutions): value = sum over
  // p < parts of src[p * part_stride + ...], added in order p = 0, 1, ...
  int parts = 1;
  std::int64_t part_stride = 0;
  int res_parts = 1;
  std::int64_t res_part_stride = 0;
};

// y = conv(input) + bias, and optionally yr = res1x1(input) + bias from the same prologue (the
// residual 1x1 projection of a ResidualBlock reads the same input as its first conv).
// Input-channel slices of a fused convolution and the lanes per output row of its sliced kernel.
struct SlicePlan {
  int slices = 1;
  int tpr = 0;
  // Matrix-core convolutions: partial sums left by the split K loop of the convolution and of
  // its 1x1 projection (1: reduced in place).
  bool matrix = false;
  int res_slices = 1;
};

// With sp.slices > 1 (from conv_fused_slices) the input channels are split into that many
// slices and y (and yr) receive one partial sum per slice at View::part spacing.
hipError_t conv_fused(const ConvOp& op, const ConvOp* res1x1, const ConvInput& in, View y,
                      View yr, int batch, hipStream_t stream, SlicePlan sp = SlicePlan{});

// True when conv_fused has a kernel for this convolution, input and batch (unsliced).
bool conv_fused_supported(const ConvOp& op, const ConvOp* res1x1, const ConvInput& in, View yr,
                          int batch);
// The most input-channel slices (a power of two up to max_slices) the sliced kernels can run
// this convolution with, and their lanes per row (`tpr` if non-zero, else the choice giving the
// most workgroups); slices 1 when none fits (then `in` must have single-part src and res).
SlicePlan conv_fused_slices(const ConvOp& op, const ConvOp* res1x1, const ConvInput& in, View yr,
                            int batch, int max_slices, int tpr = 0);

// Batched path (matrix cores).  y = conv(x) + bias with x a plain tensor: channels [0, split)
// from `src`, the rest from `plain`.  ic and split are multiples of 16, or split == ic (narrow
// first convolution).  When the output tiles would leave CUs idle, the K loop is split over
// workgroups whose partial tiles go to `workspace` (workspace_floats large enough) and are summed
// by a second kernel in a fixed order.
bool conv_mfma_supported(const ConvOp& op, int split);
// Convolutions with 32-channel multiples can run on the BF16 matrix cores: BF16 weights against
// the input split into two BF16 terms (`bf16_mma`), F32 weights as three products of split
// weights and split input (`f32_split`).  Otherwise they run on the F32 matrix cores (BF16
// weights widened).
// With max_parts >= 2, a split K loop writes up to max_parts partial sums in the output layout
// (y.part apart, bias in the first) instead of reducing them; conv_mfma_parts returns how many
// (1: unsplit).
hipError_t conv_mfma(const ConvOp& op, const float* src, std::int64_t src_stride, int split,
                     const float* plain, std::int64_t plain_stride, View y, int batch,
                     float* workspace, std::size_t workspace_floats, bool bf16_mma,
                     bool f32_split, hipStream_t stream, int max_parts = 0);
int conv_mfma_parts(const ConvOp& op, int split, std::int64_t src_stride, const float* plain,
                    std::int64_t plain_stride, int batch, bool bf16_mma, bool f32_split,
                    int max_parts);
// The K split conv_mfma runs with these arguments (1: none).
int conv_mfma_ksplit(const ConvOp& op, int split, std::int64_t src_stride, const float* plain,
                     std::int64_t plain_stride, int batch, std::size_t workspace_floats,
                     bool bf16_mma, bool f32_split, int max_parts);
// dst[b][0 : n) = sum over p < parts of src[b * src_stride + p * part_stride + ...), added in
// order: the plain input of a matrix-core convolution whose producer left partial sums.
hipError_t sum_parts(const float* src, std::int64_t src_stride, int parts,
                     std::int64_t part_stride, std::int64_t n, float* dst,
                     std::int64_t dst_stride, int batch, hipStream_t stream);

// The prologue of a ConvInput with `norm` on its own: dst[b][0 : split*lin) =
// mish(GN(src)) [* scale + shift] [+ res], per sample.  Batches under 256 samples and shapes
// outside the per-sample kernel's instances (split * lin > 8192, more than 32 groups, groups of
// lengths not a multiple of 4) run on norm_act_general.
hipError_t norm_act(const ConvInput& in, int lin, float* dst, std::int64_t dst_stride, int batch,
                    hipStream_t stream);

// General-shape path (conv_general.hip): any kernel size, length and width the checkpoint format
// admits, for convolutions neither conv_fused nor conv_mfma has an instance for.  y = conv(x) +
// bias with x a plain tensor (channels [0, split) from `src`, the rest from `plain`); the
// reduction is split over workgroups through `workspace` when the tiles leave CUs idle.
hipError_t conv_general(const ConvOp& op, const float* src, std::int64_t src_stride, int split,
                        const float* plain, std::int64_t plain_stride, View y, int batch,
                        float* workspace, std::size_t workspace_floats, hipStream_t stream);
// The prologue with one workgroup per (sample, group): any width, length and group count.
hipError_t norm_act_general(const ConvInput& in, int lin, float* dst, std::int64_t dst_stride,
                            int batch, hipStream_t stream);

// Timestep of the n-th U-Net evaluation of a sampling call, derived on the device:
//   kTimesSingle: t = t0
//   kTimesDiffusion: t_n = (steps - 1 - n) * ratio         (diffusion.cc:984-990)
//   kTimesFlow: step s = n / stages, stage j = n % stages, dt = 1/steps, t = s dt, stage offsets
//     Euler {0}, Heun {0, dt}, RK4 {0, dt/2, dt/2, dt}   (flow.cc:291-318)
//   kTimesIndex: t_n = n (the table of every train timestep)
enum TimesMode : int { kTimesSingle = 0, kTimesDiffusion = 1, kTimesFlow = 2, kTimesIndex = 3 };
struct TimeSpec {
  int mode = kTimesSingle;
  float t0 = 0.0f;
  int steps = 1;
  int ratio = 1;
  int method = 0;  // flow: 0 Euler, 1 Heun, 2 RK4
};

// m[n][:] = mish(te2(mish(te1(emb(t_n)) + b1)) + b2) for n < count.  The embedding and hidden
// layer (5 * tdim floats) live in LDS: tdim <= kMaxTimeMlpLds / 20.
constexpr std::size_t kMaxTimeMlpLds = 160 * 1024;
hipError_t time_mlp(const TimeSpec& times, int count, const float* w1, const float* b1,
                    const float* w2, const float* b2, int tdim, float* m, hipStream_t stream);

// out[n][f] = (bias ? bias[f] : 0) + sum_k wt[k][f] * act(in[n][k]); act = mish when `mish_in`.
hipError_t film_gemm(const float* in, std::int64_t in_stride, int n, int kdim, const float* wt,
                     const float* bias, int fdim, bool mish_in, float* out,
                     std::int64_t out_stride, hipStream_t stream);

// x[b][a][t] = noise[b][t][a]; also copies into `xin` when distinct.
hipError_t begin_sample(const float* noise, float* x, float* xin, int batch, int horizon,
                        int action_dim, hipStream_t stream);

// Final GroupNorm + Mish + 1x1 conv with the sampler update fused into its epilogue:
//   eps[b][a][t] = bo[a] + sum_c wo[a][c] mish(gn(h))[b][c][t].
enum UpdateKind : int {
  kUpdateDenoise = 0,  // out[b][t][a] = eps
  kUpdateDDIM = 1,
  kUpdateDDPM = 2,
  kUpdateEuler = 3,    // x += dt * v
  kUpdateStage = 4,    // k[slot] = v; xin = x + dt * v   (Heun stage 1, RK4 stages 1-3;
                       //   dt carries the stage coefficient dt or dt/2)
  kUpdateHeun = 5,     // x += 0.5 dt (k0 + v)
  kUpdateRK4 = 6,      // x += dt/6 (k0 + 2 k1 + 2 k2 + v)
};
struct UpdateOp {
  int kind = kUpdateDDIM;
  int c0 = 0, horizon = 0, action_dim = 0;
  const float* h = nullptr;      // [B][c0][H] raw final conv output
  int hparts = 1;                // h as the sum of hparts partials hpart apart (sliced conv)
  std::int64_t hpart = 0;
  std::int64_t hstride = 0;      // floats between samples of h (0: c0 * H)
  const float* gamma = nullptr;  // final GroupNorm (8 groups) applied with Mish before the 1x1
  const float* beta = nullptr;
  int groups = 8;
  const float* wo = nullptr;     // [A][c0]
  const float* bo = nullptr;     // [A]
  float* x = nullptr;            // sampler state [B][A][H]
  float* xin = nullptr;          // U-Net input for the next NFE [B][A][H] (may equal x)
  float* kbuf = nullptr;         // [4][B][A][H] flow stages
  int slot = 0;
  float* out = nullptr;          // kUpdateDenoise output [B][H][A]
  // DDIM / DDPM scalars (host-computed as the reference does).
  float sqrt_at = 0, sqrt_bt = 0, sqrt_ap = 0, sqrt_1map = 0;
  float coef_x0 = 0, coef_x = 0, sigma = 0;
  int clip = 0;
  float clip_range = 1.0f;
  const std::uint64_t* seed = nullptr;  // DDPM seed (device, set per call)
  std::uint64_t noise_offset = 0;       // Gaussian stream index of this step's first value
  int add_noise = 0;
  float dt = 0;
  // Split update (512 final channels in 8 groups): per-sample arrival counters, zero between
  // launches, and the per-group partial outputs [B][8][A][H].  Null: one workgroup per sample.
  unsigned* done = nullptr;
  float* epart = nullptr;
};
// One block per sample.  Shapes outside the fused kernel's instances (horizon not a power of two
// up to 16, c0 > 1024, more than 64 actions or 32 groups) run on a general kernel (one wavefront
// per output value), which accepts any c0 divisible by `groups` (at most 64 groups).
hipError_t update(const UpdateOp& op, int batch, hipStream_t stream);
// True when update() runs this shape on its fused kernel (the one that sums partials of h).
bool update_fused(int c0, int groups, int horizon, int action_dim);
// The most partials of h the fused update kernel sums at final width c0.
int update_max_parts(int c0);

// action[b][t][a] = (x[b][a][t] + 1) / 2 * (max - min) + min   (or a plain transpose when
// amin == nullptr).
hipError_t finish_sample(const float* x, const float* amin, const float* amax, float* action,
                         int batch, int horizon, int action_dim, hipStream_t stream);

// ---- Persistent tick (chain.hip) ----
// One sampling tick of one sample in a single launch: kChainGrid workgroups (one per CU) run every
// convolution of every U-Net evaluation as the steps of one step table, handing activations to
// each other through device-coherent memory and per-workgroup completion counters (a step's
// workgroups request their first weights, then wait until every workgroup has finished the
// previous step).  Each workgroup computes every evaluation's sampler update itself and keeps the
// sample's state in a slot of its own, so updates need no hand-off.
constexpr int kChainGrid = 256;
constexpr int kChainFlagStride = 64;  // unsigned per workgroup counter (256 bytes apart)
constexpr int kMaxChainSteps = 64;

// One convolution of an evaluation (enqueue order).
struct ChainConv {
  ConvOp op;
  bool has_res = false;
  ConvOp res;
  ConvInput in;
  View y, yr;
  bool film = false;   // its FiLM time rows are those of the evaluation being run
  bool state = false;  // its input is the workgroup's U-Net input slot (first convolution)
};
struct ChainEval {
  const float* film_row = nullptr;  // FiLM time rows of this evaluation
  UpdateOp upd;                     // sampler update after it (x, xin, kbuf: the slot's)
};
struct ChainTick {
  const void* steps = nullptr;
  int nsteps = 0;
  const ChainEval* evals = nullptr;
  int nevals = 0;
  const float* x0 = nullptr;   // state [A][H] at the start
  const float* xin0 = nullptr; // first U-Net input [A][H]
  float* slots = nullptr;      // per workgroup: x, xin, k0 .. k3, `values` floats each
  int slot_floats = 0;
  float* x_out = nullptr;      // final state, written by workgroup 0
  unsigned* flags = nullptr;   // [kChainGrid * kChainFlagStride]
  unsigned* abort = nullptr;   // set when a wait gives up (the tick's result is then invalid)
  long long spin_limit = 0;    // polls before a wait gives up
  int values = 0;              // A * H
  int horizon = 0;
};
std::size_t chain_step_bytes();
// Horizons the tick kernel is built for.
bool chain_supported_horizon(int horizon);
// Step table of one evaluation (host memory of n * chain_step_bytes()); false, with the reason,
// when a convolution has no variant in the tick kernel.
bool chain_build(const ChainConv* convs, int n, void* steps, const char** why);
// Enqueues the counter reset and the tick kernel.
hipError_t chain_tick(const ChainTick& t, hipStream_t stream);

// Static device scratch of the allocation-free entry point (scratch.hip): kScratchBytes per GPU.
// scratch_setup returns the array's device address on `device`, which must be the current device;
// the address is looked up once per device and kept.
constexpr std::size_t kScratchBytes = std::size_t{32} << 20;
hipError_t scratch_setup(int device, void** ptr);

}  // namespace fe::hip
