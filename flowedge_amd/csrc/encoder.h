// Observation encoder device operations (encoder.hip): the Diffusion Policy RGB encoder's 2-D
// convolutions, GroupNorm passes and keypoint head, enqueue-only on a caller stream.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace fe::hip::enc {

// Partial sums of a split reduction: up to 32 for outputs of at most kSmallOutput values (the
// late, small-spatial layers, where adding them is cheap), up to 8 otherwise.
constexpr int kMaxParts = 32;
constexpr int kMaxPartsLarge = 8;
constexpr std::int64_t kSmallOutput = 32768;
constexpr int kMaxHeadPos = 1024;    // feature-map positions the keypoint head takes
constexpr int kMaxHeadInputs = 1024; // keypoint coordinates (2 per keypoint) it takes

// Reduction indices per step of the convolution; the weights are repacked step-major.
constexpr int kReduceChunk = 16;

// y (+ p * ypart for split p) = conv2d(x) of `n` images, no bias.  x is read through a view of
// vh x vw pixels at (top, left) of each xh x xw input plane (the center crop of the stem);
// padding `pad` zeros around the view.
struct ConvArgs {
  // [steps][cout][kReduceChunk]: w[s][o][j] is the weight of output o at reduction index
  // k = s * kReduceChunk + j = tap * cin + input channel (zero for k >= kh * kw * cin).
  const float* w = nullptr;
  const float* x = nullptr;
  std::int64_t xs = 0;       // floats between images
  std::int64_t xplane = 0;   // floats between channels (xh * xw)
  int xw = 0;                // input row length
  int top = 0, left = 0, vh = 0, vw = 0;
  int cin = 0, cout = 0, kh = 0, kw = 0, stride = 1, pad = 0;
  int hout = 0, wout = 0, n = 0;
  float* y = nullptr;
  std::int64_t ys = 0;       // floats between images of the output
  std::int64_t ypart = 0;    // floats between partial sums (split reduction)
  // Planned by plan_conv: column tile, tiles, reduction steps and split.
  int nt = 64, mtiles = 0, ntiles = 0, steps = 0, ksplit = 1, per = 0;
};

// Fills the plan fields of `a` (shape fields set).
void plan_conv(ConvArgs& a);
// Partial sums conv() leaves for this shape (1: the output itself).
int conv_parts(const ConvArgs& shape);
hipError_t conv(const ConvArgs& a, hipStream_t stream);

enum NormMode : int {
  kNormStemPool = 0,  // dst = maxpool3x3s2(relu(GN(src)))
  kNormMid = 1,       // dst = relu(GN(src))
  kNormEndPlain = 2,  // dst = relu(GN(src) + res)                (block input as residual)
  kNormEndGn = 3,     // dst = relu(GN(src) + GN_r(res))          (1x1 projection residual)
};

// GroupNorm with `groups` groups over c channels of h x w of n images.  src (and res in
// kNormEndGn) are sums of `parts` partials, which the pass adds (writing the sum over the first
// partial) before the statistics.
struct NormArgs {
  int mode = kNormMid;
  int n = 0, c = 0, h = 0, w = 0, groups = 0;
  float* src = nullptr;
  std::int64_t src_stride = 0;
  int parts = 1;
  std::int64_t part_stride = 0;
  const float* gamma = nullptr;
  const float* beta = nullptr;
  float* res = nullptr;
  std::int64_t res_stride = 0;
  int res_parts = 1;
  std::int64_t res_part_stride = 0;
  const float* rgamma = nullptr;
  const float* rbeta = nullptr;
  float* dst = nullptr;
  std::int64_t dst_stride = 0;
  double* stats = nullptr;  // workspace of norm_chunks(a) * 4 doubles per (image, group)
};
// Statistics workgroups per (image, group) of the pass.
int norm_chunks(const NormArgs& a);
// One launch for groups of at most 8192 values outside the stem mode (a workgroup per group);
// else two: fp64 statistics per chunk of each group (adding the partials), then one lane per
// output value.
hipError_t norm(const NormArgs& a, hipStream_t stream);

// Per image: keypoint logits = nets_w [k][c] x (feature maps [c][hw]) + nets_b, softmax over the
// hw positions, expected (x, y) on grid [hw][2] into kp [n][2k] (workspace), then
// y = relu(out_w [fout][2k] kp + out_b), written at y + image * y_stride + y_offset.
struct HeadArgs {
  const float* x = nullptr;
  std::int64_t x_stride = 0;
  int n = 0, c = 0, hw = 0, k = 0, fout = 0;
  const float* nets_w = nullptr;
  const float* nets_b = nullptr;
  const float* grid = nullptr;
  const float* out_w = nullptr;
  const float* out_b = nullptr;
  float* kp = nullptr;
  float* y = nullptr;
  std::int64_t y_stride = 0, y_offset = 0;
};
hipError_t head(const HeadArgs& a, hipStream_t stream);

}  // namespace fe::hip::enc
