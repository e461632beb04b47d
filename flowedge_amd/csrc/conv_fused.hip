// Host side of the fused convolution: launch planning and dispatch to the kernel instances
// (conv_kernel.h describes the kernel).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "conv_kernel.h"
#include "kernels.h"

namespace fe::hip {
namespace {

using namespace conv;

struct LaunchPlan {
  int vec = 4;
  int tpr = 64;
  int nch = 1;
  int tiles = 0;
  int blocks = 0;
};

bool lin_ok(int lin) { return lin == 1 || lin == 2 || lin == 4 || lin == 8 || lin == 16; }

// Lanes per row and chunks per lane: the fewest lanes per row (most rows per tile) whose chunk
// count fits the register budget while leaving at least one row tile per CU; shapes with fewer
// rows take the lane count with the most tiles.  Tiles are then spread evenly over at most one
// workgroup per CU.
bool plan_conv(const ConvOp& op, bool res, int split, bool norm, LaunchPlan& p) {
  if (!lin_ok(op.lin) || op.ic <= 0 || op.oc <= 0 || split <= 0 || split > op.ic) return false;
  if (op.mode == kConvSame) {
    if (op.k != 3 && op.k != 5) return false;
  } else if (op.mode == kConvDown) {
    if (op.k != 3 || op.lin < 2 || res) return false;
  } else if (op.mode == kConvTranspose) {
    if (op.k != 4 || res) return false;
  } else {
    return false;
  }
  if (op.lout != lout_of(op.mode, op.lin)) return false;
  p.vec = (op.ic % 4 == 0 && split % 4 == 0) ? 4 : 1;
  if (p.vec == 1 && (norm || op.mode != kConvSame)) return false;
  if (op.ic * op.lin > kMaxStageFloats) return false;
  if (norm && split * op.lin > kMaxNormFloats) return false;
  const int nv = op.ic / p.vec;
  const int budget = chunk_budget(op.k, op.lin, res, p.vec);
  int best = -1, best_tiles = 0;
  for (int tpr = kWave; tpr <= kThreads; tpr *= 2) {
    const int nch = (nv + tpr - 1) / tpr;
    if (nch > budget) continue;
    const int rpt = kThreads / tpr;
    const int tiles = (op.oc + rpt - 1) / rpt;
    if (tiles >= kMaxBlocks) {
      best = tpr;
      break;
    }
    if (tiles > best_tiles) {
      best = tpr;
      best_tiles = tiles;
    }
  }
  if (best < 0) return false;
  p.tpr = best;
  p.nch = (nv + best - 1) / best;
  p.tiles = (op.oc + kThreads / best - 1) / (kThreads / best);
  const int per = (p.tiles + kMaxBlocks - 1) / kMaxBlocks;  // tiles per workgroup
  p.blocks = (p.tiles + per - 1) / per;
  return true;
}

int prologue_of(const ConvInput& in) {
  if (!in.norm) return kProPlain;
  if (in.film_time != nullptr && in.res == nullptr) return kProFilm;
  if (in.film_time == nullptr && in.res != nullptr) return kProResid;
  return -1;
}

// Every condition conv_fused needs; `p` receives the launch plan.
bool fused_plan(const ConvOp& op, const ConvOp* res1x1, const ConvInput& in, View yr, int batch,
                LaunchPlan& p) {
  const bool res = res1x1 != nullptr;
  if (!plan_conv(op, res, in.split, in.norm, p)) return false;
  if (prologue_of(in) < 0) return false;
  if (in.norm && (in.groups <= 0 || in.groups > kMaxGroups || in.split % in.groups != 0 ||
                  (in.split / in.groups * op.lin) % 4 != 0))
    return false;
  if (in.split < op.ic && in.plain == nullptr) return false;
  if (res && (res1x1->k != 1 || res1x1->ic != op.ic || res1x1->oc != op.oc || yr.p == nullptr))
    return false;
  if (batch <= 0 || batch > 65535) return false;
  // Weight tensors are addressed with 32-bit buffer offsets (out-of-range marker at 2 GiB).
  const std::uint64_t wbytes = static_cast<std::uint64_t>(op.oc) * op.k * op.ic * (op.bf16 ? 2 : 4);
  const std::uint64_t rwbytes =
      res ? static_cast<std::uint64_t>(op.oc) * op.ic * (res1x1->bf16 ? 2 : 4) : 0;
  if (wbytes >= kOutOfRange || rwbytes >= kOutOfRange) return false;
  if (res && p.vec == 4 && res1x1->bf16 != op.bf16) return false;
  return true;
}

// Plan of the sliced kernel with S input-channel slices: each slice holds whole GroupNorm groups
// of the normalised part (or lies in the plain part), stages at most kSliceFloats floats, and
// the rows (slice_tpr lanes) fit the chunk budget.  Tiles of a slice are spread over at most
// kMaxBlocks / S workgroups.
bool plan_slices(const ConvOp& op, bool res, const ConvInput& in, int S, int tpr, LaunchPlan& p) {
  if (!slice_instance(op.mode, op.k, op.lin, res)) return false;
  if (tpr != 16 && tpr != 32 && tpr != 64) return false;
  if (!slice_tpr_ok(op.mode, op.lin, res, tpr)) return false;
  if (S < 2 || S > kMaxSlices || op.ic % S != 0) return false;
  const int ics = op.ic / S;
  if (ics % 4 != 0 || ics * op.lin > kSliceFloats || in.split % ics != 0) return false;
  if (in.norm && ics % (in.split / in.groups) != 0) return false;
  if (in.parts < 1 || in.parts > kMaxSlices || in.res_parts < 1 || in.res_parts > kMaxSlices)
    return false;
  const int nch = (ics / 4 + tpr - 1) / tpr;
  if (nch > slice_budget(op.k, op.lin, res, tpr)) return false;
  p.vec = 4;
  p.tpr = tpr;
  p.nch = nch;
  const int rpt = kThreads / tpr;
  p.tiles = (op.oc + rpt - 1) / rpt;
  const int cap = kMaxBlocks / S;                    // workgroups per slice
  const int per = (p.tiles + cap - 1) / cap;         // tiles per workgroup
  p.blocks = (p.tiles + per - 1) / per;
  return true;
}

ConvInput single_part(ConvInput in) {
  in.parts = 1;
  in.res_parts = 1;
  return in;
}

}  // namespace

SlicePlan conv_fused_slices(const ConvOp& op, const ConvOp* res1x1, const ConvInput& in, View yr,
                            int batch, int max_slices, int tpr) {
  SlicePlan best;
  LaunchPlan p;
  if (!fused_plan(op, res1x1, single_part(in), yr, batch, p) || p.vec != 4) return best;
  // The most slices with any lane count; among lane counts, the most workgroups (up to one per
  // CU), then the fewest lanes per row (more weight chunks in flight per lane).
  for (int S = kMaxSlices; S >= 2; S /= 2) {
    if (S > max_slices) continue;
    int wgs = 0;
    for (int t = 16; t <= 64; t *= 2) {
      LaunchPlan q;
      if ((tpr != 0 && t != tpr) || !plan_slices(op, res1x1 != nullptr, in, S, t, q)) continue;
      const int n = q.blocks * S;
      if (n > wgs) {
        wgs = n;
        best.slices = S;
        best.res_slices = S;
        best.tpr = t;
      }
    }
    if (wgs > 0) return best;
  }
  return best;
}

bool conv_fused_supported(const ConvOp& op, const ConvOp* res1x1, const ConvInput& in, View yr,
                          int batch) {
  LaunchPlan p;
  return fused_plan(op, res1x1, in, yr, batch, p);
}

namespace conv {

bool fused_args(const ConvOp& op, const ConvOp* res1x1, const ConvInput& in, View y, View yr,
                int batch, Args& a, int& vec, int& pro) {
  const bool res = res1x1 != nullptr;
  LaunchPlan p;
  if (!fused_plan(op, res1x1, in, yr, batch, p)) return false;
  pro = prologue_of(in);
  vec = p.vec;
  const std::uint64_t wbytes = static_cast<std::uint64_t>(op.oc) * op.k * op.ic * (op.bf16 ? 2 : 4);
  const std::uint64_t rwbytes =
      res ? static_cast<std::uint64_t>(op.oc) * op.ic * (res1x1->bf16 ? 2 : 4) : 0;
  a = Args{};
  a.wbytes = static_cast<unsigned>(wbytes);
  a.rwbytes = static_cast<unsigned>(rwbytes);
  a.w = op.w;
  a.bias = op.b;
  a.y = y.p;
  a.ys = y.stride;
  a.bf16 = op.bf16 ? 1 : 0;
  if (res) {
    a.rw = res1x1->w;
    a.rbias = res1x1->b;
    a.yr = yr.p;
    a.yrs = yr.stride;
    a.rbf16 = res1x1->bf16 ? 1 : 0;
  }
  a.oc = op.oc;
  a.ic = op.ic;
  a.tiles = p.tiles;
  a.blocks = p.blocks;
  a.tpr = p.tpr;
  a.nch = p.nch;
  a.in = in;
  return true;
}

}  // namespace conv

hipError_t conv_fused(const ConvOp& op, const ConvOp* res1x1, const ConvInput& in, View y,
                      View yr, int batch, hipStream_t stream, SlicePlan sp) {
  const bool res = res1x1 != nullptr;
  Args a;
  int vec = 4, pro = 0;
  const int slices = sp.slices;
  if (slices > 1) {
    // The unsliced checks, then the slice plan.
    LaunchPlan p;
    if (!conv::fused_args(op, res1x1, single_part(in), y, yr, batch, a, vec, pro) || vec != 4 ||
        !plan_slices(op, res, in, slices, sp.tpr, p))
      return hipErrorInvalidValue;
    a.in = in;
    a.slices = slices;
    a.ics = op.ic / slices;
    a.tpr = p.tpr;
    a.nch = p.nch;
    a.tiles = p.tiles;
    a.blocks = p.blocks;
    a.ypart = y.part;
    a.yrpart = yr.part;
    return launch_slice(op.mode, op.k, op.lin, pro, res, a, batch, stream);
  }
  // The unsliced kernel reads single tensors only.
  if (in.parts != 1 || in.res_parts != 1) return hipErrorInvalidValue;
  if (!conv::fused_args(op, res1x1, in, y, yr, batch, a, vec, pro)) return hipErrorInvalidValue;
  if (op.mode == kConvSame)
    return op.k == 5 ? launch_same5(op.lin, vec, pro, res, a, batch, stream)
                     : launch_same3(op.lin, vec, pro, res, a, batch, stream);
  return launch_resample(op.mode, op.lin, pro, a, batch, stream);
}

}  // namespace fe::hip
