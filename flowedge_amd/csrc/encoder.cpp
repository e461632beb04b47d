// Host side and C ABI of the observation encoder: the Diffusion Policy RGB encoder (LeRobot's
// DiffusionRgbEncoder: center crop, resnet18 trunk with GroupNorm, spatial-softmax keypoints,
// linear + ReLU) that the reference's LeRobot integration runs through torch to build the head's
// condition (integrations/lerobot/src/flowedge_lerobot/observation.py:152-216).  Here it runs on
// the GPU:
//   * load: read the encoder tensors (LeRobot names under a prefix, "diffusion.rgb_encoder." in a
//     LeRobot model.safetensors), check the resnet18 structure, plan ONE device arena for the
//     repacked weights (convolutions step-major over tap * C + channel) and the activations of `max_images` images,
//     one hipMalloc, uploads;
//   * encode: one hipGraph replay per image count (captured on first use): 40 launches of
//     encoder.hip's convolution, GroupNorm and head kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/flowedge.h"
#include "encoder.h"
#include "safetensors.h"

namespace fe::abi {
void set_error(const std::string& msg);
void clear_error();
void count_device_alloc();
}  // namespace fe::abi

namespace {

using fe::abi::clear_error;
using fe::abi::set_error;
namespace enc = fe::hip::enc;

constexpr int kStages = 4;
constexpr int kBlocks = 2;
constexpr std::size_t kAlign = 256;

struct ConvW {
  std::size_t off = 0;  // [cout][kh * kw][cin] fp32 in the arena
  int cin = 0, cout = 0, k = 0, stride = 1, pad = 0;
};
struct NormW {
  std::size_t gamma = 0, beta = 0;
};
struct BlockW {
  ConvW c1, c2, ds;
  NormW n1, n2, nd;
  bool proj = false;
  int cin = 0, cout = 0, hin = 0, win = 0, hout = 0, wout = 0;
};

struct Layout {
  int channels = 0;                 // image channels
  int img_h = 0, img_w = 0;         // camera image
  int top = 0, left = 0, vh = 0, vw = 0;  // center-crop view
  int stem_c = 0, stem_h = 0, stem_w = 0, pool_h = 0, pool_w = 0;
  int keypoints = 0, feature = 0, fmap_c = 0, fmap_h = 0, fmap_w = 0;
};

}  // namespace

struct FeEncoder {
  Layout L;
  std::size_t max_images = 0;
  char* arena = nullptr;
  std::size_t arena_bytes = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  float last_ms = -1.0f;
  float* pin = nullptr;  // host staging: images then features
  ConvW stem;
  NormW stem_n;
  BlockW blocks[kStages][kBlocks];
  std::size_t nets_w = 0, nets_b = 0, grid = 0, out_w = 0, out_b = 0;
  // Workspace offsets.
  std::size_t images = 0, stem_parts = 0, x0 = 0, x1 = 0, a1 = 0, h1 = 0, h2 = 0, hd = 0;
  std::size_t stats = 0;  // GroupNorm chunk statistics (doubles)
  std::size_t features = 0;
  std::size_t kp = 0;       // keypoint coordinates [n][2K]
  std::size_t act_max = 0;  // floats of the largest block activation per image
  std::map<std::size_t, hipGraphExec_t> graphs;

  float* p(std::size_t off) const { return reinterpret_cast<float*>(arena + off); }

  ~FeEncoder() {
    for (auto& g : graphs) (void)hipGraphExecDestroy(g.second);
    if (ev0) (void)hipEventDestroy(ev0);
    if (ev1) (void)hipEventDestroy(ev1);
    if (stream) (void)hipStreamDestroy(stream);
    if (arena) (void)hipFree(arena);
    if (pin) (void)hipHostFree(pin);
  }
};

namespace {

struct Plan {
  std::size_t size = 0;
  std::size_t take(std::size_t bytes) {
    const std::size_t off = (size + kAlign - 1) / kAlign * kAlign;
    size = off + bytes;
    return off;
  }
};

int conv_out(int in, int k, int stride, int pad) { return (in + 2 * pad - k) / stride + 1; }

// Host copies of the tensors to upload (fp32), with their arena offsets.
struct Upload {
  std::size_t off;
  std::vector<float> data;
};

struct Builder {
  const fe::Checkpoint& ck;
  std::string prefix;
  FeEncoder& e;
  Plan plan;
  std::vector<Upload> uploads;
  std::string err;

  const fe::TensorInfo* get(const std::string& name, std::initializer_list<std::size_t> shape) {
    const fe::TensorInfo* t = ck.find(prefix + name);
    if (t == nullptr) {
      err = "Missing encoder tensor: " + prefix + name;
      return nullptr;
    }
    if (!std::equal(t->shape.begin(), t->shape.end(), shape.begin(), shape.end())) {
      err = "Encoder tensor " + prefix + name + " has an unexpected shape";
      return nullptr;
    }
    return t;
  }

  static std::vector<float> widen(const fe::TensorInfo* t) {
    std::vector<float> v(t->elements());
    if (!t->bf16) {
      std::memcpy(v.data(), t->data, v.size() * 4);
    } else {
      const auto* bits = static_cast<const std::uint16_t*>(t->data);
      for (std::size_t i = 0; i < v.size(); ++i) {
        const std::uint32_t u = static_cast<std::uint32_t>(bits[i]) << 16;
        std::memcpy(&v[i], &u, 4);
      }
    }
    return v;
  }

  std::size_t raw(const fe::TensorInfo* t) {
    Upload u{plan.take(t->elements() * 4), widen(t)};
    const std::size_t off = u.off;
    uploads.push_back(std::move(u));
    return off;
  }

  // A convolution weight [O][C][k][k] repacked step-major: [steps][O][kReduceChunk] over the
  // reduction index tap * C + channel, zero past its end.
  bool conv(const std::string& name, int cin, int cout, int k, int stride, int pad, ConvW& c) {
    const fe::TensorInfo* t = get(name, {static_cast<std::size_t>(cout),
                                         static_cast<std::size_t>(cin),
                                         static_cast<std::size_t>(k),
                                         static_cast<std::size_t>(k)});
    if (t == nullptr) return false;
    const std::vector<float> w = widen(t);
    const int taps = k * k;
    const int kdim = taps * cin;
    const int steps = (kdim + enc::kReduceChunk - 1) / enc::kReduceChunk;
    std::vector<float> r(static_cast<std::size_t>(steps) * cout * enc::kReduceChunk, 0.0f);
    for (int o = 0; o < cout; ++o)
      for (int kk = 0; kk < kdim; ++kk) {
        const int tap = kk / cin, ci = kk % cin;
        const int s = kk / enc::kReduceChunk, j = kk % enc::kReduceChunk;
        r[(static_cast<std::size_t>(s) * cout + o) * enc::kReduceChunk + j] =
            w[(static_cast<std::size_t>(o) * cin + ci) * taps + tap];
      }
    c.off = plan.take(r.size() * 4);
    c.cin = cin;
    c.cout = cout;
    c.k = k;
    c.stride = stride;
    c.pad = pad;
    uploads.push_back(Upload{c.off, std::move(r)});
    return true;
  }

  bool gn(const std::string& name, int ch, NormW& n) {
    if (ch % 16 != 0) {
      err = "Encoder width " + std::to_string(ch) + " is not a multiple of 16 (GroupNorm(C/16))";
      return false;
    }
    const fe::TensorInfo* g = get(name + ".weight", {static_cast<std::size_t>(ch)});
    const fe::TensorInfo* b = g ? get(name + ".bias", {static_cast<std::size_t>(ch)}) : nullptr;
    if (b == nullptr) return false;
    n.gamma = raw(g);
    n.beta = raw(b);
    return true;
  }

  bool build(int img_h, int img_w, int crop_h, int crop_w) {
    Layout& L = e.L;
    const fe::TensorInfo* stem = ck.find(prefix + "backbone.0.weight");
    if (stem == nullptr || stem->shape.size() != 4 || stem->shape[2] != 7 || stem->shape[3] != 7) {
      err = "Missing or malformed encoder stem " + prefix + "backbone.0.weight ([C][3][7][7])";
      return false;
    }
    L.stem_c = static_cast<int>(stem->shape[0]);
    L.channels = static_cast<int>(stem->shape[1]);
    L.img_h = img_h;
    L.img_w = img_w;
    L.vh = crop_h > 0 ? crop_h : img_h;
    L.vw = crop_w > 0 ? crop_w : img_w;
    if (L.vh > img_h || L.vw > img_w || L.vh < 8 || L.vw < 8) {
      err = "Encoder crop must fit the image and be at least 8 x 8";
      return false;
    }
    // torchvision CenterCrop: int(round((size - crop) / 2)), rounding half to even.
    L.top = static_cast<int>(std::nearbyint((img_h - L.vh) / 2.0));
    L.left = static_cast<int>(std::nearbyint((img_w - L.vw) / 2.0));
    if (!conv("backbone.0.weight", L.channels, L.stem_c, 7, 2, 3, e.stem) ||
        !gn("backbone.1", L.stem_c, e.stem_n))
      return false;
    L.stem_h = conv_out(L.vh, 7, 2, 3);
    L.stem_w = conv_out(L.vw, 7, 2, 3);
    L.pool_h = conv_out(L.stem_h, 3, 2, 1);
    L.pool_w = conv_out(L.stem_w, 3, 2, 1);
    int cin = L.stem_c, h = L.pool_h, w = L.pool_w;
    std::size_t act_max = static_cast<std::size_t>(cin) * h * w;
    for (int s = 0; s < kStages; ++s) {
      const fe::TensorInfo* c1 = ck.find(prefix + "backbone." + std::to_string(4 + s) + ".0.conv1.weight");
      if (c1 == nullptr || c1->shape.size() != 4) {
        err = "Missing encoder stage " + std::to_string(s + 1);
        return false;
      }
      const int cout = static_cast<int>(c1->shape[0]);
      for (int blk = 0; blk < kBlocks; ++blk) {
        BlockW& b = e.blocks[s][blk];
        const std::string p = "backbone." + std::to_string(4 + s) + "." + std::to_string(blk) + ".";
        const int stride = (s > 0 && blk == 0) ? 2 : 1;
        b.cin = blk == 0 ? cin : cout;
        b.cout = cout;
        b.hin = h;
        b.win = w;
        b.hout = conv_out(h, 3, stride, 1);
        b.wout = conv_out(w, 3, stride, 1);
        if (!conv(p + "conv1.weight", b.cin, cout, 3, stride, 1, b.c1) || !gn(p + "bn1", cout, b.n1) ||
            !conv(p + "conv2.weight", cout, cout, 3, 1, 1, b.c2) || !gn(p + "bn2", cout, b.n2))
          return false;
        b.proj = ck.find(prefix + p + "downsample.0.weight") != nullptr;
        if (b.proj) {
          if (!conv(p + "downsample.0.weight", b.cin, cout, 1, stride, 0, b.ds) ||
              !gn(p + "downsample.1", cout, b.nd))
            return false;
        } else if (b.cin != cout || stride != 1) {
          err = "Encoder block " + p + " changes shape without a downsample projection";
          return false;
        }
        h = b.hout;
        w = b.wout;
        act_max = std::max(act_max, static_cast<std::size_t>(cout) * h * w);
      }
      cin = cout;
    }
    L.fmap_c = cin;
    L.fmap_h = h;
    L.fmap_w = w;
    e.act_max = act_max;
    const fe::TensorInfo* nets = ck.find(prefix + "pool.nets.weight");
    if (nets == nullptr || nets->shape.size() != 4 || nets->shape[1] != static_cast<std::size_t>(cin) ||
        nets->shape[2] != 1 || nets->shape[3] != 1) {
      err = "Missing or malformed " + prefix + "pool.nets.weight ([K][C][1][1])";
      return false;
    }
    L.keypoints = static_cast<int>(nets->shape[0]);
    const int f = 2 * L.keypoints;
    const fe::TensorInfo* nb = get("pool.nets.bias", {static_cast<std::size_t>(L.keypoints)});
    const fe::TensorInfo* ow = nb ? ck.find(prefix + "out.weight") : nullptr;
    if (ow == nullptr || ow->shape.size() != 2 || ow->shape[1] != static_cast<std::size_t>(f)) {
      if (err.empty()) err = "Missing or malformed " + prefix + "out.weight ([F][2K])";
      return false;
    }
    L.feature = static_cast<int>(ow->shape[0]);
    const fe::TensorInfo* ob = get("out.bias", {static_cast<std::size_t>(L.feature)});
    if (ob == nullptr) return false;
    if (h * w > enc::kMaxHeadPos || 2 * L.keypoints > enc::kMaxHeadInputs) {
      err = "Encoder feature map too large for the keypoint head";
      return false;
    }
    e.nets_w = raw(nets);
    e.nets_b = raw(nb);
    e.out_w = raw(ow);
    e.out_b = raw(ob);
    // The SpatialSoftmax position grid: the checkpoint's buffer when present, else
    // np.meshgrid(linspace(-1, 1, W), linspace(-1, 1, H)) (x along the width).
    const std::size_t hw = static_cast<std::size_t>(h) * w;
    const fe::TensorInfo* g = ck.find(prefix + "pool.pos_grid");
    if (g != nullptr) {
      if (g->shape.size() != 2 || g->shape[0] != hw || g->shape[1] != 2) {
        err = "Encoder " + prefix + "pool.pos_grid does not match the feature map";
        return false;
      }
      e.grid = raw(g);
    } else {
      std::vector<float> grid(2 * hw);
      for (int y = 0; y < h; ++y)
        for (int x = 0; x < w; ++x) {
          grid[2 * (y * w + x)] = static_cast<float>(w > 1 ? -1.0 + 2.0 * x / (w - 1) : -1.0);
          grid[2 * (y * w + x) + 1] = static_cast<float>(h > 1 ? -1.0 + 2.0 * y / (h - 1) : -1.0);
        }
      e.grid = plan.take(grid.size() * 4);
      uploads.push_back(Upload{e.grid, std::move(grid)});
    }
    // Workspace for max_images images.  A convolution's partial sums are laid out
    // [part][image][C][H][W]; the buffers hold the largest parts * n * C*H*W of any convolution
    // at any image count n (large image counts need no split).
    const std::size_t M = e.max_images;
    std::size_t stem_need = 0, conv_need = 0;
    auto need = [&](const ConvW& c, int hin, int win) {
      std::size_t m = 0;
      for (std::size_t n = 1; n <= M; ++n) {
        enc::ConvArgs a;
        a.cin = c.cin;
        a.cout = c.cout;
        a.kh = a.kw = c.k;
        a.stride = c.stride;
        a.pad = c.pad;
        a.hout = conv_out(hin, c.k, c.stride, c.pad);
        a.wout = conv_out(win, c.k, c.stride, c.pad);
        a.n = static_cast<int>(n);
        enc::plan_conv(a);
        const std::size_t act = static_cast<std::size_t>(c.cout) * a.hout * a.wout;
        m = std::max(m, static_cast<std::size_t>(a.ksplit) * n * act);
      }
      return m;
    };
    stem_need = need(e.stem, L.vh, L.vw);
    for (int s = 0; s < kStages; ++s)
      for (int blk = 0; blk < kBlocks; ++blk) {
        const BlockW& b = e.blocks[s][blk];
        conv_need = std::max({conv_need, need(b.c1, b.hin, b.win), need(b.c2, b.hout, b.wout),
                              b.proj ? need(b.ds, b.hin, b.win) : std::size_t{0}});
      }
    e.images = plan.take(M * L.channels * img_h * img_w * 4);
    e.stem_parts = plan.take(stem_need * 4);
    e.x0 = plan.take(M * act_max * 4);
    e.x1 = plan.take(M * act_max * 4);
    e.a1 = plan.take(M * act_max * 4);
    e.h1 = plan.take(conv_need * 4);
    e.h2 = plan.take(conv_need * 4);
    e.hd = plan.take(conv_need * 4);
    e.features = plan.take(M * L.feature * 4);
    e.kp = plan.take(M * 2 * L.keypoints * 4);
    // GroupNorm statistics: the most (group, chunk) pairs of any pass (the stem's, whose groups
    // hold the most values), 4 doubles each.
    enc::NormArgs big;
    big.c = 16;
    big.groups = 1;
    big.h = L.stem_h;
    big.w = L.stem_w;
    const std::size_t pairs = static_cast<std::size_t>(enc::norm_chunks(big)) * 32;
    e.stats = plan.take(M * pairs * 4 * sizeof(double));
    return true;
  }
};

#define FE_ENC_TRY(expr)                      \
  do {                                        \
    const hipError_t fe_st_ = (expr);         \
    if (fe_st_ != hipSuccess) return fe_st_;  \
  } while (0)

// A convolution of `n` images from x (c x h x w planes of the view) into partial sums at y.
hipError_t enqueue_conv(FeEncoder& e, const ConvW& c, const float* x, int xh, int xw, int top,
                        int left, int vh, int vw, int n, float* y, int& parts,
                        std::int64_t& part, std::int64_t& ys) {
  enc::ConvArgs a;
  a.w = e.p(c.off);
  a.x = x;
  a.xplane = static_cast<std::int64_t>(xh) * xw;
  a.xs = a.xplane * c.cin;
  a.xw = xw;
  a.top = top;
  a.left = left;
  a.vh = vh;
  a.vw = vw;
  a.cin = c.cin;
  a.cout = c.cout;
  a.kh = a.kw = c.k;
  a.stride = c.stride;
  a.pad = c.pad;
  a.hout = conv_out(vh, c.k, c.stride, c.pad);
  a.wout = conv_out(vw, c.k, c.stride, c.pad);
  a.n = n;
  enc::plan_conv(a);
  ys = static_cast<std::int64_t>(c.cout) * a.hout * a.wout;
  part = ys * n;
  a.y = y;
  a.ys = ys;
  a.ypart = part;
  parts = a.ksplit;
  return enc::conv(a, e.stream);
}

// The whole encoder for n images already in e.images; features to e.features.
hipError_t enqueue_encoder(FeEncoder& e, int n) {
  const Layout& L = e.L;
  int parts = 1;
  std::int64_t part = 0, ys = 0;
  FE_ENC_TRY(enqueue_conv(e, e.stem, e.p(e.images), L.img_h, L.img_w, L.top, L.left, L.vh, L.vw,
                          n, e.p(e.stem_parts), parts, part, ys));
  enc::NormArgs sn;
  sn.mode = enc::kNormStemPool;
  sn.n = n;
  sn.c = L.stem_c;
  sn.h = L.stem_h;
  sn.w = L.stem_w;
  sn.groups = L.stem_c / 16;
  sn.src = e.p(e.stem_parts);
  sn.src_stride = ys;
  sn.parts = parts;
  sn.part_stride = part;
  sn.gamma = e.p(e.stem_n.gamma);
  sn.beta = e.p(e.stem_n.beta);
  sn.dst = e.p(e.x0);
  sn.dst_stride = static_cast<std::int64_t>(L.stem_c) * L.pool_h * L.pool_w;
  sn.stats = reinterpret_cast<double*>(e.arena + e.stats);
  FE_ENC_TRY(enc::norm(sn, e.stream));
  float* x = e.p(e.x0);
  float* nx = e.p(e.x1);
  for (int s = 0; s < kStages; ++s)
    for (int blk = 0; blk < kBlocks; ++blk) {
      const BlockW& b = e.blocks[s][blk];
      const std::int64_t in_act = static_cast<std::int64_t>(b.cin) * b.hin * b.win;
      const std::int64_t out_act = static_cast<std::int64_t>(b.cout) * b.hout * b.wout;
      int p1 = 1, p2 = 1, pd = 1;
      std::int64_t s1 = 0, s2 = 0, sd = 0, y1 = 0, y2 = 0, yd = 0;
      FE_ENC_TRY(enqueue_conv(e, b.c1, x, b.hin, b.win, 0, 0, b.hin, b.win, n, e.p(e.h1), p1, s1,
                              y1));
      enc::NormArgs m;
      m.mode = enc::kNormMid;
      m.n = n;
      m.c = b.cout;
      m.h = b.hout;
      m.w = b.wout;
      m.groups = b.cout / 16;
      m.src = e.p(e.h1);
      m.src_stride = y1;
      m.parts = p1;
      m.part_stride = s1;
      m.gamma = e.p(b.n1.gamma);
      m.beta = e.p(b.n1.beta);
      m.dst = e.p(e.a1);
      m.dst_stride = out_act;
      m.stats = reinterpret_cast<double*>(e.arena + e.stats);
      FE_ENC_TRY(enc::norm(m, e.stream));
      FE_ENC_TRY(enqueue_conv(e, b.c2, e.p(e.a1), b.hout, b.wout, 0, 0, b.hout, b.wout, n,
                              e.p(e.h2), p2, s2, y2));
      enc::NormArgs t = m;
      t.src = e.p(e.h2);
      t.src_stride = y2;
      t.parts = p2;
      t.part_stride = s2;
      t.gamma = e.p(b.n2.gamma);
      t.beta = e.p(b.n2.beta);
      t.dst = nx;
      if (b.proj) {
        FE_ENC_TRY(enqueue_conv(e, b.ds, x, b.hin, b.win, 0, 0, b.hin, b.win, n, e.p(e.hd), pd,
                                sd, yd));
        t.mode = enc::kNormEndGn;
        t.res = e.p(e.hd);
        t.res_stride = yd;
        t.res_parts = pd;
        t.res_part_stride = sd;
        t.rgamma = e.p(b.nd.gamma);
        t.rbeta = e.p(b.nd.beta);
      } else {
        t.mode = enc::kNormEndPlain;
        t.res = x;
        t.res_stride = in_act;
      }
      FE_ENC_TRY(enc::norm(t, e.stream));
      std::swap(x, nx);
    }
  enc::HeadArgs h;
  h.x = x;
  h.x_stride = static_cast<std::int64_t>(L.fmap_c) * L.fmap_h * L.fmap_w;
  h.n = n;
  h.c = L.fmap_c;
  h.hw = L.fmap_h * L.fmap_w;
  h.k = L.keypoints;
  h.fout = L.feature;
  h.nets_w = e.p(e.nets_w);
  h.nets_b = e.p(e.nets_b);
  h.grid = e.p(e.grid);
  h.out_w = e.p(e.out_w);
  h.out_b = e.p(e.out_b);
  h.kp = e.p(e.kp);
  h.y = e.p(e.features);
  h.y_stride = L.feature;
  return enc::head(h, e.stream);
}

// The captured graph of n images (captured on first use).
hipError_t graph_for(FeEncoder& e, std::size_t n, hipGraphExec_t& exec) {
  auto it = e.graphs.find(n);
  if (it != e.graphs.end()) {
    exec = it->second;
    return hipSuccess;
  }
  hipGraph_t g = nullptr;
  FE_ENC_TRY(hipStreamBeginCapture(e.stream, hipStreamCaptureModeThreadLocal));
  const hipError_t st = enqueue_encoder(e, static_cast<int>(n));
  const hipError_t st2 = hipStreamEndCapture(e.stream, &g);
  if (st != hipSuccess || st2 != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    return st != hipSuccess ? st : st2;
  }
  const hipError_t st3 = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  FE_ENC_TRY(st3);
  e.graphs[n] = exec;
  return hipSuccess;
}

int fail(const char* what, hipError_t st) {
  set_error(std::string(what) + ": " + hipGetErrorString(st));
  return FE_STATUS_RESOURCE_EXHAUSTED;
}

}  // namespace

extern "C" {

fe_encoder* fe_encoder_load(const char* path, const char* prefix, size_t image_height,
                            size_t image_width, size_t crop_height, size_t crop_width,
                            size_t max_images) {
  clear_error();
  if (path == nullptr || image_height == 0 || image_width == 0 || image_height > 4096 ||
      image_width > 4096 || max_images == 0 || max_images > 64 || crop_height > image_height ||
      crop_width > image_width || (crop_height == 0) != (crop_width == 0)) {
    set_error("Invalid arguments to fe_encoder_load");
    return nullptr;
  }
  std::string err;
  std::shared_ptr<const fe::Checkpoint> ck = fe::Checkpoint::open(path, err);
  if (!ck) {
    set_error(err);
    return nullptr;
  }
  auto e = std::make_unique<FeEncoder>();
  e->max_images = max_images;
  Builder b{*ck, prefix != nullptr ? prefix : "", *e, Plan{}, {}, {}};
  if (!b.build(static_cast<int>(image_height), static_cast<int>(image_width),
               static_cast<int>(crop_height), static_cast<int>(crop_width))) {
    set_error(b.err);
    return nullptr;
  }
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
    set_error("No HIP device available (the observation encoder runs on the GPU only)");
    return nullptr;
  }
  e->arena_bytes = b.plan.size;
  hipError_t st = hipMalloc(reinterpret_cast<void**>(&e->arena), e->arena_bytes);
  if (st != hipSuccess) {
    e->arena = nullptr;
    fail("Encoder arena allocation failed", st);
    return nullptr;
  }
  fe::abi::count_device_alloc();
  for (const Upload& u : b.uploads)
    if ((st = hipMemcpy(e->arena + u.off, u.data.data(), u.data.size() * 4,
                        hipMemcpyHostToDevice)) != hipSuccess) {
      fail("Encoder weight upload failed", st);
      return nullptr;
    }
  const std::size_t pin_floats =
      max_images * (static_cast<std::size_t>(e->L.channels) * image_height * image_width +
                    static_cast<std::size_t>(e->L.feature));
  void* pin = nullptr;
  if ((st = hipHostMalloc(&pin, pin_floats * 4, hipHostMallocDefault)) != hipSuccess) {
    fail("Encoder pinned staging allocation failed", st);
    return nullptr;
  }
  e->pin = static_cast<float*>(pin);
  if ((st = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking)) != hipSuccess ||
      (st = hipEventCreate(&e->ev0)) != hipSuccess || (st = hipEventCreate(&e->ev1)) != hipSuccess) {
    fail("Encoder stream creation failed", st);
    return nullptr;
  }
  return e.release();
}

void fe_encoder_free(fe_encoder* encoder) { delete encoder; }

int fe_encoder_shape(const fe_encoder* encoder, size_t* channels, size_t* feature_dim,
                     size_t* keypoints) {
  clear_error();
  if (encoder == nullptr) {
    set_error("Invalid arguments to fe_encoder_shape");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  if (channels) *channels = static_cast<size_t>(encoder->L.channels);
  if (feature_dim) *feature_dim = static_cast<size_t>(encoder->L.feature);
  if (keypoints) *keypoints = static_cast<size_t>(encoder->L.keypoints);
  return FE_STATUS_OK;
}

int fe_encoder_encode_device(fe_encoder* encoder, const float* images_dev, size_t n,
                             float* features_dev, size_t out_stride, size_t out_offset) {
  clear_error();
  if (encoder == nullptr || images_dev == nullptr || features_dev == nullptr || n == 0 ||
      n > encoder->max_images || out_stride < out_offset + encoder->L.feature) {
    set_error("Invalid arguments to fe_encoder_encode_device");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  FeEncoder& e = *encoder;
  const Layout& L = e.L;
  const std::size_t img = static_cast<std::size_t>(L.channels) * L.img_h * L.img_w;
  hipError_t st;
  hipGraphExec_t exec = nullptr;
  if ((st = graph_for(e, n, exec)) != hipSuccess) return fail("Encoder graph capture failed", st);
  hipStream_t s = e.stream;
  if ((st = hipMemcpyAsync(e.p(e.images), images_dev, n * img * 4, hipMemcpyDeviceToDevice, s)) !=
          hipSuccess ||
      (st = hipEventRecord(e.ev0, s)) != hipSuccess || (st = hipGraphLaunch(exec, s)) != hipSuccess ||
      (st = hipEventRecord(e.ev1, s)) != hipSuccess ||
      (st = hipMemcpy2DAsync(features_dev + out_offset, out_stride * 4, e.p(e.features),
                             static_cast<std::size_t>(L.feature) * 4,
                             static_cast<std::size_t>(L.feature) * 4, n, hipMemcpyDeviceToDevice,
                             s)) != hipSuccess)
    return fail("Encoder execution failed", st);
  if ((st = hipStreamSynchronize(s)) != hipSuccess) return fail("Encoder execution failed", st);
  float ms = 0.0f;
  if (hipEventElapsedTime(&ms, e.ev0, e.ev1) == hipSuccess) e.last_ms = ms;
  return FE_STATUS_OK;
}

int fe_encoder_encode(fe_encoder* encoder, const float* images, size_t n, float* features) {
  clear_error();
  if (encoder == nullptr || images == nullptr || features == nullptr || n == 0 ||
      n > encoder->max_images) {
    set_error("Invalid arguments to fe_encoder_encode");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  FeEncoder& e = *encoder;
  const Layout& L = e.L;
  const std::size_t img = static_cast<std::size_t>(L.channels) * L.img_h * L.img_w;
  for (std::size_t i = 0; i < n * img; ++i)
    if (!std::isfinite(images[i])) {
      set_error("Observation images contain non-finite values");
      return FE_STATUS_INVALID_ARGUMENT;
    }
  hipError_t st;
  hipGraphExec_t exec = nullptr;
  if ((st = graph_for(e, n, exec)) != hipSuccess) return fail("Encoder graph capture failed", st);
  float* pin_img = e.pin;
  float* pin_feat = e.pin + e.max_images * img;
  std::memcpy(pin_img, images, n * img * 4);
  hipStream_t s = e.stream;
  if ((st = hipMemcpyAsync(e.p(e.images), pin_img, n * img * 4, hipMemcpyHostToDevice, s)) !=
          hipSuccess ||
      (st = hipEventRecord(e.ev0, s)) != hipSuccess || (st = hipGraphLaunch(exec, s)) != hipSuccess ||
      (st = hipEventRecord(e.ev1, s)) != hipSuccess ||
      (st = hipMemcpyAsync(pin_feat, e.p(e.features), n * L.feature * 4, hipMemcpyDeviceToHost,
                           s)) != hipSuccess ||
      (st = hipStreamSynchronize(s)) != hipSuccess)
    return fail("Encoder execution failed", st);
  float ms = 0.0f;
  if (hipEventElapsedTime(&ms, e.ev0, e.ev1) == hipSuccess) e.last_ms = ms;
  std::memcpy(features, pin_feat, n * L.feature * 4);
  return FE_STATUS_OK;
}

float fe_encoder_last_device_ms(const fe_encoder* encoder) {
  return encoder != nullptr ? encoder->last_ms : -1.0f;
}

size_t fe_encoder_device_bytes(const fe_encoder* encoder) {
  return encoder != nullptr ? encoder->arena_bytes : 0;
}

}  // extern "C"
