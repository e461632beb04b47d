// CPU oracle for the Diffusion Policy Conv1D U-Net path — TEST INFRASTRUCTURE ONLY.
//
// This file restates, in plain C++ of its own, the algorithm of FlowEdge's CPU Diffusion Policy
// path so that the HIP implementation can be checked against it.  Only the test suite, the smoke
// check and the `cpu_baseline` leg of bench.py load it; the shipped library never links it and
// never falls back to it.
//
// Restated reference semantics (file:line in elprofesoriqo/FlowEdge):
//   config parse / validation ........ src/core/heads/diffusion/diffusion.cc:391-427
//   squaredcos alphas_cumprod ........ diffusion.cc:186-191, 529-541 (beta in double, product in float)
//   splitmix64 + Box-Muller .......... diffusion.cc:193-231
//   residual block ................... diffusion.cc:724-773
//   U-Net orchestration .............. diffusion.cc:793-914
//   DDIM / DDPM loop + unnormalize ... diffusion.cc:916-1035 (host path, 979-1034)
//   conv1d (im2col+GEMM / direct) .... src/core/kernels/diffusion_ops.cc:82-163
//   conv_transpose1d (k-major) ....... diffusion_ops.cc:165-268, repack diffusion.cc:496-521
//   group_norm (fp64 statistics) ..... diffusion_ops.cc:270-350 (scalar-path accumulation)
//   film ............................. diffusion_ops.cc:352-377
//   timestep embedding ............... diffusion_ops.cc:379-396
//   mish (libm form) ................. src/core/kernels/cpu/kernels_scalar.cc:83-87
//   matmul (4x8-lane accumulators) ... kernels_avx2.cc:175-204, 517-602, 727-773
//   task split ....................... src/core/kernels/kernels.h:25-47, arena/thread_pool.h:67-86
//   flow ODE update (Euler/Heun/RK4) . src/core/heads/flow/flow.cc:291-318, kernels/span_ops.h:27-52
//
// Extensions beyond the reference (each is a composition of the pieces above):
//   * dp.meta[12] == 1 ("velocity"): the U-Net is used as a flow-matching velocity field
//     v(x,t|c) = denoise(c, x, t) with continuous t, driven by the flow-head ODE update; the
//     result is x(1) with no unnormalize (flow.cc:321).
//   * BF16 conv weights: widened to F32 at load, so the oracle is the F32 path on BF16-rounded
//     values (the reference accepts BF16 only for linears, diffusion.cc:656-660, 678-683).
//   * Batches: B independent batch-1 samples (the reference has no batch argument).
//
// Mish: the reference's x86 path evaluates 8-wide blocks with Cephes exp/log polynomials and its
// scalar tails with libm; this oracle uses the libm form for every element (see mish1 below).

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <limits>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace {

// ------------------------------------------------------------------------------------------
// Minimal safetensors reader (F32 / BF16 tensors only).
// ------------------------------------------------------------------------------------------
struct Tensor {
  std::string name;
  bool bf16 = false;
  std::vector<std::size_t> shape;
  std::vector<float> data;  // widened to F32
  std::size_t elements() const {
    std::size_t n = 1;
    for (std::size_t s : shape) n *= s;
    return n;
  }
};

bool parse_u64_list(const std::string& text, std::size_t pos, std::vector<std::uint64_t>& out) {
  out.clear();
  pos = text.find('[', pos);
  if (pos == std::string::npos) return false;
  ++pos;
  std::uint64_t value = 0;
  bool have = false;
  for (; pos < text.size(); ++pos) {
    const char c = text[pos];
    if (c >= '0' && c <= '9') {
      value = value * 10 + static_cast<std::uint64_t>(c - '0');
      have = true;
    } else if (c == ',' || c == ']') {
      if (have) out.push_back(value);
      value = 0;
      have = false;
      if (c == ']') return true;
    } else if (c != ' ' && c != '\n' && c != '\t') {
      return false;
    }
  }
  return false;
}

float bf16_bits_to_f32(std::uint16_t bits) {
  const std::uint32_t wide = static_cast<std::uint32_t>(bits) << 16u;
  float f;
  std::memcpy(&f, &wide, sizeof f);
  return f;
}

bool read_safetensors(const char* path, std::vector<Tensor>& tensors) {
  FILE* f = std::fopen(path, "rb");
  if (!f) return false;
  std::uint64_t header_len = 0;
  if (std::fread(&header_len, 8, 1, f) != 1 || header_len > (1ull << 30)) {
    std::fclose(f);
    return false;
  }
  std::string header(header_len, '\0');
  if (std::fread(header.data(), 1, header_len, f) != header_len) {
    std::fclose(f);
    return false;
  }
  const long data_start = static_cast<long>(8 + header_len);
  // Walk top-level "name": { ... } entries.
  std::size_t p = header.find('{');
  if (p == std::string::npos) {
    std::fclose(f);
    return false;
  }
  ++p;
  while (true) {
    const std::size_t q0 = header.find('"', p);
    if (q0 == std::string::npos) break;
    const std::size_t q1 = header.find('"', q0 + 1);
    if (q1 == std::string::npos) break;
    const std::string name = header.substr(q0 + 1, q1 - q0 - 1);
    const std::size_t ob = header.find('{', q1);
    if (ob == std::string::npos) break;
    int depth = 1;
    std::size_t e = ob + 1;
    for (; e < header.size() && depth > 0; ++e) depth += (header[e] == '{') - (header[e] == '}');
    const std::string obj = header.substr(ob, e - ob);
    p = e;
    if (name == "__metadata__") continue;
    Tensor t;
    t.name = name;
    const bool is_f32 = obj.find("\"F32\"") != std::string::npos;
    t.bf16 = obj.find("\"BF16\"") != std::string::npos;
    if (!is_f32 && !t.bf16) continue;
    std::vector<std::uint64_t> shape, offs;
    if (!parse_u64_list(obj, obj.find("\"shape\""), shape) ||
        !parse_u64_list(obj, obj.find("\"data_offsets\""), offs) || offs.size() != 2 ||
        offs[1] < offs[0]) {
      std::fclose(f);
      return false;
    }
    for (std::uint64_t s : shape) t.shape.push_back(static_cast<std::size_t>(s));
    const std::size_t n = t.elements();
    const std::size_t esize = t.bf16 ? 2 : 4;
    if (n * esize != offs[1] - offs[0]) {
      std::fclose(f);
      return false;
    }
    t.data.resize(n);
    if (std::fseek(f, data_start + static_cast<long>(offs[0]), SEEK_SET) != 0) {
      std::fclose(f);
      return false;
    }
    if (t.bf16) {
      std::vector<std::uint16_t> raw(n);
      if (n && std::fread(raw.data(), 2, n, f) != n) {
        std::fclose(f);
        return false;
      }
      for (std::size_t i = 0; i < n; ++i) t.data[i] = bf16_bits_to_f32(raw[i]);
    } else if (n && std::fread(t.data.data(), 4, n, f) != n) {
      std::fclose(f);
      return false;
    }
    tensors.push_back(std::move(t));
  }
  std::fclose(f);
  return !tensors.empty();
}

// ------------------------------------------------------------------------------------------
// Worker pool: contiguous chunks of [0,total), as parallel_for (thread_pool.h:67-86).
// ------------------------------------------------------------------------------------------
class Pool {
 public:
  explicit Pool(unsigned workers) : n_(workers) {
    for (unsigned i = 0; i < workers; ++i) threads_.emplace_back([this, i] { loop(i); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> lk(m_);
      stop_ = true;
      ++epoch_;
    }
    cv_.notify_all();
    for (auto& t : threads_) t.join();
  }
  unsigned size() const { return n_; }
  // Runs fn(lo,hi) over `tasks` chunks on the workers (caller waits, as the reference pool).
  void run(std::size_t total, unsigned tasks, const std::function<void(std::size_t, std::size_t)>& fn) {
    const std::size_t n = std::min<std::size_t>({static_cast<std::size_t>(n_), tasks, total});
    if (n <= 1) {
      fn(0, total);
      return;
    }
    const std::size_t sz = (total + n - 1) / n;
    std::unique_lock<std::mutex> lk(m_);
    fn_ = &fn;
    chunk_ = sz;
    total_ = total;
    active_ = static_cast<unsigned>(n);
    remaining_ = static_cast<unsigned>(n);
    ++epoch_;
    cv_.notify_all();
    done_cv_.wait(lk, [this] { return remaining_ == 0; });
    fn_ = nullptr;
  }

 private:
  void loop(unsigned idx) {
    std::uint64_t seen = 0;
    while (true) {
      const std::function<void(std::size_t, std::size_t)>* fn;
      std::size_t lo, hi;
      {
        std::unique_lock<std::mutex> lk(m_);
        cv_.wait(lk, [&] { return epoch_ != seen; });
        seen = epoch_;
        if (stop_) return;
        if (idx >= active_) continue;
        fn = fn_;
        lo = idx * chunk_;
        hi = std::min(total_, lo + chunk_);
      }
      if (lo < hi) (*fn)(lo, hi);
      {
        std::lock_guard<std::mutex> lk(m_);
        if (--remaining_ == 0) done_cv_.notify_one();
      }
    }
  }
  unsigned n_;
  std::vector<std::thread> threads_;
  std::mutex m_;
  std::condition_variable cv_, done_cv_;
  std::uint64_t epoch_ = 0;
  bool stop_ = false;
  const std::function<void(std::size_t, std::size_t)>* fn_ = nullptr;
  std::size_t chunk_ = 0, total_ = 0;
  unsigned active_ = 0, remaining_ = 0;
};

// Power-of-two task count from pool capacity and work size (kernels.h:25-47).
unsigned task_count(const Pool* pool, std::size_t rows, std::size_t in_dim, std::size_t out_dim) {
  const unsigned available = pool ? pool->size() : 0u;
  if (available < 2u || rows == 0 || in_dim == 0 || out_dim < 128) return 1u;
  const std::size_t work = rows * in_dim * out_dim;
  const std::size_t work_limited = 1 + (work - 1) / 786432;
  const std::size_t output_limited = out_dim / 64;
  const unsigned useful = static_cast<unsigned>(
      std::min<std::size_t>({static_cast<std::size_t>(available), work_limited, output_limited}));
  if (useful < 2u) return 1u;
  unsigned p = 1;
  while (p * 2 <= useful) p *= 2;
  return p;
}

void parallel_for(Pool* pool, std::size_t total, unsigned tasks,
                  const std::function<void(std::size_t, std::size_t)>& fn) {
  if (pool && tasks > 1u)
    pool->run(total, tasks, fn);
  else
    fn(0, total);
}

// ------------------------------------------------------------------------------------------
// Elementwise math.
// ------------------------------------------------------------------------------------------
// mish(v) = v * tanh(softplus(v)), softplus = max(v,0) + log1p(e^-|v|), evaluated with libm
// as the reference's scalar kernel and its SIMD tails (kernels_scalar.cc:83-87,
// kernels_avx2.cc:160-163) and its CUDA kernel (kernels_cuda.cu:126-133).  The reference's
// 8-wide AVX2 blocks use Cephes exp/log and tanh = 1 - 2/(1 + e^{2s}), which differs from this by
// up to ~1.3e-6 absolute for negative inputs (cancellation in 1 - 2/(1+e^{2s}) when s -> 0).
float mish1(float v) {
  return v * std::tanh(std::fmax(v, 0.0f) + std::log1p(std::exp(-std::fabs(v))));
}

void mish(float* x, std::size_t n) {
  for (std::size_t i = 0; i < n; ++i) x[i] = mish1(x[i]);
}

// LeRobot sinusoidal position embedding (diffusion_ops.cc:379-396).
void timestep_embedding(float t, float* out, std::size_t dim) {
  const std::size_t half = dim / 2;
  if (half == 1) {
    out[0] = std::sin(t);
    out[1] = std::cos(t);
    return;
  }
  const float factor = std::log(10000.0f) / static_cast<float>(half - 1);
  for (std::size_t i = 0; i < half; ++i) {
    const float freq = std::exp(-factor * static_cast<float>(i));
    const float phase = t * freq;
    out[i] = std::sin(phase);
    out[half + i] = std::cos(phase);
  }
}

// ------------------------------------------------------------------------------------------
// matmul: out[r][o] = sum_i in[r][i] * W[o][i], W row-major [out][in].
// Four 8-lane accumulators over 32-wide blocks, then one 8-lane accumulator, then a scalar
// tail (kernels_avx2.cc:175-204); rows are processed in blocks of four sharing each weight row.
// ------------------------------------------------------------------------------------------
inline float hsum8(const float* a) {
  // (lo4 + hi4) then pairwise, as hsum8 in kernels_avx2.cc.
  const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
  return (s0 + s1) + (s2 + s3);
}

void dot_rows(const float* const* in, int nr, const float* w, std::size_t n, float* res) {
  float acc[4][32];
  for (int r = 0; r < nr; ++r)
    for (int j = 0; j < 32; ++j) acc[r][j] = 0.0f;
  std::size_t i = 0;
  for (; i + 32 <= n; i += 32)
    for (int r = 0; r < nr; ++r) {
      const float* a = in[r] + i;
      for (int j = 0; j < 32; ++j) acc[r][j] = std::fma(a[j], w[i + j], acc[r][j]);
    }
  for (int r = 0; r < nr; ++r) {
    float v[8];
    for (int j = 0; j < 8; ++j)
      v[j] = (acc[r][j] + acc[r][8 + j]) + (acc[r][16 + j] + acc[r][24 + j]);
    std::size_t k = i;
    for (; k + 8 <= n; k += 8)
      for (int j = 0; j < 8; ++j) v[j] = std::fma(in[r][k + j], w[k + j], v[j]);
    float s = hsum8(v);
    for (; k < n; ++k) s += in[r][k] * w[k];
    res[r] = s;
  }
}

void matmul(const float* in, const float* w, float* out, std::size_t rows, std::size_t in_dim,
            std::size_t out_dim, Pool* pool) {
  const unsigned tasks = task_count(pool, rows, in_dim, out_dim);
  parallel_for(pool, out_dim, tasks, [&](std::size_t lo, std::size_t hi) {
    for (std::size_t o = lo; o < hi; ++o) {
      const float* wr = w + o * in_dim;
      for (std::size_t r0 = 0; r0 < rows; r0 += 4) {
        const int nr = static_cast<int>(std::min<std::size_t>(4, rows - r0));
        const float* rp[4];
        for (int r = 0; r < nr; ++r) rp[r] = in + (r0 + r) * in_dim;
        float res[4];
        dot_rows(rp, nr, wr, in_dim, res);
        for (int r = 0; r < nr; ++r) out[(r0 + r) * out_dim + o] = res[r];
      }
    }
  });
}

// ------------------------------------------------------------------------------------------
// Convolutions, [channels][length] activations, PyTorch cross-correlation semantics.
// ------------------------------------------------------------------------------------------
// diffusion_ops.cc:82-163: im2col [L_out][IC*K] + GEMM when IC*K >= 32, else direct loop.
void conv1d(const float* x, const float* weight, const float* bias, float* y, std::size_t ic,
            std::size_t oc, std::size_t lin, std::size_t lout, std::size_t k, std::size_t stride,
            std::size_t pad, Pool* pool, std::vector<float>& ws) {
  const std::size_t cols = ic * k;
  if (cols >= 32) {
    ws.resize(lout * cols + lout * oc);
    float* packed = ws.data();
    float* gemm = packed + lout * cols;
    for (std::size_t ot = 0; ot < lout; ++ot) {
      float* row = packed + ot * cols;
      const std::ptrdiff_t origin =
          static_cast<std::ptrdiff_t>(ot * stride) - static_cast<std::ptrdiff_t>(pad);
      for (std::size_t c = 0; c < ic; ++c)
        for (std::size_t kk = 0; kk < k; ++kk) {
          const std::ptrdiff_t idx = origin + static_cast<std::ptrdiff_t>(kk);
          row[c * k + kk] =
              (idx >= 0 && idx < static_cast<std::ptrdiff_t>(lin)) ? x[c * lin + idx] : 0.0f;
        }
    }
    matmul(packed, weight, gemm, lout, cols, oc, pool);
    for (std::size_t o = 0; o < oc; ++o)
      for (std::size_t ot = 0; ot < lout; ++ot) y[o * lout + ot] = gemm[ot * oc + o] + bias[o];
    return;
  }
  const unsigned tasks = task_count(pool, lout, ic * k, oc);
  parallel_for(pool, oc, tasks, [&](std::size_t lo, std::size_t hi) {
    for (std::size_t o = lo; o < hi; ++o) {
      float* out = y + o * lout;
      for (std::size_t ot = 0; ot < lout; ++ot) out[ot] = bias[o];
      for (std::size_t c = 0; c < ic; ++c)
        for (std::size_t kk = 0; kk < k; ++kk) {
          const float wv = weight[(o * ic + c) * k + kk];
          for (std::size_t ot = 0; ot < lout; ++ot) {
            const std::ptrdiff_t idx = static_cast<std::ptrdiff_t>(ot * stride + kk) -
                                       static_cast<std::ptrdiff_t>(pad);
            if (idx >= 0 && idx < static_cast<std::ptrdiff_t>(lin)) out[ot] += x[c * lin + idx] * wv;
          }
        }
    }
  });
}

// diffusion_ops.cc:165-231 with load-time k-major weights [K][OC][IC] (diffusion.cc:496-521):
// per tap, GEMM [L_in][IC] x [OC][IC]^T, scattered to output position it*stride + k - pad.
void conv_transpose1d_kmajor(const float* x, const float* wk, const float* bias, float* y,
                             std::size_t ic, std::size_t oc, std::size_t lin, std::size_t lout,
                             std::size_t k, std::size_t stride, std::size_t pad, Pool* pool,
                             std::vector<float>& ws) {
  ws.resize(lin * ic + lin * oc);
  float* xt = ws.data();
  float* gemm = xt + lin * ic;
  for (std::size_t c = 0; c < ic; ++c)
    for (std::size_t it = 0; it < lin; ++it) xt[it * ic + c] = x[c * lin + it];
  for (std::size_t o = 0; o < oc; ++o)
    for (std::size_t ot = 0; ot < lout; ++ot) y[o * lout + ot] = bias[o];
  for (std::size_t kk = 0; kk < k; ++kk) {
    matmul(xt, wk + kk * oc * ic, gemm, lin, ic, oc, pool);
    for (std::size_t it = 0; it < lin; ++it) {
      const std::ptrdiff_t origin =
          static_cast<std::ptrdiff_t>(it * stride + kk) - static_cast<std::ptrdiff_t>(pad);
      if (origin < 0 || origin >= static_cast<std::ptrdiff_t>(lout)) continue;
      for (std::size_t o = 0; o < oc; ++o) y[o * lout + origin] += gemm[it * oc + o];
    }
  }
}

// GroupNorm over one [C][L] sample, double-precision sum / sum of squares,
// var = E[x^2] - mean^2 clamped at 0, eps 1e-5 (diffusion_ops.cc:270-350).
void group_norm(float* x, const float* w, const float* b, std::size_t c, std::size_t len,
                std::size_t groups, float eps = 1e-5f) {
  const std::size_t cpg = c / groups;
  for (std::size_t g = 0; g < groups; ++g) {
    double sum = 0.0, sq = 0.0;
    for (std::size_t i = g * cpg * len; i < (g + 1) * cpg * len; ++i) {
      const double v = static_cast<double>(x[i]);
      sum += v;
      sq += v * v;
    }
    const double count = static_cast<double>(cpg * len);
    const double mean = sum / count;
    const double var = std::max(0.0, sq / count - mean * mean);
    const float inv = static_cast<float>(1.0 / std::sqrt(var + static_cast<double>(eps)));
    const float mean_f = static_cast<float>(mean);
    for (std::size_t ch = g * cpg; ch < (g + 1) * cpg; ++ch) {
      const float scale = inv * w[ch];
      const float shift = b[ch];
      for (std::size_t t = 0; t < len; ++t)
        x[ch * len + t] = std::fma(x[ch * len + t] - mean_f, scale, shift);
    }
  }
}

// ------------------------------------------------------------------------------------------
// Model.
// ------------------------------------------------------------------------------------------
struct Conv {
  const float* w = nullptr;  // [OC][IC][K] (ConvTranspose: k-major [K][OC][IC])
  const float* b = nullptr;
  std::size_t ic = 0, oc = 0, k = 0;
};
struct Norm {
  const float* w = nullptr;
  const float* b = nullptr;
};
struct Linear {
  const float* w = nullptr;
  const float* b = nullptr;
  std::size_t in = 0, out = 0;
};
struct Residual {
  Conv c1, c2, res;
  Norm n1, n2;
  Linear film;
  bool identity = false;
};

double alpha_bar(double time) {
  const double phase = ((time + 0.008) / 1.008) * (3.14159265358979323846 / 2.0);
  const double c = std::cos(phase);
  return c * c;
}

// splitmix64 stream and Box-Muller with a cached spare (diffusion.cc:193-231).
class Gaussian {
 public:
  explicit Gaussian(std::uint64_t seed) : state_(seed + 0x9e3779b97f4a7c15ULL) {}
  float next() {
    if (has_spare_) {
      has_spare_ = false;
      return spare_;
    }
    const float first = std::max(uniform(), std::numeric_limits<float>::min());
    const float second = uniform();
    const float radius = std::sqrt(-2.0f * std::log(first));
    const float angle = 2.0f * 3.14159265358979323846f * second;
    spare_ = radius * std::sin(angle);
    has_spare_ = true;
    return radius * std::cos(angle);
  }

 private:
  std::uint64_t integer() {
    state_ += 0x9e3779b97f4a7c15ULL;
    std::uint64_t v = state_;
    v = (v ^ (v >> 30u)) * 0xbf58476d1ce4e5b9ULL;
    v = (v ^ (v >> 27u)) * 0x94d049bb133111ebULL;
    return v ^ (v >> 31u);
  }
  float uniform() { return static_cast<float>((integer() >> 40u) + 1u) / 16777217.0f; }
  std::uint64_t state_;
  float spare_ = 0.0f;
  bool has_spare_ = false;
};

bool size_value(float v, std::size_t& out) {
  if (!std::isfinite(v) || v < 0.0f || std::floor(v) != v || v > 4294967295.0f) return false;
  out = static_cast<std::size_t>(v);
  return true;
}

struct Model {
  std::vector<Tensor> tensors;
  std::size_t A = 0, H = 0, action_steps = 0, obs = 0, cond = 0, stages = 0, K = 0, G = 0,
              tdim = 0, T = 0, pred = 0;
  bool clip = false;
  float clip_range = 1.0f;
  std::size_t dims[8] = {};
  Linear te1, te2;
  Residual down[8][2];
  Conv ds[8];
  Residual mid[2];
  Residual up[7][2];
  Conv us[7];
  std::vector<float> us_kmajor[7];
  Conv fconv, fout;
  Norm fnorm;
  const float* amin = nullptr;
  const float* amax = nullptr;
  std::vector<float> alphas;
  Pool* pool = nullptr;
  std::string error;

  const Tensor* find(const std::string& name) const {
    for (const auto& t : tensors)
      if (t.name == name) return &t;
    return nullptr;
  }
  bool vec(const std::string& name, std::size_t n, const float*& out) {
    const Tensor* t = find(name);
    if (!t || t->bf16 || t->shape.size() != 1 || t->shape[0] != n) return fail("bad vector " + name);
    out = t->data.data();
    return true;
  }
  bool fail(const std::string& m) {
    if (error.empty()) error = m;
    return false;
  }
  bool conv(const std::string& p, std::size_t oc, std::size_t ic, std::size_t k, Conv& c) {
    const Tensor* w = find(p + ".w");
    if (!w || w->shape.size() != 3 || w->shape[0] != oc || w->shape[1] != ic || w->shape[2] != k)
      return fail("bad conv " + p);
    c.w = w->data.data();
    c.oc = oc;
    c.ic = ic;
    c.k = k;
    return vec(p + ".b", oc, c.b);
  }
  bool linear(const std::string& p, std::size_t out, std::size_t in, Linear& l) {
    const Tensor* w = find(p + ".w");
    if (!w || w->shape.size() != 2 || w->shape[0] != out || w->shape[1] != in)
      return fail("bad linear " + p);
    l.w = w->data.data();
    l.in = in;
    l.out = out;
    return vec(p + ".b", out, l.b);
  }
  bool norm(const std::string& p, std::size_t c, Norm& n) {
    return vec(p + ".w", c, n.w) && vec(p + ".b", c, n.b);
  }
  bool residual(const std::string& p, std::size_t ic, std::size_t oc, Residual& r) {
    if (!conv(p + ".c1", oc, ic, K, r.c1) || !norm(p + ".n1", oc, r.n1) ||
        !linear(p + ".film", 2 * oc, tdim + cond, r.film) || !conv(p + ".c2", oc, oc, K, r.c2) ||
        !norm(p + ".n2", oc, r.n2))
      return false;
    r.identity = ic == oc;
    return r.identity || conv(p + ".res", oc, ic, 1, r.res);
  }

  // diffusion.cc:383-541 (+ prediction type 1 = velocity, the flow U-Net extension).
  bool init() {
    const Tensor* meta = find("dp.meta");
    const Tensor* dt = find("dp.dims");
    if (!meta || meta->shape.size() != 1 || meta->shape[0] != 16 || meta->bf16)
      return fail("missing or malformed dp.meta");
    if (!dt || dt->shape.size() != 1 || dt->bf16) return fail("missing or malformed dp.dims");
    const float* m = meta->data.data();
    std::size_t schema, beta, norm_type, clip_i;
    if (!size_value(m[0], schema) || !size_value(m[1], A) || !size_value(m[2], H) ||
        !size_value(m[3], action_steps) || !size_value(m[4], obs) || !size_value(m[5], cond) ||
        !size_value(m[6], stages) || !size_value(m[7], K) || !size_value(m[8], G) ||
        !size_value(m[9], tdim) || !size_value(m[10], T) || !size_value(m[11], beta) ||
        !size_value(m[12], pred) || !size_value(m[13], clip_i) || !size_value(m[15], norm_type) ||
        schema != 1 || beta != 0 || pred > 1 || norm_type != 0 || clip_i > 1 || A == 0 ||
        H == 0 || action_steps == 0 || obs == 0 || obs > H || action_steps > H - obs + 1 ||
        cond == 0 || stages < 2 || stages > 8 || K == 0 || K % 2 == 0 || G == 0 || tdim < 4 ||
        tdim % 2 != 0 || T == 0 || dt->shape[0] != stages || !std::isfinite(m[14]) ||
        m[14] <= 0.0f)
      return fail("invalid dp.meta");
    clip = clip_i != 0;
    clip_range = m[14];
    for (std::size_t s = 0; s < stages; ++s)
      if (!size_value(dt->data[s], dims[s]) || dims[s] == 0 || dims[s] % G != 0)
        return fail("invalid dp.dims");
    if (dims[0] % 8 != 0) return fail("dims[0] must be divisible by 8");
    if (H % (std::size_t{1} << (stages - 1)) != 0) return fail("horizon not divisible");
    if (!vec("dp.action_min", A, amin) || !vec("dp.action_max", A, amax)) return false;
    for (std::size_t i = 0; i < A; ++i)
      if (!std::isfinite(amin[i]) || !std::isfinite(amax[i]) || amax[i] <= amin[i])
        return fail("invalid action range");
    if (!linear("dp.te1", tdim * 4, tdim, te1) || !linear("dp.te2", tdim, tdim * 4, te2))
      return false;
    for (std::size_t s = 0; s < stages; ++s) {
      const std::size_t ic = s == 0 ? A : dims[s - 1];
      const std::size_t oc = dims[s];
      const std::string p = "dp.d" + std::to_string(s);
      if (!residual(p + ".r0", ic, oc, down[s][0]) || !residual(p + ".r1", oc, oc, down[s][1]))
        return false;
      if (s + 1 < stages && !conv(p + ".ds", oc, oc, 3, ds[s])) return false;
    }
    for (int b = 0; b < 2; ++b)
      if (!residual("dp.m" + std::to_string(b), dims[stages - 1], dims[stages - 1], mid[b]))
        return false;
    for (std::size_t s = 0; s + 1 < stages; ++s) {
      const std::size_t high = dims[stages - 1 - s], low = dims[stages - 2 - s];
      const std::string p = "dp.u" + std::to_string(s);
      if (!residual(p + ".r0", 2 * high, low, up[s][0]) || !residual(p + ".r1", low, low, up[s][1]) ||
          !conv(p + ".us", low, low, 4, us[s]))
        return false;
      // ConvTranspose storage [IC][OC][K] -> k-major [K][OC][IC].
      Conv& c = us[s];
      us_kmajor[s].resize(c.ic * c.oc * c.k);
      for (std::size_t kk = 0; kk < c.k; ++kk)
        for (std::size_t i = 0; i < c.ic; ++i)
          for (std::size_t o = 0; o < c.oc; ++o)
            us_kmajor[s][(kk * c.oc + o) * c.ic + i] = c.w[(i * c.oc + o) * c.k + kk];
      c.w = us_kmajor[s].data();
    }
    if (!conv("dp.f.c", dims[0], dims[0], K, fconv) || !norm("dp.f.n", dims[0], fnorm) ||
        !conv("dp.f.o", A, dims[0], 1, fout))
      return false;
    alphas.resize(T);
    float cumulative = 1.0f;
    for (std::size_t s = 0; s < T; ++s) {
      const double b0 = static_cast<double>(s) / static_cast<double>(T);
      const double b1 = static_cast<double>(s + 1) / static_cast<double>(T);
      const float beta_s = static_cast<float>(std::min(1.0 - alpha_bar(b1) / alpha_bar(b0), 0.999));
      cumulative *= 1.0f - beta_s;
      alphas[s] = cumulative;
    }
    return true;
  }

  // diffusion.cc:724-773.
  void residual_forward(const float* in, std::size_t len, const Residual& r, const float* cm,
                        float* out, std::vector<float>& ws) {
    const std::size_t ic = r.c1.ic, oc = r.c1.oc;
    std::vector<float> first(oc * len), mod(2 * oc);
    conv1d(in, r.c1.w, r.c1.b, first.data(), ic, oc, len, len, r.c1.k, 1, r.c1.k / 2, pool, ws);
    group_norm(first.data(), r.n1.w, r.n1.b, oc, len, G);
    mish(first.data(), first.size());
    matmul(cm, r.film.w, mod.data(), 1, r.film.in, r.film.out, pool);
    for (std::size_t i = 0; i < 2 * oc; ++i) mod[i] += r.film.b[i];
    for (std::size_t c = 0; c < oc; ++c)
      for (std::size_t t = 0; t < len; ++t)
        first[c * len + t] = std::fma(mod[c], first[c * len + t], mod[oc + c]);
    conv1d(first.data(), r.c2.w, r.c2.b, out, oc, oc, len, len, r.c2.k, 1, r.c2.k / 2, pool, ws);
    group_norm(out, r.n2.w, r.n2.b, oc, len, G);
    mish(out, oc * len);
    if (r.identity) {
      for (std::size_t i = 0; i < oc * len; ++i) out[i] += in[i];
    } else {
      conv1d(in, r.res.w, r.res.b, first.data(), ic, oc, len, len, 1, 1, 0, pool, ws);
      for (std::size_t i = 0; i < oc * len; ++i) out[i] += first[i];
    }
  }

  // diffusion.cc:793-914.  sample/eps use [H][A]; activations use [C][L].
  void denoise(const float* condv, const float* sample, float t, float* eps) {
    std::vector<float> ws;
    const std::size_t hidden = tdim * 4, feat = tdim + cond;
    std::vector<float> raw(tdim), hid(hidden), cm(feat);
    timestep_embedding(t, raw.data(), tdim);
    matmul(raw.data(), te1.w, hid.data(), 1, tdim, hidden, pool);
    for (std::size_t i = 0; i < hidden; ++i) hid[i] += te1.b[i];
    mish(hid.data(), hidden);
    matmul(hid.data(), te2.w, raw.data(), 1, hidden, tdim, pool);
    for (std::size_t i = 0; i < tdim; ++i) raw[i] += te2.b[i];
    std::copy(raw.begin(), raw.end(), cm.begin());
    std::copy(condv, condv + cond, cm.begin() + tdim);
    mish(cm.data(), feat);

    std::vector<float> x(A * H);
    for (std::size_t tt = 0; tt < H; ++tt)
      for (std::size_t c = 0; c < A; ++c) x[c * H + tt] = sample[tt * A + c];
    std::vector<float> skips[8];
    std::size_t len = H, ch = A;
    for (std::size_t s = 0; s < stages; ++s) {
      for (int b = 0; b < 2; ++b) {
        std::vector<float> o(dims[s] * len);
        residual_forward(x.data(), len, down[s][b], cm.data(), o.data(), ws);
        x.swap(o);
        ch = dims[s];
      }
      skips[s] = x;
      if (s + 1 < stages) {
        const std::size_t lo = len / 2;
        std::vector<float> o(ch * lo);
        conv1d(x.data(), ds[s].w, ds[s].b, o.data(), ch, ch, len, lo, 3, 2, 1, pool, ws);
        x.swap(o);
        len = lo;
      }
    }
    for (int b = 0; b < 2; ++b) {
      std::vector<float> o(ch * len);
      residual_forward(x.data(), len, mid[b], cm.data(), o.data(), ws);
      x.swap(o);
    }
    for (std::size_t s = 0; s + 1 < stages; ++s) {
      const std::vector<float>& skip = skips[stages - 1 - s];
      std::vector<float> cat(x.size() + skip.size());
      std::copy(x.begin(), x.end(), cat.begin());
      std::copy(skip.begin(), skip.end(), cat.begin() + x.size());
      x.swap(cat);
      for (int b = 0; b < 2; ++b) {
        const std::size_t oc = dims[stages - 2 - s];
        std::vector<float> o(oc * len);
        residual_forward(x.data(), len, up[s][b], cm.data(), o.data(), ws);
        x.swap(o);
        ch = oc;
      }
      const std::size_t lo = len * 2;
      std::vector<float> o(ch * lo);
      conv_transpose1d_kmajor(x.data(), us[s].w, us[s].b, o.data(), ch, ch, len, lo, 4, 2, 1, pool,
                              ws);
      x.swap(o);
      len = lo;
    }
    std::vector<float> fin(ch * len), res(A * len);
    conv1d(x.data(), fconv.w, fconv.b, fin.data(), ch, ch, len, len, K, 1, K / 2, pool, ws);
    group_norm(fin.data(), fnorm.w, fnorm.b, ch, len, 8);
    mish(fin.data(), fin.size());
    conv1d(fin.data(), fout.w, fout.b, res.data(), ch, A, len, len, 1, 1, 0, pool, ws);
    for (std::size_t tt = 0; tt < H; ++tt)
      for (std::size_t c = 0; c < A; ++c) eps[tt * A + c] = res[c * len + tt];
  }

  // diffusion.cc:979-1034 (host path).
  // `done` < steps stops after that many steps and returns the current sample in action units
  // (the state a resumable solve exposes between steps).
  void sample(const float* condv, const float* noise, std::size_t steps, int scheduler,
              std::uint64_t seed, float* action, std::size_t done) {
    const std::size_t n = A * H;
    std::vector<float> x(noise, noise + n), e(n);
    Gaussian gaussian(seed);
    const std::size_t ratio = T / steps;
    for (std::size_t i = 0; i < std::min(done, steps); ++i) {
      const std::size_t ts = (steps - 1 - i) * ratio;
      const std::ptrdiff_t prev = static_cast<std::ptrdiff_t>(ts) - static_cast<std::ptrdiff_t>(ratio);
      denoise(condv, x.data(), static_cast<float>(ts), e.data());
      const float at = alphas[ts];
      const float ap = prev >= 0 ? alphas[prev] : 1.0f;
      const float bt = 1.0f - at;
      if (scheduler == 0) {
        for (std::size_t v = 0; v < n; ++v) {
          float x0 = (x[v] - std::sqrt(bt) * e[v]) / std::sqrt(at);
          if (clip) x0 = std::min(std::max(x0, -clip_range), clip_range);
          x[v] = std::sqrt(ap) * x0 + std::sqrt(1.0f - ap) * e[v];
        }
      } else {
        const float ca = at / ap, cb = 1.0f - ca;
        const float oc = std::sqrt(ap) * cb / std::max(bt, 1e-20f);
        const float sc = std::sqrt(ca) * (1.0f - ap) / std::max(bt, 1e-20f);
        const float var = ((1.0f - ap) / std::max(bt, 1e-20f)) * cb;
        for (std::size_t v = 0; v < n; ++v) {
          float x0 = (x[v] - std::sqrt(bt) * e[v]) / std::sqrt(at);
          if (clip) x0 = std::min(std::max(x0, -clip_range), clip_range);
          float nx = oc * x0 + sc * x[v];
          if (prev >= 0) nx += std::sqrt(std::max(var, 1e-20f)) * gaussian.next();
          x[v] = nx;
        }
      }
    }
    for (std::size_t tt = 0; tt < H; ++tt)
      for (std::size_t c = 0; c < A; ++c) {
        const std::size_t i = tt * A + c;
        action[i] = (x[i] + 1.0f) * 0.5f * (amax[c] - amin[c]) + amin[c];
      }
  }

  // Flow-head ODE update (flow.cc:291-318, span_ops.h:27-52) with the U-Net as the velocity.
  // `done` < steps stops after that many ODE steps (flow.cc:260-318 advanced in bounded units).
  void sample_flow(const float* condv, const float* x0, std::size_t steps, int method, float* out,
                   std::size_t done) {
    const std::size_t n = A * H;
    std::vector<float> x(x0, x0 + n), k1(n), k2(n), k3(n), k4(n), probe(n);
    const float dt = 1.0f / static_cast<float>(steps);
    for (std::size_t s = 0; s < std::min(done, steps); ++s) {
      const float t = static_cast<float>(s) * dt;
      denoise(condv, x.data(), t, k1.data());
      if (method == 0) {
        for (std::size_t i = 0; i < n; ++i) x[i] += dt * k1[i];
      } else if (method == 1) {
        for (std::size_t i = 0; i < n; ++i) probe[i] = x[i] + dt * k1[i];
        denoise(condv, probe.data(), t + dt, k2.data());
        for (std::size_t i = 0; i < n; ++i) x[i] += 0.5f * dt * (k1[i] + k2[i]);
      } else {
        const float h = 0.5f * dt;
        for (std::size_t i = 0; i < n; ++i) probe[i] = x[i] + h * k1[i];
        denoise(condv, probe.data(), t + h, k2.data());
        for (std::size_t i = 0; i < n; ++i) probe[i] = x[i] + h * k2[i];
        denoise(condv, probe.data(), t + h, k3.data());
        for (std::size_t i = 0; i < n; ++i) probe[i] = x[i] + dt * k3[i];
        denoise(condv, probe.data(), t + dt, k4.data());
        for (std::size_t i = 0; i < n; ++i)
          x[i] += (dt / 6.0f) * (k1[i] + 2.0f * k2[i] + 2.0f * k3[i] + k4[i]);
      }
    }
    std::copy(x.begin(), x.end(), out);
  }
};

struct Handle {
  Model model;
  Pool* pool = nullptr;
  unsigned threads = 0;
};

thread_local std::string g_error;

}  // namespace

extern "C" {

const char* dpo_last_error(void) { return g_error.c_str(); }

// Load a dp.* safetensors checkpoint.  `threads` = worker threads for intra-op parallelism
// (0 = caller thread only, as the reference pool).
void* dpo_load(const char* path, unsigned threads) {
  g_error.clear();
  auto* h = new Handle();
  if (!read_safetensors(path, h->model.tensors)) {
    g_error = "cannot read safetensors";
    delete h;
    return nullptr;
  }
  if (!h->model.init()) {
    g_error = h->model.error;
    delete h;
    return nullptr;
  }
  h->threads = threads;
  if (threads > 0) h->pool = new Pool(threads);
  h->model.pool = h->pool;
  return h;
}

void dpo_free(void* handle) {
  auto* h = static_cast<Handle*>(handle);
  if (!h) return;
  delete h->pool;
  delete h;
}

// Fills [A, H, cond, stages, K, G, tdim, T, clip, pred, action_steps, obs] and dims[8].
int dpo_config(void* handle, std::uint64_t* out12, std::uint64_t* dims8, float* clip_range) {
  auto* h = static_cast<Handle*>(handle);
  if (!h) return 1;
  const Model& m = h->model;
  const std::uint64_t v[12] = {m.A, m.H, m.cond, m.stages, m.K, m.G, m.tdim, m.T, m.clip ? 1u : 0u,
                               m.pred, m.action_steps, m.obs};
  std::memcpy(out12, v, sizeof v);
  for (int i = 0; i < 8; ++i) dims8[i] = m.dims[i];
  *clip_range = m.clip_range;
  return 0;
}

int dpo_alphas_cumprod(void* handle, float* out) {
  auto* h = static_cast<Handle*>(handle);
  if (!h) return 1;
  std::copy(h->model.alphas.begin(), h->model.alphas.end(), out);
  return 0;
}

int dpo_denoise(void* handle, const float* cond, const float* sample, float t, float* eps) {
  auto* h = static_cast<Handle*>(handle);
  if (!h || !cond || !sample || !eps || !std::isfinite(t)) return 1;
  h->model.denoise(cond, sample, t, eps);
  return 0;
}

int dpo_sample(void* handle, const float* cond, const float* noise, std::size_t steps,
               int scheduler, std::uint64_t seed, float* action) {
  auto* h = static_cast<Handle*>(handle);
  if (!h || !cond || !noise || !action || steps == 0 || steps > h->model.T) return 1;
  if (scheduler != 0 && scheduler != 1) return 5;
  if (h->model.pred != 0) return 4;
  h->model.sample(cond, noise, steps, scheduler, seed, action, steps);
  return 0;
}

// The first `done` steps of dpo_sample / dpo_sample_flow (done <= steps).
int dpo_sample_partial(void* handle, const float* cond, const float* noise, std::size_t steps,
                       int scheduler, std::uint64_t seed, std::size_t done, float* action) {
  auto* h = static_cast<Handle*>(handle);
  if (!h || !cond || !noise || !action || steps == 0 || steps > h->model.T || done > steps)
    return 1;
  if (scheduler != 0 && scheduler != 1) return 5;
  if (h->model.pred != 0) return 4;
  h->model.sample(cond, noise, steps, scheduler, seed, action, done);
  return 0;
}

int dpo_sample_flow_partial(void* handle, const float* cond, const float* x0, std::size_t steps,
                            int method, std::size_t done, float* out) {
  auto* h = static_cast<Handle*>(handle);
  if (!h || !cond || !x0 || !out || steps == 0 || done > steps) return 1;
  if (method < 0 || method > 2) return 5;
  if (h->model.pred != 1) return 4;
  h->model.sample_flow(cond, x0, steps, method, out, done);
  return 0;
}

int dpo_sample_flow(void* handle, const float* cond, const float* x0, std::size_t steps,
                    int method, float* out) {
  auto* h = static_cast<Handle*>(handle);
  if (!h || !cond || !x0 || !out || steps == 0) return 1;
  if (method < 0 || method > 2) return 5;
  if (h->model.pred != 1) return 4;
  h->model.sample_flow(cond, x0, steps, method, out, steps);
  return 0;
}

// B independent samples spread over `workers` threads with shared weights (the reference's
// multi-engine model); each sample runs single-threaded.  kind 0 = DDIM/DDPM, 1 = flow.
int dpo_sample_batch(void* handle, std::size_t batch, const float* cond, const float* noise,
                     std::size_t steps, int kind, int mode, std::uint64_t seed, float* out,
                     unsigned workers) {
  auto* h = static_cast<Handle*>(handle);
  if (!h || batch == 0) return 1;
  Model& m = h->model;
  const std::size_t n = m.A * m.H;
  Pool* saved = m.pool;
  m.pool = nullptr;
  std::atomic<std::size_t> next{0};
  auto worker = [&]() {
    for (std::size_t b = next.fetch_add(1); b < batch; b = next.fetch_add(1)) {
      if (kind == 0)
        m.sample(cond + b * m.cond, noise + b * n, steps, mode, seed, out + b * n, steps);
      else
        m.sample_flow(cond + b * m.cond, noise + b * n, steps, mode, out + b * n, steps);
    }
  };
  std::vector<std::thread> th;
  for (unsigned i = 1; i < std::max(1u, workers); ++i) th.emplace_back(worker);
  worker();
  for (auto& t : th) t.join();
  m.pool = saved;
  return 0;
}

// ---- op-level entry points for unit tests ----
void dpo_mish(float* x, std::size_t n) { mish(x, n); }
void dpo_timestep_embedding(float t, float* out, std::size_t dim) { timestep_embedding(t, out, dim); }
void dpo_matmul(const float* in, const float* w, float* out, std::size_t rows, std::size_t in_dim,
                std::size_t out_dim) {
  matmul(in, w, out, rows, in_dim, out_dim, nullptr);
}
void dpo_conv1d(const float* x, const float* w, const float* b, float* y, std::size_t ic,
                std::size_t oc, std::size_t lin, std::size_t lout, std::size_t k,
                std::size_t stride, std::size_t pad) {
  std::vector<float> ws;
  conv1d(x, w, b, y, ic, oc, lin, lout, k, stride, pad, nullptr, ws);
}
// Weights in PyTorch ConvTranspose1d storage [IC][OC][K]; repacked k-major here.
void dpo_conv_transpose1d(const float* x, const float* w, const float* b, float* y,
                          std::size_t ic, std::size_t oc, std::size_t lin, std::size_t lout,
                          std::size_t k, std::size_t stride, std::size_t pad) {
  std::vector<float> wk(ic * oc * k), ws;
  for (std::size_t kk = 0; kk < k; ++kk)
    for (std::size_t i = 0; i < ic; ++i)
      for (std::size_t o = 0; o < oc; ++o) wk[(kk * oc + o) * ic + i] = w[(i * oc + o) * k + kk];
  conv_transpose1d_kmajor(x, wk.data(), b, y, ic, oc, lin, lout, k, stride, pad, nullptr, ws);
}
void dpo_group_norm(float* x, const float* w, const float* b, std::size_t c, std::size_t len,
                    std::size_t groups) {
  group_norm(x, w, b, c, len, groups);
}
// Gaussian stream of `n` values from `seed` (diffusion.cc:193-231).
void dpo_gaussian(std::uint64_t seed, float* out, std::size_t n) {
  Gaussian g(seed);
  for (std::size_t i = 0; i < n; ++i) out[i] = g.next();
}

}  // extern "C"
