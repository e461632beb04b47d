// Host runtime and C ABI of the MI355X Diffusion Policy engine.
//
// Mirrors the reference's split (src/core/api/engine.cc -> runtime/engine_runtime.cc ->
// heads/diffusion/diffusion.cc) for the Diffusion Policy path:
//   * load: mmap the dp.* checkpoint, validate dp.meta exactly as diffusion.cc:391-427 does
//     (plus prediction type 1 = velocity for the flow-ODE U-Net), plan ONE device arena for
//     repacked weights, FiLM tables, activations of `max_batch` samples and I/O buffers, then a
//     single hipMalloc and the uploads;
//   * sample: host -> pinned staging -> H2D, one hipGraph replay of the whole sampling loop (all
//     U-Net evaluations plus the DDIM/DDPM/ODE updates), D2H -> host.  A graph is captured once per
//     (kind, batch, steps, mode) and cached; replays allocate nothing.
//   * errors: int status codes and a thread-local message as engine.cc:22-26, 507-540.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <list>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "../../include/flowedge.h"
#include "kernels.h"
#include "safetensors.h"

namespace {

// ---------------------------------------------------------------------------------------------
// Thread-local last error (engine.cc:22-26): reset to "" at each ABI entry.
// ---------------------------------------------------------------------------------------------
thread_local const char* t_error = "";
thread_local std::string t_error_buf;

void set_error(const char* msg) { t_error = msg; }
void set_error(const std::string& msg) {
  t_error_buf = msg;
  t_error = t_error_buf.c_str();
}
void clear_error() { t_error = ""; }

std::atomic<std::uint64_t> g_device_allocs{0};

bool env_flag(const char* name) {
  const char* v = std::getenv(name);
  return v != nullptr && v[0] == '1' && v[1] == '\0';
}

constexpr unsigned kMaxPoolThreads = 8;  // engine_runtime.h:39
constexpr std::size_t kMaxStages = 8;    // diffusion.h:41
constexpr std::size_t kSplitKFloats = 1024 * 64 * 128;  // split-K partials: <= 1024 tiles of 64 x 128
// Largest batch whose convolutions run input-channel sliced (on the fused kernels; the matrix
// cores take over from 5 samples with F32 weights, 8 with BF16 weights).
// Smallest convolution (multiply-adds x 2, whole batch) whose 1x1 projection is forked to the
// side stream: the fork and join cost tens of microseconds of graph synchronization.
constexpr double kForkMinFlops = 2e10;

constexpr std::size_t kSliceBatch = 8;
// Largest batch whose matrix-core convolutions leave the partial sums of a split K loop in the
// output tensor for their consumers to add (larger batches split K rarely; those that do reduce
// through the split-K workspace).
constexpr std::size_t kPartBatch = 64;
constexpr std::size_t kFinalNormGroups = 8;  // diffusion.cc:28
constexpr std::size_t kAlign = 256;

// ---------------------------------------------------------------------------------------------
// Configuration (diffusion.h:19-33 / diffusion.cc:391-427).
// ---------------------------------------------------------------------------------------------
struct Config {
  std::size_t action_dim = 0, horizon = 0, action_steps = 0, obs_steps = 0, cond_dim = 0,
              stages = 0, kernel = 0, groups = 0, tdim = 0, train_timesteps = 0;
  std::size_t prediction = 0;  // 0 epsilon, 1 velocity
  bool clip = false;
  float clip_range = 1.0f;
  std::size_t dims[kMaxStages] = {};
};

bool size_value(float v, std::size_t& out) {
  if (!std::isfinite(v) || v < 0.0f || std::floor(v) != v || v > 4294967295.0f) return false;
  out = static_cast<std::size_t>(v);
  return true;
}

bool f32_vector(const fe::TensorInfo* t, std::size_t n) {
  return t != nullptr && !t->bf16 && t->shape.size() == 1 && t->shape[0] == n;
}

bool parse_config(const fe::Checkpoint& ck, Config& c, std::string& err) {
  const fe::TensorInfo* meta = ck.find("dp.meta");
  const fe::TensorInfo* dims = ck.find("dp.dims");
  if (!f32_vector(meta, 16) || dims == nullptr || dims->bf16 || dims->shape.size() != 1) {
    err = "Checkpoint has no valid Diffusion Policy head (dp.meta / dp.dims)";
    return false;
  }
  const float* m = static_cast<const float*>(meta->data);
  std::size_t schema, beta, norm, clip;
  const bool ok =
      size_value(m[0], schema) && size_value(m[1], c.action_dim) && size_value(m[2], c.horizon) &&
      size_value(m[3], c.action_steps) && size_value(m[4], c.obs_steps) &&
      size_value(m[5], c.cond_dim) && size_value(m[6], c.stages) && size_value(m[7], c.kernel) &&
      size_value(m[8], c.groups) && size_value(m[9], c.tdim) &&
      size_value(m[10], c.train_timesteps) && size_value(m[11], beta) &&
      size_value(m[12], c.prediction) && size_value(m[13], clip) && size_value(m[15], norm) &&
      schema == 1 && beta == 0 && c.prediction <= 1 && norm == 0 && clip <= 1 &&
      c.action_dim > 0 && c.horizon > 0 && c.action_steps > 0 && c.obs_steps > 0 &&
      c.obs_steps <= c.horizon && c.action_steps <= c.horizon - c.obs_steps + 1 &&
      c.cond_dim > 0 && c.stages >= 2 && c.stages <= kMaxStages && c.kernel > 0 &&
      c.kernel % 2 == 1 && c.groups > 0 && c.tdim >= 4 && c.tdim % 2 == 0 &&
      c.train_timesteps > 0 && dims->shape[0] == c.stages && std::isfinite(m[14]) && m[14] > 0.0f;
  if (!ok) {
    err = "Invalid dp.meta";
    return false;
  }
  c.clip = clip != 0;
  c.clip_range = m[14];
  const float* d = static_cast<const float*>(dims->data);
  for (std::size_t s = 0; s < c.stages; ++s)
    if (!size_value(d[s], c.dims[s]) || c.dims[s] == 0 || c.dims[s] % c.groups != 0) {
      err = "Invalid dp.dims";
      return false;
    }
  if (c.dims[0] % kFinalNormGroups != 0 || c.horizon % (std::size_t{1} << (c.stages - 1)) != 0) {
    err = "Invalid U-Net widths or horizon";
    return false;
  }
  return true;
}

// Limits of the device path beyond the reference's own validation (parse_config).  Shapes the
// specialised kernels have no instance for run on the general kernels, so only sizes that no
// kernel addresses are refused.
bool supported_shape(const Config& c, std::string& err) {
  if (5 * c.tdim * sizeof(float) > fe::hip::kMaxTimeMlpLds) {
    err = "Unsupported timestep embedding width (at most 8192)";
    return false;
  }
  // Widths, lengths and channel counts are kernel arguments of type int.
  std::size_t widest = c.cond_dim;
  for (std::size_t s = 0; s < c.stages; ++s) widest = std::max(widest, 2 * c.dims[s]);
  if (widest > (std::size_t{1} << 24) || c.horizon > (std::size_t{1} << 24) ||
      c.action_dim > (std::size_t{1} << 24) || c.kernel > 4095) {
    err = "Unsupported U-Net size";
    return false;
  }
  return true;
}

// ---------------------------------------------------------------------------------------------
// Arena planning: every buffer is an offset into one allocation.
// ---------------------------------------------------------------------------------------------
struct Plan {
  std::size_t size = 0;
  std::size_t take(std::size_t bytes) {
    const std::size_t off = (size + kAlign - 1) / kAlign * kAlign;
    size = off + bytes;
    return off;
  }
};

struct ConvSlot {
  fe::hip::ConvOp op;
  std::size_t w_off = 0, b_off = 0;
  const fe::TensorInfo* w_src = nullptr;
  const fe::TensorInfo* b_src = nullptr;
  bool transpose_storage = false;  // ConvTranspose1d [IC][OC][K]
  bool force_f32 = false;          // widened to fp32 in the arena (read by the fused epilogue)
};

struct NormSlot {
  std::size_t g_off = 0, b_off = 0;
  const fe::TensorInfo* g_src = nullptr;
  const fe::TensorInfo* b_src = nullptr;
};

struct Block {
  ConvSlot c1, c2, res;
  NormSlot n1, n2;
  bool identity = false;
  std::size_t ic = 0, oc = 0, len = 0;
  std::size_t film_off = 0;  // row offset of this block's 2*oc FiLM outputs
  const fe::TensorInfo* film_w = nullptr;
  const fe::TensorInfo* film_b = nullptr;
  int id = 0;  // index of the block's activation buffers in Work
};

// Residual blocks of a U-Net: 2 per down stage, 2 mid, 2 per up stage.
constexpr std::size_t kMaxBlocks = 4 * kMaxStages + 2;

// Per-call device buffers (the reference's WorkspacePlan, diffusion.cc:90-126,283-381): byte
// offsets from a workspace base, planned for a batch size and a number of FiLM time rows.  The
// engine's arena holds one Work for its max batch; the allocation-free denoise entry point plans
// another one inside the library's static scratch array.
struct Work {
  std::size_t size = 0;
  std::size_t batch = 0, film_rows = 0, splitk_floats = 0;
  std::size_t time_m = 0, film_table = 0, film_cond = 0;  // [rows][tdim], [rows][F], [B][F]
  std::size_t x_state = 0, x_in = 0, k_stages = 0;        // [B][A][H], [B][A][H], [4][B][A][H]
  std::size_t in_cond = 0, in_noise = 0, out_action = 0;  // caller I/O staged on the device
  std::size_t seed = 0;                                    // DDPM seed (8 bytes)
  std::size_t concat[kMaxStages] = {};  // up stage u input [x ; skip] buffer [B][2*high][len]
  std::size_t ds_out[kMaxStages] = {};  // downsample outputs [B][C][len/2]
  std::size_t us_out[kMaxStages] = {};  // sliced upsample outputs (partials) [B][S][C][2 len]
  // Raw convolution outputs (h1, h2, r, ds_out, us_out, fconv_out) hold, for batches up to
  // slice_batch (fused kernels) and part_batch (matrix cores), kMaxSlices partial sums per
  // sample ([B][kMaxSlices][C][L]).
  std::size_t slice_batch = 0, part_batch = 0;
  std::size_t h1[kMaxBlocks] = {}, h2[kMaxBlocks] = {};  // raw conv outputs [B][oc][len]
  std::size_t r[kMaxBlocks] = {};     // residual projection [B][oc][len] (non-identity blocks)
  std::size_t xmat[kMaxBlocks] = {};  // materialised block input [B][ic][len] (identity blocks)
  std::size_t final_in = 0, fconv_out = 0;  // [B][dims0][H]
  std::size_t xnorm = 0;   // batched path: normalised input of one convolution
  std::size_t splitk = 0;  // batched path: split-K partial tiles
  std::size_t upd_part = 0;  // split update: per-group partial outputs [B][8][A][H]
};

struct GraphEntry {
  int kind = 0, mode = 0;
  std::size_t batch = 0, steps = 0;
  hipGraphExec_t exec = nullptr;
  int chain_table = -1;  // persistent tick: index of its evaluation table, else -1
};

}  // namespace

// ---------------------------------------------------------------------------------------------
// Engine.
// ---------------------------------------------------------------------------------------------
struct FeWeights {
  std::shared_ptr<const fe::Checkpoint> ck;
};

struct FeEngine {
  Config cfg;
  unsigned threads = 0;
  int device = 0;
  std::size_t max_batch = 0;
  std::size_t values = 0;  // H * A
  bool bf16_convs = false, any_bf16 = false;

  // Arena: the weights region (load-time constants) followed by the workspace `w` for max_batch.
  char* arena = nullptr;
  std::size_t arena_bytes = 0;
  char* ws = nullptr;  // workspace base of `w`
  Work w;
  // The engine's own workspace base, and the split update's per-sample arrival counters (after
  // the workspace in the arena; zeroed at load, left at zero by every split update launch).
  char* own_ws = nullptr;
  unsigned* upd_done = nullptr;
  // This device's static scratch array (allocation-free entry point), set up at load.
  void* scratch = nullptr;
  hipError_t scratch_status = hipErrorNotInitialized;
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  // Side stream for a matrix-core convolution's 1x1 projection, forked from and joined back to
  // `stream` (in a captured graph: two parallel nodes).
  hipStream_t side = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  float last_ms = -1.0f;
  bool timed = false;

  // Host pinned staging.
  float* pin_cond = nullptr;
  float* pin_noise = nullptr;
  float* pin_action = nullptr;
  std::uint64_t* pin_seed = nullptr;

  // Layout.
  std::size_t te1w = 0, te1b = 0, te2w = 0, te2b = 0;
  std::size_t film_wt = 0, film_wc = 0, film_bias = 0, film_total = 0;
  std::size_t amin = 0, amax = 0;
  Block down[kMaxStages][2];
  ConvSlot ds[kMaxStages];
  Block mid[2];
  Block up[kMaxStages][2];
  ConvSlot us[kMaxStages];
  ConvSlot fconv, fout;
  NormSlot fnorm;
  int blocks = 0;  // residual blocks (Work buffer ids 0 .. blocks-1)
  std::size_t max_nfe = 0;
  std::size_t ddim_table = 0;  // FiLM time rows for every train timestep [T][F] (epsilon models)
  // Velocity models: FiLM time rows of the flow solves sampled so far, per (steps, method), in a
  // pool of flow_pool_rows rows [row][F] (DDIM's table counterpart; the solve's evaluation times
  // depend on its step count and method).
  struct FlowTable {
    std::size_t steps = 0;
    int method = 0;
    std::size_t row0 = 0;
  };
  std::size_t flow_pool = 0, flow_pool_rows = 0, flow_pool_used = 0;
  std::vector<FlowTable> flow_tables;
  std::size_t mfma_batch = 4;  // batches of at least this many samples use the matrix cores
  // Input-channel slicing of the fused convolutions (batches below mfma_batch, up to the Work's
  // slice_batch): on when every convolution of the model runs fused and the final update sums
  // partials; slice_max (FLOWEDGE_SLICES, default kMaxSlices; 1 turns slicing off) caps it.
  bool slice_ok = false;
  // Matrix-core convolutions leave split-K partial sums for their consumers (batches from
  // mfma_batch up to the Work's part_batch): on when every convolution runs on the matrix cores
  // there and the update sums partials; FLOWEDGE_MM_PARTS=0 turns it off.
  bool mm_parts_ok = false;
  int slice_max = fe::hip::kMaxSlices;
  int slice_tpr = 0;  // lanes per row of the sliced kernels (FLOWEDGE_SLICE_TPR; 0: per shape)
  std::size_t records_batch = 0;  // batch conv_records were listed for (0: none)
  int records_mode = -1;          // and their partial-sum mode (0 none, 1 sliced, 2 matrix)
  bool bf16_mma = true;        // BF16 weights on the BF16 matrix cores (split input)
  bool f32_split = false;      // F32 weights on the BF16 matrix cores (split weights and input)

  std::list<GraphEntry> graphs;  // most recently used first
  std::uint64_t captures = 0;    // graphs captured and instantiated so far

  // Persistent batch-1 tick (chain.hip): one launch runs every evaluation of a tick.
  bool chain_on = false;          // B=1 sampling ticks use the tick kernel
  std::string chain_why = "not built";  // why they do not
  int chain_nsteps = 0;
  std::size_t chain_steps = 0;    // step table [kMaxChainSteps]
  std::size_t chain_flags = 0, chain_abort = 0, chain_slots = 0;
  std::size_t chain_tables = 0;   // kChainTables evaluation tables of kMaxChainEvals entries
  int chain_slot_floats = 0;
  std::uint64_t chain_abandoned = 0;  // ticks the kernel gave up on (re-run on per-layer graphs)
  unsigned* pin_status = nullptr;     // the tick's abort flag, copied back after each tick

  // Model identity (engine_runtime.cc:159-161).
  std::array<std::uint8_t, 16> digest{};
  std::uint32_t precision = 0;

  // The one resumable solve of this engine (engine.h:321-366; engine_runtime.cc:494-561).
  // `graphs[0]` starts the solve from the input buffers, `graphs[1 + i]` runs step i and writes
  // the current action; they are kept while later solves have the same kind, step count and mode.
  // Any other sampling or denoising call reuses the state buffers and ends the solve.
  struct Solve {
    bool active = false, cancelled = false, tracking = false;
    int kind = 0, mode = 0;
    std::size_t steps = 0, next = 0;
    std::uint64_t timestamp_ns = 0, deadline_ns = 0, generation = 0;
    int g_kind = -1, g_mode = -1;
    std::size_t g_steps = 0;
    std::vector<hipGraphExec_t> graphs;
    std::size_t remaining() const { return steps - next; }
  } solve;
  // Highest generation announced by fe_engine_cancel_before or a tracked begin; the only state
  // another thread may touch while a solve advances.
  std::atomic<std::uint64_t> latest_generation{0};

  // Diagnostics: every fused convolution of one U-Net evaluation, recorded from an eager run.
  struct ConvRecord {
    std::string name;
    fe::hip::ConvOp op;
    bool has_res = false;
    fe::hip::ConvOp res;
    fe::hip::ConvInput in;
    fe::hip::View y, yr;
    fe::hip::SlicePlan slices;
    std::uint64_t weight_bytes = 0;  // weights + biases
    std::uint64_t sample_bytes = 0;  // activations and per-channel parameters, per sample
  };
  std::vector<ConvRecord> conv_records;
  bool recording = false;  // conv() keeps the arguments of every convolution it enqueues
  bool dry = false;        // and enqueues nothing (the U-Net walk only lists its convolutions)

  template <typename T = float>
  T* ptr(std::size_t off) const {
    return reinterpret_cast<T*>(arena + off);
  }
  // A workspace buffer of the current Work.
  template <typename T = float>
  T* wp(std::size_t off) const {
    return reinterpret_cast<T*>(ws + off);
  }

  ~FeEngine() {
    for (auto& g : graphs)
      if (g.exec) (void)hipGraphExecDestroy(g.exec);
    for (hipGraphExec_t g : solve.graphs)
      if (g) (void)hipGraphExecDestroy(g);
    if (ev0) (void)hipEventDestroy(ev0);
    if (ev1) (void)hipEventDestroy(ev1);
    if (fork) (void)hipEventDestroy(fork);
    if (join) (void)hipEventDestroy(join);
    if (side) (void)hipStreamDestroy(side);
    if (stream) (void)hipStreamDestroy(stream);
    if (arena) (void)hipFree(arena);
    if (pin_cond) (void)hipHostFree(pin_cond);
  }
};

// ABI layouts fixed by protocol/contracts.h:139-142.
static_assert(sizeof(fe_model_digest) == 16);
static_assert(sizeof(fe_model_metadata) == 96);
static_assert(sizeof(fe_condition_metadata) == 88);
static_assert(sizeof(fe_action_metadata) == 80);

namespace {

constexpr std::size_t kGraphCache = 32;
// Persistent ticks: one evaluation table per cached graph, of at most this many evaluations
// (longer solves run on per-layer graphs).
constexpr std::size_t kChainTables = kGraphCache;
constexpr std::size_t kMaxChainEvals = 128;
// Velocity models: FiLM time rows kept for flow solves (RK4-4 takes 16, Euler-10 10; pusht-size
// rows are 115 KB each).
constexpr std::size_t kFlowPoolRows = 256;

void end_solve(FeEngine* e);

// Sizing and validation of the weights; fills the slots and offsets.
struct Builder {
  FeEngine& e;
  const fe::Checkpoint& ck;
  Plan plan;
  std::string err;

  bool conv(const std::string& p, std::size_t oc, std::size_t ic, std::size_t k, int mode,
            ConvSlot& s, bool transpose_storage = false, bool force_f32 = false) {
    const fe::TensorInfo* w = ck.find(p + ".w");
    const fe::TensorInfo* b = ck.find(p + ".b");
    if (w == nullptr || w->shape.size() != 3 || w->shape[0] != (transpose_storage ? ic : oc) ||
        w->shape[1] != (transpose_storage ? oc : ic) || w->shape[2] != k || !f32_vector(b, oc)) {
      err = "Missing or malformed convolution " + p;
      return false;
    }
    s.w_src = w;
    s.b_src = b;
    s.transpose_storage = transpose_storage;
    s.force_f32 = force_f32;
    s.op.bf16 = w->bf16 && !force_f32;
    s.op.mode = mode;
    s.op.k = static_cast<int>(k);
    s.op.ic = static_cast<int>(ic);
    s.op.oc = static_cast<int>(oc);
    s.w_off = plan.take(w->elements() * (s.op.bf16 ? 2 : 4));
    s.b_off = plan.take(oc * 4);
    if (w->bf16) e.bf16_convs = true, e.any_bf16 = true;
    return true;
  }

  bool norm(const std::string& p, std::size_t c, NormSlot& n) {
    n.g_src = ck.find(p + ".w");
    n.b_src = ck.find(p + ".b");
    if (!f32_vector(n.g_src, c) || !f32_vector(n.b_src, c)) {
      err = "Missing or malformed GroupNorm " + p;
      return false;
    }
    n.g_off = plan.take(c * 4);
    n.b_off = plan.take(c * 4);
    return true;
  }

  bool linear_shape(const std::string& p, std::size_t out, std::size_t in,
                    const fe::TensorInfo*& w, const fe::TensorInfo*& b) {
    w = ck.find(p + ".w");
    b = ck.find(p + ".b");
    if (w == nullptr || w->shape.size() != 2 || w->shape[0] != out || w->shape[1] != in ||
        !f32_vector(b, out)) {
      err = "Missing or malformed linear " + p;
      return false;
    }
    if (w->bf16) e.any_bf16 = true;
    return true;
  }

  bool block(const std::string& p, std::size_t ic, std::size_t oc, std::size_t len, Block& blk) {
    const Config& c = e.cfg;
    blk.ic = ic;
    blk.oc = oc;
    blk.len = len;
    blk.identity = ic == oc;
    if (!conv(p + ".c1", oc, ic, c.kernel, fe::hip::kConvSame, blk.c1) ||
        !norm(p + ".n1", oc, blk.n1) ||
        !linear_shape(p + ".film", 2 * oc, c.tdim + c.cond_dim, blk.film_w, blk.film_b) ||
        !conv(p + ".c2", oc, oc, c.kernel, fe::hip::kConvSame, blk.c2) ||
        !norm(p + ".n2", oc, blk.n2))
      return false;
    if (!blk.identity && !conv(p + ".res", oc, ic, 1, fe::hip::kConvSame, blk.res)) return false;
    blk.film_off = e.film_total;
    e.film_total += 2 * oc;
    blk.id = e.blocks++;
    for (ConvSlot* s : {&blk.c1, &blk.c2, &blk.res}) {
      s->op.lin = static_cast<int>(len);
      s->op.lout = static_cast<int>(len);
    }
    return true;
  }

  bool build() {
    Config& c = e.cfg;
    const fe::TensorInfo *w, *b;
    if (!linear_shape("dp.te1", 4 * c.tdim, c.tdim, w, b)) return false;
    e.te1w = plan.take(w->elements() * 4);
    e.te1b = plan.take(b->elements() * 4);
    if (!linear_shape("dp.te2", c.tdim, 4 * c.tdim, w, b)) return false;
    e.te2w = plan.take(w->elements() * 4);
    e.te2b = plan.take(b->elements() * 4);
    const fe::TensorInfo* amin = ck.find("dp.action_min");
    const fe::TensorInfo* amax = ck.find("dp.action_max");
    if (!f32_vector(amin, c.action_dim) || !f32_vector(amax, c.action_dim)) {
      err = "Missing or malformed action range";
      return false;
    }
    const float* mn = static_cast<const float*>(amin->data);
    const float* mx = static_cast<const float*>(amax->data);
    for (std::size_t i = 0; i < c.action_dim; ++i)
      if (!std::isfinite(mn[i]) || !std::isfinite(mx[i]) || mx[i] <= mn[i]) {
        err = "Invalid action range";
        return false;
      }
    e.amin = plan.take(c.action_dim * 4);
    e.amax = plan.take(c.action_dim * 4);

    // Down path.
    std::size_t len = c.horizon;
    for (std::size_t s = 0; s < c.stages; ++s) {
      const std::size_t ic = s == 0 ? c.action_dim : c.dims[s - 1];
      const std::string p = "dp.d" + std::to_string(s);
      if (!block(p + ".r0", ic, c.dims[s], len, e.down[s][0]) ||
          !block(p + ".r1", c.dims[s], c.dims[s], len, e.down[s][1]))
        return false;
      if (s + 1 < c.stages) {
        if (!conv(p + ".ds", c.dims[s], c.dims[s], 3, fe::hip::kConvDown, e.ds[s])) return false;
        e.ds[s].op.lin = static_cast<int>(len);
        e.ds[s].op.lout = static_cast<int>(len / 2);
        len /= 2;
      }
    }
    const std::size_t bottom = c.dims[c.stages - 1];
    for (int m = 0; m < 2; ++m)
      if (!block("dp.m" + std::to_string(m), bottom, bottom, len, e.mid[m])) return false;
    for (std::size_t u = 0; u + 1 < c.stages; ++u) {
      const std::size_t high = c.dims[c.stages - 1 - u], low = c.dims[c.stages - 2 - u];
      const std::string p = "dp.u" + std::to_string(u);
      if (!block(p + ".r0", 2 * high, low, len, e.up[u][0]) ||
          !block(p + ".r1", low, low, len, e.up[u][1]) ||
          !conv(p + ".us", low, low, 4, fe::hip::kConvTranspose, e.us[u], true))
        return false;
      e.us[u].op.lin = static_cast<int>(len);
      e.us[u].op.lout = static_cast<int>(2 * len);
      len *= 2;
    }
    if (!conv("dp.f.c", c.dims[0], c.dims[0], c.kernel, fe::hip::kConvSame, e.fconv) ||
        !norm("dp.f.n", c.dims[0], e.fnorm) ||
        !conv("dp.f.o", c.action_dim, c.dims[0], 1, fe::hip::kConvSame, e.fout, false, true))
      return false;
    e.fconv.op.lin = e.fconv.op.lout = static_cast<int>(c.horizon);
    e.fout.op.lin = e.fout.op.lout = static_cast<int>(c.horizon);

    // FiLM tables: W_t^T [tdim][F], W_c^T [cond][F], bias [F].
    const std::size_t F = e.film_total;
    e.film_wt = plan.take(c.tdim * F * 4);
    e.film_wc = plan.take(c.cond_dim * F * 4);
    e.film_bias = plan.take(F * 4);
    if (c.prediction == 0) e.ddim_table = plan.take(c.train_timesteps * F * 4);
    if (c.prediction == 1) {
      e.flow_pool_rows = kFlowPoolRows;
      e.flow_pool = plan.take(kFlowPoolRows * F * 4);
    }
    // U-Net evaluations per call: diffusion <= T steps, flow RK4 4 per step.
    e.max_nfe = std::max<std::size_t>(c.train_timesteps, 1024);
    // Persistent tick: step table, per-workgroup counters and state slots (x, xin and four flow
    // stages), evaluation tables.
    const std::size_t v = c.horizon * c.action_dim;
    if (fe::hip::chain_supported_horizon(static_cast<int>(c.horizon)) && c.action_dim <= 64) {
      e.chain_steps = plan.take(fe::hip::kMaxChainSteps * fe::hip::chain_step_bytes());
      e.chain_flags = plan.take(fe::hip::kChainGrid * fe::hip::kChainFlagStride * 4);
      e.chain_abort = plan.take(4);
      e.chain_slot_floats = static_cast<int>((6 * v + 63) / 64 * 64);
      e.chain_slots = plan.take(static_cast<std::size_t>(fe::hip::kChainGrid) *
                                e.chain_slot_floats * 4);
      e.chain_tables = plan.take(kChainTables * kMaxChainEvals * sizeof(fe::hip::ChainEval));
    }
    return true;
  }
};

// Workspace of `batch` samples with `rows` FiLM time rows and up to `splitk_floats` of split-K
// partials.  Raw conv outputs per block; a block input is materialised (by the next op's prologue)
// only when it is needed again as an identity residual.
Work plan_work(const FeEngine& e, std::size_t batch, std::size_t rows, std::size_t splitk_floats) {
  const Config& c = e.cfg;
  const std::size_t B = batch, F = e.film_total, v = c.horizon * c.action_dim;
  Plan plan;
  Work w;
  w.batch = batch;
  w.film_rows = rows;
  w.splitk_floats = splitk_floats;
  w.time_m = plan.take(rows * c.tdim * 4);
  w.film_table = plan.take(rows * F * 4);
  w.film_cond = plan.take(B * F * 4);
  w.x_state = plan.take(B * v * 4);
  w.x_in = plan.take(B * v * 4);
  w.k_stages = plan.take(4 * B * v * 4);
  w.in_cond = plan.take(B * c.cond_dim * 4);
  w.in_noise = plan.take(B * v * 4);
  w.out_action = plan.take(B * v * 4);
  w.seed = plan.take(8);
  for (std::size_t u = 0; u + 1 < c.stages; ++u) {
    const Block& r0 = e.up[u][0];
    w.concat[u] = plan.take(B * r0.ic * r0.len * 4);
  }
  w.slice_batch = std::min(B, kSliceBatch);
  w.part_batch = std::min(B, kPartBatch);
  const std::size_t PB =
      std::max(B, static_cast<std::size_t>(fe::hip::kMaxSlices) *
                      std::max(w.slice_batch, w.part_batch));
  auto acts = [&](const Block& blk) {
    w.h1[blk.id] = plan.take(PB * blk.oc * blk.len * 4);
    w.h2[blk.id] = plan.take(PB * blk.oc * blk.len * 4);
    if (!blk.identity) w.r[blk.id] = plan.take(PB * blk.oc * blk.len * 4);
    else w.xmat[blk.id] = plan.take(B * blk.ic * blk.len * 4);
  };
  for (std::size_t s = 0; s < c.stages; ++s) {
    for (int k = 0; k < 2; ++k) acts(e.down[s][k]);
    if (s + 1 < c.stages) w.ds_out[s] = plan.take(PB * c.dims[s] * (e.down[s][1].len / 2) * 4);
  }
  for (int m = 0; m < 2; ++m) acts(e.mid[m]);
  for (std::size_t u = 0; u + 1 < c.stages; ++u) {
    for (int k = 0; k < 2; ++k) acts(e.up[u][k]);
    w.us_out[u] = plan.take(PB * e.us[u].op.oc * e.us[u].op.lout * 4);
  }
  w.final_in = plan.take(B * c.dims[0] * c.horizon * 4);
  w.fconv_out = plan.take(PB * c.dims[0] * c.horizon * 4);
  // Largest normalised activation (width * length of any block output).
  std::size_t norm_floats = 0;
  for (std::size_t st = 0; st < c.stages; ++st)
    norm_floats = std::max(norm_floats, c.dims[st] * (c.horizon >> st));
  w.xnorm = plan.take(B * norm_floats * 4);
  w.splitk = plan.take(splitk_floats * 4);
  w.upd_part = plan.take(B * kFinalNormGroups * v * 4);
  w.size = plan.size;
  return w;
}

// ---------------------------------------------------------------------------------------------
// Uploads with repacking.
// ---------------------------------------------------------------------------------------------
hipError_t upload(void* dst, const void* src, std::size_t bytes) {
  return hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
}

void widen(const fe::TensorInfo* t, std::vector<float>& out) {
  const std::size_t n = t->elements();
  out.resize(n);
  if (!t->bf16) {
    std::memcpy(out.data(), t->data, n * 4);
  } else {
    const auto* bits = static_cast<const std::uint16_t*>(t->data);
    for (std::size_t i = 0; i < n; ++i) {
      const std::uint32_t w = static_cast<std::uint32_t>(bits[i]) << 16;
      std::memcpy(&out[i], &w, 4);
    }
  }
}

// Conv [OC][IC][K] (or ConvTranspose [IC][OC][K]) -> [OC][K][IC], keeping the storage dtype.
hipError_t upload_conv(FeEngine& e, const ConvSlot& s) {
  const auto* w = s.w_src;
  const std::size_t oc = s.op.oc, ic = s.op.ic, k = s.op.k;
  const std::size_t src_esz = w->bf16 ? 2 : 4;
  const std::size_t esz = s.op.bf16 ? 2 : 4;
  std::vector<char> packed(oc * ic * k * esz);
  const char* src = static_cast<const char*>(w->data);
  for (std::size_t o = 0; o < oc; ++o)
    for (std::size_t kk = 0; kk < k; ++kk)
      for (std::size_t i = 0; i < ic; ++i) {
        const std::size_t from = s.transpose_storage ? (i * oc + o) * k + kk : (o * ic + i) * k + kk;
        char* dst = &packed[((o * k + kk) * ic + i) * esz];
        if (esz == src_esz) {
          std::memcpy(dst, src + from * src_esz, esz);
        } else {  // BF16 -> F32
          std::uint16_t bits;
          std::memcpy(&bits, src + from * 2, 2);
          const std::uint32_t wide = static_cast<std::uint32_t>(bits) << 16;
          std::memcpy(dst, &wide, 4);
        }
      }
  hipError_t st = upload(e.ptr<char>(s.w_off), packed.data(), packed.size());
  if (st != hipSuccess) return st;
  return upload(e.ptr<char>(s.b_off), s.b_src->data, oc * 4);
}

hipError_t upload_norm(FeEngine& e, const NormSlot& n) {
  hipError_t st = upload(e.ptr<char>(n.g_off), n.g_src->data, n.g_src->bytes);
  if (st != hipSuccess) return st;
  return upload(e.ptr<char>(n.b_off), n.b_src->data, n.b_src->bytes);
}

hipError_t upload_block(FeEngine& e, const Block& b, std::vector<float>& wt, std::vector<float>& wc,
                        std::vector<float>& bias) {
  hipError_t st;
  if ((st = upload_conv(e, b.c1)) != hipSuccess || (st = upload_conv(e, b.c2)) != hipSuccess ||
      (st = upload_norm(e, b.n1)) != hipSuccess || (st = upload_norm(e, b.n2)) != hipSuccess)
    return st;
  if (!b.identity && (st = upload_conv(e, b.res)) != hipSuccess) return st;
  // FiLM linear [2 oc][tdim + cond] split into the transposed time and condition tables.
  std::vector<float> w;
  widen(b.film_w, w);
  const std::size_t F = e.film_total, td = e.cfg.tdim, cd = e.cfg.cond_dim;
  const float* bb = static_cast<const float*>(b.film_b->data);
  for (std::size_t r = 0; r < 2 * b.oc; ++r) {
    const std::size_t f = b.film_off + r;
    for (std::size_t k = 0; k < td; ++k) wt[k * F + f] = w[r * (td + cd) + k];
    for (std::size_t k = 0; k < cd; ++k) wc[k * F + f] = w[r * (td + cd) + td + k];
    bias[f] = bb[r];
  }
  return hipSuccess;
}

hipError_t upload_weights(FeEngine& e, const fe::Checkpoint& ck) {
  const Config& c = e.cfg;
  hipError_t st;
  std::vector<float> tmp;
  auto linear = [&](const char* name, std::size_t woff, std::size_t boff) -> hipError_t {
    const std::string p(name);
    widen(ck.find(p + ".w"), tmp);
    hipError_t s = upload(e.ptr<char>(woff), tmp.data(), tmp.size() * 4);
    if (s != hipSuccess) return s;
    const fe::TensorInfo* b = ck.find(p + ".b");
    return upload(e.ptr<char>(boff), b->data, b->bytes);
  };
  if ((st = linear("dp.te1", e.te1w, e.te1b)) != hipSuccess) return st;
  if ((st = linear("dp.te2", e.te2w, e.te2b)) != hipSuccess) return st;
  if ((st = upload(e.ptr<char>(e.amin), ck.find("dp.action_min")->data, c.action_dim * 4)) !=
          hipSuccess ||
      (st = upload(e.ptr<char>(e.amax), ck.find("dp.action_max")->data, c.action_dim * 4)) !=
          hipSuccess)
    return st;
  const std::size_t F = e.film_total;
  std::vector<float> wt(c.tdim * F), wc(c.cond_dim * F), bias(F);
  for (std::size_t s = 0; s < c.stages; ++s) {
    for (int k = 0; k < 2; ++k)
      if ((st = upload_block(e, e.down[s][k], wt, wc, bias)) != hipSuccess) return st;
    if (s + 1 < c.stages && (st = upload_conv(e, e.ds[s])) != hipSuccess) return st;
  }
  for (int m = 0; m < 2; ++m)
    if ((st = upload_block(e, e.mid[m], wt, wc, bias)) != hipSuccess) return st;
  for (std::size_t u = 0; u + 1 < c.stages; ++u) {
    for (int k = 0; k < 2; ++k)
      if ((st = upload_block(e, e.up[u][k], wt, wc, bias)) != hipSuccess) return st;
    if ((st = upload_conv(e, e.us[u])) != hipSuccess) return st;
  }
  if ((st = upload_conv(e, e.fconv)) != hipSuccess || (st = upload_norm(e, e.fnorm)) != hipSuccess ||
      (st = upload_conv(e, e.fout)) != hipSuccess)
    return st;
  if ((st = upload(e.ptr<char>(e.film_wt), wt.data(), wt.size() * 4)) != hipSuccess ||
      (st = upload(e.ptr<char>(e.film_wc), wc.data(), wc.size() * 4)) != hipSuccess ||
      (st = upload(e.ptr<char>(e.film_bias), bias.data(), bias.size() * 4)) != hipSuccess)
    return st;
  return hipSuccess;
}

// Fills device pointers of the conv ops once the arena base is known.
void bind(FeEngine& e, ConvSlot& s) {
  s.op.w = e.arena + s.w_off;
  s.op.b = e.ptr(s.b_off);
}

void bind_all(FeEngine& e) {
  const Config& c = e.cfg;
  auto blk = [&](Block& b) {
    bind(e, b.c1);
    bind(e, b.c2);
    if (!b.identity) bind(e, b.res);
  };
  for (std::size_t s = 0; s < c.stages; ++s) {
    blk(e.down[s][0]);
    blk(e.down[s][1]);
    if (s + 1 < c.stages) bind(e, e.ds[s]);
  }
  blk(e.mid[0]);
  blk(e.mid[1]);
  for (std::size_t u = 0; u + 1 < c.stages; ++u) {
    blk(e.up[u][0]);
    blk(e.up[u][1]);
    bind(e, e.us[u]);
  }
  bind(e, e.fconv);
  bind(e, e.fout);
}

// ---------------------------------------------------------------------------------------------
// Enqueue helpers.
// ---------------------------------------------------------------------------------------------
#define FE_TRY(expr)                         \
  do {                                       \
    const hipError_t fe_st_ = (expr);        \
    if (fe_st_ != hipSuccess) return fe_st_; \
  } while (0)

hipError_t dispatch_conv(FeEngine& e, const fe::hip::ConvOp& op, const fe::hip::ConvOp* res,
                         const fe::hip::ConvInput& in, fe::hip::View y, fe::hip::View yr,
                         int batch, hipStream_t s, fe::hip::SlicePlan slices = {});
enum class ConvPath : int { kFused = 0, kMatrix = 1, kGeneral = 2 };
ConvPath conv_path(const FeEngine& e, const fe::hip::ConvOp& op, const fe::hip::ConvOp* res,
                   const fe::hip::ConvInput& in, fe::hip::View yr, int batch);

// Launches one fused convolution (`slices` input-channel slices); while recording, also keeps its
// arguments and algorithmic bytes (each weight and bias once, each activation and per-channel
// parameter once per sample).
hipError_t conv(FeEngine& e, const std::string& site, const fe::hip::ConvOp& op,
                const fe::hip::ConvOp* res, const fe::hip::ConvInput& in, fe::hip::View y,
                fe::hip::View yr, int batch, hipStream_t s, fe::hip::SlicePlan slices = {}) {
  if (e.recording) {
    FeEngine::ConvRecord r;
    const char* kind = !in.norm ? "plain" : (in.film_time != nullptr ? "film" : "resid");
    const char* mode = op.mode == fe::hip::kConvSame ? "" : (op.mode == fe::hip::kConvDown ? " down" : " up");
    char shape[128];
    std::snprintf(shape, sizeof shape, " [%d<-%d K%d L%d%s %s%s]", op.oc, op.ic, op.k, op.lin, mode,
                  kind, res != nullptr ? " +1x1" : "");
    r.name = site + shape;
    r.op = op;
    r.has_res = res != nullptr;
    if (res != nullptr) r.res = *res;
    r.in = in;
    r.y = y;
    r.yr = yr;
    r.slices = slices;
    const std::uint64_t es = op.bf16 ? 2 : 4;
    r.weight_bytes = static_cast<std::uint64_t>(op.oc) * op.k * op.ic * es + op.oc * 4ull;
    std::uint64_t sb = static_cast<std::uint64_t>(op.ic) * op.lin * 4 +
                       static_cast<std::uint64_t>(op.oc) * op.lout * 4;
    if (res != nullptr) {
      r.weight_bytes += static_cast<std::uint64_t>(res->oc) * res->ic * (res->bf16 ? 2 : 4) +
                        res->oc * 4ull;
      sb += static_cast<std::uint64_t>(res->oc) * op.lout * 4;
    }
    if (in.norm) {
      sb += 2ull * in.split * 4;                                   // gamma, beta
      if (in.film_time != nullptr) sb += 4ull * in.split * 4;      // time and condition FiLM rows
      if (in.res != nullptr) sb += static_cast<std::uint64_t>(in.split) * op.lin * 4;
      if (in.mat != nullptr) sb += static_cast<std::uint64_t>(in.split) * op.lin * 4;
    }
    r.sample_bytes = sb;
    e.conv_records.push_back(std::move(r));
  }
  if (e.dry) return hipSuccess;
  return dispatch_conv(e, op, res, in, y, yr, batch, s, slices);
}

// Kernels a convolution runs on at this batch size: the fused weight-streaming kernels (few
// samples), the matrix cores (many samples), or the general-shape kernels when neither has an
// instance for the shape.
ConvPath conv_path(const FeEngine& e, const fe::hip::ConvOp& op, const fe::hip::ConvOp* res,
                   const fe::hip::ConvInput& in, fe::hip::View yr, int batch) {
  using namespace fe::hip;
  const bool plain_ok = in.split == op.ic || in.plain != nullptr;
  const bool mm_ok = plain_ok && conv_mfma_supported(op, in.split) &&
                     (res == nullptr || conv_mfma_supported(*res, in.split));
  const bool fused_ok = conv_fused_supported(op, res, in, yr, batch);
  if (mm_ok && (static_cast<std::size_t>(batch) >= e.mfma_batch || !fused_ok))
    return ConvPath::kMatrix;
  return fused_ok ? ConvPath::kFused : ConvPath::kGeneral;
}

// Runs one fused convolution on the kernels chosen for this batch size.  Sliced convolutions
// run on the fused kernels; matrix-core convolutions may leave split-K partial sums (`slices`,
// planned by plan_of) and add those of their input in the GroupNorm pass (or a summing pass for
// plain inputs); the general kernels read single tensors.
hipError_t dispatch_conv(FeEngine& e, const fe::hip::ConvOp& op, const fe::hip::ConvOp* res,
                         const fe::hip::ConvInput& in, fe::hip::View y, fe::hip::View yr,
                         int batch, hipStream_t s, fe::hip::SlicePlan slices) {
  using namespace fe::hip;
  if (!slices.matrix && (slices.slices > 1 || in.parts > 1 || in.res_parts > 1))
    return conv_fused(op, res, in, y, yr, batch, s, slices);
  const ConvPath path = conv_path(e, op, res, in, yr, batch);
  if (path == ConvPath::kGeneral && (in.parts > 1 || in.res_parts > 1)) return hipErrorInvalidValue;
  if (path == ConvPath::kGeneral) {
    // General shapes: the prologue as its own pass, then the FP32 implicit GEMM.
    const float* src = in.src;
    std::int64_t ss = in.src_stride;
    if (in.norm) {
      float* dst = in.mat != nullptr ? in.mat : e.wp(e.w.xnorm);
      const std::int64_t ds =
          in.mat != nullptr ? in.mat_stride : static_cast<std::int64_t>(in.split) * op.lin;
      FE_TRY(norm_act(in, op.lin, dst, ds, batch, s));
      src = dst;
      ss = ds;
    }
    float* ws = e.wp(e.w.splitk);
    const std::size_t wsf = e.w.splitk_floats;
    FE_TRY(conv_general(op, src, ss, in.split, in.plain, in.plain_stride, y, batch, ws, wsf, s));
    if (res != nullptr)
      FE_TRY(conv_general(*res, src, ss, in.split, in.plain, in.plain_stride, yr, batch, ws, wsf,
                          s));
    return hipSuccess;
  }
  if (path == ConvPath::kMatrix) {
    // Many samples: the prologue as its own pass (adding the producer's partial sums), then
    // implicit GEMMs on the matrix cores.
    const float* src = in.src;
    std::int64_t ss = in.src_stride;
    if (in.norm) {
      float* dst = in.mat != nullptr ? in.mat : e.wp(e.w.xnorm);
      const std::int64_t ds =
          in.mat != nullptr ? in.mat_stride : static_cast<std::int64_t>(in.split) * op.lin;
      FE_TRY(norm_act(in, op.lin, dst, ds, batch, s));
      src = dst;
      ss = ds;
    } else if (in.parts > 1) {
      const std::int64_t n = static_cast<std::int64_t>(in.split) * op.lin;
      FE_TRY(sum_parts(in.src, in.src_stride, in.parts, in.part_stride, n, e.wp(e.w.xnorm), n,
                       batch, s));
      src = e.wp(e.w.xnorm);
      ss = n;
    }
    float* ws = e.wp(e.w.splitk);
    const std::size_t wsf = e.w.splitk_floats;
    const int mp = slices.matrix ? slices.slices : 0;
    const int mpr = slices.matrix ? slices.res_slices : 0;
    if (res != nullptr && e.side != nullptr &&
        2.0 * op.oc * op.ic * op.k * op.lout * batch >= kForkMinFlops &&
        conv_mfma_ksplit(op, in.split, ss, in.plain, in.plain_stride, batch, wsf, e.bf16_mma,
                         e.f32_split, mp) == 1 &&
        conv_mfma_ksplit(*res, in.split, ss, in.plain, in.plain_stride, batch, wsf, e.bf16_mma,
                         e.f32_split, mpr) == 1) {
      // Convolutions large enough to pay for a fork (about 20 GFLOP and up) whose GEMMs need
      // no K split: the 1x1 projection reads the same staged input as the convolution and
      // writes its own output, so it runs on the side stream, forked after the prologue and
      // joined before the next layer, and fills the CUs the convolution's last wave of tiles
      // leaves idle.  Smaller ones lose to the fork's synchronization (bimanual B=64 6.32 ->
      // 6.82 ms with every projection forked, pusht B=128 +0.3%).
      FE_TRY(hipEventRecord(e.fork, s));
      FE_TRY(hipStreamWaitEvent(e.side, e.fork, 0));
      FE_TRY(conv_mfma(*res, src, ss, in.split, in.plain, in.plain_stride, yr, batch, ws, wsf,
                       e.bf16_mma, e.f32_split, e.side, mpr));
      FE_TRY(conv_mfma(op, src, ss, in.split, in.plain, in.plain_stride, y, batch, ws, wsf,
                       e.bf16_mma, e.f32_split, s, mp));
      FE_TRY(hipEventRecord(e.join, e.side));
      return hipStreamWaitEvent(s, e.join, 0);
    }
    FE_TRY(conv_mfma(op, src, ss, in.split, in.plain, in.plain_stride, y, batch, ws, wsf,
                     e.bf16_mma, e.f32_split, s, mp));
    if (res != nullptr)
      FE_TRY(conv_mfma(*res, src, ss, in.split, in.plain, in.plain_stride, yr, batch, ws, wsf,
                       e.bf16_mma, e.f32_split, s, mpr));
    return hipSuccess;
  }
  return conv_fused(op, res, in, y, yr, batch, s);
}

// True when this evaluation's convolutions run input-channel sliced.
bool sliced(const FeEngine& e, int batch) {
  return e.slice_ok && e.slice_max > 1 && batch >= 1 &&
         static_cast<std::size_t>(batch) <= e.w.slice_batch &&
         static_cast<std::size_t>(batch) < e.mfma_batch;
}

// True when this evaluation's matrix-core convolutions leave split-K partial sums.
bool mm_parts(const FeEngine& e, int batch) {
  return e.mm_parts_ok && batch >= 1 && static_cast<std::size_t>(batch) >= e.mfma_batch &&
         static_cast<std::size_t>(batch) <= e.w.part_batch;
}

// Partial sums of one convolution's output (1: a single tensor), at most `cap`: input-channel
// slices on the fused kernels, or the split K loop of a matrix-core convolution.
fe::hip::SlicePlan slices_of(const FeEngine& e, const fe::hip::ConvOp& op,
                             const fe::hip::ConvOp* res, const fe::hip::ConvInput& in, int batch,
                             int cap = fe::hip::kMaxSlices) {
  fe::hip::View yr;
  yr.p = reinterpret_cast<float*>(e.ws);  // a non-null stand-in: only its presence is checked
  if (sliced(e, batch))
    return fe::hip::conv_fused_slices(op, res, in, yr, batch, std::min(cap, e.slice_max),
                                      e.slice_tpr);
  fe::hip::SlicePlan p;
  if (!mm_parts(e, batch) || conv_path(e, op, res, in, yr, batch) != ConvPath::kMatrix) return p;
  // The GEMM reads the prologue's output (or the summed plain input) when there is one.
  const bool staged = in.norm || in.parts > 1;
  const std::int64_t ss =
      staged ? (in.norm && in.mat != nullptr ? in.mat_stride
                                             : static_cast<std::int64_t>(in.split) * op.lin)
             : in.src_stride;
  p.matrix = true;
  p.slices = fe::hip::conv_mfma_parts(op, in.split, ss, in.plain, in.plain_stride, batch,
                                      e.bf16_mma, e.f32_split, cap);
  if (res != nullptr)
    p.res_slices = fe::hip::conv_mfma_parts(*res, in.split, ss, in.plain, in.plain_stride, batch,
                                            e.bf16_mma, e.f32_split, cap);
  return p;
}

// Output view of a raw convolution output of `act` floats per sample: with slices, one partial
// sum per slice, kMaxSlices partials per sample.
fe::hip::View out_view(float* p, std::int64_t act, int slices) {
  fe::hip::View v;
  v.p = p;
  v.stride = slices > 1 ? act * fe::hip::kMaxSlices : act;
  v.part = slices > 1 ? act : 0;
  return v;
}

// How the current activation tensor is read: a plain tensor, or "virtual" as
// Y = mish(GroupNorm(src)) + res (a ResidualBlock output that is never stored whole).  `p` and
// `res` may be sums of partials (outputs of sliced convolutions).
struct Act {
  bool virt = false;
  const float* p = nullptr;  // plain tensor, or the raw source of a virtual one
  std::int64_t stride = 0;
  int parts = 1;
  std::int64_t part_stride = 0;
  const float* gamma = nullptr;
  const float* beta = nullptr;
  const float* res = nullptr;
  std::int64_t res_stride = 0;
  int res_parts = 1;
  std::int64_t res_part_stride = 0;
  int channels = 0;
};

// A plain (non-virtual) activation read from view `v` written by a convolution with `slices`.
Act plain_act(const fe::hip::View& v, int channels, int slices) {
  Act a;
  a.p = v.p;
  a.stride = v.stride;
  a.parts = slices;
  a.part_stride = v.part;
  a.channels = channels;
  return a;
}

fe::hip::ConvInput input_of(const FeEngine& e, const Act& in, float* mat, std::int64_t mat_stride) {
  fe::hip::ConvInput ci;
  ci.src = in.p;
  ci.src_stride = in.stride;
  ci.split = in.channels;
  ci.parts = in.parts;
  ci.part_stride = in.part_stride;
  if (in.virt) {
    ci.norm = true;
    ci.gamma = in.gamma;
    ci.beta = in.beta;
    ci.groups = static_cast<int>(e.cfg.groups);
    ci.res = in.res;
    ci.res_stride = in.res_stride;
    ci.res_parts = in.res_parts;
    ci.res_part_stride = in.res_part_stride;
    ci.mat = mat;
    ci.mat_stride = mat_stride;
  }
  return ci;
}

// The FiLM-conditioned conv2 input FiLM(mish(GN1(h1))) of a block whose conv1 wrote view h1.
fe::hip::ConvInput film_input(const FeEngine& e, const Block& b, const fe::hip::View& h1,
                              int parts, const float* film_row) {
  fe::hip::ConvInput c2{};
  c2.src = h1.p;
  c2.src_stride = h1.stride;
  c2.parts = parts;
  c2.part_stride = h1.part;
  c2.split = static_cast<int>(b.oc);
  c2.norm = true;
  c2.gamma = e.ptr(b.n1.g_off);
  c2.beta = e.ptr(b.n1.b_off);
  c2.groups = static_cast<int>(e.cfg.groups);
  c2.film_time = film_row;
  c2.film_cond = e.wp(e.w.film_cond);
  c2.film_cond_stride = static_cast<std::int64_t>(e.film_total);
  c2.film_off = static_cast<int>(b.film_off);
  return c2;
}

// One ResidualBlock (diffusion.cc:724-773) as two fused launches:
//   K1: [conv1 | res 1x1](prologue(input))      -> h1, r
//   K2: conv2(FiLM(mish(GN1(h1))))               -> h2
// and returns its output as the virtual Y = mish(GN2(h2)) + (identity ? input : r).  `ci` is
// the block's input descriptor (input_of, possibly with a plain second part).
hipError_t enqueue_block_in(FeEngine& e, const std::string& site, const Block& b, const Act& in,
                            const fe::hip::ConvInput& ci, int batch, const float* film_row,
                            Act& out) {
  using namespace fe::hip;
  hipStream_t s = e.stream;
  const std::int64_t act = static_cast<std::int64_t>(b.oc * b.len);
  const ConvOp* res = b.identity ? nullptr : &b.res.op;
  const SlicePlan s1 = slices_of(e, b.c1.op, res, ci, batch);
  const View v1 = out_view(e.wp(e.w.h1[b.id]), act, s1.slices);
  const View vr = b.identity ? View{} : out_view(e.wp(e.w.r[b.id]), act, s1.res_slices);
  FE_TRY(conv(e, site + ".conv1", b.c1.op, res, ci, v1, vr, batch, s, s1));
  const ConvInput c2 = film_input(e, b, v1, s1.slices, film_row);
  const SlicePlan s2 = slices_of(e, b.c2.op, nullptr, c2, batch);
  const View v2 = out_view(e.wp(e.w.h2[b.id]), act, s2.slices);
  FE_TRY(conv(e, site + ".conv2", b.c2.op, nullptr, c2, v2, View{}, batch, s, s2));
  out = plain_act(v2, static_cast<int>(b.oc), s2.slices);
  out.virt = true;
  out.gamma = e.ptr(b.n2.g_off);
  out.beta = e.ptr(b.n2.b_off);
  if (b.identity) {
    // The identity residual is the block input: the copy conv1's prologue materialised, or the
    // plain input itself.
    out.res = in.virt ? ci.mat : in.p;
    out.res_stride = in.virt ? ci.mat_stride : in.stride;
    out.res_parts = in.virt ? 1 : in.parts;
    out.res_part_stride = in.virt ? 0 : in.part_stride;
  } else {
    out.res = vr.p;
    out.res_stride = vr.stride;
    out.res_parts = s1.res_slices;
    out.res_part_stride = vr.part;
  }
  return hipSuccess;
}

hipError_t enqueue_block(FeEngine& e, const std::string& site, const Block& b, const Act& in,
                         int batch, const float* film_row, float* skip_mat,
                         std::int64_t skip_stride, Act& out) {
  // Where the (virtual) input is materialised, when something reads it again.
  float* mat = nullptr;
  std::int64_t mat_stride = 0;
  if (in.virt) {
    if (skip_mat) {
      mat = skip_mat;
      mat_stride = skip_stride;
    } else if (b.identity) {
      mat = e.wp(e.w.xmat[b.id]);
      mat_stride = static_cast<std::int64_t>(b.ic * b.len);
    }
  }
  return enqueue_block_in(e, site, b, in, input_of(e, in, mat, mat_stride), batch, film_row, out);
}

// Fields of the final GroupNorm + Mish + 1x1 conv that every update of the engine shares.
void update_base(const FeEngine& e, fe::hip::UpdateOp& upd) {
  const Config& c = e.cfg;
  upd.c0 = static_cast<int>(c.dims[0]);
  upd.horizon = static_cast<int>(c.horizon);
  upd.action_dim = static_cast<int>(c.action_dim);
  upd.h = e.wp(e.w.fconv_out);
  upd.gamma = e.ptr(e.fnorm.g_off);
  upd.beta = e.ptr(e.fnorm.b_off);
  upd.groups = static_cast<int>(kFinalNormGroups);
  upd.wo = static_cast<const float*>(e.fout.op.w);
  upd.bo = e.fout.op.b;
  // The split update keeps its counters in the engine's arena: only on the engine's workspace.
  if (e.upd_done != nullptr && e.ws == e.own_ws) {
    upd.done = e.upd_done;
    upd.epart = e.wp(e.w.upd_part);
  }
}

// One U-Net evaluation on xin (FiLM time row `film_row`), ending with `upd`
// (diffusion.cc:793-914).
hipError_t enqueue_unet(FeEngine& e, int batch, const float* film_row, fe::hip::UpdateOp upd) {
  using namespace fe::hip;
  const Config& c = e.cfg;
  hipStream_t s = e.stream;
  Act x;
  x.p = e.wp(e.w.x_in);
  x.stride = static_cast<std::int64_t>(c.action_dim * c.horizon);
  x.channels = static_cast<int>(c.action_dim);
  Act y;
  for (std::size_t st = 0; st < c.stages; ++st) {
    const std::string stage = "down" + std::to_string(st);
    FE_TRY(enqueue_block(e, stage + ".b0", e.down[st][0], x, batch, film_row, nullptr, 0, y));
    x = y;
    FE_TRY(enqueue_block(e, stage + ".b1", e.down[st][1], x, batch, film_row, nullptr, 0, y));
    x = y;
    if (st + 1 < c.stages) {
      // Downsample1d; its prologue materialises the stage output as the skip tensor of up stage
      // S-1-st (second half of that stage's input buffer).  Stage 0's skip is never read.
      const ConvSlot& d = e.ds[st];
      float* skip = nullptr;
      std::int64_t skip_stride = 0;
      if (st >= 1) {
        const std::size_t u = c.stages - 1 - st;
        skip = e.wp(e.w.concat[u]) + d.op.ic * d.op.lin;
        skip_stride = static_cast<std::int64_t>(e.up[u][0].ic * e.up[u][0].len);
      }
      ConvInput ci = input_of(e, x, skip, skip_stride);
      const std::int64_t os = static_cast<std::int64_t>(d.op.oc) * d.op.lout;
      const SlicePlan sd = slices_of(e, d.op, nullptr, ci, batch);
      const View out = out_view(e.wp(e.w.ds_out[st]), os, sd.slices);
      FE_TRY(conv(e, stage + ".downsample", d.op, nullptr, ci, out, View{}, batch, s, sd));
      x = plain_act(out, d.op.oc, sd.slices);
    }
  }
  // Mid blocks; the first one's prologue materialises the bottom stage output as the skip tensor
  // of up stage 0.
  {
    const Block& m0 = e.mid[0];
    float* skip = e.wp(e.w.concat[0]) + m0.ic * m0.len;
    const std::int64_t skip_stride = static_cast<std::int64_t>(e.up[0][0].ic * e.up[0][0].len);
    FE_TRY(enqueue_block(e, "mid0", m0, x, batch, film_row, skip, skip_stride, y));
    x = y;
    FE_TRY(enqueue_block(e, "mid1", e.mid[1], x, batch, film_row, nullptr, 0, y));
    x = y;
  }
  Act up_in;  // the previous up stage's upsample output
  for (std::size_t u = 0; u + 1 < c.stages; ++u) {
    const Block& r0 = e.up[u][0];
    const std::int64_t cs = static_cast<std::int64_t>(r0.ic * r0.len);
    const int half = static_cast<int>(r0.ic / 2);
    // Input [x ; skip]: x is the virtual mid output (u == 0) or the previous upsample output;
    // the block's input descriptor covers channels [0, half), the skip half is plain.
    Act in = u == 0 ? x : up_in;
    in.channels = half;
    ConvInput ci = input_of(e, in, nullptr, 0);
    ci.plain = e.wp(e.w.concat[u]) + half * r0.len;
    ci.plain_stride = cs;
    const std::string stage = "up" + std::to_string(u);
    FE_TRY(enqueue_block_in(e, stage + ".b0", r0, in, ci, batch, film_row, y));
    x = y;
    FE_TRY(enqueue_block(e, stage + ".b1", e.up[u][1], x, batch, film_row, nullptr, 0, y));
    x = y;
    // Upsample1d into the first half of the next up stage's input, or the final conv input; when
    // sliced, into its own partial-sum buffer.
    const ConvSlot& up = e.us[u];
    const bool last = u + 2 >= c.stages;
    ConvInput ci2 = input_of(e, x, nullptr, 0);
    const SlicePlan su = slices_of(e, up.op, nullptr, ci2, batch);
    View dst;
    if (su.slices > 1) {
      dst = out_view(e.wp(e.w.us_out[u]), static_cast<std::int64_t>(up.op.oc) * up.op.lout,
                     su.slices);
    } else if (!last) {
      dst.p = e.wp(e.w.concat[u + 1]);
      dst.stride = static_cast<std::int64_t>(e.up[u + 1][0].ic * e.up[u + 1][0].len);
    } else {
      dst.p = e.wp(e.w.final_in);
      dst.stride = static_cast<std::int64_t>(c.dims[0] * c.horizon);
    }
    FE_TRY(conv(e, stage + ".upsample", up.op, nullptr, ci2, dst, View{}, batch, s, su));
    up_in = plain_act(dst, up.op.oc, su.slices);
  }
  const std::int64_t fs = static_cast<std::int64_t>(c.dims[0] * c.horizon);
  ConvInput fi{};
  fi.src = up_in.p;
  fi.src_stride = up_in.stride;
  fi.parts = up_in.parts;
  fi.part_stride = up_in.part_stride;
  fi.split = static_cast<int>(c.dims[0]);
  // The update sums at most kMaxUpdateParts partials of the final conv output.
  const SlicePlan sf = slices_of(e, e.fconv.op, nullptr, fi, batch,
                                 update_max_parts(static_cast<int>(c.dims[0])));
  const View fo = out_view(e.wp(e.w.fconv_out), fs, sf.slices);
  FE_TRY(conv(e, "final.conv", e.fconv.op, nullptr, fi, fo, View{}, batch, s, sf));
  update_base(e, upd);
  upd.hparts = sf.slices;
  upd.hpart = fo.part;
  upd.hstride = fo.stride;
  if (e.dry) return hipSuccess;
  return update(upd, batch, s);
}

// FiLM tables for `count` U-Net evaluations and the per-sample condition part.
// FiLM time rows W_t mish(temb_mlp(t_n)) + b for `count` U-Net evaluations into `table`.
// The time MLP output already carries its Mish (the reference applies Mish to the whole FiLM
// input [t_emb ; cond] once, diffusion.cc:818-820), so the projection splits exactly into a time
// part and a condition part.
hipError_t enqueue_film_time(FeEngine& e, const fe::hip::TimeSpec& ts, int count, float* table) {
  using namespace fe::hip;
  const Config& c = e.cfg;
  const int F = static_cast<int>(e.film_total);
  FE_TRY(time_mlp(ts, count, e.ptr(e.te1w), e.ptr(e.te1b), e.ptr(e.te2w), e.ptr(e.te2b),
                  static_cast<int>(c.tdim), e.wp(e.w.time_m), e.stream));
  return film_gemm(e.wp(e.w.time_m), static_cast<std::int64_t>(c.tdim), count,
                   static_cast<int>(c.tdim), e.ptr(e.film_wt), e.ptr(e.film_bias), F, false, table,
                   F, e.stream);
}

// Condition part W_c mish(cond_b) for every sample; once per sampling call (the condition is
// the same for every U-Net evaluation of a call).  `cond` defaults to the staged input buffer.
hipError_t enqueue_film_cond(FeEngine& e, int batch, const float* cond = nullptr) {
  const Config& c = e.cfg;
  const int F = static_cast<int>(e.film_total);
  return fe::hip::film_gemm(cond != nullptr ? cond : e.wp(e.w.in_cond),
                            static_cast<std::int64_t>(c.cond_dim), batch,
                            static_cast<int>(c.cond_dim), e.ptr(e.film_wc), nullptr, F, true,
                            e.wp(e.w.film_cond), F, e.stream);
}

hipError_t enqueue_film(FeEngine& e, const fe::hip::TimeSpec& ts, int count, int batch,
                        const float* cond = nullptr) {
  FE_TRY(enqueue_film_time(e, ts, count, e.wp(e.w.film_table)));
  return enqueue_film_cond(e, batch, cond);
}

// DDIM/DDPM sampling (diffusion.cc:916-1035) for `batch` samples, in three parts so that a
// resumable solve can replay them separately: the start (noise into the state, FiLM condition
// part), step i, and the readout of the current action (unnormalised state).
hipError_t enqueue_diffusion_start(FeEngine& e, int batch) {
  using namespace fe::hip;
  const Config& c = e.cfg;
  FE_TRY(begin_sample(e.wp(e.w.in_noise), e.wp(e.w.x_state), e.wp(e.w.x_in), batch,
                      static_cast<int>(c.horizon), static_cast<int>(c.action_dim), e.stream));
  return enqueue_film_cond(e, batch);
}

// The update after step i of a DDIM/DDPM solve of `steps` steps and the timestep that step
// evaluates (diffusion.cc:928-1024); the scalars are computed on the host as the reference does.
fe::hip::UpdateOp diffusion_update(FeEngine& e, std::size_t steps, int scheduler,
                                   const float* alphas, std::size_t i, std::size_t& t_out) {
  using namespace fe::hip;
  const Config& c = e.cfg;
  const std::size_t ratio = c.train_timesteps / steps;
  const std::size_t t = (steps - 1 - i) * ratio;
  const std::ptrdiff_t prev = static_cast<std::ptrdiff_t>(t) - static_cast<std::ptrdiff_t>(ratio);
  const float at = alphas[t];
  const float ap = prev >= 0 ? alphas[prev] : 1.0f;
  const float bt = 1.0f - at;
  UpdateOp u{};
  u.x = e.wp(e.w.x_state);
  u.xin = e.wp(e.w.x_in);
  u.sqrt_at = std::sqrt(at);
  u.sqrt_bt = std::sqrt(bt);
  u.clip = c.clip ? 1 : 0;
  u.clip_range = c.clip_range;
  if (scheduler == FE_DIFFUSION_DDIM) {
    u.kind = kUpdateDDIM;
    u.sqrt_ap = std::sqrt(ap);
    u.sqrt_1map = std::sqrt(1.0f - ap);
  } else {
    // diffusion.cc:1006-1023.  Only the last step (t < ratio) draws no noise, so step i starts at
    // Gaussian draw i * H * A of the sample's stream.
    const float ca = at / ap, cb = 1.0f - ca;
    u.kind = kUpdateDDPM;
    u.coef_x0 = std::sqrt(ap) * cb / std::max(bt, 1e-20f);
    u.coef_x = std::sqrt(ca) * (1.0f - ap) / std::max(bt, 1e-20f);
    const float var = ((1.0f - ap) / std::max(bt, 1e-20f)) * cb;
    u.sigma = std::sqrt(std::max(var, 1e-20f));
    u.seed = e.wp<std::uint64_t>(e.w.seed);
    u.add_noise = prev >= 0 ? 1 : 0;
    u.noise_offset = static_cast<std::uint64_t>(i) * e.values;
  }
  t_out = t;
  return u;
}

hipError_t enqueue_diffusion_step(FeEngine& e, int batch, std::size_t steps, int scheduler,
                                  const float* alphas, std::size_t i) {
  std::size_t t = 0;
  const fe::hip::UpdateOp u = diffusion_update(e, steps, scheduler, alphas, i, t);
  const float* row = e.ptr(e.ddim_table) + t * e.film_total;
  return enqueue_unet(e, batch, row, u);
}

hipError_t enqueue_diffusion_readout(FeEngine& e, int batch) {
  const Config& c = e.cfg;
  return fe::hip::finish_sample(e.wp(e.w.x_state), e.ptr(e.amin), e.ptr(e.amax),
                                e.wp(e.w.out_action), batch, static_cast<int>(c.horizon),
                                static_cast<int>(c.action_dim), e.stream);
}

hipError_t enqueue_diffusion(FeEngine& e, int batch, std::size_t steps, int scheduler,
                             const float* alphas) {
  FE_TRY(enqueue_diffusion_start(e, batch));
  for (std::size_t i = 0; i < steps; ++i)
    FE_TRY(enqueue_diffusion_step(e, batch, steps, scheduler, alphas, i));
  return enqueue_diffusion_readout(e, batch);
}

// Flow-ODE sampling (flow.cc:291-318) with the U-Net as velocity field, in the same three parts.
// `film` holds the FiLM time rows of every evaluation of the solve (flow_table); when it is null
// the start computes them into the workspace.
std::size_t flow_stages(int method) {
  return method == FE_SOLVER_RK4 ? 4 : (method == FE_SOLVER_HEUN ? 2 : 1);
}

hipError_t enqueue_flow_start(FeEngine& e, int batch, std::size_t steps, int method,
                              const float* film) {
  using namespace fe::hip;
  const Config& c = e.cfg;
  FE_TRY(begin_sample(e.wp(e.w.in_noise), e.wp(e.w.x_state), e.wp(e.w.x_in), batch,
                      static_cast<int>(c.horizon), static_cast<int>(c.action_dim), e.stream));
  if (film != nullptr) return enqueue_film_cond(e, batch);
  TimeSpec ts;
  ts.mode = kTimesFlow;
  ts.steps = static_cast<int>(steps);
  ts.method = method;
  return enqueue_film(e, ts, static_cast<int>(steps * flow_stages(method)), batch);
}

// The update after stage j of a flow step (flow.cc:291-318, span_ops.h:27-52).
fe::hip::UpdateOp flow_update(FeEngine& e, std::size_t steps, int method, int j) {
  using namespace fe::hip;
  const int stages = static_cast<int>(flow_stages(method));
  const float dt = 1.0f / static_cast<float>(steps);
  const float half_dt = 0.5f * dt;
  {
    UpdateOp u{};
    u.x = e.wp(e.w.x_state);
    u.xin = e.wp(e.w.x_in);
    u.kbuf = e.wp(e.w.k_stages);
    u.dt = dt;
    if (stages == 1) {
      u.kind = kUpdateEuler;
    } else if (stages == 2) {
      if (j == 0) {
        u.kind = kUpdateStage;
        u.slot = 0;
        u.dt = dt;
      } else {
        u.kind = kUpdateHeun;
      }
    } else {
      if (j < 3) {
        u.kind = kUpdateStage;
        u.slot = j;
        u.dt = j < 2 ? half_dt : dt;
      } else {
        u.kind = kUpdateRK4;
      }
    }
    return u;
  }
}

// The FiLM time rows a solve reads: its table, or the workspace rows its start computes.
const float* flow_rows(const FeEngine& e, const float* film) {
  return film != nullptr ? film : e.wp(e.w.film_table);
}

hipError_t enqueue_flow_step(FeEngine& e, int batch, std::size_t steps, int method,
                             std::size_t step, const float* film) {
  const int stages = static_cast<int>(flow_stages(method));
  for (int j = 0; j < stages; ++j) {
    const fe::hip::UpdateOp u = flow_update(e, steps, method, j);
    const std::size_t n = step * static_cast<std::size_t>(stages) + static_cast<std::size_t>(j);
    FE_TRY(enqueue_unet(e, batch, flow_rows(e, film) + n * e.film_total, u));
  }
  return hipSuccess;
}

hipError_t enqueue_flow_readout(FeEngine& e, int batch) {
  // flow.cc:321: the flow head returns x(1) as is (no unnormalisation).
  const Config& c = e.cfg;
  return fe::hip::finish_sample(e.wp(e.w.x_state), nullptr, nullptr, e.wp(e.w.out_action), batch,
                                static_cast<int>(c.horizon), static_cast<int>(c.action_dim),
                                e.stream);
}

hipError_t enqueue_flow(FeEngine& e, int batch, std::size_t steps, int method,
                        const float* film) {
  FE_TRY(enqueue_flow_start(e, batch, steps, method, film));
  for (std::size_t s = 0; s < steps; ++s)
    FE_TRY(enqueue_flow_step(e, batch, steps, method, s, film));
  return enqueue_flow_readout(e, batch);
}

std::vector<float> alphas_cumprod(std::size_t T) {
  // diffusion.cc:186-191, 529-541: beta in double, cumulative product in float.
  auto abar = [](double t) {
    const double c = std::cos(((t + 0.008) / 1.008) * (3.14159265358979323846 / 2.0));
    return c * c;
  };
  std::vector<float> a(T);
  float cum = 1.0f;
  for (std::size_t s = 0; s < T; ++s) {
    const double b0 = static_cast<double>(s) / static_cast<double>(T);
    const double b1 = static_cast<double>(s + 1) / static_cast<double>(T);
    const float beta = static_cast<float>(std::min(1.0 - abar(b1) / abar(b0), 0.999));
    cum *= 1.0f - beta;
    a[s] = cum;
  }
  return a;
}

// Captures what `body` enqueues on the engine stream into an instantiated graph.
template <typename Body>
hipError_t capture_graph(FeEngine& e, Body&& body, hipGraphExec_t& exec) {
  exec = nullptr;
  FE_TRY(hipStreamBeginCapture(e.stream, hipStreamCaptureModeThreadLocal));
  hipError_t st = body();
  hipGraph_t graph = nullptr;
  const hipError_t end = hipStreamEndCapture(e.stream, &graph);
  if (st != hipSuccess || end != hipSuccess) {
    if (graph) (void)hipGraphDestroy(graph);
    return st != hipSuccess ? st : end;
  }
  st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (st != hipSuccess) exec = nullptr;
  else ++e.captures;
  return st;
}

// U-Net evaluations of a sampling call.
std::size_t evaluations(int kind, std::size_t steps, int mode) {
  return kind == 0 ? steps : steps * flow_stages(mode);
}

// Fills evaluation table `table` of the persistent tick for this solve: each evaluation's FiLM
// time rows and the update after it, computed exactly as the per-layer graphs compute them.
hipError_t fill_chain_table(FeEngine& e, int kind, std::size_t steps, int mode, int table,
                            const float* film) {
  using namespace fe::hip;
  const Config& c = e.cfg;
  std::vector<ChainEval> evals;
  if (kind == 0) {
    const std::vector<float> alphas = alphas_cumprod(c.train_timesteps);
    for (std::size_t i = 0; i < steps; ++i) {
      std::size_t t = 0;
      ChainEval ev;
      ev.upd = diffusion_update(e, steps, mode, alphas.data(), i, t);
      update_base(e, ev.upd);
      ev.film_row = e.ptr(e.ddim_table) + t * e.film_total;
      evals.push_back(ev);
    }
  } else {
    const int stages = static_cast<int>(flow_stages(mode));
    for (std::size_t st = 0; st < steps; ++st)
      for (int j = 0; j < stages; ++j) {
        ChainEval ev;
        ev.upd = flow_update(e, steps, mode, j);
        update_base(e, ev.upd);
        ev.film_row = flow_rows(e, film) + (st * stages + j) * e.film_total;
        evals.push_back(ev);
      }
  }
  ChainEval* dst = e.ptr<ChainEval>(e.chain_tables) + static_cast<std::size_t>(table) * kMaxChainEvals;
  return hipMemcpy(dst, evals.data(), evals.size() * sizeof(ChainEval), hipMemcpyHostToDevice);
}

// One batch-1 tick on the persistent kernel: the solve's start (noise into the state, FiLM rows),
// the tick kernel, the readout, and a copy of the tick's abort flag to the host.
hipError_t enqueue_chain_tick(FeEngine& e, int kind, std::size_t steps, int mode, int table,
                              const float* film) {
  using namespace fe::hip;
  FE_TRY(kind == 0 ? enqueue_diffusion_start(e, 1) : enqueue_flow_start(e, 1, steps, mode, film));
  ChainTick t;
  t.steps = e.ptr<char>(e.chain_steps);
  t.nsteps = e.chain_nsteps;
  t.evals = e.ptr<ChainEval>(e.chain_tables) + static_cast<std::size_t>(table) * kMaxChainEvals;
  t.nevals = static_cast<int>(evaluations(kind, steps, mode));
  t.x0 = e.wp(e.w.x_state);
  t.xin0 = e.wp(e.w.x_in);
  t.slots = e.ptr(e.chain_slots);
  t.slot_floats = e.chain_slot_floats;
  t.x_out = e.wp(e.w.x_state);
  t.flags = e.ptr<unsigned>(e.chain_flags);
  t.abort = e.ptr<unsigned>(e.chain_abort);
  t.spin_limit = 1ll << 22;
  t.values = static_cast<int>(e.values);
  t.horizon = static_cast<int>(e.cfg.horizon);
  FE_TRY(chain_tick(t, e.stream));
  FE_TRY(kind == 0 ? enqueue_diffusion_readout(e, 1) : enqueue_flow_readout(e, 1));
  return hipMemcpyAsync(e.pin_status, e.ptr(e.chain_abort), 4, hipMemcpyDeviceToHost, e.stream);
}

// Drops the cached persistent-tick graphs (after a tick was abandoned).
void drop_chain_graphs(FeEngine& e) {
  for (auto it = e.graphs.begin(); it != e.graphs.end();) {
    if (it->chain_table >= 0) {
      (void)hipGraphExecDestroy(it->exec);
      it = e.graphs.erase(it);
    } else {
      ++it;
    }
  }
}

// The FiLM time rows of a flow solve of `steps` steps with `method` (nullptr for diffusion
// models and for solves with more evaluations than the pool holds; their graphs compute the rows).
// Computed once per (steps, method) on the engine stream, outside any capture, and kept.  When
// the pool is full it starts over, and the sampling graphs that read the old rows are dropped.
hipError_t flow_table(FeEngine& e, std::size_t steps, int method, const float*& film) {
  film = nullptr;
  const std::size_t n = evaluations(1, steps, method);
  if (e.flow_pool_rows == 0 || n > e.flow_pool_rows) return hipSuccess;
  float* pool = e.ptr(e.flow_pool);
  for (const FeEngine::FlowTable& t : e.flow_tables)
    if (t.steps == steps && t.method == method) {
      film = pool + t.row0 * e.film_total;
      return hipSuccess;
    }
  if (e.flow_pool_used + n > e.flow_pool_rows) {
    for (auto it = e.graphs.begin(); it != e.graphs.end();) {
      if (it->kind == 1) {
        (void)hipGraphExecDestroy(it->exec);
        it = e.graphs.erase(it);
      } else {
        ++it;
      }
    }
    e.flow_tables.clear();
    e.flow_pool_used = 0;
  }
  FeEngine::FlowTable t;
  t.steps = steps;
  t.method = method;
  t.row0 = e.flow_pool_used;
  fe::hip::TimeSpec ts;
  ts.mode = fe::hip::kTimesFlow;
  ts.steps = static_cast<int>(steps);
  ts.method = method;
  FE_TRY(enqueue_film_time(e, ts, static_cast<int>(n), pool + t.row0 * e.film_total));
  e.flow_tables.push_back(t);
  e.flow_pool_used += n;
  film = pool + t.row0 * e.film_total;
  return hipSuccess;
}

// Returns the cached graph for this shape, capturing it on first use.  Batch-1 solves of up to
// kMaxChainEvals evaluations run as one persistent tick when the engine has a step table.
hipError_t get_graph(FeEngine& e, int kind, std::size_t batch, std::size_t steps, int mode,
                     hipGraphExec_t& exec, bool* chained = nullptr) {
  const bool chain =
      e.chain_on && batch == 1 && evaluations(kind, steps, mode) <= kMaxChainEvals;
  if (chained != nullptr) *chained = chain;
  for (auto it = e.graphs.begin(); it != e.graphs.end(); ++it)
    if (it->kind == kind && it->batch == batch && it->steps == steps && it->mode == mode &&
        (it->chain_table >= 0) == chain) {
      e.graphs.splice(e.graphs.begin(), e.graphs, it);
      exec = it->exec;
      return hipSuccess;
    }
  if (e.graphs.size() >= kGraphCache) {
    (void)hipGraphExecDestroy(e.graphs.back().exec);
    e.graphs.pop_back();
  }
  const float* film = nullptr;
  if (kind == 1) FE_TRY(flow_table(e, steps, mode, film));
  int table = -1;
  if (chain) {
    std::vector<bool> used(kChainTables, false);
    for (const GraphEntry& g : e.graphs)
      if (g.chain_table >= 0) used[static_cast<std::size_t>(g.chain_table)] = true;
    for (std::size_t i = 0; i < kChainTables && table < 0; ++i)
      if (!used[i]) table = static_cast<int>(i);
    FE_TRY(fill_chain_table(e, kind, steps, mode, table, film));
  }
  hipGraphExec_t inst = nullptr;
  FE_TRY(capture_graph(
      e,
      [&]() {
        if (chain) return enqueue_chain_tick(e, kind, steps, mode, table, film);
        if (kind == 0) {
          const std::vector<float> alphas = alphas_cumprod(e.cfg.train_timesteps);
          return enqueue_diffusion(e, static_cast<int>(batch), steps, mode, alphas.data());
        }
        return enqueue_flow(e, static_cast<int>(batch), steps, mode, film);
      },
      inst));
  e.graphs.push_front(GraphEntry{kind, mode, batch, steps, inst, table});
  exec = inst;
  return hipSuccess;
}

int hip_fail(const char* what, hipError_t st) {
  set_error(std::string(what) + ": " + hipGetErrorString(st));
  return FE_STATUS_RESOURCE_EXHAUSTED;
}

// Partial-sum mode of an evaluation of `batch` samples: 0 single tensors, 1 input-channel sliced
// fused kernels, 2 matrix-core split-K partials.
int parts_mode(const FeEngine& e, int batch) {
  return sliced(e, batch) ? 1 : (mm_parts(e, batch) ? 2 : 0);
}

// Lists the convolutions of one U-Net evaluation the first time a diagnostic asks for them, by
// walking the U-Net without enqueueing anything, with the arguments an evaluation of `batch`
// samples uses (they depend on the batch only through the partial-sum plan: the listing is
// taken at batch 1 unless matrix-core partials are on).
int ensure_conv_records(FeEngine* e, std::size_t batch = 1) {
  const int mode = parts_mode(*e, static_cast<int>(batch));
  const std::size_t walk = mode == 2 ? batch : 1;
  if (!e->conv_records.empty() && e->records_mode == mode && e->records_batch == walk)
    return FE_STATUS_OK;
  e->conv_records.clear();
  using namespace fe::hip;
  UpdateOp u{};
  u.kind = kUpdateDenoise;
  u.out = e->wp(e->w.out_action);
  const bool saved_slice = e->slice_ok, saved_mm = e->mm_parts_ok;
  e->slice_ok = saved_slice && mode == 1;
  e->mm_parts_ok = saved_mm && mode == 2;
  e->recording = true;
  e->dry = true;
  const hipError_t st = enqueue_unet(*e, static_cast<int>(walk), e->wp(e->w.film_table), u);
  e->recording = false;
  e->dry = false;
  e->slice_ok = saved_slice;
  e->mm_parts_ok = saved_mm;
  e->records_mode = mode;
  e->records_batch = walk;
  if (st != hipSuccess) {
    e->conv_records.clear();
    e->records_mode = -1;
    return hip_fail("Diagnostic U-Net walk failed", st);
  }
  return FE_STATUS_OK;
}

// Partial sums instead of whole tensors between convolutions:
//  - input-channel slicing, when every convolution of the model runs on the fused kernels below
//    the matrix-core threshold (and not with the persistent tick, which runs unsliced kernels);
//  - matrix-core split-K partials, when every convolution runs on the matrix cores from the
//    threshold on;
// both only when the update is the fused instance that sums partials of the final conv.
void decide_partials(FeEngine& e) {
  e.slice_ok = false;
  e.mm_parts_ok = false;
  const char* v = std::getenv("FLOWEDGE_SLICES");
  if (v != nullptr && *v != '\0') {
    char* end = nullptr;
    const long n = std::strtol(v, &end, 10);
    e.slice_max = (end && *end == '\0' && n >= 1) ? static_cast<int>(std::min<long>(n, fe::hip::kMaxSlices)) : 1;
  }
  v = std::getenv("FLOWEDGE_SLICE_TPR");
  if (v != nullptr && (std::strcmp(v, "16") == 0 || std::strcmp(v, "32") == 0 ||
                       std::strcmp(v, "64") == 0))
    e.slice_tpr = std::atoi(v);
  v = std::getenv("FLOWEDGE_MM_PARTS");
  const bool mm_wanted = !(v != nullptr && std::strcmp(v, "0") == 0);
  const char* p = std::getenv("FLOWEDGE_PERSISTENT");
  if (p != nullptr && std::strcmp(p, "1") == 0) return;
  const Config& c = e.cfg;
  if (!fe::hip::update_fused(static_cast<int>(c.dims[0]), static_cast<int>(kFinalNormGroups),
                             static_cast<int>(c.horizon), static_cast<int>(c.action_dim)))
    return;
  if (ensure_conv_records(&e) != FE_STATUS_OK) {
    clear_error();
    return;
  }
  bool fused = e.mfma_batch > 1 && e.slice_max > 1;
  bool matrix = mm_wanted && e.mfma_batch <= kPartBatch;
  for (const FeEngine::ConvRecord& r : e.conv_records) {
    const fe::hip::ConvOp* res = r.has_res ? &r.res : nullptr;
    fused = fused && conv_path(e, r.op, res, r.in, r.yr, 1) == ConvPath::kFused;
    matrix = matrix && conv_path(e, r.op, res, r.in, r.yr, static_cast<int>(e.mfma_batch)) ==
                           ConvPath::kMatrix;
  }
  e.mm_parts_ok = matrix;
  if (!fused) return;
  // A sliced walk: every convolution left unsliced must read single tensors (the unsliced
  // kernels do not sum partials).
  e.slice_ok = true;
  if (ensure_conv_records(&e, 1) != FE_STATUS_OK) {
    clear_error();
    e.slice_ok = false;
    return;
  }
  for (const FeEngine::ConvRecord& r : e.conv_records)
    if (r.slices.slices == 1 && (r.in.parts != 1 || r.in.res_parts != 1)) {
      e.slice_ok = false;
      return;
    }
}

// Validates a sampling request (engine_runtime.cc:446-470 + extensions).

int check_sample(const FeEngine* e, int kind, std::size_t batch, std::size_t steps, int mode) {
  if (kind == 0) {
    if (e->cfg.prediction != 0) {
      set_error("Model has no Diffusion Policy head to sample from");
      return FE_STATUS_UNSUPPORTED_MODEL;
    }
    if (mode != FE_DIFFUSION_DDIM && mode != FE_DIFFUSION_DDPM) {
      set_error("Diffusion scheduler must be FE_DIFFUSION_DDIM or FE_DIFFUSION_DDPM");
      return FE_STATUS_INVALID_SOLVER;
    }
    if (steps == 0 || steps > e->cfg.train_timesteps) {
      set_error("Diffusion inference steps must be between 1 and the training timestep count");
      return FE_STATUS_INVALID_ARGUMENT;
    }
  } else {
    if (e->cfg.prediction != 1) {
      set_error("Model has no flow head to sample from");
      return FE_STATUS_UNSUPPORTED_MODEL;
    }
    if (mode < FE_SOLVER_EULER || mode > FE_SOLVER_RK4) {
      set_error("Invalid solver method");
      return FE_STATUS_INVALID_SOLVER;
    }
    const std::size_t stages = mode == FE_SOLVER_RK4 ? 4 : (mode == FE_SOLVER_HEUN ? 2 : 1);
    if (steps == 0 || steps * stages > e->max_nfe) {
      set_error("Flow solver steps out of range");
      return FE_STATUS_INVALID_ARGUMENT;
    }
  }
  if (batch == 0 || batch > e->max_batch) {
    set_error("Batch size must be between 1 and the engine's max batch");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  return FE_STATUS_OK;
}

// Replays the sampling graph; inputs already in the engine's device input buffers.  `chained`
// tells whether it was a persistent tick (whose abort flag the caller checks after the sync).
int run_graph(FeEngine* e, int kind, std::size_t batch, std::size_t steps, int mode,
              bool& chained) {
  hipGraphExec_t exec = nullptr;
  hipError_t st = get_graph(*e, kind, batch, steps, mode, exec, &chained);
  if (st != hipSuccess) return hip_fail("Failed to build sampling graph", st);
  if ((st = hipEventRecord(e->ev0, e->stream)) != hipSuccess ||
      (st = hipGraphLaunch(exec, e->stream)) != hipSuccess ||
      (st = hipEventRecord(e->ev1, e->stream)) != hipSuccess)
    return hip_fail("Sampling graph launch failed", st);
  e->timed = true;
  return FE_STATUS_OK;
}

// After a synchronised persistent tick: true when the kernel abandoned it (a workgroup never
// started, e.g. other work held CUs).  The engine then stops using the tick kernel and the caller
// runs the call again on the per-layer graphs (its inputs are still in the device buffers).
bool chain_abandoned(FeEngine* e, bool chained) {
  if (!chained || *e->pin_status == 0) return false;
  e->chain_on = false;
  e->chain_why = "a persistent tick was abandoned (not every workgroup was resident)";
  ++e->chain_abandoned;
  drop_chain_graphs(*e);
  return true;
}

int sample_host(FeEngine* e, int kind, const float* cond, const float* noise, std::size_t batch,
                std::size_t steps, int mode, std::uint64_t seed, float* action) {
  const int rc = check_sample(e, kind, batch, steps, mode);
  if (rc != FE_STATUS_OK) return rc;
  end_solve(e);
  hipError_t st = hipSetDevice(e->device);
  if (st != hipSuccess) return hip_fail("hipSetDevice", st);
  const Config& c = e->cfg;
  const std::size_t nc = batch * c.cond_dim, nv = batch * e->values;
  std::memcpy(e->pin_cond, cond, nc * 4);
  std::memcpy(e->pin_noise, noise, nv * 4);
  *e->pin_seed = seed;
  if ((st = hipMemcpyAsync(e->wp(e->w.in_cond), e->pin_cond, nc * 4, hipMemcpyHostToDevice,
                           e->stream)) != hipSuccess ||
      (st = hipMemcpyAsync(e->wp(e->w.in_noise), e->pin_noise, nv * 4, hipMemcpyHostToDevice,
                           e->stream)) != hipSuccess ||
      (st = hipMemcpyAsync(e->wp(e->w.seed), e->pin_seed, 8, hipMemcpyHostToDevice,
                           e->stream)) != hipSuccess)
    return hip_fail("Input upload failed", st);
  bool chained = false;
  for (int attempt = 0; attempt < 2; ++attempt) {
    const int r = run_graph(e, kind, batch, steps, mode, chained);
    if (r != FE_STATUS_OK) return r;
    if ((st = hipMemcpyAsync(e->pin_action, e->wp(e->w.out_action), nv * 4,
                             hipMemcpyDeviceToHost, e->stream)) != hipSuccess ||
        (st = hipStreamSynchronize(e->stream)) != hipSuccess)
      return hip_fail("Sampling failed", st);
    if (!chain_abandoned(e, chained)) break;
  }
  std::memcpy(action, e->pin_action, nv * 4);
  return FE_STATUS_OK;
}

// ---- Resumable solves (engine.h:321-366, engine_runtime.cc:494-561, flow.cc:210-318) ----

void drop_solve_graphs(FeEngine::Solve& v) {
  for (hipGraphExec_t g : v.graphs)
    if (g) (void)hipGraphExecDestroy(g);
  v.graphs.clear();
  v.g_kind = v.g_mode = -1;
  v.g_steps = 0;
}

// Ends the resumable solve because another call is about to reuse its state buffers.
void end_solve(FeEngine* e) {
  FeEngine::Solve& v = e->solve;
  v.active = v.cancelled = v.tracking = false;
  v.steps = v.next = 0;
}

// Raises the engine's latest generation to `generation` (engine_runtime.cc:512-519, 554-561).
void raise_generation(FeEngine* e, std::uint64_t generation) {
  std::uint64_t seen = e->latest_generation.load(std::memory_order_relaxed);
  while (seen < generation &&
         !e->latest_generation.compare_exchange_weak(seen, generation, std::memory_order_release,
                                                     std::memory_order_relaxed)) {
  }
}

// Step graphs of one batch-1 solve shape: [0] = start + readout, [1 + i] = step i + readout.
hipError_t build_solve_graphs(FeEngine& e, int kind, std::size_t steps, int mode) {
  FeEngine::Solve& v = e.solve;
  if (v.g_kind == kind && v.g_steps == steps && v.g_mode == mode) return hipSuccess;
  drop_solve_graphs(v);
  const std::vector<float> alphas =
      kind == 0 ? alphas_cumprod(e.cfg.train_timesteps) : std::vector<float>();
  v.graphs.reserve(steps + 1);
  for (std::size_t g = 0; g <= steps; ++g) {
    hipGraphExec_t exec = nullptr;
    const hipError_t st = capture_graph(
        e,
        [&]() -> hipError_t {
          if (kind == 0) {
            FE_TRY(g == 0 ? enqueue_diffusion_start(e, 1)
                          : enqueue_diffusion_step(e, 1, steps, mode, alphas.data(), g - 1));
            return enqueue_diffusion_readout(e, 1);
          }
          // A solve computes its own rows (a later call may reset the table pool mid-solve).
          FE_TRY(g == 0 ? enqueue_flow_start(e, 1, steps, mode, nullptr)
                        : enqueue_flow_step(e, 1, steps, mode, g - 1, nullptr));
          return enqueue_flow_readout(e, 1);
        },
        exec);
    if (st != hipSuccess) {
      drop_solve_graphs(v);
      return st;
    }
    v.graphs.push_back(exec);
  }
  v.g_kind = kind;
  v.g_steps = steps;
  v.g_mode = mode;
  return hipSuccess;
}

struct SolveRequest {
  int kind = 0, mode = 0;
  std::size_t steps = 0;
  std::uint64_t seed = 0;
  bool tracking = false;
  std::uint64_t generation = 0, timestamp_ns = 0, deadline_ns = 0;
};

int solve_begin(FeEngine* e, const float* cond, const float* noise, const SolveRequest& r) {
  const int rc = check_sample(e, r.kind, 1, r.steps, r.mode);
  if (rc != FE_STATUS_OK) return rc;
  hipError_t st = hipSetDevice(e->device);
  if (st != hipSuccess) return hip_fail("hipSetDevice", st);
  end_solve(e);
  FeEngine::Solve& v = e->solve;
  v.kind = r.kind;
  v.mode = r.mode;
  v.tracking = r.tracking;
  v.generation = r.generation;
  v.timestamp_ns = r.timestamp_ns;
  v.deadline_ns = r.deadline_ns;
  if (r.tracking) raise_generation(e, r.generation);
  const char* const failed = r.kind == 1 ? "Failed to initialize resumable flow sampler"
                                         : "Failed to initialize resumable diffusion sampler";
  if ((st = build_solve_graphs(*e, r.kind, r.steps, r.mode)) != hipSuccess)
    return hip_fail(failed, st);
  std::memcpy(e->pin_cond, cond, e->cfg.cond_dim * 4);
  std::memcpy(e->pin_noise, noise, e->values * 4);
  *e->pin_seed = r.seed;
  if ((st = hipMemcpyAsync(e->wp(e->w.in_cond), e->pin_cond, e->cfg.cond_dim * 4,
                           hipMemcpyHostToDevice, e->stream)) != hipSuccess ||
      (st = hipMemcpyAsync(e->wp(e->w.in_noise), e->pin_noise, e->values * 4,
                           hipMemcpyHostToDevice, e->stream)) != hipSuccess ||
      (st = hipMemcpyAsync(e->wp(e->w.seed), e->pin_seed, 8, hipMemcpyHostToDevice,
                           e->stream)) != hipSuccess ||
      (st = hipGraphLaunch(v.graphs[0], e->stream)) != hipSuccess ||
      (st = hipStreamSynchronize(e->stream)) != hipSuccess)
    return hip_fail(failed, st);
  v.steps = r.steps;
  v.next = 0;
  v.active = true;
  return FE_STATUS_OK;
}

// Runs at most `budget` steps and copies the current action out (flow.cc:260-318).  A tracked
// solve checks for cancellation before every step and waits for each step, so that a
// cancellation from another thread stops it at the next step boundary.
int solve_advance(FeEngine* e, int kind, std::size_t budget, float* action,
                  std::size_t& remaining) {
  FeEngine::Solve& v = e->solve;
  // Messages as engine_runtime.cc:535-550 for flow solves.
  const char* const cancelled = kind == 1 ? "Flow solve was cancelled by a newer generation"
                                          : "Diffusion solve was cancelled by a newer generation";
  if (v.cancelled) {
    set_error(cancelled);
    remaining = v.remaining();
    return FE_STATUS_CANCELLED;
  }
  if (!v.active || v.kind != kind) {
    set_error(kind == 1 ? "No resumable flow sample is active"
                        : "No resumable diffusion sample is active");
    return FE_STATUS_NO_ACTIVE_OPERATION;
  }
  hipError_t st = hipSetDevice(e->device);
  if (st != hipSuccess) return hip_fail("hipSetDevice", st);
  const std::size_t todo = std::min(budget, v.remaining());
  for (std::size_t k = 0; k < todo; ++k) {
    if (v.tracking && e->latest_generation.load(std::memory_order_acquire) > v.generation) {
      v.cancelled = true;
      v.active = false;
      break;
    }
    if ((st = hipGraphLaunch(v.graphs[1 + v.next], e->stream)) != hipSuccess ||
        (v.tracking && (st = hipStreamSynchronize(e->stream)) != hipSuccess)) {
      v.active = false;
      return hip_fail("Resumable sampler step failed", st);
    }
    ++v.next;
  }
  const std::size_t nv = e->values;
  if ((st = hipMemcpyAsync(e->pin_action, e->wp(e->w.out_action), nv * 4, hipMemcpyDeviceToHost,
                           e->stream)) != hipSuccess ||
      (st = hipStreamSynchronize(e->stream)) != hipSuccess) {
    v.active = false;
    return hip_fail("Resumable sampler step failed", st);
  }
  std::memcpy(action, e->pin_action, nv * 4);
  remaining = v.remaining();
  if (v.cancelled) {
    set_error(cancelled);
    return FE_STATUS_CANCELLED;
  }
  return FE_STATUS_OK;
}

// Evaluations per solver step (engine.cc:51-59); a DDIM/DDPM step is one evaluation.
std::uint64_t nfe_for(std::size_t steps, int kind, int mode) {
  const std::uint64_t per = kind == 1 ? flow_stages(mode) : 1;
  return steps > UINT64_MAX / per ? UINT64_MAX : static_cast<std::uint64_t>(steps) * per;
}

// Smallest batch that runs the convolutions on the matrix cores (FLOWEDGE_MFMA_BATCH; 0 = by
// weight type: 4 samples for F32 convolutions, 5 for BF16, where streaming half the bytes keeps
// the sliced batch-1 kernels ahead one sample longer; measured crossovers: pusht B=4 7.31 ms
// sliced against 6.32 on the matrix cores, bimanual B=4 3.91 against 4.48 and B=6 5.33 against
// 4.56; a value above the max batch keeps every batch on the weight-streaming kernels).
std::size_t env_mfma_batch() {
  const char* v = std::getenv("FLOWEDGE_MFMA_BATCH");
  if (v == nullptr || *v == '\0') return 0;
  char* end = nullptr;
  const unsigned long n = std::strtoul(v, &end, 10);
  return (end && *end == '\0') ? n : 0;
}

// FLOWEDGE_SIDE_STREAM=0 keeps every matrix-core projection on the engine stream.
bool side_streams() {
  const char* v = std::getenv("FLOWEDGE_SIDE_STREAM");
  return v == nullptr || std::strcmp(v, "0") != 0;
}

// FLOWEDGE_SPLIT_UPDATE=0 keeps the final update on one workgroup per sample.
bool split_update() {
  const char* v = std::getenv("FLOWEDGE_SPLIT_UPDATE");
  return v == nullptr || std::strcmp(v, "0") != 0;
}

std::size_t env_max_batch() {
  const char* v = std::getenv("FLOWEDGE_MAX_BATCH");
  if (v == nullptr || *v == '\0') return 256;
  char* end = nullptr;
  const unsigned long n = std::strtoul(v, &end, 10);
  return (end && *end == '\0' && n > 0 && n <= 65535) ? n : 0;
}

// Builds the persistent tick's step table from the U-Net's convolutions at batch 1 (the listing
// the diagnostics use); leaves chain_on false, with the reason, when the tick kernel cannot run
// this model or this device.
void build_chain(FeEngine& e) {
  using namespace fe::hip;
  // Opt-in: on MI355X the per-layer graphs are as fast (pusht DDIM-10 B=1: 3.465 against
  // 3.485 ms device p50), so they stay the default.
  const char* v = std::getenv("FLOWEDGE_PERSISTENT");
  if (v == nullptr || std::strcmp(v, "1") != 0) {
    e.chain_why = "not requested (FLOWEDGE_PERSISTENT=1 at load selects it)";
    return;
  }
  if (e.chain_steps == 0) {
    e.chain_why = "horizon or action count outside the tick kernel's instances";
    return;
  }
  if (e.mfma_batch <= 1) {
    e.chain_why = "batch 1 runs on the matrix cores (FLOWEDGE_MFMA_BATCH)";
    return;
  }
  if (e.cfg.dims[0] > 1024) {  // the update's per-workgroup channel capacity (update_body.h)
    e.chain_why = "final width above 1024";
    return;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, e.device) != hipSuccess ||
      cus < kChainGrid) {
    e.chain_why = "fewer compute units than the tick kernel's workgroups";
    return;
  }
  if (ensure_conv_records(&e) != FE_STATUS_OK) {
    e.chain_why = "convolution listing failed";
    clear_error();
    return;
  }
  std::vector<ChainConv> convs;
  for (std::size_t i = 0; i < e.conv_records.size(); ++i) {
    const FeEngine::ConvRecord& r = e.conv_records[i];
    ChainConv c;
    c.op = r.op;
    c.has_res = r.has_res;
    c.res = r.res;
    c.in = r.in;
    c.y = r.y;
    c.yr = r.yr;
    c.film = r.in.film_time != nullptr;
    c.state = i == 0;
    if (c.state && r.in.src != e.wp(e.w.x_in)) {
      e.chain_why = "first convolution does not read the U-Net input";
      return;
    }
    convs.push_back(c);
  }
  const int n = static_cast<int>(convs.size());
  std::vector<char> host(static_cast<std::size_t>(n) * chain_step_bytes());
  const char* why = "";
  if (!chain_build(convs.data(), n, host.data(), &why)) {
    e.chain_why = why;
    return;
  }
  if (hipMemcpy(e.ptr<char>(e.chain_steps), host.data(), host.size(), hipMemcpyHostToDevice) !=
      hipSuccess) {
    e.chain_why = "step table upload failed";
    return;
  }
  e.chain_nsteps = n;
  e.chain_on = true;
  e.chain_why = "";
}

fe_engine* create_engine(std::shared_ptr<const fe::Checkpoint> ck, unsigned threads) {
  if (threads > kMaxPoolThreads) {
    set_error("Worker thread count must be from 0 through 8");
    return nullptr;
  }
  if (!ck) {
    set_error("Invalid null model weights");
    return nullptr;
  }
  if (env_flag("FLOWEDGE_CUDA_FORCE_HOST")) {
    set_error("FLOWEDGE_CUDA_FORCE_HOST=1 but this library has no host kernels: the U-Net runs "
              "only on the GPU");
    return nullptr;
  }
  std::unique_ptr<FeEngine> e;
  try {
    e.reset(new FeEngine());
  } catch (const std::bad_alloc&) {
    set_error("Out of host memory");
    return nullptr;
  }
  e->threads = threads;
  std::string err;
  if (!parse_config(*ck, e->cfg, err) || !supported_shape(e->cfg, err)) {
    set_error(err);
    return nullptr;
  }
  e->max_batch = env_max_batch();
  e->mfma_batch = env_mfma_batch();
  {
    // FLOWEDGE_MFMA_BF16=0 keeps BF16 weights on the F32 matrix cores (widened, as F32 weights).
    const char* v = std::getenv("FLOWEDGE_MFMA_BF16");
    e->bf16_mma = !(v != nullptr && std::strcmp(v, "0") == 0);
    // FLOWEDGE_MFMA_F32_SPLIT=1 runs F32 weights on the BF16 matrix cores as three split products.
    v = std::getenv("FLOWEDGE_MFMA_F32_SPLIT");
    e->f32_split = v != nullptr && std::strcmp(v, "1") == 0;
  }
  if (e->max_batch == 0) {
    set_error("FLOWEDGE_MAX_BATCH must be an integer from 1 through 65535");
    return nullptr;
  }
  e->values = e->cfg.horizon * e->cfg.action_dim;
  e->digest = ck->digest();
  e->precision = ck->precision();
  Builder builder{*e, *ck, Plan{}, {}};
  if (!builder.build()) {
    set_error(builder.err);
    return nullptr;
  }
  const std::size_t work_base = (builder.plan.size + kAlign - 1) / kAlign * kAlign;
  e->w = plan_work(*e, e->max_batch, e->max_nfe, kSplitKFloats);
  const std::size_t done_off = work_base + (e->w.size + kAlign - 1) / kAlign * kAlign;
  e->arena_bytes = done_off + e->max_batch * sizeof(unsigned);
  // Measured crossovers (DDIM-10 ticks): the fused weight-streaming kernels stay faster through
  // 4 samples with F32 weights and 7 with BF16 weights.
  if (e->mfma_batch == 0) e->mfma_batch = e->bf16_convs ? 5 : 4;

  int count = 0;
  hipError_t st = hipGetDeviceCount(&count);
  if (st != hipSuccess || count == 0) {
    set_error("No HIP device available (the Diffusion Policy engine runs on the GPU only)");
    return nullptr;
  }
  if ((st = hipGetDevice(&e->device)) != hipSuccess) {
    hip_fail("hipGetDevice", st);
    return nullptr;
  }
  // Device address of this GPU's static scratch array (used only by the allocation-free entry
  // point, which reports a failure here when it is called).
  e->scratch_status = fe::hip::scratch_setup(e->device, &e->scratch);
  if (env_flag("FLOWEDGE_HIP_FAIL_ALLOC")) {
    set_error("Device arena allocation failed (FLOWEDGE_HIP_FAIL_ALLOC=1)");
    return nullptr;
  }
  st = hipMalloc(reinterpret_cast<void**>(&e->arena), e->arena_bytes);
  if (st != hipSuccess) {
    e->arena = nullptr;
    hip_fail("Device arena allocation failed", st);
    return nullptr;
  }
  g_device_allocs.fetch_add(1);
  e->ws = e->arena + work_base;
  e->own_ws = e->ws;
  if (split_update()) {
    e->upd_done = reinterpret_cast<unsigned*>(e->arena + done_off);
    if ((st = hipMemset(e->upd_done, 0, e->max_batch * sizeof(unsigned))) != hipSuccess) {
      hip_fail("Device arena initialisation failed", st);
      return nullptr;
    }
  }
  const std::size_t B = e->max_batch, nv = B * e->values, nc = B * e->cfg.cond_dim;
  const std::size_t pin_bytes = (nc + 2 * nv) * 4 + 64;
  void* pin = nullptr;
  if ((st = hipHostMalloc(&pin, pin_bytes, hipHostMallocDefault)) != hipSuccess) {
    hip_fail("Pinned staging allocation failed", st);
    return nullptr;
  }
  e->pin_cond = static_cast<float*>(pin);
  e->pin_noise = e->pin_cond + nc;
  e->pin_action = e->pin_noise + nv;
  e->pin_seed = reinterpret_cast<std::uint64_t*>(
      (reinterpret_cast<std::uintptr_t>(e->pin_action + nv) + 15) & ~std::uintptr_t{15});
  e->pin_status = reinterpret_cast<unsigned*>(e->pin_seed + 1);
  *e->pin_status = 0;
  if ((st = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking)) != hipSuccess ||
      (st = hipEventCreate(&e->ev0)) != hipSuccess || (st = hipEventCreate(&e->ev1)) != hipSuccess ||
      (side_streams() &&
       ((st = hipStreamCreateWithFlags(&e->side, hipStreamNonBlocking)) != hipSuccess ||
        (st = hipEventCreateWithFlags(&e->fork, hipEventDisableTiming)) != hipSuccess ||
        (st = hipEventCreateWithFlags(&e->join, hipEventDisableTiming)) != hipSuccess))) {
    hip_fail("Stream creation failed", st);
    return nullptr;
  }
  bind_all(*e);
  if ((st = upload_weights(*e, *ck)) != hipSuccess) {
    hip_fail("Weight upload failed", st);
    return nullptr;
  }
  if (e->cfg.prediction == 0) {
    // FiLM time rows for every train timestep, computed once on the device.
    fe::hip::TimeSpec ts;
    ts.mode = fe::hip::kTimesIndex;
    if ((st = enqueue_film_time(*e, ts, static_cast<int>(e->cfg.train_timesteps),
                                e->ptr(e->ddim_table))) != hipSuccess ||
        (st = hipStreamSynchronize(e->stream)) != hipSuccess) {
      hip_fail("FiLM time table failed", st);
      return nullptr;
    }
  }
  build_chain(*e);
  decide_partials(*e);
  return e.release();
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// C ABI.
// ---------------------------------------------------------------------------------------------
extern "C" {

const char* fe_engine_last_error(void) { return t_error; }

fe_weights* fe_weights_load(const char* path) {
  clear_error();
  if (path == nullptr) {
    set_error("Invalid null model path");
    return nullptr;
  }
  std::string err;
  auto ck = fe::Checkpoint::open(path, err);
  if (!ck) {
    set_error(err);
    return nullptr;
  }
  return new (std::nothrow) FeWeights{std::move(ck)};
}

size_t fe_weights_size_bytes(const fe_weights* weights) {
  return weights != nullptr && weights->ck ? weights->ck->weight_bytes() : 0;
}

void fe_weights_free(fe_weights* weights) { delete weights; }

int fe_weights_model_digest(const fe_weights* weights, fe_model_digest* digest) {
  clear_error();
  if (weights == nullptr || weights->ck == nullptr || digest == nullptr) {
    set_error("Invalid arguments to fe_weights_model_digest");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  std::memcpy(digest->bytes, weights->ck->digest().data(), FE_MODEL_DIGEST_BYTES);
  return FE_STATUS_OK;
}

static bool env_threads(unsigned& out) {
  const char* v = std::getenv("FLOWEDGE_THREADS");
  if (v == nullptr || *v == '\0') {
    out = 0;
    return true;
  }
  char* end = nullptr;
  const unsigned long n = std::strtoul(v, &end, 10);
  if (!end || *end != '\0' || n > kMaxPoolThreads) {
    set_error("FLOWEDGE_THREADS must be an integer from 0 through 8");
    return false;
  }
  out = static_cast<unsigned>(n);
  return true;
}

fe_engine* fe_engine_create_from_weights(const fe_weights* weights, unsigned worker_threads) {
  clear_error();
  if (weights == nullptr) {
    set_error("Invalid null model weights");
    return nullptr;
  }
  return create_engine(weights->ck, worker_threads);
}

fe_engine* fe_engine_create_from_weights_auto(const fe_weights* weights) {
  clear_error();
  if (weights == nullptr) {
    set_error("Invalid null model weights");
    return nullptr;
  }
  unsigned threads = 0;
  return env_threads(threads) ? create_engine(weights->ck, threads) : nullptr;
}

fe_engine* fe_engine_load_with_threads(const char* path, unsigned worker_threads) {
  clear_error();
  if (path == nullptr) {
    set_error("Invalid null model path");
    return nullptr;
  }
  std::string err;
  auto ck = fe::Checkpoint::open(path, err);
  if (!ck) {
    set_error(err);
    return nullptr;
  }
  return create_engine(std::move(ck), worker_threads);
}

fe_engine* fe_engine_load(const char* path) {
  clear_error();
  unsigned threads = 0;
  if (!env_threads(threads)) return nullptr;
  if (path == nullptr) {
    set_error("Invalid null model path");
    return nullptr;
  }
  std::string err;
  auto ck = fe::Checkpoint::open(path, err);
  if (!ck) {
    set_error(err);
    return nullptr;
  }
  return create_engine(std::move(ck), threads);
}

void fe_engine_free(fe_engine* engine) {
  if (engine) (void)hipSetDevice(engine->device);
  delete engine;
}

unsigned fe_engine_thread_count(const fe_engine* engine) {
  return engine != nullptr ? engine->threads : 0u;
}

int fe_engine_cuda_resident(const fe_engine* engine) { return engine != nullptr ? 1 : 0; }

int fe_engine_model_metadata(const fe_engine* engine, fe_model_metadata* metadata) {
  clear_error();
  if (engine == nullptr || metadata == nullptr) {
    set_error("Invalid arguments to fe_engine_model_metadata");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  fe_model_metadata m{};
  m.struct_size = sizeof(m);
  m.protocol_version = FE_PROTOCOL_VERSION;
  m.architecture = FE_ARCH_DIFFUSION_HEAD;
  m.precision = engine->precision;
  std::memcpy(m.model_digest.bytes, engine->digest.data(), FE_MODEL_DIGEST_BYTES);
  m.action_dim = engine->cfg.action_dim;
  m.condition_dim = engine->cfg.cond_dim;
  *metadata = m;
  return FE_STATUS_OK;
}

size_t fe_engine_action_dim(const fe_engine* engine) {
  return engine != nullptr ? engine->cfg.action_dim : 0;
}

size_t fe_engine_action_horizon(const fe_engine* engine) {
  return engine != nullptr ? engine->cfg.horizon : 0;
}

size_t fe_engine_condition_dim(const fe_engine* engine) {
  return engine != nullptr ? engine->cfg.cond_dim : 0;
}

int fe_engine_diffusion_metadata(const fe_engine* engine, fe_diffusion_metadata* metadata) {
  clear_error();
  if (engine == nullptr || metadata == nullptr) {
    set_error("Invalid arguments to fe_engine_diffusion_metadata");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  fe_diffusion_metadata m{};
  m.struct_size = sizeof(m);
  m.protocol_version = FE_PROTOCOL_VERSION;
  m.clip_sample = engine->cfg.clip ? 1u : 0u;
  m.action_dim = engine->cfg.action_dim;
  m.condition_dim = engine->cfg.cond_dim;
  m.horizon = engine->cfg.horizon;
  m.action_steps = engine->cfg.action_steps;
  m.observation_steps = engine->cfg.obs_steps;
  m.train_timesteps = engine->cfg.train_timesteps;
  m.clip_sample_range = engine->cfg.clip_range;
  *metadata = m;
  return FE_STATUS_OK;
}

int fe_engine_sample_diffusion_batch(fe_engine* engine, const float* condition,
                                     const float* noise, size_t batch, size_t steps,
                                     int scheduler, uint64_t seed, float* action) {
  clear_error();
  if (engine == nullptr || condition == nullptr || noise == nullptr || action == nullptr ||
      steps == 0 || batch == 0) {
    set_error("Invalid arguments to fe_engine_sample_diffusion");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  if (scheduler != FE_DIFFUSION_DDIM && scheduler != FE_DIFFUSION_DDPM) {
    set_error("Diffusion scheduler must be FE_DIFFUSION_DDIM or FE_DIFFUSION_DDPM");
    return FE_STATUS_INVALID_SOLVER;
  }
  return sample_host(engine, 0, condition, noise, batch, steps, scheduler, seed, action);
}

int fe_engine_sample_diffusion(fe_engine* engine, const float* condition, const float* noise,
                               size_t steps, int scheduler, uint64_t seed, float* action) {
  return fe_engine_sample_diffusion_batch(engine, condition, noise, 1, steps, scheduler, seed,
                                          action);
}

int fe_engine_sample_condition_batch(fe_engine* engine, const float* condition,
                                     const float* noise, size_t batch, size_t steps, int method,
                                     float* action) {
  clear_error();
  if (engine == nullptr || condition == nullptr || noise == nullptr || action == nullptr ||
      steps == 0 || batch == 0) {
    set_error("Invalid arguments to fe_engine_sample_condition");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  if (method < FE_SOLVER_EULER || method > FE_SOLVER_RK4) {
    set_error("Invalid solver method");
    return FE_STATUS_INVALID_SOLVER;
  }
  return sample_host(engine, 1, condition, noise, batch, steps, method, 0, action);
}

int fe_engine_sample_condition(fe_engine* engine, const float* condition, const float* noise,
                               size_t steps, int method, float* action) {
  return fe_engine_sample_condition_batch(engine, condition, noise, 1, steps, method, action);
}

int fe_engine_diffusion_denoise_batch(fe_engine* engine, const float* condition,
                                      const float* normalized_sample, size_t batch,
                                      float timestep, float* predicted_noise) {
  clear_error();
  if (engine == nullptr || condition == nullptr || normalized_sample == nullptr ||
      predicted_noise == nullptr || !std::isfinite(timestep) || batch == 0) {
    set_error("Invalid arguments to fe_engine_diffusion_denoise");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  if (engine->cfg.prediction != 0) {
    set_error("Model has no Diffusion Policy head");  // engine_runtime.cc:476-479
    return FE_STATUS_UNSUPPORTED_MODEL;
  }
  if (batch > engine->max_batch) {
    set_error("Batch size must be between 1 and the engine's max batch");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  FeEngine* e = engine;
  hipError_t st = hipSetDevice(e->device);
  if (st != hipSuccess) return hip_fail("hipSetDevice", st);
  end_solve(e);
  const Config& c = e->cfg;
  const std::size_t nc = batch * c.cond_dim, nv = batch * e->values;
  std::memcpy(e->pin_cond, condition, nc * 4);
  std::memcpy(e->pin_noise, normalized_sample, nv * 4);
  using namespace fe::hip;
  if ((st = hipMemcpyAsync(e->wp(e->w.in_cond), e->pin_cond, nc * 4, hipMemcpyHostToDevice,
                           e->stream)) != hipSuccess ||
      (st = hipMemcpyAsync(e->wp(e->w.in_noise), e->pin_noise, nv * 4, hipMemcpyHostToDevice,
                           e->stream)) != hipSuccess)
    return hip_fail("Input upload failed", st);
  const int b = static_cast<int>(batch);
  TimeSpec ts;
  ts.mode = kTimesSingle;
  ts.t0 = timestep;
  UpdateOp u{};
  u.kind = kUpdateDenoise;
  u.out = e->wp(e->w.out_action);
  if ((st = begin_sample(e->wp(e->w.in_noise), e->wp(e->w.x_in), e->wp(e->w.x_in), b,
                         static_cast<int>(c.horizon), static_cast<int>(c.action_dim),
                         e->stream)) != hipSuccess ||
      (st = enqueue_film(*e, ts, 1, b)) != hipSuccess ||
      (st = enqueue_unet(*e, b, e->wp(e->w.film_table), u)) != hipSuccess ||
      (st = hipMemcpyAsync(e->pin_action, e->wp(e->w.out_action), nv * 4, hipMemcpyDeviceToHost,
                           e->stream)) != hipSuccess ||
      (st = hipStreamSynchronize(e->stream)) != hipSuccess)
    return hip_fail("Diffusion denoiser execution failed", st);
  std::memcpy(predicted_noise, e->pin_action, nv * 4);
  return FE_STATUS_OK;
}

int fe_engine_diffusion_denoise(fe_engine* engine, const float* condition,
                                const float* normalized_sample, float timestep,
                                float* predicted_noise) {
  return fe_engine_diffusion_denoise_batch(engine, condition, normalized_sample, 1, timestep,
                                           predicted_noise);
}

int fe_engine_diffusion_denoise_noalloc(fe_engine* engine, const float* condition_dev,
                                        const float* sample_dev, size_t batch, float timestep,
                                        float* predicted_noise_dev, void* stream) {
  clear_error();
  if (engine == nullptr || condition_dev == nullptr || sample_dev == nullptr ||
      predicted_noise_dev == nullptr || !std::isfinite(timestep) || batch == 0 ||
      batch > 65535) {
    set_error("Invalid arguments to fe_engine_diffusion_denoise_noalloc");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  FeEngine* e = engine;
  if (e->cfg.prediction != 0) {
    set_error("Model has no Diffusion Policy head");
    return FE_STATUS_UNSUPPORTED_MODEL;
  }
  if (e->scratch == nullptr) {
    return hip_fail("Device scratch of the allocation-free entry point is unavailable",
                    e->scratch_status);
  }
  // The whole workspace of one evaluation of `batch` samples lives in the scratch array; what is
  // left of it holds split-K partials (fewer partials only means fewer K splits).
  Work w = plan_work(*e, batch, 1, 0);
  const std::size_t base = (w.size + kAlign - 1) / kAlign * kAlign;
  if (w.size > fe::hip::kScratchBytes) {
    set_error("Batch too large for the allocation-free scratch: " + std::to_string(w.size) +
              " bytes needed, " + std::to_string(fe::hip::kScratchBytes) + " available");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  const std::size_t spare = fe::hip::kScratchBytes > base ? fe::hip::kScratchBytes - base : 0;
  w = plan_work(*e, batch, 1, std::min(kSplitKFloats, spare / 4));
  hipError_t st = hipSetDevice(e->device);
  if (st != hipSuccess) return hip_fail("hipSetDevice", st);
  // Enqueue one evaluation against the scratch workspace on the caller's stream (or the engine's);
  // the engine's own workspace and any resumable solve are left untouched.
  char* const saved_ws = e->ws;
  const Work saved_w = e->w;
  const hipStream_t saved_stream = e->stream;
  e->ws = static_cast<char*>(e->scratch);
  e->w = w;
  if (stream != nullptr) e->stream = static_cast<hipStream_t>(stream);
  using namespace fe::hip;
  const int b = static_cast<int>(batch);
  TimeSpec ts;
  ts.mode = kTimesSingle;
  ts.t0 = timestep;
  UpdateOp u{};
  u.kind = kUpdateDenoise;
  u.out = predicted_noise_dev;
  st = begin_sample(sample_dev, e->wp(e->w.x_in), e->wp(e->w.x_in), b,
                    static_cast<int>(e->cfg.horizon), static_cast<int>(e->cfg.action_dim),
                    e->stream);
  if (st == hipSuccess) st = enqueue_film(*e, ts, 1, b, condition_dev);
  if (st == hipSuccess) st = enqueue_unet(*e, b, e->wp(e->w.film_table), u);
  e->ws = saved_ws;
  e->w = saved_w;
  e->stream = saved_stream;
  if (st == hipSuccess && stream == nullptr) st = hipStreamSynchronize(e->stream);
  if (st != hipSuccess) return hip_fail("Diffusion denoiser execution failed", st);
  return FE_STATUS_OK;
}

int fe_engine_sample_device(fe_engine* engine, int kind, const float* condition_dev,
                            const float* noise_dev, size_t batch, size_t steps, int mode,
                            uint64_t seed, float* action_dev) {
  clear_error();
  if (engine == nullptr || condition_dev == nullptr || noise_dev == nullptr ||
      action_dev == nullptr || (kind != 0 && kind != 1)) {
    set_error("Invalid arguments to fe_engine_sample_device");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  FeEngine* e = engine;
  const int rc = check_sample(e, kind, batch, steps, mode);
  if (rc != FE_STATUS_OK) return rc;
  hipError_t st = hipSetDevice(e->device);
  if (st != hipSuccess) return hip_fail("hipSetDevice", st);
  end_solve(e);
  const std::size_t nc = batch * e->cfg.cond_dim, nv = batch * e->values;
  *e->pin_seed = seed;
  if ((st = hipMemcpyAsync(e->wp(e->w.in_cond), condition_dev, nc * 4, hipMemcpyDeviceToDevice,
                           e->stream)) != hipSuccess ||
      (st = hipMemcpyAsync(e->wp(e->w.in_noise), noise_dev, nv * 4, hipMemcpyDeviceToDevice,
                           e->stream)) != hipSuccess ||
      (st = hipMemcpyAsync(e->wp(e->w.seed), e->pin_seed, 8, hipMemcpyHostToDevice,
                           e->stream)) != hipSuccess)
    return hip_fail("Input copy failed", st);
  bool chained = false;
  for (int attempt = 0; attempt < 2; ++attempt) {
    const int r = run_graph(e, kind, batch, steps, mode, chained);
    if (r != FE_STATUS_OK) return r;
    if ((st = hipMemcpyAsync(action_dev, e->wp(e->w.out_action), nv * 4,
                             hipMemcpyDeviceToDevice, e->stream)) != hipSuccess ||
        (st = hipStreamSynchronize(e->stream)) != hipSuccess)
      return hip_fail("Sampling failed", st);
    if (!chain_abandoned(e, chained)) break;
  }
  return FE_STATUS_OK;
}

int fe_engine_prepare(fe_engine* engine, int kind, size_t batch, size_t steps, int mode) {
  clear_error();
  if (engine == nullptr || (kind != 0 && kind != 1)) {
    set_error("Invalid arguments to fe_engine_prepare");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  const int rc = check_sample(engine, kind, batch, steps, mode);
  if (rc != FE_STATUS_OK) return rc;
  hipError_t st = hipSetDevice(engine->device);
  if (st != hipSuccess) return hip_fail("hipSetDevice", st);
  hipGraphExec_t exec = nullptr;
  st = get_graph(*engine, kind, batch, steps, mode, exec);
  return st == hipSuccess ? FE_STATUS_OK : hip_fail("Failed to build sampling graph", st);
}

// ---- Resumable solves (engine.h:321-366) ----

int fe_engine_flow_begin(fe_engine* engine, const float* condition, const float* noise,
                         size_t steps, int method) {
  clear_error();
  if (engine == nullptr || condition == nullptr || noise == nullptr || steps == 0) {
    set_error("Invalid arguments to fe_engine_flow_begin");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  if (method < FE_SOLVER_EULER || method > FE_SOLVER_RK4) {
    set_error("Invalid solver method");
    return FE_STATUS_INVALID_SOLVER;
  }
  SolveRequest r;
  r.kind = 1;
  r.mode = method;
  r.steps = steps;
  return solve_begin(engine, condition, noise, r);
}

int fe_engine_make_condition_metadata(const fe_engine* engine, uint64_t timestamp_ns,
                                      uint64_t deadline_ns, uint64_t generation, size_t steps,
                                      int method, fe_condition_metadata* metadata) {
  clear_error();
  if (engine == nullptr || metadata == nullptr || steps == 0 ||
      (deadline_ns != 0 && deadline_ns < timestamp_ns)) {
    set_error("Invalid arguments to fe_engine_make_condition_metadata");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  if (method < FE_SOLVER_EULER || method > FE_SOLVER_RK4) {
    set_error("Invalid solver method");
    return FE_STATUS_INVALID_SOLVER;
  }
  fe_condition_metadata m{};
  m.struct_size = sizeof(m);
  m.protocol_version = FE_PROTOCOL_VERSION;
  m.solver = static_cast<uint32_t>(method);
  std::memcpy(m.model_digest.bytes, engine->digest.data(), FE_MODEL_DIGEST_BYTES);
  m.timestamp_ns = timestamp_ns;
  m.deadline_ns = deadline_ns;
  m.generation = generation;
  m.condition_dim = engine->cfg.cond_dim;
  m.action_dim = engine->cfg.action_dim;
  m.solver_steps = steps;
  m.remaining_nfe = nfe_for(steps, 1, method);
  *metadata = m;
  return FE_STATUS_OK;
}

int fe_engine_flow_begin_request(fe_engine* engine, const float* condition, const float* noise,
                                 const fe_condition_metadata* metadata) {
  clear_error();
  if (engine == nullptr || condition == nullptr || noise == nullptr || metadata == nullptr ||
      metadata->struct_size < sizeof(*metadata) ||
      metadata->protocol_version != FE_PROTOCOL_VERSION || metadata->reserved != 0 ||
      metadata->solver_steps == 0 || metadata->solver_steps > SIZE_MAX) {
    set_error("Invalid versioned flow request metadata");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  const int method = static_cast<int>(metadata->solver);
  if (metadata->solver > static_cast<uint32_t>(FE_SOLVER_RK4)) {
    set_error("Invalid solver method in flow request metadata");
    return FE_STATUS_INVALID_SOLVER;
  }
  if (std::memcmp(metadata->model_digest.bytes, engine->digest.data(), FE_MODEL_DIGEST_BYTES) !=
          0 ||
      metadata->condition_dim != engine->cfg.cond_dim ||
      metadata->action_dim != engine->cfg.action_dim ||
      metadata->remaining_nfe != nfe_for(static_cast<size_t>(metadata->solver_steps), 1, method) ||
      (metadata->deadline_ns != 0 && metadata->deadline_ns < metadata->timestamp_ns)) {
    set_error("Flow request metadata is incompatible with this model");
    return FE_STATUS_INCOMPATIBLE_STATE;
  }
  SolveRequest r;
  r.kind = 1;
  r.mode = method;
  r.steps = static_cast<size_t>(metadata->solver_steps);
  r.tracking = true;
  r.generation = metadata->generation;
  r.timestamp_ns = metadata->timestamp_ns;
  r.deadline_ns = metadata->deadline_ns;
  return solve_begin(engine, condition, noise, r);
}

void fe_engine_cancel_before(fe_engine* engine, uint64_t generation) {
  if (engine != nullptr) raise_generation(engine, generation);
}

int fe_engine_flow_advance(fe_engine* engine, size_t step_budget, float* action,
                           size_t* steps_remaining) {
  clear_error();
  if (engine == nullptr || action == nullptr || step_budget == 0) {
    set_error("Invalid arguments to fe_engine_flow_advance");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  size_t remaining = 0;
  const int rc = solve_advance(engine, 1, step_budget, action, remaining);
  if ((rc == FE_STATUS_OK || rc == FE_STATUS_CANCELLED) && steps_remaining != nullptr)
    *steps_remaining = remaining;
  return rc;
}

int fe_engine_flow_action_metadata(const fe_engine* engine, fe_action_metadata* metadata) {
  clear_error();
  if (engine == nullptr || metadata == nullptr) {
    set_error("Invalid arguments to fe_engine_flow_action_metadata");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  const FeEngine::Solve& v = engine->solve;
  fe_action_metadata m{};
  m.struct_size = sizeof(m);
  m.protocol_version = FE_PROTOCOL_VERSION;
  m.solver = static_cast<uint32_t>(v.mode);
  // engine_runtime.cc:294-301.
  m.status = v.cancelled ? FE_ACTION_CANCELLED
             : !v.active ? FE_ACTION_FAILED
             : v.remaining() == 0 ? FE_ACTION_COMPLETE
                                  : FE_ACTION_RUNNING;
  std::memcpy(m.model_digest.bytes, engine->digest.data(), FE_MODEL_DIGEST_BYTES);
  m.timestamp_ns = v.timestamp_ns;
  m.deadline_ns = v.deadline_ns;
  m.generation = v.generation;
  m.condition_dim = engine->cfg.cond_dim;
  m.action_dim = engine->cfg.action_dim;
  m.remaining_nfe = nfe_for(v.remaining(), v.kind, v.mode);
  *metadata = m;
  return FE_STATUS_OK;
}

int fe_engine_diffusion_begin(fe_engine* engine, const float* condition, const float* noise,
                              size_t steps, int scheduler, uint64_t seed) {
  clear_error();
  if (engine == nullptr || condition == nullptr || noise == nullptr || steps == 0) {
    set_error("Invalid arguments to fe_engine_diffusion_begin");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  if (scheduler != FE_DIFFUSION_DDIM && scheduler != FE_DIFFUSION_DDPM) {
    set_error("Diffusion scheduler must be FE_DIFFUSION_DDIM or FE_DIFFUSION_DDPM");
    return FE_STATUS_INVALID_SOLVER;
  }
  SolveRequest r;
  r.kind = 0;
  r.mode = scheduler;
  r.steps = steps;
  r.seed = seed;
  return solve_begin(engine, condition, noise, r);
}

int fe_engine_diffusion_begin_generation(fe_engine* engine, const float* condition,
                                         const float* noise, size_t steps, int scheduler,
                                         uint64_t seed, uint64_t generation) {
  clear_error();
  if (engine == nullptr || condition == nullptr || noise == nullptr || steps == 0) {
    set_error("Invalid arguments to fe_engine_diffusion_begin_generation");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  if (scheduler != FE_DIFFUSION_DDIM && scheduler != FE_DIFFUSION_DDPM) {
    set_error("Diffusion scheduler must be FE_DIFFUSION_DDIM or FE_DIFFUSION_DDPM");
    return FE_STATUS_INVALID_SOLVER;
  }
  SolveRequest r;
  r.kind = 0;
  r.mode = scheduler;
  r.steps = steps;
  r.seed = seed;
  r.tracking = true;
  r.generation = generation;
  return solve_begin(engine, condition, noise, r);
}

int fe_engine_diffusion_advance(fe_engine* engine, size_t step_budget, float* action,
                                size_t* steps_remaining) {
  clear_error();
  if (engine == nullptr || action == nullptr || step_budget == 0) {
    set_error("Invalid arguments to fe_engine_diffusion_advance");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  size_t remaining = 0;
  const int rc = solve_advance(engine, 0, step_budget, action, remaining);
  if ((rc == FE_STATUS_OK || rc == FE_STATUS_CANCELLED) && steps_remaining != nullptr)
    *steps_remaining = remaining;
  return rc;
}

size_t fe_engine_max_batch(const fe_engine* engine) {
  return engine != nullptr ? engine->max_batch : 0;
}

size_t fe_engine_device_bytes(const fe_engine* engine) {
  return engine != nullptr ? engine->arena_bytes : 0;
}

uint64_t fe_device_alloc_count(void) { return g_device_allocs.load(); }

uint64_t fe_engine_graph_captures(const fe_engine* engine) {
  return engine != nullptr ? engine->captures : 0;
}

int fe_engine_persistent_tick(const fe_engine* engine) {
  return engine != nullptr && engine->chain_on ? 1 : 0;
}

const char* fe_engine_persistent_tick_reason(const fe_engine* engine) {
  return engine != nullptr ? engine->chain_why.c_str() : "no engine";
}

int fe_engine_conv_count(fe_engine* engine, size_t* count) {
  clear_error();
  if (engine == nullptr || count == nullptr) {
    set_error("Invalid arguments to fe_engine_conv_count");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  const int rc = ensure_conv_records(engine);
  if (rc != FE_STATUS_OK) return rc;
  *count = engine->conv_records.size();
  return FE_STATUS_OK;
}

int fe_engine_conv_info(fe_engine* engine, size_t index, char* name, size_t name_capacity,
                        uint64_t* weight_bytes, uint64_t* sample_bytes) {
  clear_error();
  if (engine == nullptr) {
    set_error("Invalid arguments to fe_engine_conv_info");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  const int rc = ensure_conv_records(engine);
  if (rc != FE_STATUS_OK) return rc;
  if (index >= engine->conv_records.size()) {
    set_error("Convolution index out of range");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  const FeEngine::ConvRecord& r = engine->conv_records[index];
  if (name != nullptr && name_capacity > 0) {
    const std::size_t n = std::min(name_capacity - 1, r.name.size());
    std::memcpy(name, r.name.data(), n);
    name[n] = '\0';
  }
  if (weight_bytes != nullptr) *weight_bytes = r.weight_bytes;
  if (sample_bytes != nullptr) *sample_bytes = r.sample_bytes;
  return FE_STATUS_OK;
}

int fe_engine_conv_path(fe_engine* engine, size_t index, size_t batch, int* path) {
  clear_error();
  if (engine == nullptr || path == nullptr || batch == 0 || batch > engine->max_batch) {
    set_error("Invalid arguments to fe_engine_conv_path");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  const int rc = ensure_conv_records(engine, batch);
  if (rc != FE_STATUS_OK) return rc;
  if (index >= engine->conv_records.size()) {
    set_error("Convolution index out of range");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  const FeEngine::ConvRecord& r = engine->conv_records[index];
  *path = static_cast<int>(conv_path(*engine, r.op, r.has_res ? &r.res : nullptr, r.in, r.yr,
                                     static_cast<int>(batch)));
  return FE_STATUS_OK;
}

int fe_engine_conv_slices(fe_engine* engine, size_t index, size_t batch, int* slices) {
  clear_error();
  if (engine == nullptr || slices == nullptr || batch == 0 || batch > engine->max_batch) {
    set_error("Invalid arguments to fe_engine_conv_slices");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  const int rc = ensure_conv_records(engine, batch);
  if (rc != FE_STATUS_OK) return rc;
  if (index >= engine->conv_records.size()) {
    set_error("Convolution index out of range");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  *slices = engine->conv_records[index].slices.slices;
  return FE_STATUS_OK;
}

int fe_engine_time_convs(fe_engine* engine, const size_t* indices, size_t n, size_t batch,
                         size_t iters, float* avg_us) {
  clear_error();
  if (engine == nullptr || indices == nullptr || n == 0 || iters == 0 || avg_us == nullptr ||
      batch == 0 || batch > engine->max_batch) {
    set_error("Invalid arguments to fe_engine_time_convs");
    return FE_STATUS_INVALID_ARGUMENT;
  }
  FeEngine* e = engine;
  const int rc = ensure_conv_records(e, batch);
  if (rc != FE_STATUS_OK) return rc;
  for (size_t i = 0; i < n; ++i)
    if (indices[i] >= e->conv_records.size()) {
      set_error("Convolution index out of range");
      return FE_STATUS_INVALID_ARGUMENT;
    }
  hipError_t st = hipSetDevice(e->device);
  if (st != hipSuccess) return hip_fail("hipSetDevice", st);
  const int b = static_cast<int>(batch);
  auto round = [&]() -> hipError_t {
    for (size_t i = 0; i < n; ++i) {
      const FeEngine::ConvRecord& r = e->conv_records[indices[i]];
      const hipError_t s2 = dispatch_conv(*e, r.op, r.has_res ? &r.res : nullptr, r.in, r.y,
                                          r.yr, b, e->stream, r.slices);
      if (s2 != hipSuccess) return s2;
    }
    return hipSuccess;
  };
  if ((st = round()) != hipSuccess || (st = hipEventRecord(e->ev0, e->stream)) != hipSuccess)
    return hip_fail("Convolution timing failed", st);
  for (size_t it = 0; it < iters; ++it)
    if ((st = round()) != hipSuccess) return hip_fail("Convolution timing failed", st);
  float ms = 0.0f;
  if ((st = hipEventRecord(e->ev1, e->stream)) != hipSuccess ||
      (st = hipEventSynchronize(e->ev1)) != hipSuccess ||
      (st = hipEventElapsedTime(&ms, e->ev0, e->ev1)) != hipSuccess)
    return hip_fail("Convolution timing failed", st);
  e->timed = false;  // the events no longer bracket a sampling graph
  *avg_us = ms * 1000.0f / static_cast<float>(iters * n);
  return FE_STATUS_OK;
}

float fe_engine_last_device_ms(const fe_engine* engine) {
  if (engine == nullptr || !engine->timed) return -1.0f;
  float ms = -1.0f;
  if (hipEventElapsedTime(&ms, engine->ev0, engine->ev1) != hipSuccess) return -1.0f;
  return ms;
}

}  // extern "C"

// The thread-local error and the allocation counter, for the library's other C ABI translation
// units (the observation encoder).
namespace fe::abi {
void set_error(const std::string& msg) { ::set_error(msg); }
void clear_error() { ::clear_error(); }
void count_device_alloc() { g_device_allocs.fetch_add(1); }
}  // namespace fe::abi
