/*
 * FlowEdge-compatible C ABI for the Diffusion Policy U-Net action head on AMD Instinct MI355X.
 *
 * Drop-in surface: every declaration below that carries a reference citation has the same name,
 * argument meaning, status codes and thread-local error behaviour as elprofesoriqo/FlowEdge's
 * `src/core/api/engine.h` (cited as engine.h:line).  The library behind it keeps the model
 * weights and all scratch in one device arena allocated at load, and runs each sampling call as
 * one hipGraph replay of hand-written gfx950 kernels.  Host buffers are caller-owned float
 * arrays; sample/action buffers use [horizon][action_dim] order.
 *
 * Extensions (no reference counterpart) are grouped at the end and say so.
 */
#ifndef FLOWEDGE_AMD_H
#define FLOWEDGE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct FeEngine fe_engine;
typedef struct FeWeights fe_weights;

/* engine.h:16-21 */
enum {
  FE_SOLVER_EULER = 0,
  FE_SOLVER_HEUN = 1,
  FE_SOLVER_RK4 = 2,
};

/* engine.h:23-27 */
enum {
  FE_DIFFUSION_DDIM = 0,
  FE_DIFFUSION_DDPM = 1,
};

/* protocol/contracts.h:10-30 */
enum {
  FE_PROTOCOL_VERSION = 1,
  FE_MODEL_DIGEST_BYTES = 16,
};
enum {
  FE_ARCH_UNKNOWN = 0,
  FE_ARCH_DIFFUSION_HEAD = 4,
};
enum {
  FE_PRECISION_UNKNOWN = 0,
  FE_PRECISION_F32 = 1,
  FE_PRECISION_BF16 = 2,
  FE_PRECISION_MIXED = 3,
};

/* protocol/contracts.h:36-42 — status of a resumable solve's current action. */
enum {
  FE_ACTION_RUNNING = 0,
  FE_ACTION_COMPLETE = 1,
  FE_ACTION_CANCELLED = 2,
  FE_ACTION_FAILED = 3,
};

/* engine.h:29-43 */
typedef struct fe_diffusion_metadata {
  uint32_t struct_size;
  uint32_t protocol_version;
  uint32_t clip_sample;
  uint32_t reserved;
  uint64_t action_dim;
  uint64_t condition_dim;
  uint64_t horizon;
  uint64_t action_steps;
  uint64_t observation_steps;
  uint64_t train_timesteps;
  float clip_sample_range;
  float reserved_float;
} fe_diffusion_metadata;

/* protocol/contracts.h:62-83 */
typedef struct fe_model_digest {
  uint8_t bytes[FE_MODEL_DIGEST_BYTES];
} fe_model_digest;
typedef struct fe_model_metadata {
  uint32_t struct_size;
  uint32_t protocol_version;
  uint32_t architecture;
  uint32_t precision;
  fe_model_digest model_digest;
  uint64_t d_model;
  uint64_t n_layers;
  uint64_t d_inner;
  uint64_t d_state;
  uint64_t d_conv;
  uint64_t action_dim;
  uint64_t condition_dim;
  uint64_t decode_snapshot_bytes;
} fe_model_metadata;

/* protocol/contracts.h:105-134 — versioned request and action metadata of resumable solves. */
typedef struct fe_condition_metadata {
  uint32_t struct_size;
  uint32_t protocol_version;
  uint32_t solver;
  uint32_t reserved;
  fe_model_digest model_digest;
  uint64_t timestamp_ns;
  uint64_t deadline_ns;
  uint64_t generation;
  uint64_t condition_dim;
  uint64_t action_dim;
  uint64_t solver_steps;
  uint64_t remaining_nfe;
} fe_condition_metadata;
typedef struct fe_action_metadata {
  uint32_t struct_size;
  uint32_t protocol_version;
  uint32_t solver;
  uint32_t status;
  fe_model_digest model_digest;
  uint64_t timestamp_ns;
  uint64_t deadline_ns;
  uint64_t generation;
  uint64_t condition_dim;
  uint64_t action_dim;
  uint64_t remaining_nfe;
} fe_action_metadata;

/* engine.h:46-59 */
enum {
  FE_STATUS_OK = 0,
  FE_STATUS_INVALID_ARGUMENT = 1,
  FE_STATUS_RESOURCE_EXHAUSTED = 2,
  FE_STATUS_TOKEN_OUT_OF_RANGE = 3,
  FE_STATUS_UNSUPPORTED_MODEL = 4,
  FE_STATUS_INVALID_SOLVER = 5,
  FE_STATUS_NO_ACTIVE_OPERATION = 6,
  FE_STATUS_STATE_UNAVAILABLE = 7,
  FE_STATUS_CANCELLED = 8,
  FE_STATUS_INCOMPATIBLE_STATE = 9,
  FE_STATUS_CORRUPT_STATE = 10,
};

/* engine.h:63 — last error on this thread; valid until the next ABI call; never NULL. */
const char* fe_engine_last_error(void);

/* engine.h:71 — load a dp.* .safetensors checkpoint into one device arena; NULL on failure. */
fe_engine* fe_engine_load(const char* path);

/* engine.h:82 — `worker_threads` (0-8) is validated and reported; device execution uses none. */
fe_engine* fe_engine_load_with_threads(const char* path, unsigned worker_threads);

/* engine.h:85 — immutable host weight store shareable by several engines. */
fe_weights* fe_weights_load(const char* path);

/* engine.h:88 */
size_t fe_weights_size_bytes(const fe_weights* weights);

/* engine.h:91 */
void fe_weights_free(fe_weights* weights);

/* engine.h:94 — each engine owns its own device arena built from the shared host store. */
fe_engine* fe_engine_create_from_weights(const fe_weights* weights, unsigned worker_threads);

/* engine.h:97 */
fe_engine* fe_engine_create_from_weights_auto(const fe_weights* weights);

/* engine.h:218 */
unsigned fe_engine_thread_count(const fe_engine* engine);

/* engine.h:227 — 1 when the weights are device-resident (always, for a loaded engine). */
int fe_engine_cuda_resident(const fe_engine* engine);

/* engine.h:230 */
int fe_engine_model_metadata(const fe_engine* engine, fe_model_metadata* metadata);

/* engine.h:245 */
size_t fe_engine_action_dim(const fe_engine* engine);

/* engine.h:251 */
size_t fe_engine_action_horizon(const fe_engine* engine);

/* engine.h:254 */
int fe_engine_diffusion_metadata(const fe_engine* engine, fe_diffusion_metadata* metadata);

/* engine.h:261 */
size_t fe_engine_condition_dim(const fe_engine* engine);

/* engine.h:277-278 — DDIM/DDPM action chunk in original action units. */
int fe_engine_sample_diffusion(fe_engine* engine, const float* condition, const float* noise,
                               size_t steps, int scheduler, uint64_t seed, float* action);

/* engine.h:281-283 — one U-Net pass in normalized action space (epsilon, or velocity for a
 * flow checkpoint). */
int fe_engine_diffusion_denoise(fe_engine* engine, const float* condition,
                                const float* normalized_sample, float timestep,
                                float* predicted_noise);

/* engine.h:318-319 — flow-ODE sample.  Served by a U-Net checkpoint whose dp.meta[12] == 1
 * (velocity field v(x,t|c), continuous t in [0,1]); `noise` and `action` hold
 * [horizon][action_dim] values and the result is x(1) without unnormalisation, as the
 * reference flow head returns it (flow.cc:321). */
int fe_engine_sample_condition(fe_engine* engine, const float* condition, const float* noise,
                               size_t steps, int method, float* action);

/* engine.h:321-330 — begin a resumable flow solve (velocity checkpoints, as
 * fe_engine_sample_condition).  One resumable solve per engine: a new begin replaces it, and any
 * sampling or denoising call on the engine ends it (its buffers are reused).  Not cancellable. */
int fe_engine_flow_begin(fe_engine* engine, const float* condition, const float* noise,
                         size_t steps, int method);

/* engine.h:332-338 — request metadata for this model: digest, dimensions (action_dim per horizon
 * step), steps and remaining_nfe = steps x evaluations per step. */
int fe_engine_make_condition_metadata(const fe_engine* engine, uint64_t timestamp_ns,
                                      uint64_t deadline_ns, uint64_t generation, size_t steps,
                                      int method, fe_condition_metadata* metadata);

/* engine.h:340-342 — begin a cancellable flow solve after validating the metadata
 * (status 9 if it does not match this model). */
int fe_engine_flow_begin_request(fe_engine* engine, const float* condition, const float* noise,
                                 const fe_condition_metadata* metadata);

/* engine.h:344-348 — cancel tracked solves of a lower generation; safe to call from another
 * thread while a solve advances.  The solve stops before its next step. */
void fe_engine_cancel_before(fe_engine* engine, uint64_t generation);

/* engine.h:350-363 — run at most `step_budget` solver steps; `action` [horizon][action_dim]
 * receives the current state (the final x(1) once *steps_remaining is 0).  Status 6 when no
 * flow solve is active, 8 after a cancellation (steps_remaining is still written). */
int fe_engine_flow_advance(fe_engine* engine, size_t step_budget, float* action,
                           size_t* steps_remaining);

/* engine.h:365-366 — metadata of the current action of the engine's resumable solve. */
int fe_engine_flow_action_metadata(const fe_engine* engine, fe_action_metadata* metadata);

/* engine.h:395 */
void fe_engine_free(fe_engine* engine);

/* ---------------------------------------------------------------------------------------------
 * Extensions (no reference counterpart).
 * ------------------------------------------------------------------------------------------- */

/* Batched DDIM/DDPM: equal to `batch` independent fe_engine_sample_diffusion calls with the same
 * steps/scheduler/seed.  condition [batch][condition_dim], noise/action
 * [batch][horizon][action_dim]. */
int fe_engine_sample_diffusion_batch(fe_engine* engine, const float* condition,
                                     const float* noise, size_t batch, size_t steps,
                                     int scheduler, uint64_t seed, float* action);

/* Batched flow-ODE sample for a velocity checkpoint (see fe_engine_sample_condition). */
int fe_engine_sample_condition_batch(fe_engine* engine, const float* condition,
                                     const float* noise, size_t batch, size_t steps, int method,
                                     float* action);

/* Batched single U-Net pass. */
int fe_engine_diffusion_denoise_batch(fe_engine* engine, const float* condition,
                                      const float* normalized_sample, size_t batch,
                                      float timestep, float* predicted_noise);

/* Resumable DDIM/DDPM solve, the Diffusion Policy counterpart of fe_engine_flow_begin /
 * fe_engine_flow_advance with the same rules (one solve per engine, ended by other sampling
 * calls).  After k of n steps `action` holds the current sample x_t in action units; after all n
 * it equals fe_engine_sample_diffusion's action with the same inputs, bit for bit.  Status 6
 * when no diffusion solve is active.  fe_engine_flow_action_metadata describes this solve too
 * (`solver` = scheduler, remaining_nfe = remaining steps). */
int fe_engine_diffusion_begin(fe_engine* engine, const float* condition, const float* noise,
                              size_t steps, int scheduler, uint64_t seed);

/* As fe_engine_diffusion_begin, but cancellable: `generation` is tracked as
 * fe_engine_flow_begin_request tracks it, and fe_engine_cancel_before with a higher generation
 * stops the solve before its next step (fe_engine_diffusion_advance then returns 8). */
int fe_engine_diffusion_begin_generation(fe_engine* engine, const float* condition,
                                         const float* noise, size_t steps, int scheduler,
                                         uint64_t seed, uint64_t generation);

int fe_engine_diffusion_advance(fe_engine* engine, size_t step_budget, float* action,
                                size_t* steps_remaining);

/* The model digest that fe_engine_model_metadata reports for engines created from these
 * weights (the reference's tensor fingerprint, protocol/model_identity.cc:124-148); needs no
 * GPU, so a host process can check request metadata against a checkpoint. */
int fe_weights_model_digest(const fe_weights* weights, fe_model_digest* digest);

/* Device-resident variants: the pointers are device memory (hipMalloc) of the same shapes;
 * nothing crosses PCIe.  `kind` 0 = DDIM/DDPM (`mode` = scheduler, `seed` used by DDPM),
 * 1 = flow ODE (`mode` = solver method).  Completes before returning. */
int fe_engine_sample_device(fe_engine* engine, int kind, const float* condition_dev,
                            const float* noise_dev, size_t batch, size_t steps, int mode,
                            uint64_t seed, float* action_dev);

/* Allocation-free batched denoise.  No counterpart in the reference: for callers that cannot
 * allocate device memory during the call -- code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation.  The same U-Net evaluation as fe_engine_diffusion_denoise_batch
 * on device pointers (condition [batch][condition_dim], normalized_sample and predicted_noise
 * [batch][horizon][action_dim]), with every intermediate buffer inside the library's static
 * device scratch array (32 MiB per GPU, held until the process ends): no hipMalloc, no graph
 * capture, no allocating library call.  A batch whose buffers exceed the scratch array returns
 * status 1 before anything is enqueued (pusht-size U-Net: about 1.5 MiB per sample).  `stream` is a
 * hipStream_t to enqueue on, returning at once (capturable); NULL uses the engine's stream and
 * returns when the result is written.  Every call on one GPU shares that GPU's scratch array,
 * so calls that overlap on one GPU (other streams, other engines) race; calls on one stream are
 * ordered.  The engine's own workspace and any resumable solve are not touched. */
int fe_engine_diffusion_denoise_noalloc(fe_engine* engine, const float* condition_dev,
                                        const float* normalized_sample_dev, size_t batch,
                                        float timestep, float* predicted_noise_dev, void* stream);

/* Build (capture and instantiate) the sampling graph for this shape ahead of the first call.
 * A sampling call of a (kind, batch, steps, mode) with no cached graph captures one itself
 * (HIP-runtime host and kernel-argument allocations, about a millisecond); the engine keeps the
 * 32 most recently used.  After a shape's first call or prepare, its calls allocate nothing and
 * capture nothing while it stays cached. */
int fe_engine_prepare(fe_engine* engine, int kind, size_t batch, size_t steps, int mode);

/* Sampling graphs this engine has captured and instantiated so far (sampling, prepare and
 * resumable-solve graphs). */
uint64_t fe_engine_graph_captures(const fe_engine* engine);

/* 1 when this engine runs batch-1 sampling ticks (up to 128 U-Net evaluations) as one persistent
 * kernel launch (one workgroup per compute unit, convolution steps handed over through
 * device-coherent memory), 0 when they run as a graph of per-layer launches (the default).  Both
 * compute the same values.  FLOWEDGE_PERSISTENT=1 in the environment at load selects the
 * persistent kernel.  If a persistent tick is ever abandoned (not every workgroup became
 * resident), the engine re-runs that call on the per-layer graphs and keeps using them. */
int fe_engine_persistent_tick(const fe_engine* engine);

/* Why fe_engine_persistent_tick is 0 ("" when it is 1). */
const char* fe_engine_persistent_tick_reason(const fe_engine* engine);

/* Largest batch the arena was sized for (FLOWEDGE_MAX_BATCH at load, default 256). */
size_t fe_engine_max_batch(const fe_engine* engine);

/* Bytes of the single device arena owned by the engine. */
size_t fe_engine_device_bytes(const fe_engine* engine);

/* Device allocations made by this library in this process (one arena per engine; a sampling
 * call never allocates). */
uint64_t fe_device_alloc_count(void);

/* Device time in milliseconds of the most recent sampling graph replay (hipEvents around the
 * graph launch on the engine's stream), or -1 if none. */
float fe_engine_last_device_ms(const fe_engine* engine);

/* Diagnostics (no counterpart in the reference; for benchmarks and profiling).  The fused
 * convolutions of one U-Net evaluation, in launch order, with their batch-1 arguments, listed
 * the first time they are asked for (nothing runs on the device to list them). */
int fe_engine_conv_count(fe_engine* engine, size_t* count);

/* Name ("site [oc<-ic Kk Llin prologue]") and algorithmic bytes of convolution `index`: weights
 * and biases (read once per launch) and activations plus per-channel parameters (per sample). */
int fe_engine_conv_info(fe_engine* engine, size_t index, char* name, size_t name_capacity,
                        uint64_t* weight_bytes, uint64_t* sample_bytes);

/* Kernels convolution `index` runs on in a sampling call of `batch` samples: 0 the fused
 * weight-streaming kernels, 1 the matrix-core implicit GEMMs, 2 the general-shape kernels (shapes
 * neither of the others has an instance for). */
int fe_engine_conv_path(fe_engine* engine, size_t index, size_t batch, int* path);

/* Partial sums convolution `index` leaves in a sampling call of `batch` samples (1: a single
 * tensor).  Below the matrix-core threshold these are input-channel slices: the convolution
 * splits its input channels over workgroups (whole GroupNorm groups per slice) and leaves one
 * partial sum per slice (FLOWEDGE_SLICES at load caps the count; 1 turns slicing off).  On the
 * matrix cores they are the partial sums of a split K loop (FLOWEDGE_MM_PARTS=0: reduced in
 * place).  Consumers add the partials while reading them. */
int fe_engine_conv_slices(fe_engine* engine, size_t index, size_t batch, int* slices);

/* Launches convolutions indices[0..n) round-robin `iters` times at `batch` on the engine's stream,
 * on the kernels a sampling call of that batch uses, and returns the mean device time of one
 * launch in microseconds (hipEvents around the loop, after one untimed round).  Outputs land in
 * the engine's own buffers. */
int fe_engine_time_convs(fe_engine* engine, const size_t* indices, size_t n, size_t batch,
                         size_t iters, float* avg_us);

/* ---- Observation encoder (extension; no counterpart in the reference's C ABI) ----
 * The Diffusion Policy RGB encoder the reference's LeRobot integration runs through torch
 * (integrations/lerobot/src/flowedge_lerobot/observation.py:152-216, LeRobot's
 * DiffusionRgbEncoder): center crop, resnet18 trunk with GroupNorm(C/16), spatial-softmax
 * keypoints, linear + ReLU.  It maps normalized camera images [n][C][H][W] (float32) to image
 * features [n][F] (F = 64 for 32 keypoints), the image part of the head's condition, which
 * stacks [state, image features, environment state] per observation step (observation.py:
 * 193-216). */
typedef struct FeEncoder fe_encoder;

/* Loads the encoder tensors named with LeRobot's state-dict names under `prefix`
 * ("diffusion.rgb_encoder." in a LeRobot model.safetensors) for images of image_height x
 * image_width, center-cropped to crop_height x crop_width (0 x 0: no crop), and up to max_images
 * images per call (1-64).  One device allocation at load.  Returns NULL with the error set when
 * a tensor is missing or its shape breaks the resnet18 structure. */
fe_encoder* fe_encoder_load(const char* path, const char* prefix, size_t image_height,
                            size_t image_width, size_t crop_height, size_t crop_width,
                            size_t max_images);
void fe_encoder_free(fe_encoder* encoder);
int fe_encoder_shape(const fe_encoder* encoder, size_t* channels, size_t* feature_dim,
                     size_t* keypoints);
/* Host buffers: features[n][F] of images[n][C][H][W]; rejects non-finite pixels. */
int fe_encoder_encode(fe_encoder* encoder, const float* images, size_t n, float* features);
/* Device buffers: image i's features go to features_dev + i * out_stride + out_offset (so they
 * can land inside a condition vector); returns once they are written. */
int fe_encoder_encode_device(fe_encoder* encoder, const float* images_dev, size_t n,
                             float* features_dev, size_t out_stride, size_t out_offset);
/* Device time of the last encode (hipEvents around the encoder graph), milliseconds. */
float fe_encoder_last_device_ms(const fe_encoder* encoder);
size_t fe_encoder_device_bytes(const fe_encoder* encoder);

#ifdef __cplusplus
}
#endif

#endif /* FLOWEDGE_AMD_H */
