/* tg.h — C ABI of the MI355X (gfx950) execution backend for tensorgrad's compiled
 * training path.
 *
 * The boundary replaces the reference's worker seam: `WorkerProxy.request(...)`
 * (src/worker-proxy.ts:49-73) carrying the `Req` kinds of src/worker-protocol.ts:54-63,
 * served by the handlers in src/worker.ts:86-334 on top of src/runtime.ts. Everything
 * above it (ir.ts, trace.ts, grad.ts, dce.ts, adam.ts/sgd.ts and the public compile()
 * API) stays on the caller's side and hands over the traced IR as a JSON document:
 *
 *   { "graph":      { "ops": [OpNode...], "tensors": [{id, shape, dtype}...],
 *                     "outputs": [id], "captures": {name: id} },
 *     "paramGrads": { name: tensor id },                 // appendGrad result
 *     "writebacks": [{ "source": id, "destName": s, "destKind": "param"|"state" }],
 *     "optimizer":  null | { "kind": "adam"|"sgd", "config": WireAdamConfig|WireSGDConfig } }
 *
 * OpNode objects carry the field names of src/ir.ts:74-271 verbatim. All arguments are
 * plain pointers and sizes; host buffers are copied (the caller keeps ownership), which
 * stands in for the reference's transfer-and-detach of typed arrays.
 *
 * Every entry point returns a tg_status; on failure tg_last_error() returns a message
 * for the calling thread. TG_ABORTED corresponds to the reference's AbortError
 * (src/worker.ts:223-238, src/compile.ts:1201-1208).
 */
#ifndef TG_H
#define TG_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tg_runtime tg_runtime;

typedef enum {
  TG_OK = 0,
  TG_ABORTED = 1,          /* graph destroyed / replaced while in flight */
  TG_INVALID_ARGUMENT = 2, /* bad IR, unknown or missing names, wrong byte sizes */
  TG_DEVICE_ERROR = 3,     /* HIP error (no device, out of memory, launch failure) */
  TG_INTERNAL = 4
} tg_status;

/* Message for the last failed call on this thread ("" if none). */
const char* tg_last_error(void);

/* Number of visible HIP devices (0 without a GPU). */
int tg_device_count(void);

/* Build a runtime for a traced graph: plan device memory, lower ops to gfx950 kernels.
 * Replaces the `createRuntime` request (src/worker-protocol.ts:66-74,
 * src/worker.ts:86-122). Initial params are then loaded with tg_upload_params.
 * Each step is captured once into a hipGraph and replayed; with TG_GRAPH=0 in the
 * environment the same launches are issued directly instead (for profilers that do not
 * follow graph launches). */
tg_status tg_runtime_create(const char* ir_json, tg_runtime** out);

/* A forward-only graph sharing `parent`'s parameter buffers. Replaces `compileForward`
 * (src/worker-protocol.ts:78-82, src/worker.ts:137-170). */
tg_status tg_runtime_create_sibling(tg_runtime* parent, const char* ir_json, tg_runtime** out);

/* Destroy a runtime; destroying a parent also destroys its siblings
 * (`destroy`, src/worker.ts:321-334). In-flight calls on it return TG_ABORTED. */
void tg_destroy(tg_runtime* rt);

/* Parameter names in materialisation order (CompileResult.paramNames,
 * src/worker-protocol.ts:127-132) and their element counts. */
int tg_param_count(const tg_runtime* rt);
const char* tg_param_name(const tg_runtime* rt, int i);
int64_t tg_param_numel(const tg_runtime* rt, int i);

/* Strict upload: the n names must cover every parameter exactly once (missing and
 * unknown names both fail) — `uploadParams`, src/runtime.ts:403-429. */
tg_status tg_upload_params(tg_runtime* rt, int n, const char* const* names, const float* const* data,
                           const int64_t* numel);
/* Read every named parameter into caller buffers — `downloadParams`,
 * src/runtime.ts:431-449. */
tg_status tg_download_params(tg_runtime* rt, int n, const char* const* names, float* const* data,
                             const int64_t* numel);

/* One fused forward + backward + optimizer step (`step`, src/worker.ts:216-240): bumps
 * the optimizer step t and the PRNG counter, computes lrt / decayShrink / lr on the
 * host (src/worker.ts:187-214, src/adam.ts:134-143), uploads the user inputs (host
 * pointers, byte sizes must match), replays the captured step graph and returns the
 * scalar loss. */
tg_status tg_step(tg_runtime* rt, int n, const char* const* names, const void* const* data,
                  const int64_t* nbytes, float* loss);
/* Same, with the user inputs already resident in device memory (device pointers). */
tg_status tg_step_device(tg_runtime* rt, int n, const char* const* names, const void* const* dev_data,
                         const int64_t* nbytes, float* loss);

/* Scratch-only step. No counterpart in the reference: it is for callers that cannot
 * allocate device memory during a step (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments and results as
 * tg_step_device (device-resident user inputs); the step's launches are issued directly
 * (no graph instantiation) and every scratch buffer they use (split-K and reduction
 * partials, the embedding-gradient sort, launch-completion counters) lives in one static
 * device array of TG_SCRATCH_BYTES per GPU instead of memory the runtime allocates. The
 * call allocates nothing; graphs that need more scratch than TG_SCRATCH_BYTES are
 * rejected with TG_INVALID_ARGUMENT. All calls on one GPU share that array: calls from
 * one process are serialised; calls that overlap on one GPU from different processes
 * race. Bit-identical to tg_step_device. */
#define TG_SCRATCH_BYTES (16ll << 20)
tg_status tg_step_noalloc(tg_runtime* rt, int n, const char* const* names, const void* const* dev_data,
                          const int64_t* nbytes, float* loss);

/* Device-resident batches (no reference counterpart): copy one batch of user inputs
 * (host pointers) into device slot `slot`, then run steps from a slot without any host
 * to device copy of user data. Used by callers that prefetch, and by the benchmark. */
tg_status tg_stage_batch(tg_runtime* rt, int slot, int n, const char* const* names, const void* const* data,
                         const int64_t* nbytes);
tg_status tg_step_staged(tg_runtime* rt, int slot, float* loss);

/* Forward-only dispatch; copies the graph output into `out` (`run`,
 * src/worker.ts:242-260). */
tg_status tg_run(tg_runtime* rt, int n, const char* const* names, const void* const* data,
                 const int64_t* nbytes, void* out, int64_t out_bytes);

/* Activation captures of the last step/run (src/runtime.ts:26-75). */
int tg_capture_count(const tg_runtime* rt);
const char* tg_capture_name(const tg_runtime* rt, int i);
tg_status tg_get_capture(tg_runtime* rt, const char* name, void* out, int64_t nbytes);

/* Zero optimizer state and its step counter (`resetOptimizer`, src/worker.ts:295-302). */
tg_status tg_reset_optimizer(tg_runtime* rt);

/* Replace the learning-rate schedule (JSON number or schedule object), rebased so its
 * step 1 is the next step (`setLR`, src/worker.ts:304-319, src/lr.ts:108-112). */
tg_status tg_set_lr(tg_runtime* rt, const char* lr_json);

/* ---- optimizer state and checkpoints ---------------------------------------------
 * The reference keeps optimizer state on the GPU only and has no resume
 * (src/worker.ts:295-302 can only zero it); these entry points add export / import
 * and a checkpoint file. State tensors are the graph's state_input tensors
 * (appendAdam's adam_m_<param> / adam_v_<param>, appendSGD's velocity), listed in
 * name order. */
int tg_state_count(tg_runtime* rt);
const char* tg_state_name(tg_runtime* rt, int i);
int64_t tg_state_numel(tg_runtime* rt, int i);
/* Read the named state tensors, the optimizer step t and the PRNG seed counter. */
tg_status tg_download_state(tg_runtime* rt, int n, const char* const* names, float* const* data, const int64_t* numel,
                            int64_t* step_t, int64_t* prng_counter);
/* Strict (every state tensor exactly once, like tg_upload_params); also sets t and the
 * seed counter, so the next step runs at t + 1 with seed counter + 1. */
tg_status tg_upload_state(tg_runtime* rt, int n, const char* const* names, const float* const* data,
                          const int64_t* numel, int64_t step_t, int64_t prng_counter);
/* Write every parameter and state tensor to a safetensors file (F32; __metadata__ holds
 * the optimizer kind, t, the seed counter and the LR schedule). */
tg_status tg_save_checkpoint(tg_runtime* rt, const char* path);
/* Load a safetensors file written by tg_save_checkpoint, or any file holding exactly the
 * graph's parameters (e.g. converted pretrained weights; the optimizer state, t and the
 * seed counter are then left alone). Every parameter must be present with its shape;
 * state is all or nothing; unknown tensors (integer and bool ones included) and
 * malformed counters are errors (TG_INVALID_ARGUMENT). Nothing is written unless the
 * whole file checks out. */
tg_status tg_load_checkpoint(tg_runtime* rt, const char* path);
/* The checks of tg_load_checkpoint for the graph `ir_json` without a device (nothing is
 * allocated or loaded): writes JSON {"params", "state", "restoresCounters", "step",
 * "prngCounter"} or fails with the message a load would give. A params-only file leaves
 * the optimizer state, t and the seed counter alone. No counterpart in the reference. */
tg_status tg_check_checkpoint(const char* ir_json, const char* path, char* out_json, int64_t out_len);
/* Index a safetensors container held in memory without a device: JSON
 * {"dataStart", "tensors": [{name, dtype, shape, begin, end}], "skipped": [...],
 *  "metadata": {...}} with the checks and messages of `loadSafetensors`
 * (src/safetensors.ts:49-103): F32 tensors listed, integer / bool tensors skipped, other
 * dtypes, truncated buffers and offset / shape mismatches rejected. */
tg_status tg_safetensors_index(const void* buf, int64_t len, char* out_json, int64_t out_len);

/* ---- measurement (no reference counterpart) ---------------------------------------
 * Kernel-level schedule of the lowered step, as JSON: one entry per launch node with
 * its kind, shape summary, algorithmic FLOP and byte counts. */
tg_status tg_describe(tg_runtime* rt, char* buf, int64_t buflen);
/* Lower an IR document without touching the device (no allocation, no launches) and
 * write the same JSON schedule as tg_describe. Usable on a machine without a GPU. */
tg_status tg_plan(const char* ir_json, char* buf, int64_t buflen);
/* Replay the step `iters` times eagerly with HIP events around every launch node on
 * the runtime's stream; writes the mean duration (ms) of each node into ms_out
 * (length = node count from tg_describe). Inputs must have been set by a prior step. */
tg_status tg_profile_nodes(tg_runtime* rt, int iters, double* ms_out, int64_t n_out);
/* Run the step `iters` times eagerly, every kernel dispatched with start / end events of
 * its own (hipExtLaunchKernel), and write each launch node's mean kernel time (ms: the
 * durations of the kernels it launches, summed, without gaps between launches) into
 * ms_out (length = node count). Measurement only; no counterpart in the reference. */
tg_status tg_profile_kernels(tg_runtime* rt, int iters, double* ms_out, int64_t n_out);
/* Time `steps` graph replays (device-resident inputs from the previous step) between two
 * HIP events; returns total milliseconds. */
tg_status tg_time_replays(tg_runtime* rt, int steps, double* total_ms);
/* Time `iters` back-to-back passes over only the launch nodes whose kind (as reported by
 * tg_describe) is listed in `kinds` (comma separated; a leading '-' selects all other
 * nodes); returns milliseconds per pass and the number of launches in a pass. Used for
 * per-kernel-family roofline figures. No counterpart in the reference. */
tg_status tg_time_kinds(tg_runtime* rt, const char* kinds, int iters, double* ms_per_pass, int* launches);

#ifdef __cplusplus
}
#endif

#endif /* TG_H */
