/*
 * st_runtime.h - C ABI of the MI355X (gfx950) streaming-step backend, libstamd.so.
 *
 * This is the drop-in boundary for the reference's backend interface
 * Stream::Runtime (include/Runtime.hpp:7-46). Plain pointers and sizes only; no C++
 * types cross it. Every function returning int returns ST_OK (0) on success or a
 * nonzero ST_ERR_* code and records a message readable with st_last_error() on the
 * calling thread; this replaces the std::runtime_error the reference throws
 * (src/cuda/Runtime.cu:178-194,285-287,399-425). A C++ shim that rethrows
 * std::runtime_error(st_last_error()) restores the reference's exact interface.
 *
 * Threading: like the reference, a runtime is not thread-safe and has one outstanding
 * command at a time (docs/transport.md:14); the calling thread does any polling.
 */
#ifndef ST_RUNTIME_H
#define ST_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ST_OK = 0,
  ST_ERR_INVALID = 1,   /* bad config, tensor, option or argument */
  ST_ERR_DEVICE = 2,    /* HIP runtime failure or unsupported device */
  ST_ERR_STATE = 3,     /* stopped runtime, exhausted sequence, worker exit, timeout */
  ST_ERR_NUMERIC = 4    /* device-side watchdog (barrier timeout) tripped */
};

/* Stream::Backend (include/Runtime.hpp:7). CUDA = staged HIP kernels, GRAPH = one step
 * captured in a hipGraph (the fused kernel as a single node when blocks > 1 and the grid
 * passes the co-residency probe, otherwise the staged sequence; st_runtime_info's
 * "fused_launch" says which), FUSED = one launch of the fused kernel per step, PERSISTENT =
 * resident kernel driven through a host mailbox. CUBLAS / CUBLAS_GRAPH are the vendor GEMV
 * baselines (src/cuda/Runtime.cu:330-385): the projections run in rocBLAS (sgemv for FP32,
 * gemm_ex FP16 -> FP32 for mixed), eagerly or captured in a hipGraph; they take the
 * checkpoint's own weight storage (ST_WEIGHTS_BF16 is rejected). */
enum {
  ST_BACKEND_CUDA = 0,
  ST_BACKEND_GRAPH = 1,
  ST_BACKEND_CUBLAS = 2,
  ST_BACKEND_CUBLAS_GRAPH = 3,
  ST_BACKEND_FUSED = 4,
  ST_BACKEND_PERSISTENT = 5
};

/* Weight storage. AS_MODEL = the checkpoint's own mode (FP32, or FP16 for a "mixed"
 * checkpoint, src/cuda/Runtime.cu:231-246); BF16 = FP32 model whose weights are stored
 * as bfloat16 (round to nearest even) with FP32 activations, K/V and reductions. */
enum { ST_WEIGHTS_AS_MODEL = 0, ST_WEIGHTS_BF16 = 1 };

/* = Stream::ModelConfig (include/Model.hpp:12-18), validated like
 * ModelConfig::validate (src/runtime/Model.cpp:22-29). */
typedef struct {
  int32_t layers, width, heads, ffn, window, features;
  float epsilon;
} st_config;

/* = Stream::RuntimeOptions (include/Runtime.hpp:8-19) plus weight_dtype and initial_epoch.
 * blocks: workgroups of 512 threads; 0 selects one per compute unit.
 * mapped (src/cuda/Runtime.cu:43-48,278-280,435-450): CUDA, GRAPH, FUSED and the CUBLAS
 * backends read the event from, and write the score to, coherent host memory mapped into
 * the device (a staging kernel before and after the step; inside the captured graph for
 * GRAPH and CUBLAS_GRAPH) instead of pinned copies. The persistent worker always uses
 * mapped memory.
 * vector_matvec and fused_attention are accepted for source compatibility; this
 * backend always uses its wide-load matvec and its own windowed attention.
 * PERSISTENT only: backoff makes the worker and the host spin sleep between polls;
 * max_events > 0 ends the worker after that many RUN commands (RESET does not count);
 * initial_sequence is the mailbox's first sequence ID (the last ID is kept for STOP, so
 * values >= UINT64_MAX - 1 are rejected); idle_seconds ends a worker that receives no
 * command for that long. A call after the worker has ended fails with ST_ERR_STATE.
 * initial_epoch (extension, no counterpart in the reference): the first 32-bit epoch of the
 * device's tagged dataflow (0 selects 1). Epochs advance by 5*layers+3 per step; before they
 * would pass 0xF0000000 the runtime drains the device, zeroes the tagged vectors and restarts
 * at 1 (a persistent worker is stopped and relaunched for this). Only tests set it, to start
 * near that limit. */
typedef struct {
  int32_t backend;
  int32_t blocks;
  int32_t backoff;
  int32_t mapped;
  int32_t vector_matvec;
  int32_t fused_attention;
  uint64_t max_events;
  uint64_t initial_sequence;
  double idle_seconds;
  int32_t weight_dtype;
  uint32_t initial_epoch;
} st_options;

/* One named host tensor, FP32 values, row-major [out, in]. Names and shapes follow the
 * checkpoint manifest (reference/model.py:27-47; shape checks src/runtime/Model.cpp:120-139):
 * "input" [width, features], "final_norm" [width], "score" [1, width], and per layer
 * "layers.{l}.norm1|norm2" [width], ".q|k|v|out" [width, width], ".gate|up" [ffn, width],
 * ".down" [width, ffn]. For a mixed model the values must be FP16-representable. */
typedef struct {
  const char* name;
  int32_t rank;
  int32_t shape[2];
  const float* data;
} st_tensor;

typedef struct st_runtime st_runtime;

/* Fill *options with the reference defaults (RuntimeOptions{}: GRAPH, 1 block, ... 30 s). */
void st_options_default(st_options* options);

/* Runtime(const Model&, RuntimeOptions) - src/cuda/Runtime.cu:169-292.
 * mixed: 1 for a "mixed" checkpoint (FP16 weights, K/V and cast points). Tensors are
 * copied; the caller may free them on return. */
int st_runtime_create(const st_config* config, int32_t mixed, const st_tensor* tensors,
                      size_t tensor_count, const st_options* options, st_runtime** out);

/* ~Runtime() - stops and joins a persistent worker, frees device resources; never fails. */
void st_runtime_destroy(st_runtime* runtime);

/* float Runtime::step(const float* input) - src/cuda/Runtime.cu:430-455. Reads
 * `features` floats, writes the score. */
int st_runtime_step(st_runtime* runtime, const float* input, float* score);

/* void Runtime::reset() - src/cuda/Runtime.cu:457-464. */
int st_runtime_reset(st_runtime* runtime);

/* void Runtime::stop() - src/cuda/Runtime.cu:466-474. Idempotent. */
int st_runtime_stop(st_runtime* runtime);

/* Snapshot Runtime::snapshot() - src/cuda/Runtime.cu:548-568. keys/values receive
 * layers*width*window floats in [layer][head][slot][dim] order (FP16 cache decoded),
 * hidden receives layers*width floats. Any output pointer may be NULL. */
int st_runtime_snapshot(st_runtime* runtime, uint64_t* position, float* keys, float* values,
                        float* hidden);

/* double Runtime::deviceTrace(const float* inputs, size_t count) - src/cuda/Runtime.cu:596-630.
 * Resets state, runs `count` events from a preloaded device copy and writes the mean
 * microseconds per event. If per_event_us is not NULL it receives count per-event device
 * durations (microseconds). */
int st_runtime_device_trace(st_runtime* runtime, const float* inputs, size_t count,
                            double* us_per_event, double* per_event_us);

/* Extension with no counterpart in the reference: st_runtime_device_trace for callers that
 * cannot allocate device memory (serving loops and harnesses that forbid hipMalloc). It calls
 * no hipMalloc, hipFree or other allocating routine. It is not for use during stream or graph
 * capture: it synchronizes the runtime's stream and copies the stamps back with hipMemcpy.
 * FUSED backend only (ST_ERR_INVALID otherwise). device_events holds count*features floats in
 * device memory, row-major and unpadded, which the caller allocated and filled; the call resets
 * the state, runs the events in one launch and writes the mean and (if per_event_us is not
 * NULL) the per-event microseconds like st_runtime_device_trace. The per-step stamps go to a
 * fixed device array of the library with room for ST_NOALLOC_MAX_EVENTS + 1 stamps (8 MiB,
 * held by each GPU the library runs on until the process ends); a larger count is rejected
 * with ST_ERR_INVALID. Every call on one GPU shares that array; calls on one GPU take turns
 * (a per-device lock is held from the launch to the stamp readback), so calls from several
 * threads or runtimes on one GPU serialize instead of racing. */
#define ST_NOALLOC_MAX_EVENTS ((size_t)1 << 20)
int st_runtime_device_trace_noalloc(st_runtime* runtime, const float* device_events, size_t count,
                                    double* us_per_event, double* per_event_us);

/* Extension (no counterpart in the reference): per-launch device timing. Runs `count`
 * events from a preloaded device copy, one step per launch (FUSED: one fused-kernel launch
 * per event; CUDA/GRAPH: device-to-device staging copy plus the staged step), after a
 * reset if `reset` is nonzero, otherwise continuing the current stream state. A HIP event
 * is recorded on the runtime's stream after every step; per_event_us (may be NULL)
 * receives the count event-to-event durations, *us_per_event their mean. */
int st_runtime_device_run(st_runtime* runtime, const float* inputs, size_t count, int32_t reset,
                          double* us_per_event, double* per_event_us);

/* Extension (no counterpart in the reference): one FUSED step on `input` (advancing the
 * stream like st_runtime_step) with wall-clock stamps, for profiling. For each of the
 * 5*layers+2 phases and each of the `blocks` workgroups (phase-major) writes 8 times in
 * microseconds since workgroup 0 started the step: phase start, stream wave 1 done with the
 * phase, all stream waves done (staging of the next phase's inputs starts), staging done,
 * then three progress marks of stream wave 1 (matvec: work set up, first slab consumed, last
 * slab consumed; attention: inputs polled, partial stored, combine done), and the time stream
 * wave 1 finished issuing the next phase's prefetch; 0 where not recorded. The end of the step follows. Writes min(cap, 8*phases*blocks+1)
 * values and the full count; with cap 0 only the count is written and no step runs. */
int st_runtime_phase_times(st_runtime* runtime, const float* input, double* us, size_t cap,
                           size_t* count);

/* std::map<std::string, std::vector<float>> Runtime::traceStep(const float* input) -
 * src/cuda/Runtime.cu:476-546; staged backend (ST_BACKEND_CUDA) only, like the reference.
 * Runs one real step (advancing the stream exactly like st_runtime_step) and records the
 * named operation/cast boundaries of the reference's trace: "input.operand", ".pre_cast",
 * ".linear", "input", and per layer "layers.{l}.norm1.*", ".q|k|v.*", ".q", ".k", ".v",
 * ".attention", ".out.*", ".attention_residual", ".norm2.*", ".gate.*", ".up.*",
 * ".activation", ".down.*", ".hidden", then "final_norm.*" and "score.*". The phase outputs
 * (input, q, k, v, attention, attention_residual, activation, hidden, score.linear) are the
 * step's own values; the per-operation entries (.operand, .pre_cast, .norm, .linear) are
 * recomputed from the phase inputs by diagnostic kernels.
 * names receives a JSON object {"name": [offset, count], ...} (at most names_cap bytes,
 * NUL-terminated, full length in *names_needed); values receives the concatenated vectors
 * (values_cap must hold all; the total is written to *values_count). With names_cap and
 * values_cap both 0 only the sizes are written and no step runs. */
int st_runtime_trace_step(st_runtime* runtime, const float* input, char* names, size_t names_cap,
                          size_t* names_needed, float* values, size_t values_cap, size_t* values_count);

/* The scheduled-arrival mode of the reference's benchmark driver (bench/Main.cpp:282-342):
 * a producer thread offers event i (inputs + i*features) at time i*1e9/rate ns after the
 * schedule's start (bursty: in groups of 16 at the group's time) into a bounded queue of
 * queue_capacity, dropping it when the queue is full; the calling thread runs st_runtime_step
 * on each dequeued event in order. Every output holds `count` entries: the intended and
 * enqueue times, the submit and completion times (ns since the schedule's start; NaN for a
 * dropped event), the score (NaN when dropped) and the dropped flag. */
int st_runtime_scheduled_run(st_runtime* runtime, const float* inputs, size_t count, double rate_per_second,
                             size_t queue_capacity, int32_t bursty, double* intended_ns, double* enqueue_ns,
                             double* submit_ns, double* complete_ns, float* scores, uint8_t* dropped);

/* Json Runtime::info() const - src/cuda/Runtime.cu:570-594, as a JSON string. Writes at
 * most cap bytes (NUL-terminated) and the full length to *needed. */
int st_runtime_info_json(st_runtime* runtime, char* buffer, size_t cap, size_t* needed);

/* Json transportBench(mode, count, backoff, output) - include/Runtime.hpp:46,
 * src/cuda/Runtime.cu:703-814: `count` round trips of one transport mode, "ping-pong"
 * (host request, resident one-thread kernel answers through coherent pinned memory),
 * "gpu-ping" (the kernel initiates, the host answers), "empty" / "empty-graph" (an empty
 * kernel launched or replayed from a hipGraph, then synchronized) or "copy" (128 bytes in, an
 * echo kernel, 128 bytes out). Writes per-sample CSV rows to csv_path unless it is NULL or
 * empty, and the JSON report (p50/p99/worst microseconds, failures) like info_json. Checksum
 * failures return ST_ERR_NUMERIC. */
int st_transport_bench(const char* mode, uint64_t count, int32_t backoff, const char* csv_path, char* report,
                       size_t cap, size_t* needed);

/* Json probe() - src/cuda/Runtime.cu:134-161, as a JSON string. */
int st_probe_json(char* buffer, size_t cap, size_t* needed);

/* Extension (no counterpart in the reference, which is single-stream by design,
 * docs/Architecture.md:3): `streams` independent streams (1..256) sharing one set of
 * weights, each with its own K/V ring, hidden state and position. FP32 checkpoints with FP32
 * or bfloat16 weight storage (weight_dtype as in st_options), or mixed checkpoints (FP16
 * weights and K/V, the reference's cast points). A step advances every stream by one event;
 * the projections run as MFMA GEMMs over the streams. */
typedef struct st_batch st_batch;
int st_batch_create(const st_config* config, int32_t mixed, const st_tensor* tensors, size_t tensor_count,
                    int32_t streams, int32_t weight_dtype, st_batch** out);
/* Extension, the same batch as one resident launch per step: stream s runs the fused
 * single-stream step on its own share of the CUs (workgroups [s*per, (s+1)*per), per = the
 * CU count / streams, a multiple of 8 when at least 8), with its own state and the weights
 * shared. Each stream's scores and state are bit-identical to a single-stream runtime's (FUSED)
 * fed the same events. For small batches, which the phase-kernel graph above leaves
 * launch-bound. streams: 1..32. Every st_batch_* call below applies. */
int st_batch_create_resident(const st_config* config, int32_t mixed, const st_tensor* tensors, size_t tensor_count,
                             int32_t streams, int32_t weight_dtype, st_batch** out);
void st_batch_destroy(st_batch* batch);
/* inputs: streams*features floats (stream-major); scores: streams floats. */
int st_batch_step(st_batch* batch, const float* inputs, float* scores);
/* Zero stream `stream` (all streams when -1): K/V, hidden state and position. */
int st_batch_reset(st_batch* batch, int32_t stream);
/* State of one stream, in st_runtime_snapshot's layout; any output may be NULL. */
int st_batch_snapshot(st_batch* batch, int32_t stream, uint64_t* position, float* keys, float* values,
                      float* hidden);
/* `count` steps from a preloaded device copy of count*streams*features inputs, continuing
 * the current state; a HIP event after each step. Writes the mean microseconds per step and,
 * when per_step_us is not NULL, each step's event-to-event duration. */
int st_batch_device_run(st_batch* batch, const float* inputs, size_t count, double* us_per_step,
                        double* per_step_us);
/* Phase-kernel batches: 1 launches each step's kernels directly instead of replaying the
 * captured graph (so that a kernel trace sees plain launches; the results are the same), 0
 * restores the replay. Resident batches already launch one kernel per step: for them the call
 * changes nothing. No counterpart in the reference, which has no batched streams. */
int st_batch_set_eager(st_batch* batch, int32_t eager);

/* Message of the last failed call on this thread ("" if none). */
const char* st_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
