// The batched runtimes' interface (st_batch): BatchBase, and Batch, the graph of phase kernels
// over B independent streams sharing one weight arena. A step is a fixed sequence of 5L + 2
// kernels captured once in a hipGraph: the input projection, then per layer QKV (RMSNorm
// prologue, RoPE and ring-write epilogue), attention, OUT (+residual), gate/up (RMSNorm
// prologue, SwiGLU epilogue), down (+residual, hidden), then the final norm and the scores.
// Batch's members are defined in batch.hip, a translation unit of their own; the resident
// batches (ResidentBatch, one launch of the fused step per step) are in batch_runtime.hpp.
#pragma once

#include "host_common.hpp"
#include "batch_kernels.hpp"

#include <cstddef>
#include <cstdint>

namespace stamd {

class BatchBase {
 public:
  virtual ~BatchBase() = default;
  virtual void step(const float* inputs, float* scores) = 0;
  virtual void reset(int stream) = 0;
  virtual void snapshot(int stream, uint64_t* position, float* keys, float* values, float* hidden) = 0;
  virtual double device_run(const float* inputs, size_t count, double* per_step) = 0;
  // Launch each step's kernels directly instead of replaying a captured graph (same results).
  virtual void set_eager(bool) {}
};

class Batch : public BatchBase {
 public:
  Batch(const st_config& config, bool mixed, const st_tensor* tensors, size_t count, int streams, int weight_dtype);
  ~Batch() override;
  void step(const float* inputs, float* scores) override;
  void reset(int stream) override;
  void snapshot(int stream, uint64_t* position, float* keys, float* values, float* hidden) override;
  double device_run(const float* inputs, size_t count, double* per_step) override;
  void set_eager(bool eager) override { eager_ = eager; }

 private:
  bool eager_ = false;  // launch the step's kernels directly (for kernel traces)
  void replay() {
    if (eager_) launch();
    else HIP_CHECK(hipGraphLaunch(graph_exec_, stream_));
  }
  template <int P> void launch_sequence();
  template <int P, int E, bool kNorm, int CT, int SW>
  void project(const void* X, int ld, uint32_t woff, int N, uint32_t norm, int layer, int max_tiles = kGroupTiles);
  int group_tiles(int cols, int max_tiles) const;
  void stage_events(const float* inputs, float* block) const;
  bool wide_qkv_ = false, wide_gateup_ = false;  // two column tiles per workgroup
  size_t block_words_ = 0;  // one (layer, stream) block [H][W][dh] of the K (or V) ring, in 4-byte words
  void launch() {
    if (prec_ == kFp32) launch_sequence<kFp32>();
    else if (prec_ == kMixed) launch_sequence<kMixed>();
    else launch_sequence<kBf16w>();
  }
  void sync() { HIP_CHECK(hipStreamSynchronize(stream_)); }

  st_config c_;
  int prec_ = kFp32, streams_ = 1, streams_p_ = 16, dim_ = 0;
  StreamHandle stream_;
  GraphHandle graph_;
  GraphExecHandle graph_exec_;
  DeviceBuffer weights_, keys_, values_, hidden_, position_, in_, x_, xn_, attn_, act_, q_, score_, rope_, args_dev_;
  PinnedBuffer host_in_, host_out_;
  StepArgs offsets_{};  // weight arena offsets (shared layout with the single-stream runtime)
  BatchArgs args_{};
  const BatchArgs* dargs_ = nullptr;
};

}  // namespace stamd
