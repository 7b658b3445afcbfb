// Resident batches (included by runtime.hip, inside namespace stamd): B independent streams
// as one launch of the fused step per step. The graph of phase kernels (Batch) is declared in
// batch_api.hpp and defined in batch.hip.
#pragma once

// Streams a resident batch holds: each needs its own workgroups (8 of the 256 CUs at 32).
constexpr int kResidentMax = 32;

// B independent streams as one launch of the fused step per step (fused_streams_kernel):
// stream s runs on workgroups [s * per, (s + 1) * per) with its own state, held by a
// single-stream runtime (FUSED backend on `per` workgroups) per stream; the streams share
// stream 0's weight arena. Each stream's scores and state are bit-identical to a single-stream
// runtime's fed the same events. Every call returns with the device drained.
class ResidentBatch : public BatchBase {
 public:
  ResidentBatch(const st_config& config, bool mixed, const st_tensor* tensors, size_t count, int streams,
                int weight_dtype);
  ~ResidentBatch() override;
  void step(const float* inputs, float* scores) override;
  void reset(int stream) override;
  void snapshot(int stream, uint64_t* position, float* keys, float* values, float* hidden) override;
  double device_run(const float* inputs, size_t count, double* per_step) override;

 private:
  template <int P, int A> void launch_t(const float* events);
  void launch(const float* events) {
    lanes_[0]->dispatch([&](auto P, auto A) {
      launch_t<P.value, A.value>(events);
      return 0;
    });
  }
  st_config c_;
  int streams_ = 1, per_ = 1, fp_ = 0;
  hipStream_t stream_ = nullptr;  // stream 0's runtime stream: every launch and copy of the batch
  std::vector<std::unique_ptr<Runtime>> lanes_;
  DeviceBuffer stream_args_, in_, out_;  // stream_args_: every stream's StepArgs, contiguous
  PinnedBuffer host_in_, host_out_;
};

// Score and error word of every stream of a resident batch, gathered for one copy back.
__global__ void resident_scores_kernel(const StepArgs* args, int streams, unsigned* out) {
  const int s = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (s >= streams) return;
  const StepArgs& a = args[s];
  out[2 * s] = __builtin_bit_cast(unsigned, a.scratch[a.s_score]);
  out[2 * s + 1] = *a.error;
}

ResidentBatch::ResidentBatch(const st_config& config, bool mixed, const st_tensor* tensors, size_t count,
                             int streams, int weight_dtype)
    : c_(config), streams_(streams) {
  validate_config(c_);
  if (streams < 1 || streams > kResidentMax)
    throw Error(ST_ERR_INVALID, "Resident batches take 1 to " + std::to_string(kResidentMax) + " streams");
  int device = 0;
  HIP_CHECK(hipGetDevice(&device));
  hipDeviceProp_t prop;
  HIP_CHECK(hipGetDeviceProperties(&prop, device));
  // Workgroups per stream: an equal share of the CUs (one workgroup each), a multiple of 8
  // when at least 8, so that workgroup g of every stream runs on XCD g mod 8.
  per_ = std::min(prop.multiProcessorCount, kMaxGrid) / streams;
  if (per_ >= 8) per_ -= per_ % 8;
  if (per_ < 1) throw Error(ST_ERR_INVALID, "More streams than compute units");
  st_options o;
  st_options_default(&o);
  o.backend = ST_BACKEND_FUSED;
  o.blocks = per_;
  o.weight_dtype = weight_dtype;
  lanes_.reserve((size_t)streams);
  for (int s = 0; s < streams; s++)
    lanes_.push_back(std::make_unique<Runtime>(c_, mixed, tensors, count, o, s ? lanes_[0].get() : nullptr));
  Runtime& l0 = *lanes_[0];
  stream_ = l0.stream_;
  // The streams exchange data only within their own workgroups, but every workgroup of a
  // stream must be resident with the others of that stream: the whole launch is checked.
  if (streams * per_ > 1 && !l0.coresident(streams * per_))
    throw Error(ST_ERR_DEVICE, "The streams' workgroups are not resident at once");
  fp_ = l0.args_.features_p;
  // The streams' arguments side by side (each also stays in its runtime for reset and
  // snapshot; neither copy changes after construction).
  std::vector<StepArgs> all;
  for (auto& l : lanes_) all.push_back(l->args_);
  stream_args_.alloc(all.size() * sizeof(StepArgs));
  HIP_CHECK(hipMemcpy(stream_args_.ptr, all.data(), all.size() * sizeof(StepArgs), hipMemcpyHostToDevice));
  const size_t in_bytes = (size_t)streams * fp_ * 4;
  in_.alloc(in_bytes);
  HIP_CHECK(hipMemset(in_.ptr, 0, in_bytes));
  out_.alloc((size_t)streams * 8);
  host_in_.alloc(in_bytes);
  std::memset(host_in_.ptr, 0, in_bytes);
  host_out_.alloc((size_t)streams * 8);
}

ResidentBatch::~ResidentBatch() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  // Stream 0's runtime owns the shared weights: it goes last.
  while (!lanes_.empty()) lanes_.pop_back();
}

template <int P, int A>
void ResidentBatch::launch_t(const float* events) {
  hipLaunchKernelGGL((fused_streams_kernel<P, A>), dim3(streams_ * per_), dim3(kThreads), 0, stream_,
                     reinterpret_cast<const StepArgs*>(stream_args_.ptr), per_, events, fp_);
  HIP_CHECK(hipGetLastError());
}

void ResidentBatch::step(const float* inputs, float* scores) {
  if (!inputs || !scores) throw Error(ST_ERR_INVALID, "Null argument");
  for (auto& l : lanes_) l->reserve_epochs(1);
  float* h = reinterpret_cast<float*>(host_in_.ptr);
  for (int s = 0; s < streams_; s++)
    std::memcpy(h + (size_t)s * fp_, inputs + (size_t)s * c_.features, (size_t)c_.features * 4);
  HIP_CHECK(hipMemcpyAsync(in_.ptr, host_in_.ptr, (size_t)streams_ * fp_ * 4, hipMemcpyHostToDevice, stream_));
  launch(reinterpret_cast<const float*>(in_.ptr));
  hipLaunchKernelGGL(resident_scores_kernel, dim3(1), dim3(64), 0, stream_,
                     reinterpret_cast<const StepArgs*>(stream_args_.ptr), streams_, reinterpret_cast<unsigned*>(out_.ptr));
  HIP_CHECK(hipGetLastError());
  HIP_CHECK(hipMemcpyAsync(host_out_.ptr, out_.ptr, (size_t)streams_ * 8, hipMemcpyDeviceToHost, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
  const unsigned* o = reinterpret_cast<const unsigned*>(host_out_.ptr);
  for (int s = 0; s < streams_; s++)
    if (o[2 * s + 1])
      throw Error(ST_ERR_NUMERIC, "Device watchdog tripped on stream " + std::to_string(s) + " (error bits " +
                                      std::to_string(o[2 * s + 1]) + ")");
  for (int s = 0; s < streams_; s++) std::memcpy(scores + s, o + 2 * s, 4);
}

void ResidentBatch::reset(int stream) {
  if (stream < -1 || stream >= streams_) throw Error(ST_ERR_INVALID, "Stream index out of range");
  for (int s = 0; s < streams_; s++)
    if (stream == -1 || stream == s) lanes_[(size_t)s]->reset();
}

void ResidentBatch::snapshot(int stream, uint64_t* position, float* keys, float* values, float* hidden) {
  if (stream < 0 || stream >= streams_) throw Error(ST_ERR_INVALID, "Stream index out of range");
  lanes_[(size_t)stream]->snapshot(position, keys, values, hidden);
}

// `count` steps from a preloaded device copy of the inputs (count x streams x features,
// each row padded), continuing the current state: one launch per step, which reads its
// streams' events from the copy in place, with a HIP event after each.
double ResidentBatch::device_run(const float* inputs, size_t count, double* per_step) {
  if (!inputs || count == 0 || count > ((size_t)1 << 30) / ((size_t)streams_ * fp_))
    throw Error(ST_ERR_INVALID, "Invalid trace (empty, or more than 4 GiB of padded inputs)");
  for (auto& l : lanes_) l->reserve_epochs(count);
  std::vector<float> padded(count * (size_t)streams_ * fp_, 0.f);
  for (size_t i = 0; i < count; i++)
    for (int s = 0; s < streams_; s++)
      std::memcpy(&padded[(i * streams_ + s) * fp_], inputs + (i * streams_ + s) * c_.features,
                  (size_t)c_.features * 4);
  DeviceBuffer dev;
  dev.alloc(padded.size() * 4);
  HIP_CHECK(hipMemcpy(dev.ptr, padded.data(), padded.size() * 4, hipMemcpyHostToDevice));
  std::vector<hipEvent_t> ev(count + 1);
  for (auto& e : ev) create_timing_event(&e);
  HIP_CHECK(hipStreamSynchronize(stream_));
  HIP_CHECK(hipEventRecord(ev[0], stream_));
  for (size_t i = 0; i < count; i++) {
    launch(reinterpret_cast<const float*>(dev.ptr) + i * (size_t)streams_ * fp_);
    HIP_CHECK(hipEventRecord(ev[i + 1], stream_));
  }
  HIP_CHECK(hipStreamSynchronize(stream_));
  double total = 0;
  for (size_t i = 0; i < count; i++) {
    float ms = 0;
    HIP_CHECK(hipEventElapsedTime(&ms, ev[i], ev[i + 1]));
    if (per_step) per_step[i] = ms * 1000.0;
    total += ms * 1000.0;
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  for (auto& l : lanes_) l->check_device_error();
  return total / count;
}
