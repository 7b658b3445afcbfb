// Host side of the batched runtime (included by runtime.hip, inside namespace stamd): B
// independent streams over one weight arena. A step is a fixed kernel sequence captured once
// in a hipGraph: input projection, then per layer norm, QKV (+RoPE, ring write), attention,
// OUT (+residual), norm, gate/up (+SwiGLU), down (+residual, hidden), then the final norm and
// the scores. Each projection is a split-K MFMA GEMM followed by its reduce/epilogue kernel.
#pragma once

class Batch {
 public:
  Batch(const st_config& config, const st_tensor* tensors, size_t count, int streams, int weight_dtype);
  ~Batch();
  void step(const float* inputs, float* scores);
  void reset(int stream);
  void snapshot(int stream, uint64_t* position, float* keys, float* values, float* hidden);
  double device_run(const float* inputs, size_t count, double* per_step);

 private:
  template <int P> void launch_sequence();
  void launch() {
    if (prec_ == kFp32) launch_sequence<kFp32>();
    else launch_sequence<kBf16w>();
  }
  // K-slices of a projection with K columns: enough workgroups to spread the weight stream
  // (about 512 over N / 16 column tiles), each slice a multiple of 16 columns.
  void slices(int N, int K, int& ks, int& kc) const {
    const int tiles = N / kBatchTile;
    int want = (512 + tiles - 1) / tiles;
    const int blocks16 = K / 16;
    if (want > blocks16) want = blocks16;
    if (want < 1) want = 1;
    kc = (blocks16 + want - 1) / want * 16;
    ks = (K + kc - 1) / kc;
  }
  void sync() { HIP_CHECK(hipStreamSynchronize(stream_)); }

  st_config c_;
  int prec_ = kFp32, streams_ = 1, streams_p_ = 16, dim_ = 0;
  hipStream_t stream_ = nullptr;
  hipGraph_t graph_ = nullptr;
  hipGraphExec_t graph_exec_ = nullptr;
  DeviceBuffer weights_, keys_, values_, hidden_, position_, in_, x_, xn_, attn_, act_, q_, part_, score_, rope_,
      args_dev_;
  PinnedBuffer host_in_, host_out_;
  StepArgs offsets_{};  // weight arena offsets (shared layout with the single-stream runtime)
  BatchArgs args_{};
  const BatchArgs* dargs_ = nullptr;
};

Batch::Batch(const st_config& config, const st_tensor* tensors, size_t count, int streams, int weight_dtype)
    : c_(config) {
  validate_config(c_);
  if (streams < 1 || streams > kBatchMax)
    throw Error(ST_ERR_INVALID, "Streams must be between 1 and " + std::to_string(kBatchMax));
  if (weight_dtype != ST_WEIGHTS_AS_MODEL && weight_dtype != ST_WEIGHTS_BF16)
    throw Error(ST_ERR_INVALID, "Unknown weight storage");
  if (c_.width % kBatchTile || (2 * c_.ffn) % kBatchTile)
    throw Error(ST_ERR_INVALID, "Batched streams need width and 2*ffn to be multiples of 16");
  prec_ = weight_dtype == ST_WEIGHTS_BF16 ? kBf16w : kFp32;
  streams_ = streams;
  streams_p_ = (streams + kBatchTile - 1) / kBatchTile * kBatchTile;
  dim_ = c_.width / c_.heads;
  int device = 0;
  HIP_CHECK(hipGetDevice(&device));
  hipDeviceProp_t prop;
  HIP_CHECK(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    throw Error(ST_ERR_DEVICE, std::string("Supported target is gfx950; found ") + prop.gcnArchName);
  HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));

  // Weight arena: the single-stream layout (rows padded to 1 KiB slabs).
  const int slab = 1024 / (prec_ == kFp32 ? 4 : 2);
  offsets_.width_p = round_up(c_.width, slab);
  offsets_.ffn_p = round_up(c_.ffn, slab);
  offsets_.features_p = round_up(c_.features, slab);
  build_arena(c_, prec_, tensors, count, offsets_, weights_);

  BatchArgs& a = args_;
  a.streams = streams_;
  a.streams_p = streams_p_;
  a.layers = c_.layers;
  a.width = c_.width;
  a.heads = c_.heads;
  a.dim = dim_;
  a.ffn = c_.ffn;
  a.window = c_.window;
  a.features = c_.features;
  a.width_p = offsets_.width_p;
  a.ffn_p = offsets_.ffn_p;
  a.features_p = offsets_.features_p;
  a.xcols = std::max({a.width_p, a.ffn_p, a.features_p});
  a.epsilon = c_.epsilon;
  a.weights = offsets_.weights;
  a.w_input = offsets_.w_input;
  a.w_final_norm = offsets_.w_final_norm;
  a.w_score = offsets_.w_score;
  for (int l = 0; l < c_.layers; l++) a.layer[l] = offsets_.layer[l];

  std::vector<float> freq(dim_ / 2);
  for (int j = 0; j < dim_ / 2; j++) freq[j] = std::pow(10000.0f, -(float)(2 * j) / (float)dim_);
  rope_.alloc(freq.size() * 4);
  HIP_CHECK(hipMemcpy(rope_.ptr, freq.data(), freq.size() * 4, hipMemcpyHostToDevice));
  a.rope_freq = reinterpret_cast<const float*>(rope_.ptr);

  const size_t ring = (size_t)streams_ * c_.layers * c_.width * c_.window;
  auto zeroed = [&](DeviceBuffer& buf, size_t floats) {
    buf.alloc(floats * 4);
    HIP_CHECK(hipMemset(buf.ptr, 0, std::max<size_t>(floats * 4, 256)));
    return reinterpret_cast<float*>(buf.ptr);
  };
  a.keys = zeroed(keys_, ring);
  a.values = zeroed(values_, ring);
  a.hidden = zeroed(hidden_, (size_t)streams_ * c_.layers * c_.width);
  position_.alloc((size_t)streams_ * 8);
  HIP_CHECK(hipMemset(position_.ptr, 0, (size_t)streams_ * 8));
  a.position = reinterpret_cast<unsigned long long*>(position_.ptr);
  a.in = zeroed(in_, (size_t)streams_p_ * a.features_p);
  a.x = zeroed(x_, (size_t)streams_p_ * a.width_p);
  a.xn = zeroed(xn_, (size_t)streams_p_ * a.xcols);
  a.attn = zeroed(attn_, (size_t)streams_p_ * a.width_p);
  a.act = zeroed(act_, (size_t)streams_p_ * a.ffn_p);
  a.q = zeroed(q_, (size_t)streams_p_ * a.width);
  a.score = zeroed(score_, (size_t)streams_);
  // Split-K partials: the largest slices x Bp x N over the projections.
  size_t part = 0;
  const int shapes[5][2] = {{c_.width, a.features_p}, {3 * c_.width, a.width_p}, {c_.width, a.width_p},
                            {2 * c_.ffn, a.width_p}, {c_.width, a.ffn_p}};
  for (auto& sh : shapes) {
    int ks, kc;
    slices(sh[0], sh[1], ks, kc);
    part = std::max(part, (size_t)ks * streams_p_ * sh[0]);
  }
  a.part = zeroed(part_, part);
  host_in_.alloc((size_t)streams_p_ * a.features_p * 4);
  std::memset(host_in_.ptr, 0, (size_t)streams_p_ * a.features_p * 4);
  host_out_.alloc((size_t)streams_ * 4);

  args_dev_.alloc(sizeof(BatchArgs));
  HIP_CHECK(hipMemcpy(args_dev_.ptr, &args_, sizeof(BatchArgs), hipMemcpyHostToDevice));
  dargs_ = reinterpret_cast<const BatchArgs*>(args_dev_.ptr);

  // Warm up outside capture, restore the initial state, then capture the step sequence.
  launch();
  sync();
  reset(-1);
  HIP_CHECK(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
  launch();
  HIP_CHECK(hipStreamEndCapture(stream_, &graph_));
  HIP_CHECK(hipGraphInstantiate(&graph_exec_, graph_, nullptr, nullptr, 0));
}

Batch::~Batch() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
  if (graph_) (void)hipGraphDestroy(graph_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

template <int P>
void Batch::launch_sequence() {
  const BatchArgs& a = args_;
  auto gemm = [&](const float* X, int ldx, uint32_t woff, int ldw, int N, int K) {
    int ks, kc;
    slices(N, K, ks, kc);
    hipLaunchKernelGGL(batch_gemm<P>, dim3(N / kBatchTile, ks), dim3(64), 0, stream_, dargs_, X, ldx, woff, ldw, N, K,
                       kc, a.part);
    return ks;
  };
  auto reduce = [&](auto kernel, int layer, int N, int ks, int unit) {
    const int threads = streams_ * (N / unit);
    hipLaunchKernelGGL(kernel, dim3((threads + 255) / 256), dim3(256), 0, stream_, dargs_, layer, N, ks);
  };
  const int d = c_.width, F = c_.ffn;
  int ks = gemm(a.in, a.features_p, a.w_input, a.features_p, d, a.features_p);
  reduce(batch_reduce<kEpInput>, 0, d, ks, 1);
  for (int l = 0; l < c_.layers; l++) {
    const LayerWeights& w = a.layer[l];
    hipLaunchKernelGGL(batch_norm<P>, dim3(streams_p_), dim3(256), 0, stream_, dargs_, w.norm1);
    ks = gemm(a.xn, a.xcols, w.qkv, a.width_p, 3 * d, a.width_p);
    reduce(batch_reduce<kEpQkv>, l, 3 * d, ks, 2);
    hipLaunchKernelGGL(batch_attention, dim3(streams_ * c_.heads), dim3(64), (size_t)c_.window * 4, stream_, dargs_,
                       l);
    ks = gemm(a.attn, a.width_p, w.out, a.width_p, d, a.width_p);
    reduce(batch_reduce<kEpOut>, l, d, ks, 1);
    hipLaunchKernelGGL(batch_norm<P>, dim3(streams_p_), dim3(256), 0, stream_, dargs_, w.norm2);
    ks = gemm(a.xn, a.xcols, w.gateup, a.width_p, 2 * F, a.width_p);
    reduce(batch_reduce<kEpGateUp>, l, 2 * F, ks, 2);
    ks = gemm(a.act, a.ffn_p, w.down, a.ffn_p, d, a.ffn_p);
    reduce(batch_reduce<kEpDown>, l, d, ks, 1);
  }
  hipLaunchKernelGGL(batch_final<P>, dim3(streams_), dim3(64), 0, stream_, dargs_);
  HIP_CHECK(hipGetLastError());
}

void Batch::step(const float* inputs, float* scores) {
  if (!inputs || !scores) throw Error(ST_ERR_INVALID, "Null argument");
  const int fp = args_.features_p;
  float* h = reinterpret_cast<float*>(host_in_.ptr);
  for (int b = 0; b < streams_; b++) std::memcpy(h + (size_t)b * fp, inputs + (size_t)b * c_.features, (size_t)c_.features * 4);
  HIP_CHECK(hipMemcpyAsync(args_.in, host_in_.ptr, (size_t)streams_p_ * fp * 4, hipMemcpyHostToDevice, stream_));
  HIP_CHECK(hipGraphLaunch(graph_exec_, stream_));
  HIP_CHECK(hipMemcpyAsync(host_out_.ptr, args_.score, (size_t)streams_ * 4, hipMemcpyDeviceToHost, stream_));
  sync();
  std::memcpy(scores, host_out_.ptr, (size_t)streams_ * 4);
}

void Batch::reset(int stream) {
  if (stream < -1 || stream >= streams_) throw Error(ST_ERR_INVALID, "Stream index out of range");
  hipLaunchKernelGGL(batch_reset, dim3(256), dim3(256), 0, stream_, dargs_, stream);
  HIP_CHECK(hipGetLastError());
  sync();
}

void Batch::snapshot(int stream, uint64_t* position, float* keys, float* values, float* hidden) {
  if (stream < 0 || stream >= streams_) throw Error(ST_ERR_INVALID, "Stream index out of range");
  sync();
  const size_t ring = (size_t)c_.layers * c_.width * c_.window;
  if (position)
    HIP_CHECK(hipMemcpy(position, args_.position + stream, 8, hipMemcpyDeviceToHost));
  if (keys) HIP_CHECK(hipMemcpy(keys, args_.keys + (size_t)stream * ring, ring * 4, hipMemcpyDeviceToHost));
  if (values) HIP_CHECK(hipMemcpy(values, args_.values + (size_t)stream * ring, ring * 4, hipMemcpyDeviceToHost));
  if (hidden)
    HIP_CHECK(hipMemcpy(hidden, args_.hidden + (size_t)stream * c_.layers * c_.width, (size_t)c_.layers * c_.width * 4,
                        hipMemcpyDeviceToHost));
}

// `count` batched steps from a preloaded device copy of the inputs (count x streams x
// features), continuing the current state; one graph replay per step after a device-to-device
// copy of that step's inputs, with a HIP event after each. Returns the mean microseconds per
// step and, when per_step is not NULL, each step's event-to-event duration.
double Batch::device_run(const float* inputs, size_t count, double* per_step) {
  if (!inputs || count == 0 || count > (1u << 20)) throw Error(ST_ERR_INVALID, "Invalid trace");
  const int fp = args_.features_p;
  std::vector<float> padded(count * (size_t)streams_p_ * fp, 0.f);
  for (size_t i = 0; i < count; i++)
    for (int b = 0; b < streams_; b++)
      std::memcpy(&padded[(i * streams_p_ + b) * fp], inputs + (i * streams_ + b) * c_.features,
                  (size_t)c_.features * 4);
  DeviceBuffer dev;
  dev.alloc(padded.size() * 4);
  HIP_CHECK(hipMemcpy(dev.ptr, padded.data(), padded.size() * 4, hipMemcpyHostToDevice));
  std::vector<hipEvent_t> ev(count + 1);
  for (auto& e : ev) HIP_CHECK(hipEventCreate(&e));
  sync();
  HIP_CHECK(hipEventRecord(ev[0], stream_));
  for (size_t i = 0; i < count; i++) {
    HIP_CHECK(hipMemcpyAsync(args_.in, reinterpret_cast<float*>(dev.ptr) + i * (size_t)streams_p_ * fp,
                             (size_t)streams_p_ * fp * 4, hipMemcpyDeviceToDevice, stream_));
    HIP_CHECK(hipGraphLaunch(graph_exec_, stream_));
    HIP_CHECK(hipEventRecord(ev[i + 1], stream_));
  }
  sync();
  double total = 0;
  for (size_t i = 0; i < count; i++) {
    float ms = 0;
    HIP_CHECK(hipEventElapsedTime(&ms, ev[i], ev[i + 1]));
    if (per_step) per_step[i] = ms * 1000.0;
    total += ms * 1000.0;
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  return total / count;
}
