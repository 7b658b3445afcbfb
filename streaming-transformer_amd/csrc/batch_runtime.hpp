// Host side of the batched runtime (included by runtime.hip, inside namespace stamd): B
// independent streams over one weight arena. A step is a fixed sequence of 5L + 2 kernels
// captured once in a hipGraph: the input projection, then per layer QKV (RMSNorm prologue,
// RoPE and ring-write epilogue), attention, OUT (+residual), gate/up (RMSNorm prologue,
// SwiGLU epilogue), down (+residual, hidden), then the final norm and the scores.
#pragma once

// The batched runtimes behind st_batch: the graph of phase kernels below (Batch) and the
// resident launch of the fused step per stream (ResidentBatch).
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
  hipStream_t stream_ = nullptr;
  hipGraph_t graph_ = nullptr;
  hipGraphExec_t graph_exec_ = nullptr;
  DeviceBuffer weights_, keys_, values_, hidden_, position_, in_, x_, xn_, attn_, act_, q_, score_, rope_, args_dev_;
  PinnedBuffer host_in_, host_out_;
  StepArgs offsets_{};  // weight arena offsets (shared layout with the single-stream runtime)
  BatchArgs args_{};
  const BatchArgs* dargs_ = nullptr;
};

Batch::Batch(const st_config& config, bool mixed, const st_tensor* tensors, size_t count, int streams,
             int weight_dtype)
    : c_(config) {
  validate_config(c_);
  if (streams < 1 || streams > kBatchMax)
    throw Error(ST_ERR_INVALID, "Streams must be between 1 and " + std::to_string(kBatchMax));
  if (weight_dtype != ST_WEIGHTS_AS_MODEL && weight_dtype != ST_WEIGHTS_BF16)
    throw Error(ST_ERR_INVALID, "Unknown weight storage");
  if (c_.width % kBatchTile || (2 * c_.ffn) % kBatchTile)
    throw Error(ST_ERR_INVALID, "Batched streams need width and 2*ffn to be multiples of 16");
  if (mixed && weight_dtype == ST_WEIGHTS_BF16)
    throw Error(ST_ERR_INVALID, "bfloat16 weight storage applies to FP32 checkpoints only");
  prec_ = mixed ? kMixed : weight_dtype == ST_WEIGHTS_BF16 ? kBf16w : kFp32;
  streams_ = streams;
  // Padded batch: 16 or 32 rows, else a multiple of 64, so that every projection's batch
  // groups (1, 2 or 4 tiles of 16) divide it.
  streams_p_ = streams <= 16 ? 16 : streams <= 32 ? 32 : (streams + 63) / 64 * 64;
  dim_ = c_.width / c_.heads;
  wide_qkv_ = (3 * c_.width / kBatchTile) % 2 == 0;
  wide_gateup_ = (2 * c_.ffn / kBatchTile) % 2 == 0;
  if (dim_ % 4) throw Error(ST_ERR_INVALID, "Batched streams need a head dimension that is a multiple of 4");
  int device = 0;
  HIP_CHECK(hipGetDevice(&device));
  hipDeviceProp_t prop;
  HIP_CHECK(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    throw Error(ST_ERR_DEVICE, std::string("Supported target is gfx950; found ") + prop.gcnArchName);
  HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));

  // Weight arena: the single-stream runtime's (rows padded to 1 KiB slabs), with the
  // projection matrices in MFMA operand order (tiled).
  const int slab = 1024 / (prec_ == kFp32 ? 4 : 2);
  offsets_.width_p = round_up(c_.width, slab);
  offsets_.ffn_p = round_up(c_.ffn, slab);
  offsets_.features_p = round_up(c_.features, slab);
  build_arena(c_, prec_, tensors, count, offsets_, weights_, true);

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

  auto zeroed = [&](DeviceBuffer& buf, size_t floats) {
    buf.alloc(floats * 4);
    HIP_CHECK(hipMemset(buf.ptr, 0, std::max<size_t>(floats * 4, 256)));
    return reinterpret_cast<float*>(buf.ptr);
  };
  // K/V rings [L][B][H][W][dh]: FP32, or FP16 in mixed mode.
  block_words_ = (size_t)c_.width * c_.window * (prec_ == kMixed ? 2 : 4) / 4;
  a.keys = zeroed(keys_, (size_t)c_.layers * streams_ * block_words_);
  a.values = zeroed(values_, (size_t)c_.layers * streams_ * block_words_);
  a.hidden = zeroed(hidden_, (size_t)streams_ * c_.layers * c_.width);
  position_.alloc((size_t)streams_ * 8);
  HIP_CHECK(hipMemset(position_.ptr, 0, (size_t)streams_ * 8));
  a.position = reinterpret_cast<unsigned long long*>(position_.ptr);
  a.in = zeroed(in_, (size_t)streams_p_ * a.features_p);
  a.x = zeroed(x_, (size_t)streams_p_ * a.width_p);
  a.xn = zeroed(xn_, (size_t)streams_p_ * a.width_p);
  a.attn = zeroed(attn_, (size_t)streams_p_ * a.width_p);
  a.act = zeroed(act_, (size_t)streams_p_ * a.ffn_p);
  a.q = zeroed(q_, (size_t)streams_p_ * a.width);
  a.score = zeroed(score_, (size_t)streams_);
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

// Batch tiles per projection workgroup: the largest of 4, 2, 1 that still gives at least 256
// workgroups (one per CU), so that narrow projections at small batches spread over the chip.
// `cols` is the number of column groups (N / (16 CT)); at most `max_tiles` batch tiles.
int Batch::group_tiles(int cols, int max_tiles) const {
  const int tiles = streams_p_ / kBatchTile;
  for (int nt = std::min(kGroupTiles, max_tiles); nt > 1; nt >>= 1)
    if (tiles % nt == 0 && cols * (tiles / nt) >= 256) return nt;
  return 1;
}

template <int P, int E, bool kNorm, int CT, int SW>
void Batch::project(const void* X, int ld, uint32_t woff, int N, uint32_t norm, int layer, int max_tiles) {
  const int cols = N / (kBatchTile * CT);
  const int nt = group_tiles(cols, max_tiles);
  const dim3 grid(cols, streams_p_ / kBatchTile / nt), block(64 * kSlices / SW);
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, block, 0, stream_, dargs_, X, woff, N, ld, norm, layer); };
  if (nt == 4) go(batch_proj<P, E, kNorm, 4, CT, SW>);
  else if (nt == 2) go(batch_proj<P, E, kNorm, 2, CT, SW>);
  else go(batch_proj<P, E, kNorm, 1, CT, SW>);
}

// Workgroup shapes per projection. Every shape computes the same fixed slice tree, so the
// choice changes speed only, never a stream's bits. Small batches want many workgroups (one
// column tile and one K-slice per wave); large ones want each X fragment reused across column
// tiles: from 64 streams the wide projections (QKV, gate/up) take two column tiles and two
// K-slices per wave, and from 128 streams the narrow ones (OUT, down) take two column tiles.
// From 256 streams (16-bit operands), gate/up takes four column tiles and one K-slice per
// wave (eight waves), and QKV one batch tile per workgroup: measured on Main at 256 streams,
// gate/up 15.2 -> 12.5 us and QKV 11.6 -> 10.0 us per layer with bfloat16 weights
// (9.3 -> 8.0 and 8.5 -> 7.5 us in mixed mode), from fewer re-reads of X across column tiles
// and more workgroups respectively.
template <int P>
void Batch::launch_sequence() {
  const BatchArgs& a = args_;
  const int d = c_.width, F = c_.ffn;
  const bool wide = streams_p_ >= 64, narrow = streams_p_ >= 128 && (c_.width / kBatchTile) % 2 == 0;
  const bool huge = P != kFp32 && streams_p_ >= 256;
  // The attention loops' form (batch_attention): chunked loads for FP32 K/V with dh <= 64; for
  // FP16 K/V only from 256 streams.
  const int attn_loads = dim_ > 64 ? kAttnPerPass
                         : P == kMixed ? (streams_p_ >= 256 ? kAttnChunk4 : kAttnPerPass)
                         : streams_p_ <= 32 ? kAttnChunk8 : streams_p_ == 64 ? kAttnChunk4Early : kAttnChunk4;
  // K/V rings that do not fit in the Infinity Cache beside the weights are read with
  // non-temporal loads, so that the weights stay cached.
  const bool kv_nt = 2 * c_.layers * (size_t)streams_ * block_words_ * 4 + offsets_.weight_bytes > kInfinityCacheBytes;
  // Mixed mode casts each norm's output, so its norms run first into xn; the other modes fold
  // the norm into the projection (kNorm).
  constexpr bool kFold = P != kMixed;
  const void* nx = kFold ? a.x : a.xn;
  auto norm = [&](uint32_t w_norm) {
    if constexpr (!kFold)
      hipLaunchKernelGGL(batch_norm_mixed, dim3(streams_p_), dim3(256), 0, stream_, dargs_, w_norm);
  };
  project<P, kEpInput, false, 1, 1>(a.in, a.features_p, a.w_input, d, 0u, 0);
  for (int l = 0; l < c_.layers; l++) {
    const LayerWeights& w = a.layer[l];
    norm(w.norm1);
    if (wide && wide_qkv_)
      project<P, kEpQkv, kFold, 2, 2>(nx, a.width_p, w.qkv, 3 * d, w.norm1, l, huge ? 1 : kGroupTiles);
    else project<P, kEpQkv, kFold, 1, 1>(nx, a.width_p, w.qkv, 3 * d, w.norm1, l);
    {
      const dim3 grid(streams_ * c_.heads), block(kAttnThreads);
      const size_t lds = (size_t)c_.window * 4;
      auto attend = [&](auto nt) {
        constexpr bool kNT = decltype(nt)::value;
        if (attn_loads == kAttnChunk4)
          hipLaunchKernelGGL((batch_attention<P, kAttnChunk4, kNT>), grid, block, lds, stream_, dargs_, l);
        else if (attn_loads == kAttnChunk8)
          hipLaunchKernelGGL((batch_attention<P, kAttnChunk8, kNT>), grid, block, lds, stream_, dargs_, l);
        else if (attn_loads == kAttnChunk4Early)
          hipLaunchKernelGGL((batch_attention<P, kAttnChunk4Early, kNT>), grid, block, lds, stream_, dargs_, l);
        else
          hipLaunchKernelGGL((batch_attention<P, kAttnPerPass, kNT>), grid, block, lds, stream_, dargs_, l);
      };
      if (kv_nt) attend(std::true_type{});
      else attend(std::false_type{});
    }
    if (narrow) project<P, kEpOut, false, 2, 1>(a.attn, a.width_p, w.out, d, 0u, l);
    else project<P, kEpOut, false, 1, 1>(a.attn, a.width_p, w.out, d, 0u, l);
    norm(w.norm2);
    if (huge && (2 * F / kBatchTile) % 4 == 0) project<P, kEpGateUp, kFold, 4, 1>(nx, a.width_p, w.gateup, 2 * F, w.norm2, l);
    else if (wide && wide_gateup_) project<P, kEpGateUp, kFold, 2, 2>(nx, a.width_p, w.gateup, 2 * F, w.norm2, l);
    else project<P, kEpGateUp, kFold, 1, 1>(nx, a.width_p, w.gateup, 2 * F, w.norm2, l);
    if (narrow) project<P, kEpDown, false, 2, 1>(a.act, a.ffn_p, w.down, d, 0u, l);
    else project<P, kEpDown, false, 1, 1>(a.act, a.ffn_p, w.down, d, 0u, l);
  }
  hipLaunchKernelGGL(batch_final<P>, dim3(streams_), dim3(64), 0, stream_, dargs_);
  HIP_CHECK(hipGetLastError());
}

// The events of one step into the padded input block in the projections' operand layout.
// Four consecutive columns from a multiple of 4 are consecutive in the layout.
void Batch::stage_events(const float* inputs, float* block) const {
  const int fp = args_.features_p;
  auto at = [&](int b, int k) { return prec_ == kBf16w ? act_index<kBf16w>(b, k, fp) : act_index<kFp32>(b, k, fp); };
  for (int b = 0; b < streams_; b++) {
    const float* src = inputs + (size_t)b * c_.features;
    int k = 0;
    for (; k + 4 <= c_.features; k += 4) std::memcpy(block + at(b, k), src + k, 16);
    for (; k < c_.features; k++) block[at(b, k)] = src[k];
  }
}

void Batch::step(const float* inputs, float* scores) {
  if (!inputs || !scores) throw Error(ST_ERR_INVALID, "Null argument");
  const int fp = args_.features_p;
  float* h = reinterpret_cast<float*>(host_in_.ptr);
  stage_events(inputs, h);
  HIP_CHECK(hipMemcpyAsync(args_.in, host_in_.ptr, (size_t)streams_p_ * fp * 4, hipMemcpyHostToDevice, stream_));
  replay();
  HIP_CHECK(hipMemcpyAsync(host_out_.ptr, args_.score, (size_t)streams_ * 4, hipMemcpyDeviceToHost, stream_));
  sync();
  std::memcpy(scores, host_out_.ptr, (size_t)streams_ * 4);
}

void Batch::reset(int stream) {
  if (stream < -1 || stream >= streams_) throw Error(ST_ERR_INVALID, "Stream index out of range");
  hipLaunchKernelGGL(batch_reset, dim3(256), dim3(256), 0, stream_, dargs_, stream, block_words_);
  HIP_CHECK(hipGetLastError());
  sync();
}

void Batch::snapshot(int stream, uint64_t* position, float* keys, float* values, float* hidden) {
  if (stream < 0 || stream >= streams_) throw Error(ST_ERR_INVALID, "Stream index out of range");
  sync();
  const size_t ring = (size_t)c_.layers * c_.width * c_.window;
  if (position)
    HIP_CHECK(hipMemcpy(position, args_.position + stream, 8, hipMemcpyDeviceToHost));
  // The stream's block of each layer (layer-major rings) into [L][H][W][dh].
  auto download = [&](const void* base, float* dst) {
    if (!dst) return;
    const size_t block = block_words_ * 4, pitch = (size_t)streams_ * block;
    const char* src = reinterpret_cast<const char*>(base) + (size_t)stream * block;
    if (prec_ == kMixed) {
      std::vector<uint16_t> h(ring);
      HIP_CHECK(hipMemcpy2D(h.data(), block, src, pitch, block, c_.layers, hipMemcpyDeviceToHost));
      for (size_t i = 0; i < ring; i++) dst[i] = host_half_to_float(h[i]);
    } else {
      HIP_CHECK(hipMemcpy2D(dst, block, src, pitch, block, c_.layers, hipMemcpyDeviceToHost));
    }
  };
  download(args_.keys, keys);
  download(args_.values, values);
  if (hidden)
    HIP_CHECK(hipMemcpy(hidden, args_.hidden + (size_t)stream * c_.layers * c_.width, (size_t)c_.layers * c_.width * 4,
                        hipMemcpyDeviceToHost));
}

// `count` batched steps from a preloaded device copy of the inputs (count x streams x
// features), continuing the current state; one graph replay per step after a device-to-device
// copy of that step's inputs, with a HIP event after each. Returns the mean microseconds per
// step and, when per_step is not NULL, each step's event-to-event duration.
double Batch::device_run(const float* inputs, size_t count, double* per_step) {
  const int fp = args_.features_p;
  // The padded copy is staged on the host and the device: at most 4 GiB.
  if (!inputs || count == 0 || count > ((size_t)1 << 30) / ((size_t)streams_p_ * fp))
    throw Error(ST_ERR_INVALID, "Invalid trace (empty, or more than 4 GiB of padded inputs)");
  std::vector<float> padded(count * (size_t)streams_p_ * fp, 0.f);
  for (size_t i = 0; i < count; i++)
    stage_events(inputs + i * streams_ * c_.features, &padded[i * streams_p_ * fp]);
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
    replay();
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

// ---- resident batch

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
  for (auto& e : ev) HIP_CHECK(hipEventCreate(&e));
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
