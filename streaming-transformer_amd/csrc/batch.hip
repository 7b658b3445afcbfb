// The batched phase kernels' host sequence (Batch, declared in batch_api.hpp). A translation
// unit of its own, compiled with the kernel arguments preloaded into SGPRs (the projections'
// first loads then wait for no argument load; the single-stream fused kernel, in runtime.hip,
// is faster without).
#include "batch_api.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <type_traits>
#include <vector>

namespace stamd {

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
  stream_.create();

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
  HIP_CHECK(hipStreamEndCapture(stream_, &graph_.g));
  graph_exec_.instantiate(graph_);
}

Batch::~Batch() {
  if (stream_) (void)hipStreamSynchronize(stream_);  // before the buffers are freed
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
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, block, 0, stream_, dargs_, args_.weights, X, woff, N, ld, c_.width, norm, layer);
  };
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
  // The attention loops' form (batch_attention): chunked loads for dh <= 64, eight passes with
  // V loaded early up to 32 streams, four with V early at 64, four from 128.
  const int attn_loads = dim_ > 64 ? kAttnPerPass
                         : streams_p_ <= 32 ? kAttnChunk8Early : streams_p_ == 64 ? kAttnChunk4Early : kAttnChunk4;
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
        else if (attn_loads == kAttnChunk4Early)
          hipLaunchKernelGGL((batch_attention<P, kAttnChunk4Early, kNT>), grid, block, lds, stream_, dargs_, l);
        else if (attn_loads == kAttnChunk8Early)
          hipLaunchKernelGGL((batch_attention<P, kAttnChunk8Early, kNT>), grid, block, lds, stream_, dargs_, l);
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
  for (auto& e : ev) create_timing_event(&e);
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

}  // namespace stamd
