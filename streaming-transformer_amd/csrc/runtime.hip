// Host runtime and C ABI of libstamd.so (see include/st_runtime.h).
//
// Owns the device state of one stream: a single weight arena laid out in phase order,
// the K/V rings, an FP32 scratch arena, the epoch-tagged activation vectors, the
// device-held position and epoch. Mirrors Stream::Runtime::Impl (src/cuda/Runtime.cu:167-653) behind a C ABI.
#include "step_phases.hpp"
#include "mailbox.hpp"
#include "host_common.hpp"
#include "batch_api.hpp"
#include "diag_kernels.hpp"
#include "../../include/st_runtime.h"

#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

namespace stamd {

static thread_local std::string g_last_error;

static std::string json_escape(const std::string& s) {
  std::string o;
  for (char ch : s) {
    if (ch == '"' || ch == '\\') o += '\\';
    o += ch;
  }
  return o;
}

static std::string probe_json() {
  int device = 0, driver = 0, runtime = 0;
  HIP_CHECK(hipGetDevice(&device));
  HIP_CHECK(hipDriverGetVersion(&driver));
  HIP_CHECK(hipRuntimeGetVersion(&runtime));
  hipDeviceProp_t p;
  HIP_CHECK(hipGetDeviceProperties(&p, device));
  int wall = 0, coop = 0;
  HIP_CHECK(hipDeviceGetAttribute(&wall, hipDeviceAttributeWallClockRate, device));
  HIP_CHECK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, device));
  char bus[64] = {0};
  (void)hipDeviceGetPCIBusId(bus, sizeof(bus), device);
  // Some driver stacks report an empty marketing name; fall back to the ISA and CU count.
  std::string name = p.name;
  if (name.empty()) {
    char buf[256] = {0};
    if (hipDeviceGetName(buf, sizeof(buf), device) == hipSuccess) name = buf;
  }
  if (name.empty())
    name = std::string("AMD ") + std::string(p.gcnArchName).substr(0, std::string(p.gcnArchName).find(':')) + " (" +
           std::to_string(p.multiProcessorCount) + " CUs)";
  std::ostringstream o;
  o << "{\"gpu\": \"" << json_escape(name) << "\", \"arch\": \"" << json_escape(p.gcnArchName)
    << "\", \"device\": " << device << ", \"compute_units\": " << p.multiProcessorCount
    << ", \"lds_bytes_per_block\": " << p.sharedMemPerBlock
    << ", \"global_bytes\": " << p.totalGlobalMem << ", \"l2_bytes\": " << p.l2CacheSize
    << ", \"pci_bus\": \"" << bus << "\", \"clock_khz\": " << p.clockRate
    << ", \"memory_clock_khz\": " << p.memoryClockRate << ", \"wall_clock_khz\": " << wall
    << ", \"cooperative_launch\": " << coop << ", \"driver_version\": " << driver
    << ", \"runtime_version\": " << runtime
    << ", \"cpu_logical_count\": " << std::thread::hardware_concurrency() << "}";
  return o.str();
}

// ---------------------------------------------------------------------------------------------

// The allocation-free device trace. Stamps of the per-step wall clock go to a fixed device
// array of kNoAllocMaxEvents + 1 entries (8 MiB per GPU, held until the process ends). In
// host code the array's name only stands for the symbol: its device address on each GPU is
// looked up once (hipGetSymbolAddress, with that device current) and kept per device.
constexpr size_t kNoAllocMaxEvents = (size_t)1 << 20;
static __device__ __align__(256) unsigned long long trace_scratch[kNoAllocMaxEvents + 1];

static std::mutex g_scratch_mutex;
static std::map<int, unsigned long long*> g_scratch_ptr;  // device -> address of trace_scratch there
// device -> held by an allocation-free trace from its launch to its stamp readback, so that
// such calls on one GPU (from any runtime or thread) take turns on that GPU's array
static std::map<int, std::unique_ptr<std::mutex>> g_scratch_use;

static std::mutex& trace_scratch_use(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  std::unique_ptr<std::mutex>& m = g_scratch_use[device];
  if (!m) m = std::make_unique<std::mutex>();
  return *m;
}

// Looks up (once per device) the address of trace_scratch on the current device.
static unsigned long long* trace_scratch_address() {
  int device = 0;
  HIP_CHECK(hipGetDevice(&device));
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  auto it = g_scratch_ptr.find(device);
  if (it != g_scratch_ptr.end()) return it->second;
  void* ptr = nullptr;
  HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(trace_scratch)));
  if (!ptr) throw Error(ST_ERR_DEVICE, "No device address for the trace scratch array");
  g_scratch_ptr[device] = reinterpret_cast<unsigned long long*>(ptr);
  return g_scratch_ptr[device];
}

#include "vendor_path.hpp"

class ResidentBatch;

class Runtime {
 public:
  // share_weights: use that runtime's weight arena (same config and storage) instead of
  // building one; it must outlive this runtime.
  Runtime(const st_config& config, bool mixed, const st_tensor* tensors, size_t count,
          const st_options& options, const Runtime* share_weights = nullptr);
  ~Runtime();
  float step(const float* input);
  void reset();
  void stop();
  void snapshot(uint64_t* position, float* keys, float* values, float* hidden);
  double device_trace(const float* inputs, size_t count, double* per_event);
  // deviceTrace without allocation: events already in device memory, stamps in the
  // library's fixed device array.
  double device_trace_noalloc(const float* device_events, size_t count, double* per_event);
  double device_run(const float* inputs, size_t count, bool reset_first, double* per_event);
  size_t phase_times(const float* input, double* us, size_t cap);
  // traceStep: names and sizes of the trace entries in output order (fixed by the config).
  std::vector<std::pair<std::string, size_t>> trace_layout() const;
  std::vector<std::pair<std::string, std::vector<float>>> trace_step(const float* input);
  std::string info();
  // Scheduled arrivals (bench/Main.cpp:282-342): a producer thread offers event i at its
  // intended time into a bounded queue (dropping it when the queue is full); this thread
  // steps the runtime on each dequeued event. Times in ns since the schedule's start.
  void scheduled_run(const float* inputs, size_t count, double rate, size_t capacity, bool bursty, double* intended,
                     double* enqueue, double* submit, double* complete, float* scores, uint8_t* dropped);

 private:
  void build_weights(const st_tensor* tensors, size_t count);
  // One step on the stream: the captured graph for GRAPH / CUBLAS_GRAPH (which holds the
  // mapped staging kernels when `mapped`), else the backend's launches.
  void launch_step();
  // One step's compute launches without the graph and without mapped staging.
  void launch_compute();
  void launch_phases();
  void launch_fused(const float* event = nullptr);
  // Epochs of the tagged dataflow: `steps` steps are about to run. Rebases first when they
  // would pass kEpochLimit.
  void reserve_epochs(uint64_t steps);
  void rebase_epochs();
  unsigned per_step() const { return 5u * (unsigned)c_.layers + 3u; }
  bool tagged_steps() const { return !vendor(); }
  template <int P, int A> void launch_phases_t();
  template <int P, int A> void launch_fused_t(const float* event);
  template <int P, int A> void launch_trace_t(const float* events, int count, int stride, unsigned long long* stamps);
  template <int P, int A> int legal_blocks_t();
  // Call f(precision, attention path) with both as integral constants.
  template <class F> auto dispatch(F&& f) {
    using I = std::integral_constant<int, 0>;
    if (args_.attn_regs) {
      // One instantiation per register attention variant: 16 or 8 16-byte chunks per head
      // row, or any other count (A = 1, 2, 3).
      const int variant = attn_variant();
      const bool nt = weights_nt();
      auto with = [&](auto P) {
        if (variant == 1) return nt ? f(P, std::integral_constant<int, 1 | kWeightNt>{})
                                    : f(P, std::integral_constant<int, 1>{});
        if (variant == 2) return nt ? f(P, std::integral_constant<int, 2 | kWeightNt>{})
                                    : f(P, std::integral_constant<int, 2>{});
        return f(P, std::integral_constant<int, 3>{});
      };
      switch (prec_) {
        case kFp32: return with(std::integral_constant<int, kFp32>{});
        case kMixed: return with(std::integral_constant<int, kMixed>{});
        default: return with(std::integral_constant<int, kBf16w>{});
      }
    }
    switch (prec_) {
      case kFp32: return f(std::integral_constant<int, kFp32>{}, I{});
      case kMixed: return f(std::integral_constant<int, kMixed>{}, I{});
      default: return f(std::integral_constant<int, kBf16w>{}, I{});
    }
  }
  // Register attention variant: 1, 2, 3 for head rows of 16, 8 or another number of 16-byte
  // chunks (0: the LDS path).
  int attn_variant() const {
    if (!args_.attn_regs) return 0;
    const int chunks = dim_ * (prec_ == kMixed ? 2 : 4) / 16;
    return chunks == 16 ? 1 : chunks == 8 ? 2 : 3;
  }
  // Weights larger than the 256 MB Infinity Cache (MALL) stream with non-temporal loads (bit 2
  // of the kernels' A parameter, instantiated for variants 1 and 2): they then do not displace
  // what stays cached across steps. Smaller weight sets stay resident in the cache instead.
  bool weights_nt() const {
    const int v = attn_variant();
    return (size_t)args_.weight_bytes > ((size_t)256 << 20) && (v == 1 || v == 2);
  }
  void check_device_error();
  void sync() { HIP_CHECK(hipStreamSynchronize(stream_)); }
  bool persistent() const { return opt_.backend == ST_BACKEND_PERSISTENT; }
  bool coresident(int grid);
  // grid_ passed the co-residency probe: the FUSED, PERSISTENT and trace kernels (and GRAPH's
  // fused node) launch plainly.
  bool plain_launch_ = false;
  bool graph_fused_ = false;   // GRAPH: the captured step is the fused kernel
  bool vendor() const { return opt_.backend == ST_BACKEND_CUBLAS || opt_.backend == ST_BACKEND_CUBLAS_GRAPH; }
  void reset_device();
  void start_worker();
  void command(int cmd);
  void issue(int cmd);            // one mailbox round trip
  void restart_worker_rebased();  // stop the worker, rebase the epochs, relaunch it
  void stage_input();             // mapped: event from host-mapped memory into the device copy
  void stage_output();            // mapped: score and error bits into host-mapped memory
  Mailbox* mailbox() { return reinterpret_cast<Mailbox*>(mailbox_.ptr); }

  // Epochs stay below this bound, so the never-matching tag 0 and the all-ones sentinel of the
  // workgroup-local flags are never live epochs.
  static constexpr uint64_t kEpochLimit = 0xF0000000ull;

  st_config c_;
  st_options opt_;
  int prec_ = kFp32;
  int dim_ = 0, grid_ = 1, legal_blocks_ = 1, cus_ = 1, wall_khz_ = 100000;
  int phase_grid_ = 1;       // workgroups of a phase launch (staged sequence)
  bool phase_coop_ = false;  // phase launches are cooperative (the plain grid failed the probe)
  bool running_ = true;
  StreamHandle stream_;
  GraphHandle graph_;
  GraphExecHandle graph_exec_;
  DeviceBuffer weights_, keys_, values_, scratch_, tagged_, position_, epoch_dev_, rope_, args_dev_;
  PinnedBuffer host_in_, host_out_;
  MappedBuffer mailbox_, mapped_in_, mapped_snap_, mapped_io_;
  MailboxClient client_;     // host half of the persistent worker's mailbox protocol
  uint64_t epoch_ = 1;       // host copy of the device epoch (the next step's phase-0 epoch)
  unsigned long long* scratch_ptr_ = nullptr;  // this device's trace_scratch (allocation-free trace)
  int device_ = 0;                             // the device this runtime was created on
  uint64_t runs_done_ = 0;   // RUN commands the persistent worker has completed
  StreamHandle copy_stream_;
  StepArgs args_{};
  const StepArgs* dargs_ = nullptr;
  std::string probe_;
  std::unique_ptr<VendorPath> vendor_;  // CUBLAS / CUBLAS_GRAPH

  // A resident batch launches its streams' steps together and keeps their epochs.
  friend class ResidentBatch;
};

Runtime::Runtime(const st_config& config, bool mixed, const st_tensor* tensors, size_t count,
                 const st_options& options, const Runtime* share_weights)
    : c_(config), opt_(options) {
  validate_config(c_);
  if (options.idle_seconds <= 0 || options.idle_seconds > 3600 || options.blocks < 0)
    throw Error(ST_ERR_INVALID, "Invalid blocks or idle budget");
  if (options.initial_sequence >= std::numeric_limits<uint64_t>::max() - 1)
    throw Error(ST_ERR_INVALID, "Initial sequence must leave room for RUN and STOP");
  if ((options.backend == ST_BACKEND_CUBLAS || options.backend == ST_BACKEND_CUBLAS_GRAPH) &&
      options.weight_dtype == ST_WEIGHTS_BF16)
    throw Error(ST_ERR_INVALID, "Vendor GEMV backends take the checkpoint's own weight storage (FP32 or mixed)");
  if (options.backend < 0 || options.backend > ST_BACKEND_PERSISTENT)
    throw Error(ST_ERR_INVALID, "Unknown backend");
  if (options.weight_dtype == ST_WEIGHTS_BF16 && mixed)
    throw Error(ST_ERR_INVALID, "bfloat16 weight storage applies to FP32 checkpoints only");
  if (options.weight_dtype != ST_WEIGHTS_AS_MODEL && options.weight_dtype != ST_WEIGHTS_BF16)
    throw Error(ST_ERR_INVALID, "Unknown weight storage");
  prec_ = mixed ? kMixed : (options.weight_dtype == ST_WEIGHTS_BF16 ? kBf16w : kFp32);
  dim_ = c_.width / c_.heads;

  probe_ = probe_json();
  int device = 0;
  HIP_CHECK(hipGetDevice(&device));
  hipDeviceProp_t prop;
  HIP_CHECK(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    throw Error(ST_ERR_DEVICE, std::string("Supported target is gfx950; found ") + prop.gcnArchName);
  cus_ = prop.multiProcessorCount;
  HIP_CHECK(hipDeviceGetAttribute(&wall_khz_, hipDeviceAttributeWallClockRate, device));
  device_ = device;
  scratch_ptr_ = trace_scratch_address();
  stream_.create();
  copy_stream_.create();

  // ---- shape-derived layout
  StepArgs& a = args_;
  a.layers = c_.layers;
  a.width = c_.width;
  a.heads = c_.heads;
  a.ffn = c_.ffn;
  a.window = c_.window;
  a.features = c_.features;
  a.dim = dim_;
  a.epsilon = c_.epsilon;
  // Rows padded to whole 1 KiB slabs (zeros in weights and activations).
  const int slab = 1024 / (prec_ == kFp32 ? 4 : 2);
  a.width_p = round_up(c_.width, slab);
  a.ffn_p = round_up(c_.ffn, slab);
  a.features_p = round_up(c_.features, slab);
  // Window slots per attention item: one K (or V) block of at most kKB 1 KiB slabs in FP32.
  a.chunk = std::min(4 * kKB, kKB * 256 / dim_);
  if (a.chunk < 1) a.chunk = 1;
  {
    // Register attention: power-of-two head dim with E <= dim <= 64E (E = elements per
    // 16-byte chunk) and a K/V block that is whole 16-byte chunks.
    const int e = prec_ == kMixed ? 8 : 4;
    const int kvb = prec_ == kMixed ? 2 : 4;
    bool pow2 = (dim_ & (dim_ - 1)) == 0;
    a.attn_regs = pow2 && dim_ >= e && dim_ <= 64 * e && (a.chunk * dim_ * kvb) % 16 == 0 ? 1 : 0;
  }

  if (share_weights) {
    if (share_weights->prec_ != prec_ || share_weights->args_.width_p != a.width_p ||
        share_weights->args_.ffn_p != a.ffn_p || share_weights->args_.features_p != a.features_p ||
        share_weights->c_.layers != c_.layers)
      throw Error(ST_ERR_INVALID, "Shared weights come from a runtime of another shape or storage");
    const StepArgs& w = share_weights->args_;
    a.weights = w.weights;
    a.weight_bytes = w.weight_bytes;
    a.w_input = w.w_input;
    a.w_final_norm = w.w_final_norm;
    a.w_score = w.w_score;
    for (int l = 0; l < kMaxLayers; l++) a.layer[l] = w.layer[l];
  } else {
    build_weights(tensors, count);
  }

  // ---- state
  const size_t kvb = prec_ == kMixed ? 2 : 4;
  const size_t cache_elems = (size_t)c_.layers * c_.width * c_.window;
  keys_.alloc(cache_elems * kvb);
  values_.alloc(cache_elems * kvb);
  a.keys = keys_.ptr;
  a.values = values_.ptr;
  a.cache_bytes = (uint32_t)(cache_elems * kvb);

  int nch = (c_.window + a.chunk - 1) / a.chunk;
  uint32_t off = 0;
  auto take = [&](size_t n) {
    uint32_t o = off;
    off += (uint32_t)round_up((int)n, 64);
    return o;
  };
  int vec = std::max({a.width_p, a.ffn_p, a.features_p});
  a.s_input = take(a.features_p);
  a.s_hidden = take((size_t)c_.layers * c_.width);
  a.s_score = take(64);
  (void)vec;
  scratch_.alloc((size_t)off * 4);
  HIP_CHECK(hipMemset(scratch_.ptr, 0, (size_t)off * 4));
  a.scratch = reinterpret_cast<float*>(scratch_.ptr);
  a.scratch_bytes = off * 4;
  a.error = reinterpret_cast<unsigned*>(a.scratch + a.s_score + 1);
  a.input = a.scratch + a.s_input;

  // Epoch-tagged activation vectors (8 bytes per element), zeroed: tag 0 never matches
  // because epochs start at 1.
  uint32_t toff = 0;
  auto ttake = [&](size_t n) {
    uint32_t o = toff;
    toff += (uint32_t)round_up((int)n, 64);
    return o;
  };
  a.t_x = ttake(a.width_p);
  a.t_q = ttake(a.width_p);
  a.t_k = ttake(a.width_p);
  a.t_v = ttake(a.width_p);
  a.t_attn = ttake(a.width_p);
  a.t_act = ttake(a.ffn_p);
  a.t_done = ttake(64);
  a.t_cmd = ttake(64);
  a.t_in = ttake(a.features_p);
  a.t_wdone = ttake(kMaxGrid);
  a.t_po = ttake((size_t)c_.heads * nch * dim_);
  a.t_pm = ttake((size_t)c_.heads * nch);
  a.t_ps = ttake((size_t)c_.heads * nch);
  tagged_.alloc((size_t)toff * 8);
  HIP_CHECK(hipMemset(tagged_.ptr, 0, (size_t)toff * 8));
  a.tagged = reinterpret_cast<unsigned long long*>(tagged_.ptr);
  a.tagged_bytes = toff * 8;

  position_.alloc(8);
  HIP_CHECK(hipMemset(position_.ptr, 0, 8));
  a.position = reinterpret_cast<unsigned long long*>(position_.ptr);
  epoch_dev_.alloc(64);
  epoch_ = options.initial_epoch ? options.initial_epoch : 1u;
  const unsigned first_epoch = (unsigned)epoch_;
  HIP_CHECK(hipMemset(epoch_dev_.ptr, 0, 64));
  HIP_CHECK(hipMemcpy(epoch_dev_.ptr, &first_epoch, 4, hipMemcpyHostToDevice));
  a.epoch = reinterpret_cast<unsigned*>(epoch_dev_.ptr);

  // RoPE inverse frequencies: powf(10000, -i/dim) for even i (src/cpu/Cpu.cpp:75).
  std::vector<float> freq(dim_ / 2);
  for (int j = 0; j < dim_ / 2; j++) freq[j] = std::pow(10000.0f, -(float)(2 * j) / (float)dim_);
  rope_.alloc(freq.size() * 4);
  HIP_CHECK(hipMemcpy(rope_.ptr, freq.data(), freq.size() * 4, hipMemcpyHostToDevice));
  a.rope_freq = reinterpret_cast<const float*>(rope_.ptr);
  a.spin_limit = (unsigned long long)wall_khz_ * 1000ull * 2ull;  // 2 s per barrier wait

  host_in_.alloc((size_t)a.features_p * 4);
  std::memset(host_in_.ptr, 0, (size_t)a.features_p * 4);
  host_out_.alloc(64);
  if (options.mapped && options.backend != ST_BACKEND_PERSISTENT) {
    // The event (features_p floats, zero padding) followed by the score and the error word.
    mapped_io_.alloc((size_t)a.features_p * 4 + 64);
  }

  // ---- grid
  legal_blocks_ = dispatch([&](auto P, auto A) { return legal_blocks_t<P.value, A.value>(); });
  grid_ = options.blocks == 0 ? std::min(cus_, kMaxGrid) : options.blocks;
  if (grid_ > kMaxGrid) throw Error(ST_ERR_INVALID, "Requested grid exceeds " + std::to_string(kMaxGrid) + " workgroups");
  if ((options.backend == ST_BACKEND_FUSED || options.backend == ST_BACKEND_PERSISTENT) && grid_ > legal_blocks_)
    throw Error(ST_ERR_INVALID,
                "Requested cooperative grid exceeds actual occupancy limit " + std::to_string(legal_blocks_));
  a.grid = grid_;
  phase_grid_ = std::min(grid_, legal_blocks_);
  if (options.backend == ST_BACKEND_PERSISTENT) {
    mailbox_.alloc(sizeof(Mailbox));
    mapped_in_.alloc((size_t)c_.features * 4);
    Mailbox* mb = mailbox();
    Mailbox* dmb = reinterpret_cast<Mailbox*>(mailbox_.dev);
    client_.attach(mb, options.initial_sequence);
    a.mb_request = &dmb->request;
    a.mb_completion = &dmb->completion;
    a.mb_exited = &dmb->exited;
    a.mb_command = &dmb->command;
    a.mb_score = &dmb->score;
    a.mb_checksum = &dmb->checksum;
    a.mb_error = &dmb->error;
    a.mapped_input = reinterpret_cast<const float*>(mapped_in_.dev);
    const int kvb = prec_ == kMixed ? 2 : 4;
    mapped_snap_.alloc(kSnapKeys + 2 * (size_t)snapshot_ring_bytes(c_.layers, c_.width, c_.window, kvb) +
                       (size_t)c_.layers * c_.width * 4);
    a.mapped_snapshot = reinterpret_cast<unsigned char*>(mapped_snap_.dev);
    a.idle_ticks = (unsigned long long)(options.idle_seconds * (double)wall_khz_ * 1000.0);
    a.max_events = options.max_events;
    a.initial_sequence = options.initial_sequence;
    a.backoff = options.backoff ? 1 : 0;
  }
  args_dev_.alloc(sizeof(StepArgs));
  HIP_CHECK(hipMemcpy(args_dev_.ptr, &args_, sizeof(StepArgs), hipMemcpyHostToDevice));
  dargs_ = reinterpret_cast<const StepArgs*>(args_dev_.ptr);

  reset_device();
  if (options.backend == ST_BACKEND_CUDA && phase_grid_ > 1 && !coresident(phase_grid_)) {
    // Phase launches exchange data within the launch, so their workgroups must be resident
    // together: when a plain launch of this grid is not, launch the phases cooperatively.
    phase_coop_ = true;
  }
  // The captured graph holds one step, with the mapped staging kernels around it (the
  // reference captures stage_input and stage_output with the sequence, src/cuda/Runtime.cu:
  // 276-283). Warm up outside capture, restore the initial state, then capture.
  auto capture = [&](auto&& sequence) {
    if (tagged_steps()) reserve_epochs(1);
    sequence();
    sync();
    reset_device();
    HIP_CHECK(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
    if (opt_.mapped) stage_input();
    sequence();
    if (opt_.mapped) stage_output();
    HIP_CHECK(hipStreamEndCapture(stream_, &graph_.g));
    graph_exec_.instantiate(graph_);
  };
  if (vendor()) {
    vendor_ = std::make_unique<VendorPath>(c_, prec_ == kMixed, args_, tensors, count, stream_);
    if (options.backend == ST_BACKEND_CUBLAS_GRAPH) capture([&] { vendor_->launch(); });
  }
  if (options.backend == ST_BACKEND_GRAPH) {
    // The graph holds the fused kernel as a single plain node when the grid is resident all
    // at once (bit-identical to the phase sequence), else the phase sequence, on the largest
    // grid (halving from the requested one) that a plain launch keeps resident: captured
    // launches cannot be cooperative.
    graph_fused_ = grid_ > 1 && grid_ <= legal_blocks_ && coresident(grid_);
    if (graph_fused_) plain_launch_ = true;
    while (!graph_fused_ && phase_grid_ > 1 && !coresident(phase_grid_)) phase_grid_ /= 2;
    capture([&] {
      if (graph_fused_) launch_fused();
      else launch_phases();
    });
  }
  // FUSED, PERSISTENT and the device trace launch grid_ workgroups plainly when the probe
  // shows them resident at once. A cooperative launch is the fallback only: it takes the
  // device's global wave sync resource, which one process holds at a time, so while another
  // process holds it a cooperative launch fails (hipErrorIllegalState).
  if (!plain_launch_ && grid_ > 1 && options.backend != ST_BACKEND_GRAPH && !vendor())
    plain_launch_ = coresident(grid_);
  if (persistent()) {
    if (epoch_ + 2ull * per_step() > kEpochLimit) rebase_epochs();
    start_worker();
  }
}

// Co-residency probe: one plain launch of `grid` workgroups with the fused kernel's footprint
// (kThreads threads and LdsAll in LDS, which leaves room for one workgroup per CU). Every
// workgroup counts itself in and waits, for at most 50 ms, until all have arrived. True when
// they all did: the grid then runs at once without a cooperative launch, whose dispatch costs
// about 15 us per step on this stack.
__global__ __launch_bounds__(kThreads) void coresidency_kernel(unsigned* arrived, unsigned grid, unsigned long long ticks,
                                                                unsigned* failed) {
  __shared__ LdsAll lds;
  if (threadIdx.x == 0) {
    *reinterpret_cast<volatile int*>(&lds.cmd) = (int)blockIdx.x;  // keeps the LDS allocation
    __hip_atomic_fetch_add(arrived, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long start = wall_clock64();
    while (__hip_atomic_load(arrived, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < grid) {
      if (wall_clock64() - start > ticks) {
        __hip_atomic_fetch_or(failed, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(8);
    }
  }
}

bool Runtime::coresident(int grid) {
  DeviceBuffer words;
  words.alloc(256);
  HIP_CHECK(hipMemset(words.ptr, 0, 256));
  unsigned* w = reinterpret_cast<unsigned*>(words.ptr);
  const unsigned long long ticks = (unsigned long long)wall_khz_ * 50ull;  // 50 ms
  hipLaunchKernelGGL(coresidency_kernel, dim3(grid), dim3(kThreads), 0, stream_, w, (unsigned)grid, ticks, w + 32);
  HIP_CHECK(hipGetLastError());
  sync();
  unsigned failed = 0;
  HIP_CHECK(hipMemcpy(&failed, w + 32, 4, hipMemcpyDeviceToHost));
  return failed == 0;
}

Runtime::~Runtime() {
  // Join a persistent worker before anything it uses is freed (src/cuda/Runtime.cu:294-299).
  try {
    stop();
  } catch (...) {
  }
  if (stream_) (void)hipStreamSynchronize(stream_);
  vendor_.reset();  // the rocBLAS handle refers to the stream, which the members release after it
}

template <int P, int A>
int Runtime::legal_blocks_t() {
  int per_cu = 0, trace_per_cu = 0, phase_per_cu = 0, worker_per_cu = 0;
  HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fused_kernel<P, A>, kThreads, 0));
  HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&trace_per_cu, trace_kernel<P, A>, kThreads, 0));
  HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&phase_per_cu, phase_kernel<P, A>, kThreads, 0));
  HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&worker_per_cu, persistent_kernel<P, A>, kThreads, 0));
  return std::max(1, std::min({per_cu, trace_per_cu, phase_per_cu, worker_per_cu}) * cus_);
}

// Weight arena in phase order: input, then per layer norm1, norm2, qkv (stacked q;k;v),
// out, gateup (row 2i = gate i, row 2i+1 = up i), down; then final_norm, score.
// Rows are padded with zeros to a multiple of 16 bytes.
// The weight arena (also used by the batched runtime): rows padded to whole 1 KiB slabs, q/k/v
// stacked, gate and up rows interleaved per unit; offsets recorded in args_. The row lengths
// args_.width_p, ffn_p and features_p must be set.
// The weight arena. Matrices are row-major with rows padded to the slab, or, with `tiled`
// (the batched runtime's MFMA projections), in operand order: 16-row tiles, then blocks of KB
// columns, then the 64 lanes of an MFMA operand (row r mod 16 + 16 x column group), KB / 4
// values each, so that a wave loads one block as one contiguous run of 64 x 16 bytes (a
// row-major operand makes every lane's 16 bytes a separate access for the L1, whose rate of
// accesses then bounds the projections). KB is 16 for the FP32 MFMA (FP32 weights, and the
// mixed mode's input projection) and 32 for the 16-bit MFMAs.
void build_arena(const st_config& c_, int prec_, const st_tensor* tensors, size_t count, StepArgs& args_,
                 DeviceBuffer& weights_, bool tiled) {
  std::map<std::string, const st_tensor*> byname;
  for (size_t i = 0; i < count; i++) {
    if (!tensors[i].name || !tensors[i].data) throw Error(ST_ERR_INVALID, "Null tensor");
    if (!byname.emplace(tensors[i].name, &tensors[i]).second)
      throw Error(ST_ERR_INVALID, std::string("Duplicate tensor: ") + tensors[i].name);
  }
  auto get = [&](const std::string& name, std::vector<int> shape) -> const st_tensor* {
    auto it = byname.find(name);
    if (it == byname.end()) throw Error(ST_ERR_INVALID, "Missing tensor: " + name);
    const st_tensor* t = it->second;
    std::vector<int> actual(t->shape, t->shape + std::max(0, std::min(2, t->rank)));
    if (t->rank != (int)shape.size() || actual != shape) throw Error(ST_ERR_INVALID, "Shape mismatch: " + name);
    return t;
  };
  const int wb = prec_ == kFp32 ? 4 : 2;
  std::vector<unsigned char> host;
  auto align = [&]() { host.resize((host.size() + 255) / 256 * 256, 0); };
  auto put = [&](float v) {
    if (prec_ == kFp32) {
      unsigned char b[4];
      std::memcpy(b, &v, 4);
      host.insert(host.end(), b, b + 4);
    } else {
      uint16_t h;
      if (prec_ == kMixed) {
        h = host_half_bits(v);
        if (host_half_to_float(h) != v && !std::isnan(v))
          throw Error(ST_ERR_INVALID, "Mixed checkpoint tensor value is not FP16-representable");
      } else {
        h = host_bf16_bits(v);
      }
      host.push_back((unsigned char)(h & 0xff));
      host.push_back((unsigned char)(h >> 8));
    }
  };
  // Rows of `cols` values padded to `cols_p`, appended to a row-major matrix.
  auto add_rows = [&](std::vector<float>& m, const float* data, int rows, int cols, int cols_p) {
    for (int r = 0; r < rows; r++) {
      m.insert(m.end(), data + (size_t)r * cols, data + (size_t)r * cols + cols);
      m.insert(m.end(), (size_t)(cols_p - cols), 0.f);
    }
  };
  auto put_matrix = [&](const std::vector<float>& m, int cols_p, bool fp32_mfma) {
    if (!tiled) {
      for (float v : m) put(v);
      return;
    }
    const int kb_cols = fp32_mfma ? 16 : 32, per_lane = kb_cols / 4;
    const int rows = (int)(m.size() / cols_p);
    for (int t = 0; t < rows / 16; t++)
      for (int kb = 0; kb < cols_p / kb_cols; kb++)
        for (int lane = 0; lane < 64; lane++)
          for (int e = 0; e < per_lane; e++)
            put(m[(size_t)(t * 16 + lane % 16) * cols_p + kb * kb_cols + lane / 16 * per_lane + e]);
  };
  const bool fp32_mfma = prec_ == kFp32;
  auto put_rows = [&](const float* data, int rows, int cols, int cols_p, bool fp32) {
    std::vector<float> m;
    add_rows(m, data, rows, cols, cols_p);
    put_matrix(m, cols_p, fp32);
  };
  auto put_vector = [&](const float* data, int n) {
    for (int i = 0; i < n; i++) put(data[i]);
  };
  StepArgs& a = args_;
  const int d = c_.width, f = c_.ffn;
  align();
  a.w_input = (uint32_t)host.size();
  put_rows(get("input", {d, c_.features})->data, d, c_.features, a.features_p, prec_ != kBf16w);
  for (int l = 0; l < c_.layers; l++) {
    std::string p = "layers." + std::to_string(l) + ".";
    LayerWeights& lw = a.layer[l];
    align();
    lw.norm1 = (uint32_t)host.size();
    put_vector(get(p + "norm1", {d})->data, d);
    align();
    lw.norm2 = (uint32_t)host.size();
    put_vector(get(p + "norm2", {d})->data, d);
    align();
    lw.qkv = (uint32_t)host.size();
    {
      std::vector<float> m;
      for (const char* part : {"q", "k", "v"}) add_rows(m, get(p + part, {d, d})->data, d, d, a.width_p);
      put_matrix(m, a.width_p, fp32_mfma);
    }
    align();
    lw.out = (uint32_t)host.size();
    put_rows(get(p + "out", {d, d})->data, d, d, a.width_p, fp32_mfma);
    align();
    lw.gateup = (uint32_t)host.size();
    const float* gate = get(p + "gate", {f, d})->data;
    const float* up = get(p + "up", {f, d})->data;
    {
      std::vector<float> m;
      for (int r = 0; r < f; r++) {
        add_rows(m, gate + (size_t)r * d, 1, d, a.width_p);
        add_rows(m, up + (size_t)r * d, 1, d, a.width_p);
      }
      put_matrix(m, a.width_p, fp32_mfma);
    }
    align();
    lw.down = (uint32_t)host.size();
    put_rows(get(p + "down", {d, f})->data, d, f, a.ffn_p, fp32_mfma);
  }
  align();
  a.w_final_norm = (uint32_t)host.size();
  put_vector(get("final_norm", {d})->data, d);
  align();
  a.w_score = (uint32_t)host.size();
  {
    std::vector<float> m;
    add_rows(m, get("score", {1, d})->data, 1, d, a.width_p);
    for (float v : m) put(v);  // a vector (the final phase reads it as one)
  }
  align();
  host.resize(host.size() + 256, 0);
  if (host.size() > (size_t)std::numeric_limits<int>::max())
    throw Error(ST_ERR_INVALID, "Weight arena exceeds 2 GiB");
  (void)wb;
  weights_.alloc(host.size());
  HIP_CHECK(hipMemcpy(weights_.ptr, host.data(), host.size(), hipMemcpyHostToDevice));
  a.weights = reinterpret_cast<const char*>(weights_.ptr);
  a.weight_bytes = (uint32_t)host.size();
}

void Runtime::build_weights(const st_tensor* tensors, size_t count) {
  build_arena(c_, prec_, tensors, count, args_, weights_);
}

template <int P, int A>
void Runtime::launch_phases_t() {
  const int nph = 5 * c_.layers + 2;
  // Attention chunks of one head are combined by polling partials written in the same
  // launch, so every workgroup of a launch must be resident at once: phase_grid_ passed the
  // co-residency probe, or the launches are cooperative.
  for (int ph = 0; ph < nph; ph++) {
    int grid = ph == nph - 1 ? 1 : phase_grid_;
    if (phase_coop_ && grid > 1) {
      const StepArgs* args = dargs_;
      void* params[] = {&args, &ph};
      HIP_CHECK(hipLaunchCooperativeKernel(reinterpret_cast<void*>(phase_kernel<P, A>), dim3(grid), dim3(kThreads),
                                           params, 0, stream_));
    } else {
      hipLaunchKernelGGL((phase_kernel<P, A>), dim3(grid), dim3(kThreads), 0, stream_, dargs_, ph);
    }
  }
  HIP_CHECK(hipGetLastError());
}

void Runtime::launch_phases() {
  dispatch([&](auto P, auto A) { launch_phases_t<P.value, A.value>(); return 0; });
}

template <int P, int A>
void Runtime::launch_fused_t(const float* event) {
  if (grid_ == 1 || plain_launch_) {
    // One workgroup, or a grid the co-residency probe showed to be resident all at once.
    hipLaunchKernelGGL((fused_kernel<P, A>), dim3(grid_), dim3(kThreads), 0, stream_, dargs_, event);
  } else {
    void* params[] = {&dargs_, &event};
    HIP_CHECK(hipLaunchCooperativeKernel(reinterpret_cast<void*>(fused_kernel<P, A>), dim3(grid_),
                                         dim3(kThreads), params, 0, stream_));
  }
  HIP_CHECK(hipGetLastError());
}

void Runtime::launch_fused(const float* event) {
  dispatch([&](auto P, auto A) { launch_fused_t<P.value, A.value>(event); return 0; });
}

void Runtime::launch_step() {
  if (opt_.backend == ST_BACKEND_GRAPH || opt_.backend == ST_BACKEND_CUBLAS_GRAPH) {
    HIP_CHECK(hipGraphLaunch(graph_exec_, stream_));
    return;
  }
  if (opt_.mapped) stage_input();
  launch_compute();
  if (opt_.mapped) stage_output();
}

void Runtime::launch_compute() {
  if (opt_.backend == ST_BACKEND_FUSED || (opt_.backend == ST_BACKEND_GRAPH && graph_fused_)) launch_fused();
  else if (vendor()) vendor_->launch();
  else launch_phases();
}

// Mapped staging kernels (the reference's stage_input / stage_output, src/cuda/Runtime.cu:
// 43-48): the event is read from host memory mapped into the device, the score and the
// error word are written back there.
// The event crosses PCIe as one 16-byte load per thread: a padded row of up to 1024 floats in
// a single round trip from host memory (n4: 16-byte pieces).
__global__ void stage_input_kernel(const float4* mapped, float4* input, int n4) {
  for (int i = threadIdx.x; i < n4; i += blockDim.x) input[i] = mapped[i];
}
__global__ void stage_output_kernel(const float* score_and_error, float* mapped) {
  if (threadIdx.x < 2) mapped[threadIdx.x] = score_and_error[threadIdx.x];
}

void Runtime::stage_input() {
  hipLaunchKernelGGL(stage_input_kernel, dim3(1), dim3(256), 0, stream_, reinterpret_cast<const float4*>(mapped_io_.dev),
                     reinterpret_cast<float4*>(args_.scratch + args_.s_input), args_.features_p / 4);
  HIP_CHECK(hipGetLastError());
}

void Runtime::stage_output() {
  hipLaunchKernelGGL(stage_output_kernel, dim3(1), dim3(64), 0, stream_, args_.scratch + args_.s_score,
                     reinterpret_cast<float*>(mapped_io_.dev) + args_.features_p);
  HIP_CHECK(hipGetLastError());
}

void Runtime::rebase_epochs() {
  // Drain the device, zero every tag (tag 0 never matches a live epoch), restart at 1.
  sync();
  HIP_CHECK(hipMemsetAsync(tagged_.ptr, 0, args_.tagged_bytes, stream_));
  const unsigned one = 1;
  HIP_CHECK(hipMemcpyAsync(epoch_dev_.ptr, &one, 4, hipMemcpyHostToDevice, stream_));
  sync();
  epoch_ = 1;
}

void Runtime::reserve_epochs(uint64_t steps) {
  const uint64_t need = steps * per_step();
  if (need >= kEpochLimit) throw Error(ST_ERR_INVALID, "Too many steps in one launch for the 32-bit epoch range");
  if (epoch_ + need > kEpochLimit) rebase_epochs();
  epoch_ += need;
}

void Runtime::check_device_error() {
  unsigned err = 0;
  HIP_CHECK(hipMemcpy(&err, args_.error, 4, hipMemcpyDeviceToHost));
  if (err) throw Error(ST_ERR_NUMERIC, "Device watchdog tripped (error bits " + std::to_string(err) + ")");
}

float Runtime::step(const float* input) {
  if (!running_) throw Error(ST_ERR_STATE, "Runtime is stopped");
  if (!input) throw Error(ST_ERR_INVALID, "Null input");
  if (persistent()) {
    std::memcpy(mapped_in_.ptr, input, (size_t)c_.features * 4);
    command(kCmdRun);
    return mailbox()->score;
  }
  if (tagged_steps()) reserve_epochs(1);
  const float* out;
  if (opt_.mapped) {
    std::memcpy(mapped_io_.ptr, input, (size_t)c_.features * 4);
    launch_step();  // staging kernels included
    sync();
    out = reinterpret_cast<const float*>(mapped_io_.ptr) + args_.features_p;
  } else {
    std::memcpy(host_in_.ptr, input, (size_t)c_.features * 4);
    HIP_CHECK(hipMemcpyAsync(args_.scratch + args_.s_input, host_in_.ptr, (size_t)args_.features_p * 4,
                             hipMemcpyHostToDevice, stream_));
    launch_step();
    HIP_CHECK(hipMemcpyAsync(host_out_.ptr, args_.scratch + args_.s_score, 8, hipMemcpyDeviceToHost, stream_));
    sync();
    out = reinterpret_cast<const float*>(host_out_.ptr);
  }
  unsigned err;
  std::memcpy(&err, out + 1, 4);
  if (err) throw Error(ST_ERR_NUMERIC, "Device watchdog tripped (error bits " + std::to_string(err) + ")");
  return out[0];
}

void Runtime::reset_device() {
  hipLaunchKernelGGL(reset_kernel, dim3(std::max(1, std::min(cus_, 1024))), dim3(256), 0, stream_, dargs_);
  HIP_CHECK(hipGetLastError());
  sync();
}

void Runtime::reset() {
  if (!running_) throw Error(ST_ERR_STATE, "Runtime is stopped");
  if (persistent()) command(kCmdReset);
  else reset_device();
}

// Runtime::stop (src/cuda/Runtime.cu:466-474): a live persistent worker gets STOP, then the
// stream is joined. Idempotent.
void Runtime::stop() {
  if (!running_) return;
  if (persistent() && !__atomic_load_n(&mailbox()->exited, __ATOMIC_ACQUIRE)) command(kCmdStop);
  sync();
  running_ = false;
}

template <int P, int A>
static void launch_persistent_t(int grid, bool plain, const StepArgs* dargs, hipStream_t stream) {
  if (grid == 1 || plain) {
    hipLaunchKernelGGL((persistent_kernel<P, A>), dim3(grid), dim3(kThreads), 0, stream, dargs);
  } else {
    void* params[] = {&dargs};
    HIP_CHECK(hipLaunchCooperativeKernel(reinterpret_cast<void*>(persistent_kernel<P, A>), dim3(grid), dim3(kThreads),
                                         params, 0, stream));
  }
  HIP_CHECK(hipGetLastError());
}

void Runtime::start_worker() {
  dispatch([&](auto P, auto A) {
    launch_persistent_t<P.value, A.value>(grid_, plain_launch_, dargs_, stream_);
    return 0;
  });
}

// The worker's epochs would pass kEpochLimit: stop it (a STOP round trip; the runtime stays
// running), rebase, and relaunch it continuing the mailbox sequence and the RUN budget. The
// device state (K/V, hidden, position) is untouched.
void Runtime::restart_worker_rebased() {
  issue(kCmdStop);
  sync();
  rebase_epochs();
  mailbox()->exited = 0;
  args_.initial_sequence = client_.sequence();
  args_.max_events = opt_.max_events ? opt_.max_events - runs_done_ : 0;
  HIP_CHECK(hipMemcpy(args_dev_.ptr, &args_, sizeof(StepArgs), hipMemcpyHostToDevice));
  start_worker();
}

// One command through the mailbox (src/cuda/Runtime.cu:398-428, docs/transport.md:9-16): the
// input and command are written before the request word is released; the worker's
// completion word is acquired before the score is read. The last sequence ID is kept for
// STOP. Every command uses one step's worth of epochs.
void Runtime::command(int cmd) {
  if (!running_) throw Error(ST_ERR_STATE, "Persistent runtime is stopped");
  try {
    client_.check(cmd);
  } catch (const MailboxError& e) {
    if (e.kind == MailboxError::kExited) {
      sync();
      running_ = false;
    }
    throw Error(ST_ERR_STATE, e.what());
  }
  // Room for this command and a later STOP; the rebase itself uses one STOP's worth.
  const uint64_t maximum = std::numeric_limits<uint64_t>::max();
  if (cmd != kCmdStop && epoch_ + 2ull * per_step() > kEpochLimit && client_.sequence() + 2 < maximum)
    restart_worker_rebased();
  issue(cmd);
  if (cmd == kCmdRun) runs_done_++;
}

void Runtime::issue(int cmd) {
  epoch_ += per_step();
  // The worker's launch has ended when its stream is idle (a HIP error there is reported).
  auto finished = [&]() {
    const hipError_t status = hipStreamQuery(stream_);
    if (status == hipErrorNotReady) return false;
    HIP_CHECK(status);
    return true;
  };
  try {
    client_.issue(cmd, opt_.backoff != 0, opt_.idle_seconds + 30, finished);
  } catch (const MailboxError& e) {
    if (e.kind == MailboxError::kExited || e.kind == MailboxError::kExitedBeforeCompletion) running_ = false;
    throw Error(e.kind == MailboxError::kWatchdog ? ST_ERR_NUMERIC : ST_ERR_STATE, e.what());
  }
}

// Snapshot (src/cuda/Runtime.cu:548-568). With a live persistent worker, the worker itself
// copies the state into mapped host memory (a SNAPSHOT command): a device-to-host copy on
// another queue would wait for the resident worker to end. Otherwise the state is copied
// after the stream has drained.
void Runtime::snapshot(uint64_t* position, float* keys, float* values, float* hidden) {
  if (persistent() && running_ && !__atomic_load_n(&mailbox()->exited, __ATOMIC_ACQUIRE)) {
    command(kCmdSnapshot);
    const unsigned char* s = reinterpret_cast<const unsigned char*>(mapped_snap_.ptr);
    const size_t n = (size_t)c_.layers * c_.width * c_.window;
    const size_t ring = snapshot_ring_bytes(c_.layers, c_.width, c_.window, prec_ == kMixed ? 2 : 4);
    if (position) std::memcpy(position, s, 8);
    auto decode = [&](const unsigned char* src, float* dst) {
      if (!dst) return;
      if (prec_ == kMixed) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(src);
        for (size_t i = 0; i < n; i++) dst[i] = host_half_to_float(h[i]);
      } else {
        std::memcpy(dst, src, n * 4);
      }
    };
    decode(s + kSnapKeys, keys);
    decode(s + kSnapKeys + ring, values);
    if (hidden) std::memcpy(hidden, s + kSnapKeys + 2 * ring, (size_t)c_.layers * c_.width * 4);
    return;
  }
  sync();
  auto copy = [&](void* dst, const void* src, size_t bytes) {
    HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, copy_stream_));
    HIP_CHECK(hipStreamSynchronize(copy_stream_));
  };
  if (position) copy(position, args_.position, 8);
  const size_t n = (size_t)c_.layers * c_.width * c_.window;
  auto download = [&](const void* src, float* dst) {
    if (!dst) return;
    if (prec_ == kMixed) {
      std::vector<uint16_t> h(n);
      copy(h.data(), src, n * 2);
      for (size_t i = 0; i < n; i++) dst[i] = host_half_to_float(h[i]);
    } else {
      copy(dst, src, n * 4);
    }
  };
  download(args_.keys, keys);
  download(args_.values, values);
  if (hidden) copy(hidden, args_.scratch + args_.s_hidden, (size_t)c_.layers * c_.width * 4);
}

template <int P, int A>
void Runtime::launch_trace_t(const float* events, int count, int stride, unsigned long long* stamps) {
  if (grid_ == 1 || plain_launch_) {
    hipLaunchKernelGGL((trace_kernel<P, A>), dim3(grid_), dim3(kThreads), 0, stream_, dargs_, events, count, stride,
                       stamps);
  } else {
    void* params[] = {&dargs_, &events, &count, &stride, &stamps};
    HIP_CHECK(hipLaunchCooperativeKernel(reinterpret_cast<void*>(trace_kernel<P, A>), dim3(grid_),
                                         dim3(kThreads), params, 0, stream_));
  }
  HIP_CHECK(hipGetLastError());
}

double Runtime::device_trace(const float* inputs, size_t count, double* per_event) {
  if (!running_) throw Error(ST_ERR_STATE, "Runtime is stopped");
  if (persistent()) throw Error(ST_ERR_INVALID, "Device traces run on launch-per-step backends, not the persistent worker");
  const int fp = args_.features_p;
  // The padded copy is staged on the host and the device: at most 4 GiB.
  if (!inputs || count == 0 || count > ((size_t)1 << 30) / (size_t)fp)
    throw Error(ST_ERR_INVALID, "Invalid trace (empty, or more than 4 GiB of padded inputs)");
  std::vector<float> padded(count * (size_t)fp, 0.f);
  for (size_t i = 0; i < count; i++)
    std::memcpy(&padded[i * fp], inputs + i * c_.features, (size_t)c_.features * 4);
  DeviceBuffer trace;
  trace.alloc(padded.size() * 4);
  HIP_CHECK(hipMemcpy(trace.ptr, padded.data(), padded.size() * 4, hipMemcpyHostToDevice));
  reset();
  if (tagged_steps()) reserve_epochs(count);
  std::vector<double> durations(count);
  double mean = 0;
  if (opt_.backend == ST_BACKEND_FUSED) {
    DeviceBuffer stamps;
    stamps.alloc((count + 1) * 8);
    const float* ev = reinterpret_cast<const float*>(trace.ptr);
    auto* st_ptr = (unsigned long long*)stamps.ptr;
    dispatch([&](auto P, auto A) { launch_trace_t<P.value, A.value>(ev, (int)count, fp, st_ptr); return 0; });
    sync();
    std::vector<unsigned long long> st(count + 1);
    HIP_CHECK(hipMemcpy(st.data(), stamps.ptr, st.size() * 8, hipMemcpyDeviceToHost));
    for (size_t i = 0; i < count; i++) durations[i] = (double)(st[i + 1] - st[i]) * 1000.0 / wall_khz_;
    mean = (double)(st[count] - st[0]) * 1000.0 / wall_khz_ / count;
  } else {
    std::vector<hipEvent_t> ev(count + 1);
    for (auto& e : ev) create_timing_event(&e);
    HIP_CHECK(hipEventRecord(ev[0], stream_));
    for (size_t i = 0; i < count; i++) {
      HIP_CHECK(hipMemcpyAsync(args_.scratch + args_.s_input, reinterpret_cast<float*>(trace.ptr) + i * fp,
                               (size_t)fp * 4, hipMemcpyDeviceToDevice, stream_));
      // A mapped graph stages host I/O inside the capture: run the compute launches instead
      // (the reference does the same, src/cuda/Runtime.cu:617-622).
      if (opt_.mapped) launch_compute();
      else launch_step();
      HIP_CHECK(hipEventRecord(ev[i + 1], stream_));
    }
    sync();
    for (size_t i = 0; i < count; i++) {
      float ms = 0;
      HIP_CHECK(hipEventElapsedTime(&ms, ev[i], ev[i + 1]));
      durations[i] = ms * 1000.0;
    }
    float total = 0;
    HIP_CHECK(hipEventElapsedTime(&total, ev[0], ev[count]));
    mean = total * 1000.0 / count;
    for (auto& e : ev) (void)hipEventDestroy(e);
  }
  check_device_error();
  if (per_event) std::copy(durations.begin(), durations.end(), per_event);
  return mean;
}

double Runtime::device_trace_noalloc(const float* device_events, size_t count, double* per_event) {
  if (!running_) throw Error(ST_ERR_STATE, "Runtime is stopped");
  if (opt_.backend != ST_BACKEND_FUSED)
    throw Error(ST_ERR_INVALID, "The allocation-free device trace runs on the fused backend only");
  if (!device_events || count == 0) throw Error(ST_ERR_INVALID, "Invalid trace (null or empty)");
  if (count > kNoAllocMaxEvents)
    throw Error(ST_ERR_INVALID, "Allocation-free device trace is limited to " + std::to_string(kNoAllocMaxEvents) +
                                    " events per call (its stamp array is fixed)");
  hipPointerAttribute_t attr{};
  if (hipPointerGetAttributes(&attr, device_events) != hipSuccess) {
    (void)hipGetLastError();  // an unknown pointer is an argument error, not a device one
    throw Error(ST_ERR_INVALID, "Events must be in device memory");
  }
  if (attr.type != hipMemoryTypeDevice) throw Error(ST_ERR_INVALID, "Events must be in device memory");
  unsigned long long* stamps = scratch_ptr_;
  // One call at a time per GPU on the shared stamp array (launch to readback).
  std::lock_guard<std::mutex> turn(trace_scratch_use(device_));
  reset();
  reserve_epochs(count);
  const int stride = c_.features;
  dispatch([&](auto P, auto A) { launch_trace_t<P.value, A.value>(device_events, (int)count, stride, stamps); return 0; });
  sync();
  check_device_error();
  // Stamps 1..count land in per_event (as 64-bit words) and become durations in place, last
  // first, so that stamp i is still unread when duration i is written.
  unsigned long long first = 0, last = 0;
  HIP_CHECK(hipMemcpy(&first, stamps, 8, hipMemcpyDeviceToHost));
  HIP_CHECK(hipMemcpy(&last, stamps + count, 8, hipMemcpyDeviceToHost));
  if (per_event) {
    static_assert(sizeof(double) == sizeof(unsigned long long), "stamps and durations share storage");
    HIP_CHECK(hipMemcpy(per_event, stamps + 1, count * 8, hipMemcpyDeviceToHost));
    unsigned long long* words = reinterpret_cast<unsigned long long*>(per_event);
    for (size_t i = count; i-- > 0;) {
      const unsigned long long hi = words[i], lo = i ? words[i - 1] : first;
      per_event[i] = (double)(hi - lo) * 1000.0 / wall_khz_;
    }
  }
  return (double)(last - first) * 1000.0 / wall_khz_ / (double)count;
}

// Per-launch device timing over a preloaded trace: one step per launch (FUSED: one
// cooperative launch reading the event in place; CUDA/GRAPH: D2D staging copy + phases),
// with a HIP event recorded on the runtime's stream after every step.
double Runtime::device_run(const float* inputs, size_t count, bool reset_first, double* per_event) {
  if (!running_) throw Error(ST_ERR_STATE, "Runtime is stopped");
  if (persistent()) throw Error(ST_ERR_INVALID, "Device runs use launch-per-step backends, not the persistent worker");
  const int fp = args_.features_p;
  // The padded copy is staged on the host and the device: at most 4 GiB.
  if (!inputs || count == 0 || count > ((size_t)1 << 30) / (size_t)fp)
    throw Error(ST_ERR_INVALID, "Invalid trace (empty, or more than 4 GiB of padded inputs)");
  std::vector<float> padded(count * (size_t)fp, 0.f);
  for (size_t i = 0; i < count; i++)
    std::memcpy(&padded[i * fp], inputs + i * c_.features, (size_t)c_.features * 4);
  DeviceBuffer trace;
  trace.alloc(padded.size() * 4);
  HIP_CHECK(hipMemcpy(trace.ptr, padded.data(), padded.size() * 4, hipMemcpyHostToDevice));
  if (reset_first) reset();
  if (tagged_steps()) reserve_epochs(count);
  std::vector<hipEvent_t> ev(count + 1);
  for (auto& e : ev) create_timing_event(&e);
  const float* base = reinterpret_cast<const float*>(trace.ptr);
  HIP_CHECK(hipEventRecord(ev[0], stream_));
  for (size_t i = 0; i < count; i++) {
    if (opt_.backend == ST_BACKEND_FUSED) {
      launch_fused(base + i * fp);
    } else {
      HIP_CHECK(hipMemcpyAsync(args_.scratch + args_.s_input, base + i * fp, (size_t)fp * 4,
                               hipMemcpyDeviceToDevice, stream_));
      if (opt_.mapped) launch_compute();
      else launch_step();
    }
    HIP_CHECK(hipEventRecord(ev[i + 1], stream_));
  }
  sync();
  double total_ms = 0;
  for (size_t i = 0; i < count; i++) {
    float ms = 0;
    HIP_CHECK(hipEventElapsedTime(&ms, ev[i], ev[i + 1]));
    if (per_event) per_event[i] = ms * 1000.0;
    total_ms += ms;
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  check_device_error();
  return total_ms * 1000.0 / count;
}

void Runtime::scheduled_run(const float* inputs, size_t count, double rate, size_t capacity, bool bursty,
                            double* intended, double* enqueue, double* submit, double* complete, float* scores,
                            uint8_t* dropped) {
  if (!inputs || !intended || !enqueue || !submit || !complete || !scores || !dropped)
    throw Error(ST_ERR_INVALID, "Null argument");
  if (count == 0 || !(rate > 0) || !std::isfinite(rate) || capacity == 0)
    throw Error(ST_ERR_INVALID, "Invalid rate, count or queue capacity");
  using clock = std::chrono::steady_clock;
  std::vector<size_t> queue(capacity);
  std::atomic<size_t> head{0}, tail{0};
  std::atomic<bool> done{false}, cancel{false};
  // The schedule starts 100 ms from now, so the producer is running before the first event.
  const auto epoch = clock::now() + std::chrono::milliseconds(100);
  auto ns_since = [&](clock::time_point t) { return std::chrono::duration<double, std::nano>(t - epoch).count(); };
  std::exception_ptr producer_error;
  std::thread producer([&] {
    try {
      for (size_t i = 0; i < count && !cancel.load(std::memory_order_relaxed); i++) {
        const double at = (double)(bursty ? (i / 16) * 16 : i) * 1e9 / rate;
        intended[i] = at;
        const auto when = epoch + std::chrono::nanoseconds((long long)at);
        while (clock::now() < when && !cancel.load(std::memory_order_relaxed)) std::this_thread::yield();
        enqueue[i] = ns_since(clock::now());
        const size_t write = tail.load(std::memory_order_relaxed);
        if (write - head.load(std::memory_order_acquire) == capacity) {
          dropped[i] = 1;
        } else {
          dropped[i] = 0;
          queue[write % capacity] = i;
          tail.store(write + 1, std::memory_order_release);
        }
      }
    } catch (...) {
      producer_error = std::current_exception();
    }
    done.store(true, std::memory_order_release);
  });
  try {
    while (true) {
      const size_t read = head.load(std::memory_order_relaxed);
      if (read == tail.load(std::memory_order_acquire)) {
        // Re-read the tail after seeing `done`, so the last queued event is not lost.
        if (done.load(std::memory_order_acquire) && read == tail.load(std::memory_order_acquire)) break;
        std::this_thread::yield();
        continue;
      }
      const size_t i = queue[read % capacity];
      head.store(read + 1, std::memory_order_release);
      submit[i] = ns_since(clock::now());
      scores[i] = step(inputs + i * (size_t)c_.features);
      complete[i] = ns_since(clock::now());
    }
  } catch (...) {
    cancel.store(true, std::memory_order_relaxed);  // a failed step ends the schedule early
    producer.join();
    throw;
  }
  producer.join();
  if (producer_error) std::rethrow_exception(producer_error);
  for (size_t i = 0; i < count; i++) {
    if (!dropped[i]) continue;
    submit[i] = std::nan("");
    complete[i] = std::nan("");
    scores[i] = std::nanf("");
  }
}

// Trace of one step (Runtime::traceStep, src/cuda/Runtime.cu:476-546), on the staged backend
// like the reference. The step runs in the phase kernels, one launch at a time, so it leaves
// exactly the state and score of an ordinary step; after each phase its output vector (x, q,
// k, v, attention, activation, hidden, score) is read back. The per-operation entries that the
// phases keep internal (".operand", ".pre_cast", ".norm", ".linear") are recomputed by the
// diagnostic kernels from the captured phase inputs.
std::vector<std::pair<std::string, size_t>> Runtime::trace_layout() const {
  const size_t d = c_.width, F = c_.ffn, f = c_.features;
  std::vector<std::pair<std::string, size_t>> l;
  auto linear = [&](const std::string& n, size_t rows, size_t cols) {
    l.push_back({n + ".operand", cols});
    l.push_back({n + ".pre_cast", rows});
    l.push_back({n + ".linear", rows});
  };
  auto norm = [&](const std::string& n) {
    l.push_back({n + ".operand", d});
    l.push_back({n + ".pre_cast", d});
    l.push_back({n + ".norm", d});
  };
  linear("input", d, f);
  l.push_back({"input", d});
  for (int layer = 0; layer < c_.layers; layer++) {
    const std::string p = "layers." + std::to_string(layer) + ".";
    norm(p + "norm1");
    linear(p + "q", d, d);
    linear(p + "k", d, d);
    linear(p + "v", d, d);
    l.push_back({p + "q", d});
    l.push_back({p + "k", d});
    l.push_back({p + "v", d});
    l.push_back({p + "attention", d});
    linear(p + "out", d, d);
    l.push_back({p + "attention_residual", d});
    norm(p + "norm2");
    linear(p + "gate", F, d);
    linear(p + "up", F, d);
    l.push_back({p + "activation", F});
    linear(p + "down", d, F);
    l.push_back({p + "hidden", d});
  }
  norm("final_norm");
  linear("score", 1, d);
  return l;
}

std::vector<std::pair<std::string, std::vector<float>>> Runtime::trace_step(const float* input) {
  if (!running_) throw Error(ST_ERR_STATE, "Runtime is stopped");
  if (opt_.backend != ST_BACKEND_CUDA) throw Error(ST_ERR_INVALID, "traceStep requires the staged backend (CUDA)");
  if (!input) throw Error(ST_ERR_INVALID, "Null input");
  const int d = c_.width, F = c_.ffn, f = c_.features;
  const StepArgs& a = args_;
  std::map<std::string, std::vector<float>> t;
  const size_t wide = (size_t)std::max({3 * d, 2 * F, f, d});
  DeviceBuffer operand, pre, out;
  operand.alloc(wide * 4);
  pre.alloc(wide * 4);
  out.alloc(wide * 4);
  float* dop = reinterpret_cast<float*>(operand.ptr);
  float* dpre = reinterpret_cast<float*>(pre.ptr);
  float* dout = reinterpret_cast<float*>(out.ptr);
  auto fetch = [&](const float* src, size_t n) {
    std::vector<float> v(n);
    HIP_CHECK(hipMemcpy(v.data(), src, n * 4, hipMemcpyDeviceToHost));
    return v;
  };
  auto tagged = [&](uint32_t off, size_t n) {
    std::vector<unsigned long long> w(n);
    HIP_CHECK(hipMemcpy(w.data(), a.tagged + off, n * 8, hipMemcpyDeviceToHost));
    std::vector<float> v(n);
    for (size_t i = 0; i < n; i++) {
      const uint32_t bits = (uint32_t)(w[i] & 0xffffffffull);
      std::memcpy(&v[i], &bits, 4);
    }
    return v;
  };
  auto run_phase = [&](int ph) {
    dispatch([&](auto P, auto A) {
      const int grid = ph == 5 * c_.layers + 1 ? 1 : phase_grid_;
      if (phase_coop_ && grid > 1) {
        const StepArgs* args = dargs_;
        void* params[] = {&args, &ph};
        HIP_CHECK(hipLaunchCooperativeKernel(reinterpret_cast<void*>(phase_kernel<P.value, A.value>), dim3(grid),
                                             dim3(kThreads), params, 0, stream_));
      } else {
        hipLaunchKernelGGL((phase_kernel<P.value, A.value>), dim3(grid), dim3(kThreads), 0, stream_, dargs_, ph);
      }
      return 0;
    });
    HIP_CHECK(hipGetLastError());
    sync();
  };
  // pre_cast / cast of one projection of `operand` (host vector) over arena rows.
  auto linear = [&](const std::string& n, const std::vector<float>& v, uint32_t woff, int ld, int first, int stride,
                    int rows, bool final) {
    t[n + ".operand"] = v;
    HIP_CHECK(hipMemcpy(dop, v.data(), v.size() * 4, hipMemcpyHostToDevice));
    dispatch([&](auto P, auto) {
      hipLaunchKernelGGL((diag_linear<P.value>), dim3((rows + 3) / 4), dim3(256), 0, stream_, a.weights, woff, ld,
                         first, stride, rows, (int)v.size(), dop, dpre, dout, final ? 1 : 0);
      return 0;
    });
    HIP_CHECK(hipGetLastError());
    sync();
    t[n + ".pre_cast"] = fetch(dpre, rows);
    t[n + ".linear"] = fetch(dout, rows);
    return t[n + ".linear"];
  };
  auto norm = [&](const std::string& n, const std::vector<float>& x, uint32_t w_norm) {
    t[n + ".operand"] = x;
    HIP_CHECK(hipMemcpy(dop, x.data(), x.size() * 4, hipMemcpyHostToDevice));
    dispatch([&](auto P, auto) {
      hipLaunchKernelGGL((diag_norm<P.value>), dim3(1), dim3(256), 0, stream_, a.weights, w_norm, d, c_.epsilon, dop,
                         dpre, dout);
      return 0;
    });
    HIP_CHECK(hipGetLastError());
    sync();
    t[n + ".pre_cast"] = fetch(dpre, d);
    t[n + ".norm"] = fetch(dout, d);
    return t[n + ".norm"];
  };

  reserve_epochs(1);
  std::memcpy(host_in_.ptr, input, (size_t)f * 4);
  HIP_CHECK(hipMemcpyAsync(a.scratch + a.s_input, host_in_.ptr, (size_t)a.features_p * 4, hipMemcpyHostToDevice,
                           stream_));
  sync();
  linear("input", std::vector<float>(input, input + f), a.w_input, a.features_p, 0, 1, d, false);
  run_phase(0);
  std::vector<float> x = tagged(a.t_x, d);
  t["input"] = x;
  for (int l = 0; l < c_.layers; l++) {
    const std::string p = "layers." + std::to_string(l) + ".";
    const LayerWeights& w = a.layer[l];
    const std::vector<float> n1 = norm(p + "norm1", x, w.norm1);
    linear(p + "q", n1, w.qkv, a.width_p, 0, 1, d, false);
    linear(p + "k", n1, w.qkv, a.width_p, d, 1, d, false);
    linear(p + "v", n1, w.qkv, a.width_p, 2 * d, 1, d, false);
    run_phase(1 + 5 * l);
    t[p + "q"] = tagged(a.t_q, d);
    t[p + "k"] = tagged(a.t_k, d);
    t[p + "v"] = tagged(a.t_v, d);
    run_phase(2 + 5 * l);
    const std::vector<float> attention = tagged(a.t_attn, d);
    t[p + "attention"] = attention;
    linear(p + "out", attention, w.out, a.width_p, 0, 1, d, false);
    run_phase(3 + 5 * l);
    x = tagged(a.t_x, d);
    t[p + "attention_residual"] = x;
    const std::vector<float> n2 = norm(p + "norm2", x, w.norm2);
    linear(p + "gate", n2, w.gateup, a.width_p, 0, 2, F, false);
    linear(p + "up", n2, w.gateup, a.width_p, 1, 2, F, false);
    run_phase(4 + 5 * l);
    const std::vector<float> act = tagged(a.t_act, F);
    t[p + "activation"] = act;
    linear(p + "down", act, w.down, a.ffn_p, 0, 1, d, false);
    run_phase(5 + 5 * l);
    x = tagged(a.t_x, d);
    t[p + "hidden"] = x;
  }
  const std::vector<float> fin = norm("final_norm", x, a.w_final_norm);
  t["score.operand"] = fin;
  run_phase(5 * c_.layers + 1);
  check_device_error();
  const std::vector<float> score = fetch(a.scratch + a.s_score, 1);
  t["score.pre_cast"] = score;  // the score has no cast
  t["score.linear"] = score;
  std::vector<std::pair<std::string, std::vector<float>>> result;
  for (const auto& [name, n] : trace_layout()) {
    auto it = t.find(name);
    if (it == t.end() || it->second.size() != n) throw Error(ST_ERR_DEVICE, "Trace entry missing: " + name);
    result.push_back({name, std::move(it->second)});
  }
  return result;
}

// One fused step with wall-clock stamps. For each phase and workgroup writes kStamps times
// in microseconds since workgroup 0 started the step (slots as in stamp()); 0 where not
// recorded; then the end of the step.
size_t Runtime::phase_times(const float* input, double* us, size_t cap) {
  if (!running_) throw Error(ST_ERR_STATE, "Runtime is stopped");
  if (opt_.backend != ST_BACKEND_FUSED) throw Error(ST_ERR_INVALID, "Phase stamps require the fused backend");
  const int nph = 5 * c_.layers + 2;
  const size_t n = (size_t)kStamps * nph * grid_ + 1;
  if (cap == 0) return n;  // size query: no step
  DeviceBuffer stamps, args;
  stamps.alloc(n * 8);
  HIP_CHECK(hipMemset(stamps.ptr, 0, n * 8));
  StepArgs prof = args_;
  prof.stamps = reinterpret_cast<unsigned long long*>(stamps.ptr);
  args.alloc(sizeof(StepArgs));
  HIP_CHECK(hipMemcpy(args.ptr, &prof, sizeof(StepArgs), hipMemcpyHostToDevice));
  reserve_epochs(1);
  std::memcpy(host_in_.ptr, input, (size_t)c_.features * 4);
  HIP_CHECK(hipMemcpyAsync(args_.scratch + args_.s_input, host_in_.ptr, (size_t)args_.features_p * 4,
                           hipMemcpyHostToDevice, stream_));
  const StepArgs* saved = dargs_;
  dargs_ = reinterpret_cast<const StepArgs*>(args.ptr);
  try {
    launch_fused();
    sync();
  } catch (...) {
    dargs_ = saved;
    throw;
  }
  dargs_ = saved;
  check_device_error();
  std::vector<unsigned long long> st(n);
  HIP_CHECK(hipMemcpy(st.data(), stamps.ptr, n * 8, hipMemcpyDeviceToHost));
  // Stamps hold the low 32 bits of the wall clock (the step is far shorter than a wrap).
  for (size_t i = 0; i < n && i < cap; i++)
    us[i] = st[i] ? (double)(int32_t)((uint32_t)st[i] - (uint32_t)st[0]) * 1000.0 / wall_khz_ : 0.0;
  return n;
}

std::string Runtime::info() {
  hipFuncAttributes fa{};
  const void* fn = nullptr;
  std::string name;
  const bool fused = opt_.backend == ST_BACKEND_FUSED, worker = persistent();
  fn = dispatch([&](auto P, auto A) {
    return worker ? (const void*)persistent_kernel<P.value, A.value>
                  : fused ? (const void*)fused_kernel<P.value, A.value> : (const void*)phase_kernel<P.value, A.value>;
  });
  name = worker ? "persistent_kernel" : fused ? "fused_kernel" : "phase_kernel";
  HIP_CHECK(hipFuncGetAttributes(&fa, fn));
  static const char* backends[] = {"cuda(staged)", "graph", "cublas", "cublas-graph", "fused", "persistent"};
  static const char* precs[] = {"fp32", "mixed", "bf16w"};
  std::ostringstream o;
  o << "{\"environment\": " << probe_ << ", \"backend\": \"" << backends[opt_.backend]
    << "\", \"precision\": \"" << precs[prec_] << "\", \"blocks\": " << grid_
    << ", \"threads\": " << kThreads << ", \"legal_cooperative_blocks\": " << legal_blocks_
    << ", \"fused_launch\": \""
    << (opt_.backend == ST_BACKEND_GRAPH ? (graph_fused_ ? "graph node (plain)" : "n/a (phase sequence)")
        : opt_.backend != ST_BACKEND_FUSED ? "n/a" : plain_launch_ || grid_ == 1 ? "plain" : "cooperative")
    << "\", \"resource_kernel\": \"" << name << "\", \"registers_per_thread\": " << fa.numRegs
    << ", \"local_bytes\": " << fa.localSizeBytes << ", \"shared_bytes\": " << fa.sharedSizeBytes
    << ", \"phases_per_step\": " << 5 * c_.layers + 2 << ", \"prefetch_slabs\": " << kPF
    << ", \"attention_chunk\": " << args_.chunk << ", \"weight_arena_bytes\": " << args_.weight_bytes
    << ", \"matvec_implementation\": \"wave64 16-byte buffer loads, register ring, butterfly reduction\""
    << ", \"weight_loads\": \"" << (weights_nt() ? "non-temporal" : "temporal") << "\""
    << ", \"attention_implementation\": \"" << (args_.attn_regs ? "register" : "LDS-staged")
    << " window chunks, tagged partials combined by the chunk-0 wave\""
    << ", \"transport\": \""
    << (worker ? "mapped-system-load-store" : opt_.mapped ? "mapped-stream-sync" : "pinned-copy-stream-sync") << "\""
    << ", \"poll_policy\": \"" << (opt_.backoff ? "bounded-device-backoff-host-yield" : "tight") << "\""
    << ", \"workspace_storage\": \"FP32 with explicit FP16 rounding in mixed mode\""
    << ", \"phase_launch\": \"" << (phase_coop_ ? "cooperative" : "plain") << "\", \"phase_blocks\": " << phase_grid_
    << ", \"weights_and_kv_storage\": \""
    << (prec_ == kMixed ? "FP16/FP16" : prec_ == kBf16w ? "BF16/FP32" : "FP32/FP32") << "\"}";
  return o.str();
}

#include "batch_runtime.hpp"

}  // namespace stamd

// ---------------------------------------------------------------------------------------------
// C ABI

struct st_runtime {
  std::unique_ptr<stamd::Runtime> impl;
};

template <class F>
static int guarded(F&& f) {
  try {
    f();
    stamd::g_last_error.clear();
    return ST_OK;
  } catch (const stamd::Error& e) {
    stamd::g_last_error = e.what();
    return e.code;
  } catch (const std::exception& e) {
    stamd::g_last_error = e.what();
    return ST_ERR_DEVICE;
  } catch (...) {
    stamd::g_last_error = "unknown error";
    return ST_ERR_DEVICE;
  }
}

namespace stamd {

// ---------------------------------------------------------------------------------------------
// Transport microbenchmarks (Stream::transportBench, src/cuda/Runtime.cu:667-814): the floors
// under a step. "ping-pong": the host releases a request through coherent pinned memory and a
// resident one-thread kernel answers with a checksum of 32 mapped floats; "gpu-ping": the
// kernel initiates and the host answers; "empty" / "empty-graph": an empty kernel launched
// (or replayed from a hipGraph) and synchronized; "copy": 128 bytes host-to-device, an echo
// kernel, 128 bytes back, synchronized and compared.

struct alignas(64) PingBox {
  alignas(64) unsigned long long request;
  alignas(64) unsigned long long completion;
  alignas(64) unsigned long long exited;
  alignas(64) unsigned long long checksum;
};

__global__ void transport_empty_kernel() {}

__global__ void transport_echo_kernel(const float* in, float* out, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = in[i];
}

// One thread; every wait ends within `idle_ticks` of the wall clock (then the kernel marks
// itself exited and returns).
__global__ void transport_ping_kernel(PingBox* box, const float* input, unsigned long long count, int backoff,
                                      unsigned long long idle_ticks, int gpu_initiated, unsigned long long* ticks,
                                      int* errors) {
  if (threadIdx.x || blockIdx.x) return;
  for (unsigned long long seq = 1; seq <= count; seq++) {
    const unsigned long long start = wall_clock64();
    if (gpu_initiated) {
      __hip_atomic_store(&box->checksum, seq * 2654435761ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(&box->request, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
      while (__hip_atomic_load(&box->completion, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) != seq) {
        if (wall_clock64() - start > idle_ticks) {
          __hip_atomic_store(&box->exited, 1ull, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
          return;
        }
        if (backoff) __builtin_amdgcn_s_sleep(8);
      }
      if (__hip_atomic_load(&box->checksum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) != ((seq * 2654435761ull) ^ 0xabcdefull))
        (*errors)++;
    } else {
      while (__hip_atomic_load(&box->request, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) != seq) {
        if (wall_clock64() - start > idle_ticks) {
          __hip_atomic_store(&box->exited, 1ull, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
          return;
        }
        if (backoff) __builtin_amdgcn_s_sleep(8);
      }
      unsigned long long sum = 0;
      for (int i = 0; i < 32; i++) sum += __builtin_bit_cast(unsigned, input[i]);
      __hip_atomic_store(&box->checksum, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(&box->completion, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    ticks[seq - 1] = wall_clock64() - start;
  }
  __hip_atomic_store(&box->exited, 1ull, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

std::string transport_bench(const std::string& mode, uint64_t count, bool backoff, const char* csv_path) {
  const bool interactive = mode == "ping-pong" || mode == "gpu-ping";
  if (!interactive && mode != "empty" && mode != "empty-graph" && mode != "copy")
    throw Error(ST_ERR_INVALID, "Unknown transport mode: " + mode);
  if (count == 0 || count > (1ull << 24)) throw Error(ST_ERR_INVALID, "Transport count must be 1 .. 2^24");
  const std::string environment = probe_json();
  int device = 0, wall_khz = 100000;
  HIP_CHECK(hipGetDevice(&device));
  HIP_CHECK(hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, device));
  // Buffers first: the stream guard below is destroyed before them, so a kernel still
  // running when an error unwinds is joined before its memory is freed.
  MappedBuffer box_buf, in_buf;
  box_buf.alloc(sizeof(PingBox));
  in_buf.alloc(32 * 4);
  PingBox* box = reinterpret_cast<PingBox*>(box_buf.ptr);
  float* input = reinterpret_cast<float*>(in_buf.ptr);
  PinnedBuffer host_in, host_out;
  host_in.alloc(128);
  host_out.alloc(128);
  DeviceBuffer d_in, d_out, d_ticks, d_errors;
  d_in.alloc(128);
  d_out.alloc(128);
  d_ticks.alloc(count * 8);
  d_errors.alloc(4);
  HIP_CHECK(hipMemset(d_errors.ptr, 0, 4));
  HIP_CHECK(hipMemset(d_ticks.ptr, 0, count * 8));
  hipStream_t stream;
  HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  struct StreamGuard {
    hipStream_t s;
    hipGraph_t g = nullptr;
    hipGraphExec_t e = nullptr;
    ~StreamGuard() {
      (void)hipStreamSynchronize(s);
      if (e) (void)hipGraphExecDestroy(e);
      if (g) (void)hipGraphDestroy(g);
      (void)hipStreamDestroy(s);
    }
  } guard{stream};
  if (mode == "empty-graph") {
    HIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    hipLaunchKernelGGL(transport_empty_kernel, dim3(1), dim3(1), 0, stream);
    HIP_CHECK(hipStreamEndCapture(stream, &guard.g));
    HIP_CHECK(hipGraphInstantiate(&guard.e, guard.g, nullptr, nullptr, 0));
  }
  if (interactive) {
    const unsigned long long idle = (unsigned long long)wall_khz * 1000ull * 30ull;  // 30 s per wait
    hipLaunchKernelGGL(transport_ping_kernel, dim3(1), dim3(1), 0, stream, reinterpret_cast<PingBox*>(box_buf.dev),
                       reinterpret_cast<const float*>(in_buf.dev), (unsigned long long)count, backoff ? 1 : 0, idle,
                       mode == "gpu-ping" ? 1 : 0, reinterpret_cast<unsigned long long*>(d_ticks.ptr),
                       reinterpret_cast<int*>(d_errors.ptr));
    HIP_CHECK(hipGetLastError());
  }
  auto wait = [&](unsigned long long* word, unsigned long long seq) {
    const auto start = std::chrono::steady_clock::now();
    uint64_t polls = 0;
    while (__atomic_load_n(word, __ATOMIC_ACQUIRE) != seq) {
      if (backoff) std::this_thread::yield();
      if ((++polls & 0xffff) == 0) {
        if (__atomic_load_n(&box->exited, __ATOMIC_ACQUIRE))
          throw Error(ST_ERR_STATE, "Ping kernel exited before the request or acknowledgement");
        if (std::chrono::steady_clock::now() - start > std::chrono::seconds(60))
          throw Error(ST_ERR_STATE, "Ping host timeout");
      }
    }
  };
  std::vector<double> samples(count);
  uint64_t failed = 0;
  const auto begin = std::chrono::steady_clock::now();
  float* hin = reinterpret_cast<float*>(host_in.ptr);
  for (uint64_t seq = 1; seq <= count; seq++) {
    unsigned long long checksum = 0;
    for (int i = 0; i < 32; i++) {
      const float v = (float)(seq % 1024 + i);
      input[i] = v;
      hin[i] = v;
      uint32_t bits;
      std::memcpy(&bits, &v, 4);
      checksum += bits;
    }
    const auto start = std::chrono::steady_clock::now();
    if (mode == "gpu-ping") {
      wait(&box->request, seq);
      const unsigned long long got = __atomic_load_n(&box->checksum, __ATOMIC_RELAXED);
      if (got != seq * 2654435761ull) failed++;
      __atomic_store_n(&box->checksum, got ^ 0xabcdefull, __ATOMIC_RELAXED);
      __atomic_store_n(&box->completion, seq, __ATOMIC_RELEASE);
    } else if (mode == "ping-pong") {
      __atomic_store_n(&box->request, seq, __ATOMIC_RELEASE);
      wait(&box->completion, seq);
      if (__atomic_load_n(&box->checksum, __ATOMIC_RELAXED) != checksum) failed++;
    } else {
      if (mode == "empty") {
        hipLaunchKernelGGL(transport_empty_kernel, dim3(1), dim3(1), 0, stream);
      } else if (mode == "empty-graph") {
        HIP_CHECK(hipGraphLaunch(guard.e, stream));
      } else {
        HIP_CHECK(hipMemcpyAsync(d_in.ptr, host_in.ptr, 128, hipMemcpyHostToDevice, stream));
        hipLaunchKernelGGL(transport_echo_kernel, dim3(1), dim3(32), 0, stream, reinterpret_cast<const float*>(d_in.ptr),
                           reinterpret_cast<float*>(d_out.ptr), 32);
        HIP_CHECK(hipMemcpyAsync(host_out.ptr, d_out.ptr, 128, hipMemcpyDeviceToHost, stream));
      }
      HIP_CHECK(hipGetLastError());
      HIP_CHECK(hipStreamSynchronize(stream));
      if (mode == "copy" && std::memcmp(host_out.ptr, host_in.ptr, 128)) failed++;
    }
    samples[seq - 1] = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - start).count();
  }
  HIP_CHECK(hipStreamSynchronize(stream));
  const double wall = std::chrono::duration<double>(std::chrono::steady_clock::now() - begin).count();
  std::vector<unsigned long long> ticks(count, 0);
  if (interactive) {
    HIP_CHECK(hipMemcpy(ticks.data(), d_ticks.ptr, count * 8, hipMemcpyDeviceToHost));
    int errors = 0;
    HIP_CHECK(hipMemcpy(&errors, d_errors.ptr, 4, hipMemcpyDeviceToHost));
    failed += (uint64_t)errors;
  }
  if (csv_path && *csv_path) {
    FILE* f = std::fopen(csv_path, "w");
    if (!f) throw Error(ST_ERR_INVALID, std::string("Cannot write ") + csv_path);
    // The reference's columns (src/cuda/Runtime.cu:803-805). The device column counts ticks of
    // the constant wall clock (its rate is "wall_clock_khz" of the environment report).
    std::fprintf(f, "sequence,host_observation_us,device_round_trip_or_wait_cycles\n");
    for (uint64_t i = 0; i < count; i++)
      std::fprintf(f, "%llu,%.17g,%llu\n", (unsigned long long)(i + 1), samples[i], (unsigned long long)ticks[i]);
    std::fclose(f);
  }
  std::vector<double> sorted = samples;
  std::sort(sorted.begin(), sorted.end());
  const double p50 = sorted[count / 2], p99 = sorted[std::min<size_t>(count - 1, (size_t)(count * 0.99))];
  std::ostringstream o;
  o.precision(17);
  o << "{\"environment\": " << environment << ", \"mode\": \"" << mode << "\", \"events\": " << count
    << ", \"failed\": " << failed << ", \"poll_policy\": \"" << (backoff ? "device-sleep-host-yield" : "tight")
    << "\", \"wall_seconds\": " << wall << ", \"p50_us\": " << p50 << ", \"p99_us\": " << p99
    << ", \"worst_us\": " << sorted.back() << ", \"boundary\": \""
    << (mode == "gpu-ping" ? "host wait+ack service observation; device round trip in the CSV"
                           : "host submission through the corresponding host-visible completion")
    << "\"}";
  if (failed) throw Error(ST_ERR_NUMERIC, "Transport checksum failure");
  return o.str();
}

}  // namespace stamd

static int write_string(const std::string& s, char* buffer, size_t cap, size_t* needed) {
  if (needed) *needed = s.size() + 1;
  if (buffer && cap) {
    size_t n = std::min(cap - 1, s.size());
    std::memcpy(buffer, s.data(), n);
    buffer[n] = 0;
  }
  return ST_OK;
}

extern "C" {

void st_options_default(st_options* o) {
  if (!o) return;
  std::memset(o, 0, sizeof(*o));
  o->backend = ST_BACKEND_GRAPH;
  o->blocks = 1;
  o->idle_seconds = 30;
}

int st_runtime_create(const st_config* config, int32_t mixed, const st_tensor* tensors, size_t count,
                      const st_options* options, st_runtime** out) {
  return guarded([&] {
    if (!config || !tensors || !out) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    *out = nullptr;
    st_options o;
    if (options) o = *options;
    else st_options_default(&o);
    auto r = std::make_unique<st_runtime>();
    r->impl = std::make_unique<stamd::Runtime>(*config, mixed != 0, tensors, count, o);
    *out = r.release();
  });
}

void st_runtime_destroy(st_runtime* r) {
  if (!r) return;
  try {
    r->impl.reset();
  } catch (...) {
  }
  delete r;
}

int st_runtime_step(st_runtime* r, const float* input, float* score) {
  return guarded([&] {
    if (!r || !score) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    *score = r->impl->step(input);
  });
}

int st_runtime_reset(st_runtime* r) {
  return guarded([&] {
    if (!r) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    r->impl->reset();
  });
}

int st_runtime_stop(st_runtime* r) {
  return guarded([&] {
    if (!r) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    r->impl->stop();
  });
}

int st_runtime_snapshot(st_runtime* r, uint64_t* position, float* keys, float* values, float* hidden) {
  return guarded([&] {
    if (!r) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    r->impl->snapshot(position, keys, values, hidden);
  });
}

int st_runtime_device_trace(st_runtime* r, const float* inputs, size_t count, double* us_per_event,
                            double* per_event_us) {
  return guarded([&] {
    if (!r || !us_per_event) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    *us_per_event = r->impl->device_trace(inputs, count, per_event_us);
  });
}

int st_runtime_device_trace_noalloc(st_runtime* r, const float* device_events, size_t count, double* us_per_event,
                                    double* per_event_us) {
  return guarded([&] {
    if (!r || !us_per_event) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    *us_per_event = r->impl->device_trace_noalloc(device_events, count, per_event_us);
  });
}

int st_runtime_device_run(st_runtime* r, const float* inputs, size_t count, int32_t reset,
                          double* us_per_event, double* per_event_us) {
  return guarded([&] {
    if (!r || !us_per_event) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    *us_per_event = r->impl->device_run(inputs, count, reset != 0, per_event_us);
  });
}

int st_runtime_phase_times(st_runtime* r, const float* input, double* us, size_t cap, size_t* count) {
  return guarded([&] {
    if (!r || !input || (!us && cap)) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    size_t n = r->impl->phase_times(input, us, cap);
    if (count) *count = n;
  });
}

int st_runtime_trace_step(st_runtime* r, const float* input, char* names, size_t names_cap, size_t* names_needed,
                          float* values, size_t values_cap, size_t* values_count) {
  return guarded([&] {
    if (!r || (!names && names_cap) || (!values && values_cap)) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    const auto layout = r->impl->trace_layout();
    std::ostringstream o;
    size_t total = 0;
    o << "{";
    for (size_t i = 0; i < layout.size(); i++) {
      o << (i ? ", " : "") << "\"" << layout[i].first << "\": [" << total << ", " << layout[i].second << "]";
      total += layout[i].second;
    }
    o << "}";
    if (values_count) *values_count = total;
    if (names_cap == 0 && values_cap == 0) {  // size query: no step
      write_string(o.str(), nullptr, 0, names_needed);
      return;
    }
    if (!input) throw stamd::Error(ST_ERR_INVALID, "Null input");
    if (values_cap < total) throw stamd::Error(ST_ERR_INVALID, "Trace value buffer too small");
    const auto trace = r->impl->trace_step(input);
    size_t off = 0;
    for (const auto& [name, v] : trace) {
      std::memcpy(values + off, v.data(), v.size() * 4);
      off += v.size();
    }
    write_string(o.str(), names, names_cap, names_needed);
  });
}

int st_transport_bench(const char* mode, uint64_t count, int32_t backoff, const char* csv_path, char* report,
                       size_t cap, size_t* needed) {
  return guarded([&] {
    if (!mode) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    write_string(stamd::transport_bench(mode, count, backoff != 0, csv_path), report, cap, needed);
  });
}

int st_runtime_scheduled_run(st_runtime* r, const float* inputs, size_t count, double rate_per_second,
                             size_t queue_capacity, int32_t bursty, double* intended_ns, double* enqueue_ns,
                             double* submit_ns, double* complete_ns, float* scores, uint8_t* dropped) {
  return guarded([&] {
    if (!r) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    r->impl->scheduled_run(inputs, count, rate_per_second, queue_capacity, bursty != 0, intended_ns, enqueue_ns,
                           submit_ns, complete_ns, scores, dropped);
  });
}

int st_runtime_info_json(st_runtime* r, char* buffer, size_t cap, size_t* needed) {
  return guarded([&] {
    if (!r) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    write_string(r->impl->info(), buffer, cap, needed);
  });
}

int st_probe_json(char* buffer, size_t cap, size_t* needed) {
  return guarded([&] { write_string(stamd::probe_json(), buffer, cap, needed); });
}

// ---- batched independent streams (extension)

struct st_batch {
  std::unique_ptr<stamd::BatchBase> impl;
};

int st_batch_create(const st_config* config, int32_t mixed, const st_tensor* tensors, size_t count, int32_t streams,
                    int32_t weight_dtype, st_batch** out) {
  return guarded([&] {
    if (!config || !tensors || !out) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    *out = nullptr;
    auto r = std::make_unique<st_batch>();
    r->impl = std::make_unique<stamd::Batch>(*config, mixed != 0, tensors, count, streams, weight_dtype);
    *out = r.release();
  });
}

int st_batch_create_resident(const st_config* config, int32_t mixed, const st_tensor* tensors, size_t count,
                             int32_t streams, int32_t weight_dtype, st_batch** out) {
  return guarded([&] {
    if (!config || !tensors || !out) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    *out = nullptr;
    auto r = std::make_unique<st_batch>();
    r->impl = std::make_unique<stamd::ResidentBatch>(*config, mixed != 0, tensors, count, streams, weight_dtype);
    *out = r.release();
  });
}

void st_batch_destroy(st_batch* r) {
  if (!r) return;
  try {
    r->impl.reset();
  } catch (...) {
  }
  delete r;
}

int st_batch_step(st_batch* r, const float* inputs, float* scores) {
  return guarded([&] {
    if (!r) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    r->impl->step(inputs, scores);
  });
}

int st_batch_reset(st_batch* r, int32_t stream) {
  return guarded([&] {
    if (!r) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    r->impl->reset(stream);
  });
}

int st_batch_snapshot(st_batch* r, int32_t stream, uint64_t* position, float* keys, float* values, float* hidden) {
  return guarded([&] {
    if (!r) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    r->impl->snapshot(stream, position, keys, values, hidden);
  });
}

int st_batch_device_run(st_batch* r, const float* inputs, size_t count, double* us_per_step, double* per_step_us) {
  return guarded([&] {
    if (!r || !us_per_step) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    *us_per_step = r->impl->device_run(inputs, count, per_step_us);
  });
}

int st_batch_set_eager(st_batch* r, int32_t eager) {
  return guarded([&] {
    if (!r) throw stamd::Error(ST_ERR_INVALID, "Null argument");
    if (eager != 0 && eager != 1) throw stamd::Error(ST_ERR_INVALID, "eager must be 0 or 1");
    r->impl->set_eager(eager != 0);
  });
}

const char* st_last_error(void) { return stamd::g_last_error.c_str(); }

}  // extern "C"
