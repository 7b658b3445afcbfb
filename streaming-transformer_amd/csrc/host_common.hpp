// Host-side pieces shared by the library's two translation units (runtime.hip: the
// single-stream runtime, the resident batches and the C ABI; batch.hip: the batched phase
// kernels and their host sequence): the error type, buffers, host-side FP16/bfloat16
// rounding, configuration checks and the weight arena's builder.
#pragma once

#include "step_device.hpp"
#include "../../include/st_runtime.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

namespace stamd {

struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define HIP_CHECK(expr)                                                                    \
  do {                                                                                     \
    hipError_t _e = (expr);                                                                \
    if (_e != hipSuccess)                                                                  \
      throw Error(ST_ERR_DEVICE, std::string(#expr) + ": " + hipGetErrorString(_e));       \
  } while (0)

// Events that only time device work between launches. Recorded without the system-scope
// fence (an L2 writeback and invalidation before every record), so consecutive steps run as they
// would untimed; the host reads results only after synchronizing the stream, which releases at
// system scope. Measured on Large FP32: 305.0 -> 303.1 us per step.
inline void create_timing_event(hipEvent_t* e) { HIP_CHECK(hipEventCreateWithFlags(e, hipEventDisableSystemFence)); }

// ---------------------------------------------------------------------------------------------
// host-side rounding (round to nearest even), matching the device conversions

inline uint16_t host_half_bits(float value) {
  uint32_t u;
  std::memcpy(&u, &value, 4);
  uint32_t sign = (u >> 16) & 0x8000u, exp = (u >> 23) & 0xffu, man = u & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    uint32_t full = man | 0x800000u;
    int shift = 14 - e;
    uint32_t half = full >> shift, rem = full & ((1u << shift) - 1u), mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1u))) half++;
    return (uint16_t)(sign | half);
  }
  uint32_t half = ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
  return (uint16_t)(sign | half);
}

inline float host_half_to_float(uint16_t bits) {
  uint32_t sign = ((uint32_t)bits & 0x8000u) << 16, exp = (bits >> 10) & 0x1fu, man = bits & 0x3ffu;
  uint32_t u;
  if (exp == 0x1fu) u = sign | 0x7f800000u | (man << 13);
  else if (exp == 0) {
    if (!man) u = sign;
    else {
      float f = (float)man * 5.9604644775390625e-8f;
      return sign ? -f : f;
    }
  } else u = sign | ((exp + 112u) << 23) | (man << 13);
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

inline uint16_t host_bf16_bits(float value) {
  uint32_t u;
  std::memcpy(&u, &value, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

inline int round_up(int v, int m) { return (v + m - 1) / m * m; }

// ---------------------------------------------------------------------------------------------

struct DeviceBuffer {
  void* ptr = nullptr;
  size_t bytes = 0;
  void alloc(size_t n) {
    bytes = n;
    HIP_CHECK(hipMalloc(&ptr, std::max<size_t>(n, 256)));
  }
  ~DeviceBuffer() {
    if (ptr) (void)hipFree(ptr);
  }
};

struct PinnedBuffer {
  void* ptr = nullptr;
  void alloc(size_t n) { HIP_CHECK(hipHostMalloc(&ptr, std::max<size_t>(n, 64), hipHostMallocDefault)); }
  ~PinnedBuffer() {
    if (ptr) (void)hipHostFree(ptr);
  }
};

// Coherent pinned host memory mapped into the device's address space (the persistent
// backend's mailbox and event buffer).
struct MappedBuffer {
  void* ptr = nullptr;
  void* dev = nullptr;
  void alloc(size_t n) {
    HIP_CHECK(hipHostMalloc(&ptr, std::max<size_t>(n, 64), hipHostMallocMapped | hipHostMallocCoherent));
    std::memset(ptr, 0, std::max<size_t>(n, 64));
    HIP_CHECK(hipHostGetDevicePointer(&dev, ptr, 0));
  }
  ~MappedBuffer() {
    if (ptr) (void)hipHostFree(ptr);
  }
};

// Owning stream and graph handles, so that a constructor that throws after creating them
// (an invalid checkpoint, a failed capture) still releases them. A stream is drained before it
// is destroyed. Declared in the order stream, graph, executable, they are destroyed in reverse.
struct StreamHandle {
  hipStream_t s = nullptr;
  StreamHandle() = default;
  StreamHandle(const StreamHandle&) = delete;
  StreamHandle& operator=(const StreamHandle&) = delete;
  void create() { HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking)); }
  operator hipStream_t() const { return s; }
  ~StreamHandle() {
    if (s) {
      (void)hipStreamSynchronize(s);
      (void)hipStreamDestroy(s);
    }
  }
};

struct GraphHandle {
  hipGraph_t g = nullptr;
  GraphHandle() = default;
  GraphHandle(const GraphHandle&) = delete;
  GraphHandle& operator=(const GraphHandle&) = delete;
  operator hipGraph_t() const { return g; }
  ~GraphHandle() {
    if (g) (void)hipGraphDestroy(g);
  }
};

struct GraphExecHandle {
  hipGraphExec_t e = nullptr;
  GraphExecHandle() = default;
  GraphExecHandle(const GraphExecHandle&) = delete;
  GraphExecHandle& operator=(const GraphExecHandle&) = delete;
  void instantiate(hipGraph_t g) { HIP_CHECK(hipGraphInstantiate(&e, g, nullptr, nullptr, 0)); }
  operator hipGraphExec_t() const { return e; }
  ~GraphExecHandle() {
    if (e) (void)hipGraphExecDestroy(e);
  }
};

inline void validate_config(const st_config& c) {
  if (c.layers < 1 || c.layers > 16 || c.width < 1 || c.width > 1024 || c.heads < 1 ||
      c.width % c.heads || (c.width / c.heads) % 2 || c.ffn < 1 || c.ffn > 4096 || c.window < 1 ||
      c.window > 4096 || c.features < 1 || c.features > 1024 || !std::isfinite(c.epsilon) ||
      c.epsilon <= 0)
    throw Error(ST_ERR_INVALID, "Invalid or unsupported model dimensions");
}

// The weight arena (defined in runtime.hip). `tiled`: the projection matrices in MFMA operand
// order, for the batched runtime.
void build_arena(const st_config& c_, int prec_, const st_tensor* tensors, size_t count, StepArgs& args_,
                 DeviceBuffer& weights_, bool tiled = false);

}  // namespace stamd
