// Diagnostic kernels of the per-operation trace (Runtime::traceStep, src/cuda/Runtime.cu:
// 476-546). The step itself runs in the staged backend's phase kernels; these kernels only
// recompute the per-operation values the phases keep internal (a norm's output before and
// after its cast, a projection's output before and after its cast) from the phase inputs
// the trace captured, for a reader who wants to see where two runs part. They write only
// their own output buffers, never the stream state.
#pragma once

#include "step_device.hpp"

namespace stamd {

// Element i of a weight row or vector in the arena, decoded to FP32.
template <int P>
__device__ __forceinline__ float diag_weight(const char* w, size_t element) {
  if constexpr (P == kFp32) return reinterpret_cast<const float*>(w)[element];
  if constexpr (P == kMixed) return half_to_float(reinterpret_cast<const uint16_t*>(w)[element]);
  return bf16_to_float(reinterpret_cast<const uint16_t*>(w)[element]);
}

// RMSNorm (src/cuda/Primitives.cuh:122-135): pre[i] = x[i] s g[i] with s = 1/sqrt(sum x^2 / d
// + eps), out = cast(pre). One workgroup of 256 threads.
template <int P>
__global__ __launch_bounds__(256) void diag_norm(const char* weights, uint32_t w_norm, int width, float epsilon,
                                                 const float* x, float* pre, float* out) {
  __shared__ float red[4];
  float s = 0.f;
  for (int i = threadIdx.x; i < width; i += blockDim.x) s += x[i] * x[i];
  s = wave_total(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  const float sum = (red[0] + red[1]) + (red[2] + red[3]);
  const float scale = 1.0f / sqrtf(sum / (float)width + epsilon);
  for (int i = threadIdx.x; i < width; i += blockDim.x) {
    const float v = x[i] * scale * diag_weight<P>(weights + w_norm, i);
    pre[i] = v;
    out[i] = cast<P>(v);
  }
}

// Projection (src/cuda/Primitives.cuh:100-120): pre[r] = sum_c W[first + r * stride][c] v[c]
// over `cols` columns of rows `ld` elements apart, out = pre if final else cast(pre). One wave
// per output row, four rows per workgroup of 256 threads.
template <int P>
__global__ __launch_bounds__(256) void diag_linear(const char* weights, uint32_t woff, int ld, int first, int stride,
                                                   int rows, int cols, const float* v, float* pre, float* out,
                                                   int final) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;  // uniform over the wave
  const size_t base = (size_t)(first + row * stride) * (size_t)ld;
  float s = 0.f;
  for (int c = lane; c < cols; c += 64) s += diag_weight<P>(weights + woff, base + c) * v[c];
  s = wave_total(s);
  if (lane == 0) {
    pre[row] = s;
    out[row] = final ? s : cast<P>(s);
  }
}

}  // namespace stamd
