// Batched independent streams on gfx950: B streams share the weights and each keeps its own
// K/V ring, hidden state and position. One step advances every stream by one event. The
// projections become skinny GEMMs [B x K] . W^T computed with MFMA (v_mfma_f32_16x16x4_f32:
// FP32 operands, FP32 accumulation; bfloat16 weights are widened exactly), split over K
// across workgroups so that small batches still spread the weight stream over the chip. A
// reduce kernel per projection adds the K-slices in a fixed order and applies the phase's
// epilogue (RoPE and ring write, residual, SwiGLU). Activations, K/V and reductions are FP32,
// so each stream follows the single-stream runtime's arithmetic up to summation order.
#pragma once

#include "step_device.hpp"

namespace stamd {

constexpr int kBatchMax = 256;   // streams per batch (16 batch tiles of 16 in the GEMM)
constexpr int kBatchTile = 16;   // MFMA rows

typedef float f4v __attribute__((ext_vector_type(4)));

struct BatchArgs {
  int streams, streams_p;  // B and B rounded up to 16
  int layers, width, heads, dim, ffn, window, features;
  int width_p, ffn_p, features_p, xcols;  // padded row lengths; xcols = widest GEMM input
  float epsilon;
  const char* weights;
  uint32_t w_input, w_final_norm, w_score;
  LayerWeights layer[kMaxLayers];
  const float* rope_freq;          // [dim / 2]
  float* keys;                     // [B][L][H][W][dh]
  float* values;
  float* hidden;                   // [B][L][d]
  unsigned long long* position;    // [B]
  float* in;                       // [Bp][features_p] events
  float* x;                        // [Bp][width_p] residual stream
  float* xn;                       // [Bp][xcols] normalized x, then the GEMM input
  float* attn;                     // [Bp][width_p] attention output
  float* act;                      // [Bp][ffn_p] SwiGLU output
  float* q;                        // [Bp][width] rotated queries
  float* part;                     // split-K partial sums [ks][Bp][N]
  float* score;                    // [B]
};

// Four consecutive weights of row `row` from column `k` (FP32 or bfloat16 storage).
template <int P>
__device__ __forceinline__ float4 load_w4(const char* w, uint32_t woff, int row, int ldw, int k) {
  const uint32_t e = (uint32_t)row * (uint32_t)ldw + (uint32_t)k;
  if constexpr (P == kFp32) {
    return *reinterpret_cast<const float4*>(w + woff + e * 4u);
  } else {
    const uint2 u = *reinterpret_cast<const uint2*>(w + woff + e * 2u);
    return make_float4(__builtin_bit_cast(float, u.x << 16), __builtin_bit_cast(float, u.x & 0xffff0000u),
                       __builtin_bit_cast(float, u.y << 16), __builtin_bit_cast(float, u.y & 0xffff0000u));
  }
}

// part[ks][b][n] = sum over k in K-slice ks of X[b][k] * W[n][k], for the 16 columns of this
// workgroup and every batch tile. One wave per workgroup; grid (N / 16, slices).
// MFMA 16x16x4 layout: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16]; register r
// of lane l holds D[4 (l / 16) + r][l % 16]. The four MFMA steps of a 16-wide k block use
// k = kb + 4 (l / 16) + c for step c, the same index for A and B.
template <int P>
__global__ __launch_bounds__(64) void batch_gemm(const BatchArgs* __restrict__ ap, const float* __restrict__ X, int ldx,
                                                 uint32_t woff, int ldw, int N, int K, int kc,
                                                 float* __restrict__ part) {
  const BatchArgs& a = *ap;
  const int lane = threadIdx.x;
  const int n0 = blockIdx.x * kBatchTile;
  const int ks = blockIdx.y;
  const int k0 = ks * kc;
  const int k1 = k0 + kc < K ? k0 + kc : K;
  const int tiles = a.streams_p / kBatchTile;
  const int r16 = lane & 15, g = lane >> 4;
  f4v acc[kBatchMax / kBatchTile];
#pragma unroll
  for (int t = 0; t < kBatchMax / kBatchTile; t++) acc[t] = f4v{0.f, 0.f, 0.f, 0.f};
  for (int kb = k0; kb < k1; kb += 16) {
    const float4 w = load_w4<P>(a.weights, woff, n0 + r16, ldw, kb + 4 * g);
#pragma unroll
    for (int t = 0; t < kBatchMax / kBatchTile; t++) {
      if (t < tiles) {
        const float4 xv = *reinterpret_cast<const float4*>(X + (size_t)(t * kBatchTile + r16) * ldx + kb + 4 * g);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.x, w.x, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.y, w.y, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.z, w.z, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv.w, w.w, acc[t], 0, 0, 0);
      }
    }
  }
  float* out = part + (size_t)ks * a.streams_p * N;
#pragma unroll
  for (int t = 0; t < kBatchMax / kBatchTile; t++)
    if (t < tiles)
#pragma unroll
      for (int r = 0; r < 4; r++) out[(size_t)(t * kBatchTile + 4 * g + r) * N + n0 + r16] = acc[t][r];
}

// Sum of the K-slices of output (b, n), in slice order.
__device__ __forceinline__ float slice_sum(const float* part, int slices, int rows, int N, int b, int n) {
  float s = part[(size_t)b * N + n];
  for (int ks = 1; ks < slices; ks++) s += part[((size_t)ks * rows + b) * N + n];
  return s;
}

enum BatchEpilogue : int { kEpInput = 0, kEpQkv, kEpOut, kEpGateUp, kEpDown };

// Reduce the K-slices of one projection and apply its epilogue; one thread per output unit
// (a row, or the row pair of a RoPE pair / gate-up pair) of a stream below B.
template <int E>
__global__ __launch_bounds__(256) void batch_reduce(const BatchArgs* __restrict__ ap, int layer, int N, int slices) {
  const BatchArgs& a = *ap;
  const int unit = (E == kEpQkv || E == kEpGateUp) ? 2 : 1;
  const int units = N / unit;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.streams * units) return;
  const int b = idx / units, u = idx - b * units;
  const int n = u * unit;
  const float s0 = slice_sum(a.part, slices, a.streams_p, N, b, n);
  const float s1 = unit == 2 ? slice_sum(a.part, slices, a.streams_p, N, b, n + 1) : 0.f;
  float* xb = a.x + (size_t)b * a.width_p;
  if constexpr (E == kEpInput) {
    xb[n] = s0;
  } else if constexpr (E == kEpQkv) {
    // src/cuda/Primitives.cuh:148-166: RoPE on adjacent pairs of q and k, then the ring write.
    const int sec = (n >= a.width) + (n >= 2 * a.width);
    const int i = n - sec * a.width;
    const unsigned long long t = a.position[b];
    float va = s0, vb = s1;
    if (sec < 2) {
      const int e = i % a.dim;
      const float angle = (float)t * a.rope_freq[e >> 1];
      const float co = cosf(angle), si = sinf(angle);
      const float ra = va * co - vb * si, rb = va * si + vb * co;
      va = ra;
      vb = rb;
    }
    if (sec == 0) {
      a.q[(size_t)b * a.width + i] = va;
      a.q[(size_t)b * a.width + i + 1] = vb;
    } else {
      const int h = i / a.dim, d = i - h * a.dim;
      const int slot = (int)(t % (unsigned long long)a.window);
      const size_t ring = ((((size_t)b * a.layers + layer) * a.heads + h) * a.window + slot) * a.dim + d;
      float* dst = sec == 1 ? a.keys : a.values;
      dst[ring] = va;
      dst[ring + 1] = vb;
    }
  } else if constexpr (E == kEpOut) {
    xb[n] = xb[n] + s0;
  } else if constexpr (E == kEpGateUp) {
    a.act[(size_t)b * a.ffn_p + u] = (s0 / (1.0f + expf(-s0))) * s1;
  } else {
    const float v = xb[n] + s0;
    xb[n] = v;
    a.hidden[((size_t)b * a.layers + layer) * a.width + n] = v;
  }
}

// RMSNorm of every stream's x into xn (src/cuda/Primitives.cuh:122-135); padding columns and
// padding streams are zero. One workgroup per row of the padded batch.
template <int P>
__global__ __launch_bounds__(256) void batch_norm(const BatchArgs* __restrict__ ap, uint32_t w_norm) {
  const BatchArgs& a = *ap;
  __shared__ float red[4];
  const int b = blockIdx.x;
  const float* xb = a.x + (size_t)b * a.width_p;
  float* out = a.xn + (size_t)b * a.xcols;
  if (b >= a.streams) {
    for (int i = threadIdx.x; i < a.width_p; i += blockDim.x) out[i] = 0.f;
    return;
  }
  float s = 0.f;
  for (int i = threadIdx.x; i < a.width; i += blockDim.x) s += xb[i] * xb[i];
  s = wave_total(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  const float sum = (red[0] + red[1]) + (red[2] + red[3]);
  const float scale = 1.0f / sqrtf(sum / (float)a.width + a.epsilon);
  for (int i = threadIdx.x; i < a.width_p; i += blockDim.x) {
    float v = 0.f;
    if (i < a.width) {
      const float w = P == kFp32 ? reinterpret_cast<const float*>(a.weights + w_norm)[i]
                                 : __builtin_bit_cast(float, (unsigned)reinterpret_cast<const unsigned short*>(a.weights + w_norm)[i] << 16);
      v = xb[i] * scale * w;
    }
    out[i] = v;
  }
}

// Attention of one (stream, head) over the stream's valid ring slots [0, valid)
// (src/cuda/Primitives.cuh:167-219): logits q.K/sqrt(dh), softmax, weighted V. One wave per
// workgroup: lane s computes the logits of slots s, s + 64, ... (a K row each, 16 bytes at a
// time); the probabilities go through LDS (dynamic, `window` floats) to the lanes that sum V
// by output coordinate.
__global__ __launch_bounds__(64) void batch_attention(const BatchArgs* __restrict__ ap, int layer) {
  const BatchArgs& a = *ap;
  extern __shared__ float pr[];
  const int b = blockIdx.x / a.heads, h = blockIdx.x - b * a.heads;
  const int lane = threadIdx.x, dim = a.dim;
  const unsigned long long t = a.position[b];
  const int valid = t + 1 < (unsigned long long)a.window ? (int)(t + 1) : a.window;
  const size_t base = (((size_t)b * a.layers + layer) * a.heads + h) * (size_t)a.window * dim;
  const float* K = a.keys + base;
  const float* V = a.values + base;
  const float* q = a.q + (size_t)b * a.width + h * dim;
  const float div = sqrtf((float)dim);
  float mx = -INFINITY;
  for (int s = lane; s < valid; s += 64) {
    const float* kr = K + (size_t)s * dim;
    float dot = 0.f;
    if ((dim & 3) == 0) {
      for (int d = 0; d < dim; d += 4) {
        const float4 kv = *reinterpret_cast<const float4*>(kr + d);
        dot += q[d] * kv.x;
        dot += q[d + 1] * kv.y;
        dot += q[d + 2] * kv.z;
        dot += q[d + 3] * kv.w;
      }
    } else {
      for (int d = 0; d < dim; d++) dot += q[d] * kr[d];
    }
    const float lg = dot / div;
    pr[s] = lg;
    mx = fmaxf(mx, lg);
  }
  mx = wave_top(mx);
  float sum = 0.f;
  for (int s = lane; s < valid; s += 64) {
    const float e = expf(pr[s] - mx);
    pr[s] = e;
    sum += e;
  }
  sum = wave_total(sum);
  __syncthreads();
  float* out = a.attn + (size_t)b * a.width_p + h * dim;
  for (int d = lane; d < dim; d += 64) {
    float o = 0.f;
    for (int s = 0; s < valid; s++) o += pr[s] * V[(size_t)s * dim + d];
    out[d] = o / sum;
  }
}

// Final RMSNorm and score of every stream (src/cuda/Runtime.cu:380-383), then the position
// advance. One wave per stream.
template <int P>
__global__ __launch_bounds__(64) void batch_final(const BatchArgs* __restrict__ ap) {
  const BatchArgs& a = *ap;
  const int b = blockIdx.x, lane = threadIdx.x;
  const float* xb = a.x + (size_t)b * a.width_p;
  float s = 0.f;
  for (int i = lane; i < a.width; i += 64) s += xb[i] * xb[i];
  const float scale = 1.0f / sqrtf(wave_total(s) / (float)a.width + a.epsilon);
  float acc = 0.f;
  for (int i = lane; i < a.width; i += 64) {
    float wn, ws;
    if constexpr (P == kFp32) {
      wn = reinterpret_cast<const float*>(a.weights + a.w_final_norm)[i];
      ws = reinterpret_cast<const float*>(a.weights + a.w_score)[i];
    } else {
      wn = __builtin_bit_cast(float, (unsigned)reinterpret_cast<const unsigned short*>(a.weights + a.w_final_norm)[i] << 16);
      ws = __builtin_bit_cast(float, (unsigned)reinterpret_cast<const unsigned short*>(a.weights + a.w_score)[i] << 16);
    }
    acc += ws * (xb[i] * scale * wn);
  }
  acc = wave_total(acc);
  if (lane == 0) {
    a.score[b] = acc;
    a.position[b] = a.position[b] + 1;
  }
}

// Zero the state of stream `stream` (every stream when negative): K/V rows, hidden, position.
__global__ void batch_reset(const BatchArgs* __restrict__ ap, int stream) {
  const BatchArgs& a = *ap;
  const int b0 = stream < 0 ? 0 : stream, b1 = stream < 0 ? a.streams : stream + 1;
  const size_t per = (size_t)a.layers * a.heads * a.window * a.dim;
  const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x, step = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)b0 * per + tid; i < (size_t)b1 * per; i += step) {
    a.keys[i] = 0.f;
    a.values[i] = 0.f;
  }
  const size_t hper = (size_t)a.layers * a.width;
  for (size_t i = (size_t)b0 * hper + tid; i < (size_t)b1 * hper; i += step) a.hidden[i] = 0.f;
  if (tid == 0)
    for (int b = b0; b < b1; b++) a.position[b] = 0;
}

}  // namespace stamd
