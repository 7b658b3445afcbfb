// Batched independent streams on gfx950: B streams share the weights and each keeps its own
// K/V ring, hidden state and position. One step advances every stream by one event. The
// projections become skinny GEMMs [B x K] . W^T on MFMA, split over K across the waves of a
// workgroup and summed in LDS in a fixed order, with the phase's epilogue (RoPE and ring write,
// residual, SwiGLU) fused. Storage modes:
//  - FP32 and bfloat16 weights: FP32 activations, K/V and reductions; RMSNorm folded into the
//    projection prologue;
//  - mixed (the reference's FP16 mode): FP16 weights and K/V ring, every value rounded to FP16
//    at the reference's cast points, so each GEMM input is exactly FP16 and runs on
//    v_mfma_f32_16x16x32_f16 with FP32 accumulation; the norms are materialized (their output
//    is cast before the projection).
// Each stream follows the single-stream runtime's arithmetic up to summation order.
#pragma once

#include "step_device.hpp"

#include <type_traits>

namespace stamd {

constexpr int kBatchMax = 256;   // streams per batch (16 batch tiles of 16 in the GEMM)
constexpr int kBatchTile = 16;   // MFMA rows

typedef float f4v __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

struct BatchArgs {
  int streams, streams_p;  // B and the padded batch (16, 32 or a multiple of 64)
  int layers, width, heads, dim, ffn, window, features;
  int width_p, ffn_p, features_p;  // padded row lengths
  float epsilon;
  const char* weights;
  uint32_t w_input, w_final_norm, w_score;
  LayerWeights layer[kMaxLayers];
  const float* rope_freq;          // [dim / 2]
  void* keys;                      // [L][B][H][W][dh], FP32 (FP16 in mixed mode): layer-major, so
                                   // that one layer's attention reads one contiguous region
  void* values;
  float* hidden;                   // [B][L][d]
  unsigned long long* position;    // [B]
  // Activations, Bp rows of the padded lengths, in the tiled layouts (act_index, half_index):
  float* in;                       // events (features_p)
  float* x;                        // residual stream (width_p)
  float* xn;                       // normalized x (mixed mode, FP16; width_p)
  float* attn;                     // attention output (FP16 in mixed mode; width_p)
  float* act;                      // SwiGLU output (FP16 in mixed mode; ffn_p)
  float* q;                        // [Bp][width] rotated queries
  float* score;                    // [B]
};

constexpr int kSlices = 8;       // K-slices of a projection, K / 8 columns each
constexpr size_t kInfinityCacheBytes = (size_t)256 << 20;  // MI355X's memory-side cache (MALL)

// Loads from the weight arena through the global address space. The arena's base arrives in
// the arguments block as a generic pointer, and a load through a generic (flat) pointer also
// counts on the LDS counter, so the compiler would wait for every outstanding load, the
// prefetched ones included, before a block's first MFMA.
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 gload16(const void* p) {
  return __builtin_bit_cast(uint4, *(const __attribute__((address_space(1))) u32x4_t*)p);
}
__device__ __forceinline__ float4 gload16f(const void* p) {
  return __builtin_bit_cast(float4, *(const __attribute__((address_space(1))) u32x4_t*)p);
}
__device__ __forceinline__ uint2 gload8(const void* p) {
  return __builtin_bit_cast(uint2, *(const __attribute__((address_space(1))) u32x2_t*)p);
}

// Activation layouts. The projections' operands (in, x, xn, attn, act) are stored the way the
// weights are (the tiled arena): 16-row tiles of streams, then blocks of KB columns, then the
// 64 lanes of the MFMA operand (stream b mod 16 + 16 x column group), so that a wave loads a
// block as contiguous 16-byte runs in lane order. `cols` is the buffer's padded row length
// (a multiple of 32).
//  - FP32 buffers for the FP32 MFMA (FP32 storage; mixed mode's x and events): KB = 16, four
//    floats per lane.
//  - FP32 buffers for the bfloat16 MFMA (bfloat16 weights): KB = 32, eight floats per lane,
//    stored as two planes of four (the lane's low and high halves), each plane 64 x 16 bytes.
//  - FP16 buffers (mixed mode's xn, attn, act): KB = 32, eight halves per lane.
// Four consecutive columns from a multiple of 4 are consecutive in every layout.
template <int P>
__host__ __device__ __forceinline__ size_t act_index(int b, int n, int cols) {
  if constexpr (P == kBf16w) {
    const int kk = n & 31;
    return ((((size_t)(b >> 4) * (cols >> 5) + (n >> 5)) * 2 + ((kk >> 2) & 1)) * 64 + (b & 15) + 16 * (kk >> 3)) * 4 +
           (kk & 3);
  } else {
    const int kk = n & 15;
    return (((size_t)(b >> 4) * (cols >> 4) + (n >> 4)) * 64 + (b & 15) + 16 * (kk >> 2)) * 4 + (kk & 3);
  }
}
__host__ __device__ __forceinline__ size_t half_index(int b, int n, int cols) {
  const int kk = n & 31;
  return (((size_t)(b >> 4) * (cols >> 5) + (n >> 5)) * 64 + (b & 15) + 16 * (kk >> 3)) * 8 + (kk & 7);
}
constexpr int kGroupTiles = 4;   // most batch tiles (16 streams each) per projection workgroup

enum BatchEpilogue : int { kEpInput = 0, kEpQkv, kEpOut, kEpGateUp, kEpDown };

// The exact three-term bfloat16 split of FP32 values, x = hi + mid + lo: truncations, hi keeps
// the top 8 significand bits, mid the next 8 of the remainder, lo the rest (at most 8 bits).
// Each term times a bfloat16 weight is exact in an FP32 accumulator.
__device__ __forceinline__ void split3(const float (&x)[8], unsigned (&ph)[4], unsigned (&pm)[4], unsigned (&pl)[4]) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    unsigned h2[2], m2[2], l2[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const float v = x[2 * i + j];
      const unsigned hb = __builtin_bit_cast(unsigned, v) & 0xffff0000u;
      const float r1 = v - __builtin_bit_cast(float, hb);
      const unsigned mb = __builtin_bit_cast(unsigned, r1) & 0xffff0000u;
      const float r2 = r1 - __builtin_bit_cast(float, mb);
      h2[j] = hb;
      m2[j] = mb;
      l2[j] = __builtin_bit_cast(unsigned, r2) & 0xffff0000u;
    }
    ph[i] = h2[1] | (h2[0] >> 16);
    pm[i] = m2[1] | (m2[0] >> 16);
    pl[i] = l2[1] | (l2[0] >> 16);
  }
}

// The K loop of one wave over its SW slices, from slice `first`, in blocks of KB columns.
// SW = 1: a ring of R fragments, unrolled so that no fragment is copied (a copy would wait for
// its loads): block j + R is loaded into the fragment of block j as soon as block j's MFMAs are
// issued, so R blocks are in flight while one computes. R = 4 for workgroups of at most two
// tiles when the slice holds a multiple of 4 blocks (it always holds an even number), else 2.
// Two kinds of empty asm statement hold the schedule: one after each prefetch (the compiler
// would otherwise see that the loads only feed the next round and move them next to their
// use), and `pin`, which passes a fragment's registers through an asm right before its MFMAs
// (the compiler would otherwise hoist the operand arithmetic of every fragment to the top of
// the round, which waits for all loads in flight). Either way every block would wait a full
// memory round trip. SW = 2: each step loads one block of each of the two slices, then runs
// both. Every form issues a slice's MFMAs in block order.
template <int R, int KB, typename Frag, typename Load, typename Pin, typename Mma>
__device__ __forceinline__ void k_ring(int k0, int nb, Load& load, Pin& pin, Mma& mma) {
  Frag f[R];
#pragma unroll
  for (int r = 0; r < R; r++) load(k0 + r * KB, f[r]);
  asm volatile("" ::: "memory");
  int j = 0;
  for (; j + R < nb; j += R) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      pin(f[r]);
      mma(0, f[r]);
      load(k0 + (j + R + r) * KB, f[r]);
      asm volatile("" ::: "memory");
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    pin(f[r]);
    mma(0, f[r]);
  }
}

__device__ __forceinline__ void pin4(uint4& v) { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)); }
__device__ __forceinline__ void pin4(float4& v) { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)); }

template <int SW, int KB, bool kSmall, typename Frag, typename Load, typename Pin, typename Mma>
__device__ __forceinline__ void k_loop(int first, int slice, Load&& load, Pin&& pin, Mma&& mma) {
  if constexpr (SW == 1) {
    const int k0 = first * slice, nb = slice / KB;
    if (kSmall && nb % 4 == 0) k_ring<4, KB, Frag>(k0, nb, load, pin, mma);
    else k_ring<2, KB, Frag>(k0, nb, load, pin, mma);
  } else {
    for (int kk = 0; kk < slice; kk += KB) {
      Frag f[SW];
#pragma unroll
      for (int i = 0; i < SW; i++) load((first + i) * slice + kk, f[i]);
#pragma unroll
      for (int i = 0; i < SW; i++) mma(i, f[i]);
    }
  }
}

// One projection Y = X . W^T over the batch, with its phase's epilogue. Workgroup: CT column
// tiles of 16 outputs and NT batch tiles of 16 streams. K is cut into 8 slices; each wave
// accumulates SW of them (8 / SW waves) for every tile pair with MFMA, reusing each X
// fragment for the CT column tiles and each weight fragment for the NT batch tiles. The slice
// partials are added in one fixed pairwise tree, ((s0 + s1) + (s2 + s3)) + ((s4 + s5) +
// (s6 + s7)), whatever NT, CT and SW are, so a stream's outputs depend only on its own row
// and are bit-identical for every batch size. The padded batch is a multiple of NT tiles, so
// the loops have no branches. X and W are in the tiled operand layout (act_index and the tiled
// arena): one 16 x KB block of either is 64 lanes' contiguous 16-byte pieces in lane order.
// X is the padded buffer of K columns; W the N x K matrix at offset `woff` of the arena
// `weights`. What the K loop's first loads need (the arena, X, the shape) comes in the kernel
// arguments, not from the arguments block, whose read would add a memory round trip before
// them.
// FP32 weights: v_mfma_f32_16x16x4_f32, k block of 16; lane l supplies A[l % 16][l / 16] and
// B[l / 16][l % 16], register r of lane l holds D[4 (l / 16) + r][l % 16]; the four MFMA
// steps use k = kb + 4 (l / 16) + c for step c, the same index for A and B.
// bfloat16 weights: v_mfma_f32_16x16x32_bf16, k block of 32, on the exact split of the FP32
// activation (3 MFMAs), so the product is the FP32 path's up to accumulation order. Lane
// (r16, g) holds k = kb + 8 g .. + 7 for both operands; the sum over k does not depend on how
// the hardware orders the lane groups.
// kNorm: X is the residual stream x and the projection consumes RMSNorm(x) . g
// (src/cuda/Primitives.cuh:122-135). The waves feed x * g to the MFMAs, accumulate the row's
// sum of squares from the same loads, and the epilogue scales the row by
// 1 / sqrt(sum / d + eps).
template <int P, int E, bool kNorm, int NT, int CT, int SW>
__global__ __launch_bounds__(64 * kSlices / SW) void batch_proj(const BatchArgs* __restrict__ ap,
                                                               const char* __restrict__ weights,
                                                               const void* __restrict__ X, uint32_t woff, int N,
                                                               int K, int width, uint32_t w_norm, int layer) {
  constexpr int kWaves = kSlices / SW;
  const BatchArgs& a = *ap;
  __shared__ float red[kWaves][NT][CT][16][17];
  __shared__ float sq[kWaves][NT][16];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n0 = blockIdx.x * kBatchTile * CT;
  const int t0 = blockIdx.y * NT;
  const int r16 = lane & 15, g = lane >> 4;
  const int slice = K / kSlices;
  const int first = wave * SW;  // the wave's first slice
  f4v acc[SW][NT][CT];
  float ss[SW][NT];
#pragma unroll
  for (int i = 0; i < SW; i++)
#pragma unroll
    for (int t = 0; t < NT; t++) {
      ss[i][t] = 0.f;
#pragma unroll
      for (int c = 0; c < CT; c++) acc[i][t][c] = f4v{0.f, 0.f, 0.f, 0.f};
    }
  static_assert(!(kNorm && P == kMixed), "mixed mode materializes its norms");
  if constexpr (P == kFp32 || (P == kMixed && E == kEpInput)) {
    // FP32 MFMA. Mixed mode takes this path for the input projection only: its operand is
    // the raw FP32 event, and its FP16 weights widen exactly.
    // Tiled operands: block (tile, k / 16) holds 64 lanes x 4 values.
    const int nkb = K / 16;
    const float* xr = reinterpret_cast<const float*>(X) + ((size_t)t0 * nkb * 64 + lane) * 4;
    const char* wr = weights + woff + ((size_t)(n0 / kBatchTile) * nkb * 64 + lane) * 4 * (P == kFp32 ? 4 : 2);
    const float* gr = reinterpret_cast<const float*>(weights + w_norm) + 4 * g;
    struct Frag {
      float4 w[CT], gn, x[NT];
    };
    auto load = [&](int k, Frag& f) {
#pragma unroll
      for (int c = 0; c < CT; c++) {
        const size_t blk = ((size_t)c * nkb + k / 16) * 256;
        if constexpr (P == kFp32) {
          f.w[c] = gload16f(reinterpret_cast<const float*>(wr) + blk);
        } else {
          const uint2 h = gload8(reinterpret_cast<const uint16_t*>(wr) + blk);
          f.w[c] = make_float4(half_to_float((unsigned short)(h.x & 0xffffu)), half_to_float((unsigned short)(h.x >> 16)),
                               half_to_float((unsigned short)(h.y & 0xffffu)), half_to_float((unsigned short)(h.y >> 16)));
        }
      }
      // The norm vector holds `width` values (a multiple of 16): a group of 4 is all in or out.
      f.gn = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (kNorm)
        if (k + 4 * g < width) f.gn = gload16f(gr + k);
#pragma unroll
      for (int t = 0; t < NT; t++) f.x[t] = *reinterpret_cast<const float4*>(xr + ((size_t)t * nkb + k / 16) * 256);
    };
    auto mma = [&](int i, const Frag& f) {
#pragma unroll
      for (int t = 0; t < NT; t++) {
        float4 x = f.x[t];
        if constexpr (kNorm) {
          ss[i][t] += x.x * x.x;
          ss[i][t] += x.y * x.y;
          ss[i][t] += x.z * x.z;
          ss[i][t] += x.w * x.w;
          x.x *= f.gn.x;
          x.y *= f.gn.y;
          x.z *= f.gn.z;
          x.w *= f.gn.w;
        }
#pragma unroll
        for (int c = 0; c < CT; c++) {
          f4v& d = acc[i][t][c];
          d = __builtin_amdgcn_mfma_f32_16x16x4f32(x.x, f.w[c].x, d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x4f32(x.y, f.w[c].y, d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x4f32(x.z, f.w[c].z, d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x4f32(x.w, f.w[c].w, d, 0, 0, 0);
        }
      }
    };
    auto pin = [&](Frag& f) {
#pragma unroll
      for (int c = 0; c < CT; c++) pin4(f.w[c]);
#pragma unroll
      for (int t = 0; t < NT; t++) pin4(f.x[t]);
      if constexpr (kNorm) pin4(f.gn);
    };
    k_loop<SW, 16, NT * CT <= 2, Frag>(first, slice, load, pin, mma);
  } else if constexpr (P == kBf16w) {
    // Tiled operands: weight block (tile, k / 32) holds 64 lanes x 8 values, activation block
    // two planes of 64 lanes x 4 floats.
    const int nkb = K / 32;
    const float* xr = reinterpret_cast<const float*>(X) + ((size_t)t0 * nkb * 128 + lane) * 4;
    const uint16_t* wr = reinterpret_cast<const uint16_t*>(weights + woff) + ((size_t)(n0 / kBatchTile) * nkb * 64 + lane) * 8;
    const uint16_t* gr = reinterpret_cast<const uint16_t*>(weights + w_norm) + 8 * g;
    struct Frag {
      uint4 w[CT], gn;
      float4 xlo[NT], xhi[NT];
    };
    auto load = [&](int k, Frag& f) {
#pragma unroll
      for (int c = 0; c < CT; c++) f.w[c] = gload16(wr + ((size_t)c * nkb + k / 32) * 512);
      f.gn = make_uint4(0u, 0u, 0u, 0u);
      if constexpr (kNorm)
        if (k + 8 * g < width) f.gn = gload16(gr + k);
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const float* p = xr + ((size_t)t * nkb + k / 32) * 512;
        f.xlo[t] = *reinterpret_cast<const float4*>(p);
        f.xhi[t] = *reinterpret_cast<const float4*>(p + 256);
      }
    };
    auto mma = [&](int i, const Frag& f) {
      float gv[8];
      if constexpr (kNorm) {
        const unsigned gu[4] = {f.gn.x, f.gn.y, f.gn.z, f.gn.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          gv[2 * j] = __builtin_bit_cast(float, gu[j] << 16);
          gv[2 * j + 1] = __builtin_bit_cast(float, gu[j] & 0xffff0000u);
        }
      }
#pragma unroll
      for (int t = 0; t < NT; t++) {
        float x[8] = {f.xlo[t].x, f.xlo[t].y, f.xlo[t].z, f.xlo[t].w, f.xhi[t].x, f.xhi[t].y, f.xhi[t].z, f.xhi[t].w};
        if constexpr (kNorm) {
#pragma unroll
          for (int j = 0; j < 8; j++) {
            ss[i][t] += x[j] * x[j];
            x[j] *= gv[j];
          }
        }
        unsigned ph[4], pm[4], pl[4];
        split3(x, ph, pm, pl);
        const bf16x8 h = __builtin_bit_cast(bf16x8, ph), m = __builtin_bit_cast(bf16x8, pm),
                     l = __builtin_bit_cast(bf16x8, pl);
#pragma unroll
        for (int c = 0; c < CT; c++) {
          const bf16x8 wb = __builtin_bit_cast(bf16x8, f.w[c]);
          f4v& d = acc[i][t][c];
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h, wb, d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(m, wb, d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(l, wb, d, 0, 0, 0);
        }
      }
    };
    auto pin = [&](Frag& f) {
#pragma unroll
      for (int c = 0; c < CT; c++) pin4(f.w[c]);
#pragma unroll
      for (int t = 0; t < NT; t++) {
        pin4(f.xlo[t]);
        pin4(f.xhi[t]);
      }
      if constexpr (kNorm) pin4(f.gn);
    };
    k_loop<SW, 32, NT * CT <= 2, Frag>(first, slice, load, pin, mma);
  } else {
    // Mixed mode: the operand is an FP16 buffer (its values are cast points) and the weights
    // are FP16; one v_mfma_f32_16x16x32_f16 per 32-k block, lane (r16, g) holding
    // k = kb + 8 g .. + 7 of both, 16 bytes each.
    // Tiled operands: block (tile, k / 32) holds 64 lanes x 8 values.
    const int nkb = K / 32;
    const uint16_t* xr = reinterpret_cast<const uint16_t*>(X) + ((size_t)t0 * nkb * 64 + lane) * 8;
    const uint16_t* wr = reinterpret_cast<const uint16_t*>(weights + woff) + ((size_t)(n0 / kBatchTile) * nkb * 64 + lane) * 8;
    struct Frag {
      uint4 w[CT], x[NT];
    };
    auto load = [&](int k, Frag& f) {
#pragma unroll
      for (int c = 0; c < CT; c++) f.w[c] = gload16(wr + ((size_t)c * nkb + k / 32) * 512);
#pragma unroll
      for (int t = 0; t < NT; t++) f.x[t] = *reinterpret_cast<const uint4*>(xr + ((size_t)t * nkb + k / 32) * 512);
    };
    auto mma = [&](int i, const Frag& f) {
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int c = 0; c < CT; c++)
          acc[i][t][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, f.x[t]),
                                                                __builtin_bit_cast(f16x8, f.w[c]), acc[i][t][c], 0, 0, 0);
    };
    auto pin = [&](Frag& f) {
#pragma unroll
      for (int c = 0; c < CT; c++) pin4(f.w[c]);
#pragma unroll
      for (int t = 0; t < NT; t++) pin4(f.x[t]);
    };
    k_loop<SW, 32, NT * CT <= 2, Frag>(first, slice, load, pin, mma);
  }
  // A wave holding two slices adds them here: the first level of the tree.
#pragma unroll
  for (int t = 0; t < NT; t++) {
#pragma unroll
    for (int c = 0; c < CT; c++) {
      f4v v = acc[0][t][c];
      if constexpr (SW == 2) v = acc[0][t][c] + acc[1][t][c];
#pragma unroll
      for (int r = 0; r < 4; r++) red[wave][t][c][4 * g + r][r16] = v[r];
    }
    if constexpr (kNorm) {
      float v = column_sum(ss[0][t], 16);
      if constexpr (SW == 2) v = v + column_sum(ss[1][t], 16);
      if (g == 0) sq[wave][t][r16] = v;
    }
  }
  __syncthreads();
  // Epilogue: one thread per output unit (a column, or the column pair of a RoPE pair /
  // gate-up pair) of a stream below B.
  constexpr int unit = (E == kEpQkv || E == kEpGateUp) ? 2 : 1;
  constexpr int per_row = kBatchTile * CT / unit;
  auto tree = [&](auto at) {
    float p[4];
#pragma unroll
    for (int k = 0; k < 4; k++) p[k] = SW == 2 ? at(k) : at(2 * k) + at(2 * k + 1);
    return (p[0] + p[1]) + (p[2] + p[3]);
  };
  for (int o = threadIdx.x; o < NT * kBatchTile * per_row; o += blockDim.x) {
    const int t = o / (kBatchTile * per_row);
    const int row = (o / per_row) % kBatchTile;
    const int cc = (o % per_row) * unit;
    const int c = cc / kBatchTile, col = cc % kBatchTile;
    const int b = (t0 + t) * kBatchTile + row;
    if (b >= a.streams) continue;
    float s0 = tree([&](int k) { return red[k][t][c][row][col]; });
    float s1 = unit == 2 ? tree([&](int k) { return red[k][t][c][row][col + 1]; }) : 0.f;
    if constexpr (kNorm) {
      const float sum = tree([&](int k) { return sq[k][t][row]; });
      const float scale = 1.0f / sqrtf(sum / (float)a.width + a.epsilon);
      s0 *= scale;
      s1 *= scale;
    }
    // Projection outputs are cast (mixed mode), then each epilogue casts where the reference
    // does (src/cuda/Primitives.cuh:148-239); cast<P> is the identity for FP32 storage.
    s0 = cast<P>(s0);
    s1 = cast<P>(s1);
    const int n = n0 + cc;
    float* xp = a.x + act_index<P>(b, n, a.width_p);  // x[b][n]
    if constexpr (E == kEpInput) {
      *xp = s0;
    } else if constexpr (E == kEpQkv) {
      // src/cuda/Primitives.cuh:148-166: RoPE on adjacent pairs of q and k, then the ring write.
      const int sec = (n >= a.width) + (n >= 2 * a.width);
      const int i = n - sec * a.width;
      const unsigned long long pos = a.position[b];
      float va = s0, vb = s1;
      if (sec < 2) {
        // No FMA contraction here: left to the compiler, it fuses one product or the other
        // depending on the kernel variant, and a stream's bits would then depend on the
        // workgroup shape chosen for its batch size.
#pragma clang fp contract(off)
        const int e = i % a.dim;
        const float angle = (float)pos * a.rope_freq[e >> 1];
        const float co = cosf(angle), si = sinf(angle);
        const float ra = va * co - vb * si, rb = va * si + vb * co;
        va = cast<P>(ra);
        vb = cast<P>(rb);
      }
      if (sec == 0) {
        a.q[(size_t)b * a.width + i] = va;
        a.q[(size_t)b * a.width + i + 1] = vb;
      } else {
        const int h = i / a.dim, d = i - h * a.dim;
        const int slot = (int)(pos % (unsigned long long)a.window);
        const size_t ring = ((((size_t)layer * a.streams + b) * a.heads + h) * a.window + slot) * a.dim + d;
        void* dst = sec == 1 ? a.keys : a.values;
        if constexpr (P == kMixed) {
          reinterpret_cast<uint16_t*>(dst)[ring] = float_to_half(va);
          reinterpret_cast<uint16_t*>(dst)[ring + 1] = float_to_half(vb);
        } else {
          reinterpret_cast<float*>(dst)[ring] = va;
          reinterpret_cast<float*>(dst)[ring + 1] = vb;
        }
      }
    } else if constexpr (E == kEpOut) {
      *xp = cast<P>(*xp + s0);
    } else if constexpr (E == kEpGateUp) {
      const float v = cast<P>((s0 / (1.0f + expf(-s0))) * s1);
      if constexpr (P == kMixed) reinterpret_cast<uint16_t*>(a.act)[half_index(b, n >> 1, a.ffn_p)] = float_to_half(v);
      else a.act[act_index<P>(b, n >> 1, a.ffn_p)] = v;
    } else {
      const float v = cast<P>(*xp + s0);
      *xp = v;
      a.hidden[((size_t)b * a.layers + layer) * a.width + n] = v;
    }
  }
}

// Four consecutive ring elements of K or V (FP32, or FP16 in mixed mode) as floats.
// Global (not flat) loads, so that they count on the vector memory counter only; kNT marks
// them non-temporal, for rings larger than the Infinity Cache (see batch_attention).
template <int P, bool kNT>
__device__ __forceinline__ float4 ring4(const void* ring, size_t i) {
  typedef const __attribute__((address_space(1))) u32x2_t g2;
  typedef const __attribute__((address_space(1))) u32x4_t g4;
  if constexpr (P == kMixed) {
    const void* p = reinterpret_cast<const uint16_t*>(ring) + i;
    const uint2 h = __builtin_bit_cast(uint2, kNT ? __builtin_nontemporal_load((g2*)p) : *(g2*)p);
    return make_float4(half_to_float((unsigned short)(h.x & 0xffffu)), half_to_float((unsigned short)(h.x >> 16)),
                       half_to_float((unsigned short)(h.y & 0xffffu)), half_to_float((unsigned short)(h.y >> 16)));
  } else {
    const void* p = reinterpret_cast<const float*>(ring) + i;
    return __builtin_bit_cast(float4, kNT ? __builtin_nontemporal_load((g4*)p) : *(g4*)p);
  }
}

// Four consecutive ring elements as loaded (FP16 pairs in mixed mode), and their FP32 values.
// The chunked attention keeps the loaded form in registers and widens at each use, so that the
// FP16 values feed mixed-precision FMAs directly (widening is exact, the results unchanged).
template <int P>
using RingRaw = std::conditional_t<P == kMixed, uint2, float4>;
template <int P, bool kNT>
__device__ __forceinline__ RingRaw<P> ring_raw(const void* ring, size_t i) {
  typedef const __attribute__((address_space(1))) u32x2_t g2;
  typedef const __attribute__((address_space(1))) u32x4_t g4;
  if constexpr (P == kMixed) {
    const void* p = reinterpret_cast<const uint16_t*>(ring) + i;
    return __builtin_bit_cast(uint2, kNT ? __builtin_nontemporal_load((g2*)p) : *(g2*)p);
  } else {
    return ring4<P, kNT>(ring, i);
  }
}
__device__ __forceinline__ const float4& widen(const float4& v) { return v; }
__device__ __forceinline__ float4 widen(uint2 h) {
  return make_float4(half_to_float((unsigned short)(h.x & 0xffffu)), half_to_float((unsigned short)(h.x >> 16)),
                     half_to_float((unsigned short)(h.y & 0xffffu)), half_to_float((unsigned short)(h.y >> 16)));
}

constexpr int kAttnThreads = 256;  // batch_attention's workgroup: four waves, 16 groups of 16 lanes

// batch_attention for dh <= 64: lane (group grp, r) holds elements 4r .. 4r + 3 of its rows,
// one 16-byte load per row, the loads of NP passes of 16 rows issued together; with kEarlyV the
// first chunk's V loads are issued before the softmax reductions. The arithmetic is the general
// loop's, in the same order: per row a dot product over the lane's four elements and a 16-lane
// sum; per group the V rows of slots grp, grp + 16, ... accumulated in slot order.
template <int P, int NP, bool kEarlyV, bool kNT>
__device__ __forceinline__ void attention_chunked(const BatchArgs& a, int b, int h, int valid, size_t base,
                                                  const float* q, float div, float* pr, float* wred,
                                                  float4 (*vred)[17]) {
  constexpr int kRows = 16 * NP;
  const int dim = a.dim;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = tid & 15, grp = tid >> 4;
  const int d = 4 * r;
  const bool in = d < dim;
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  const float4 qv = in ? *reinterpret_cast<const float4*>(q + d) : z4;
  // Slots past `valid` load slot valid - 1 and are dropped.
  auto at = [&](int s) { return base + (size_t)(s < valid ? s : valid - 1) * dim + d; };
  // V rows of a chunk; filled in place (an array filled through a lambda went to scratch).
  // K and V stay in their loaded form (RingRaw) until used.
  const RingRaw<P> zr{};
  RingRaw<P> vv[NP];
  float mx = -INFINITY;
  for (int c0 = 0; c0 < valid; c0 += kRows) {
    RingRaw<P> kv[NP];
#pragma unroll
    for (int p = 0; p < NP; p++) kv[p] = in ? ring_raw<P, kNT>(a.keys, at(c0 + 16 * p + grp)) : zr;
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const int s = c0 + 16 * p + grp;
      float dot = 0.f;
      if (in) {
        const float4& k = widen(kv[p]);
        dot += qv.x * k.x;
        dot += qv.y * k.y;
        dot += qv.z * k.z;
        dot += qv.w * k.w;
      }
      dot = group_sum(dot, 16);
      if (s < valid) {
        const float lg = dot / div;
        if (r == 0) pr[s] = lg;
        mx = fmaxf(mx, lg);
      }
    }
  }
  if constexpr (kEarlyV) {
#pragma unroll
    for (int p = 0; p < NP; p++) vv[p] = in ? ring_raw<P, kNT>(a.values, at(16 * p + grp)) : zr;
  }
  mx = wave_top(mx);
  if (lane == 0) wred[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
  float sum = 0.f;
  for (int s = tid; s < valid; s += kAttnThreads) {
    const float e = expf(pr[s] - mx);
    pr[s] = e;
    sum += e;
  }
  sum = wave_total(sum);
  __syncthreads();  // every wave has read wred (max) and written its probabilities
  if (lane == 0) wred[wave] = sum;
  __syncthreads();
  sum = (wred[0] + wred[1]) + (wred[2] + wred[3]);
  float4 o = z4;
  for (int c0 = 0; c0 < valid; c0 += kRows) {
    if (!kEarlyV || c0 > 0) {
#pragma unroll
      for (int p = 0; p < NP; p++) vv[p] = in ? ring_raw<P, kNT>(a.values, at(c0 + 16 * p + grp)) : zr;
    }
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const int s = c0 + 16 * p + grp;
      if (s < valid) {
        const float pp = pr[s];
        const float4& v = widen(vv[p]);
        o.x += pp * v.x;
        o.y += pp * v.y;
        o.z += pp * v.z;
        o.w += pp * v.w;
      }
    }
  }
  vred[grp][r] = o;
  __syncthreads();
  if (tid < 16 && 4 * tid < dim) {
    float4 acc = vred[0][tid];
    for (int k = 1; k < 16; k++) {
      const float4 v = vred[k][tid];
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    const float o4[4] = {acc.x / sum, acc.y / sum, acc.z / sum, acc.w / sum};
    // attn[b][h dh + 4 tid + j]: four consecutive elements in the tiled layouts too.
    const int n = h * dim + 4 * tid;
    const size_t oi = P == kMixed ? half_index(b, n, a.width_p) : act_index<P>(b, n, a.width_p);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if constexpr (P == kMixed) reinterpret_cast<uint16_t*>(a.attn)[oi + j] = float_to_half(o4[j]);
      else a.attn[oi + j] = o4[j];
    }
  }
}

// Attention of one (stream, head) over the stream's valid ring slots [0, valid)
// (src/cuda/Primitives.cuh:167-219): logits q.K/sqrt(dh), softmax, weighted V, cast. Slot order
// does not change the result beyond summation order. Four waves; every load is a coalesced
// row:
//  - logits: 16 lanes per K row (4 elements each, rows of up to 64 elements per pass), a
//    16-lane DPP sum, so a wave covers 4 rows per load;
//  - softmax: workgroup max and sum through LDS;
//  - values: lane group (slot s mod 16) accumulates its slots' V rows, 4 elements per lane,
//    and the 16 groups are summed in LDS in group order.
// Needs dh a multiple of 4; dynamic LDS holds `window` floats of probabilities. The rings are
// layer-major, so a layer's K and V are one contiguous region. kLoads picks the form of the
// loops, on the host, by storage and batch size; every form computes the same values in the same
// order, so a stream's bits do not depend on it:
//  - kAttnPerPass: the general loop below, one pass of 16 rows after the other (any dh);
//  - kAttnChunk4, kAttnChunk4Early, kAttnChunk8Early: dh <= 64, the loads of 4 or 8 passes
//    issued together (attention_chunked); the Early forms load the first V chunk before the
//    softmax.
// Measured on Main (one layer, W = 128): with FP32 K/V at 256 streams 23.2 us against 26.2 us
// for the per-pass loop in the former stream-major layout, at 64 streams 6.95 (4, early V)
// against 8.8, at 16 streams 5.2 (8) against 7.4 (and 8 with early V, once the K/V loads were
// global loads, 183.7 -> 181.2 us per Main step). FP16 K/V take the same forms since the
// chunked loops keep K and V in their loaded form (RingRaw) until each use: converted when
// loaded, they were slower than the per-pass loop below 256 streams (at 16 streams 9.7-10.4
// against 7.9 us per layer); kept as loaded, Main mixed steps went 204 -> 187 us at one stream,
// 214 -> 200 at 16, 237 -> 226 at 64 and 368 -> 344 at 256.
// kNT: the K and V loads are non-temporal, for rings that do not fit in the Infinity Cache
// beside the weights: a step streams them through once, and cached they would evict the
// weights the projections re-read (Main, bfloat16 weights: 454 -> 436 us per step at 256
// streams, 249 -> 241 at 64; mixed mode 400 -> 382 at 256). Rings that fit stay cached from
// step to step instead (mixed mode at 64 streams: 253 against 270 us).
enum AttnLoads : int { kAttnPerPass = 0, kAttnChunk4, kAttnChunk4Early, kAttnChunk8Early };
template <int P, int kLoads, bool kNT>
__global__ __launch_bounds__(kAttnThreads) void batch_attention(const BatchArgs* __restrict__ ap, int layer) {
  const BatchArgs& a = *ap;
  extern __shared__ float pr[];
  __shared__ float wred[kAttnThreads / 64];
  __shared__ float4 vred[16][17];
  const int b = blockIdx.x / a.heads, h = blockIdx.x - b * a.heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int dim = a.dim, r = tid & 15, grp = tid >> 4;  // 16 groups of 16 lanes
  const unsigned long long t = a.position[b];
  const int valid = t + 1 < (unsigned long long)a.window ? (int)(t + 1) : a.window;
  const size_t base = (((size_t)layer * a.streams + b) * a.heads + h) * (size_t)a.window * dim;
  const float* q = a.q + (size_t)b * a.width + h * dim;
  const float div = sqrtf((float)dim);
  if constexpr (kLoads != kAttnPerPass) {
    constexpr int np = kLoads == kAttnChunk8Early ? 8 : 4;
    attention_chunked<P, np, kLoads == kAttnChunk4Early || kLoads == kAttnChunk8Early, kNT>(a, b, h, valid, base, q,
                                                                                            div, pr, wred, vred);
    return;
  }
  float mx = -INFINITY;
  // Rows past `valid` load row valid - 1 and are dropped, so the loop body has no branch
  // around its loads and several passes of loads stay in flight.
#pragma unroll 4
  for (int s0 = 0; s0 < valid; s0 += kAttnThreads / 16) {
    const int s = s0 + grp;
    const size_t row = base + (size_t)(s < valid ? s : valid - 1) * dim;
    float dot = 0.f;
    for (int d = 4 * r; d < dim; d += 64) {
      const float4 kv = ring4<P, kNT>(a.keys, row + d);
      const float4 qv = *reinterpret_cast<const float4*>(q + d);
      dot += qv.x * kv.x;
      dot += qv.y * kv.y;
      dot += qv.z * kv.z;
      dot += qv.w * kv.w;
    }
    dot = group_sum(dot, 16);
    if (s < valid) {
      const float lg = dot / div;
      if (r == 0) pr[s] = lg;
      mx = fmaxf(mx, lg);
    }
  }
  mx = wave_top(mx);
  if (lane == 0) wred[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
  float sum = 0.f;
  for (int s = tid; s < valid; s += kAttnThreads) {
    const float e = expf(pr[s] - mx);
    pr[s] = e;
    sum += e;
  }
  sum = wave_total(sum);
  __syncthreads();  // every wave has read wred (max) and written its probabilities
  if (lane == 0) wred[wave] = sum;
  __syncthreads();
  sum = (wred[0] + wred[1]) + (wred[2] + wred[3]);
  for (int d0 = 0; d0 < dim; d0 += 64) {
    const int d = d0 + 4 * r;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    if (d < dim) {
#pragma unroll 4
      for (int s = grp; s < valid; s += 16) {
        const float p = pr[s];
        const float4 vv = ring4<P, kNT>(a.values, base + (size_t)s * dim + d);
        o.x += p * vv.x;
        o.y += p * vv.y;
        o.z += p * vv.z;
        o.w += p * vv.w;
      }
    }
    vred[grp][r] = o;
    __syncthreads();
    if (tid < 16 && d0 + 4 * tid < dim) {
      float4 acc = vred[0][tid];
      for (int k = 1; k < 16; k++) {
        const float4 v = vred[k][tid];
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
      }
      const float o4[4] = {acc.x / sum, acc.y / sum, acc.z / sum, acc.w / sum};
      const int n = h * dim + d0 + 4 * tid;
      const size_t oi = P == kMixed ? half_index(b, n, a.width_p) : act_index<P>(b, n, a.width_p);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if constexpr (P == kMixed) reinterpret_cast<uint16_t*>(a.attn)[oi + j] = float_to_half(o4[j]);
        else a.attn[oi + j] = o4[j];
      }
    }
    __syncthreads();
  }
}

// One element of a norm or score vector in the arena, decoded to FP32.
template <int P>
__device__ __forceinline__ float batch_weight(const char* w, uint32_t off, int i) {
  if constexpr (P == kFp32) return reinterpret_cast<const float*>(w + off)[i];
  if constexpr (P == kMixed) return half_to_float(reinterpret_cast<const uint16_t*>(w + off)[i]);
  return bf16_to_float(reinterpret_cast<const uint16_t*>(w + off)[i]);
}

// Mixed mode: RMSNorm of every stream's x into xn with the output cast to FP16
// (src/cuda/Primitives.cuh:122-135); padding columns and padding streams are zero. One
// workgroup of 256 threads per row of the padded batch. Every load (x and the norm vector,
// at most 4 columns per thread) is issued before the reduction, so the kernel waits one
// memory round trip; the sums keep their order.
static __global__ __launch_bounds__(256) void batch_norm_mixed(const BatchArgs* __restrict__ ap, uint32_t w_norm) {
  const BatchArgs& a = *ap;
  __shared__ float red[4];
  const int b = blockIdx.x;
  const float* x = a.x;
  uint16_t* out = reinterpret_cast<uint16_t*>(a.xn);
  auto xb = [&](int i) { return x[act_index<kMixed>(b, i, a.width_p)]; };
  if (b >= a.streams) {
    for (int i = threadIdx.x; i < a.width_p; i += blockDim.x) out[half_index(b, i, a.width_p)] = 0;
    return;
  }
  constexpr int kPer = kMaxDim / 256;
  float xv[kPer], gv[kPer];
#pragma unroll
  for (int j = 0; j < kPer; j++) {
    const int i = threadIdx.x + 256 * j;
    xv[j] = i < a.width ? xb(i) : 0.f;
    gv[j] = i < a.width ? batch_weight<kMixed>(a.weights, w_norm, i) : 0.f;
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kPer; j++)
    if (threadIdx.x + 256 * j < a.width) s += xv[j] * xv[j];
  s = wave_total(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  const float scale = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)a.width + a.epsilon);
#pragma unroll
  for (int j = 0; j < kPer; j++) {
    const int i = threadIdx.x + 256 * j;
    if (i < a.width_p) out[half_index(b, i, a.width_p)] = i < a.width ? float_to_half(xv[j] * scale * gv[j]) : 0;
  }
}

// Final RMSNorm (cast in mixed mode) and score of every stream (src/cuda/Runtime.cu:380-383;
// the score itself is not cast), then the position advance. One wave per stream.
template <int P>
__global__ __launch_bounds__(64) void batch_final(const BatchArgs* __restrict__ ap) {
  const BatchArgs& a = *ap;
  const int b = blockIdx.x, lane = threadIdx.x;
  const float* x = a.x;
  auto xb = [&](int i) { return x[act_index<P>(b, i, a.width_p)]; };
  // Unrolled so that the loads of several iterations are in flight together (the sums keep
  // their order).
  float s = 0.f;
#pragma unroll 8
  for (int i = lane; i < a.width; i += 64) s += xb(i) * xb(i);
  const float scale = 1.0f / sqrtf(wave_total(s) / (float)a.width + a.epsilon);
  float acc = 0.f;
#pragma unroll 8
  for (int i = lane; i < a.width; i += 64) {
    const float wn = batch_weight<P>(a.weights, a.w_final_norm, i), ws = batch_weight<P>(a.weights, a.w_score, i);
    acc += ws * cast<P>(xb(i) * scale * wn);
  }
  acc = wave_total(acc);
  if (lane == 0) {
    a.score[b] = acc;
    a.position[b] = a.position[b] + 1;
  }
}

// Zero the state of stream `stream` (every stream when negative): K/V rows, hidden, position.
// `block_words` is one (layer, stream) block of the K (or V) ring, [H][W][dh], in 4-byte words;
// a stream's K/V is one such block in each layer (the rings are layer-major).
static __global__ void batch_reset(const BatchArgs* __restrict__ ap, int stream, size_t block_words) {
  const BatchArgs& a = *ap;
  const int b0 = stream < 0 ? 0 : stream, b1 = stream < 0 ? a.streams : stream + 1;
  const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x, step = (size_t)gridDim.x * blockDim.x;
  unsigned* k = reinterpret_cast<unsigned*>(a.keys);
  unsigned* v = reinterpret_cast<unsigned*>(a.values);
  const size_t span = (size_t)(b1 - b0) * block_words;  // the streams' words in one layer
  for (size_t i = tid; i < (size_t)a.layers * span; i += step) {
    const size_t l = i / span, j = ((size_t)l * a.streams + b0) * block_words + i % span;
    k[j] = 0u;
    v[j] = 0u;
  }
  const size_t hper = (size_t)a.layers * a.width;
  for (size_t i = (size_t)b0 * hper + tid; i < (size_t)b1 * hper; i += step) a.hidden[i] = 0.f;
  if (tid == 0)
    for (int b = b0; b < b1; b++) a.position[b] = 0;
}

}  // namespace stamd
