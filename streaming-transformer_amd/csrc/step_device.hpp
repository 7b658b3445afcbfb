// Device code for the streaming local-causal transformer step on gfx950 (CDNA4, wave64).
//
// One step = 5*layers + 2 dependent phases:
//   INPUT            x = cast(W_input . event)                      (src/cuda/Primitives.cuh:253)
//   per layer l:
//     QKV            z = norm1(x); q,k,v = W_qkv . z; RoPE; ring write (Primitives.cuh:138-166)
//     ATTN           windowed softmax attention over the ring         (Primitives.cuh:167-219)
//     OUT            x = cast(x + cast(W_out . attn))                 (Primitives.cuh:221-226)
//     GATEUP         z = norm2(x); act = cast(silu(cast(g)) * cast(u)) (Primitives.cuh:227-239)
//     DOWN           x = cast(x + cast(W_down . act)); hidden[l] = x  (Primitives.cuh:221-229)
//   FINAL            score = W_score . norm(x) (not cast); position++   (Primitives.cuh:268-277)
//
// Workgroup shape: 512 threads = 8 wave64s. Wave 0 is the control wave: it waits on the
// grid barrier, stages the phase's input vector into LDS (agent-coherent loads) and computes
// RMSNorm there. Waves 1..7 are stream waves: each owns a list of weight rows and keeps a
// register ring of PF "slabs" (one slab = 64 lanes x 16 B = 1 KiB of one row) so the next
// phase's weights are already in flight while the control wave waits on the barrier.
//
// Every output row is reduced by one wave with a fixed lane->column mapping and a fixed
// butterfly, so results are bit-identical whichever workgroup computes the row and whatever
// the grid size: staged, graph, fused and persistent execution agree exactly.
//
// Cross-workgroup data (activations, K/V ring, attention partials, barrier flags) is written
// with agent-scope write-through stores (sc1) and read with agent-scope loads, so no L2
// writeback/invalidate fences are needed between phases.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mailbox.hpp"  // the mailbox commands (kCmd*) shared with the host

namespace stamd {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kStreamWaves = kWaves - 1;
#ifndef STAMD_PF
#define STAMD_PF 8
#endif
constexpr int kPF = STAMD_PF;      // register ring depth (slabs) per stream wave
constexpr int kKB = kPF >= 16 ? 8 : kPF / 2;  // ring slabs per attention K (or V) block
static_assert(2 * kKB <= kPF, "an attention item's K and V blocks fit in the ring");
#ifndef STAMD_POLL_STAMPS
#define STAMD_POLL_STAMPS 0
#endif
constexpr int kStampPhases = 128;  // phases of a step that record stamps (profiling only)
constexpr int kStamps = STAMD_POLL_STAMPS ? 16 : 8;         // wall-clock stamps per phase and workgroup (profiling only)
constexpr int kMaxGrid = 1024;     // largest grid accepted
constexpr int kMaxLayers = 16;
constexpr int kXs = 4096 + 64;     // LDS activation vector capacity (floats)
constexpr int kAttnLds = 2304;     // per stream wave K/V staging (floats): CH*(dh+4) <= 2304
constexpr int kMaxDim = 1024;

enum Precision : int { kFp32 = 0, kMixed = 1, kBf16w = 2 };
enum PhaseKind : int { kInput = 0, kQkv, kAttn, kOut, kGateUp, kDown, kFinal };
enum ErrorBits : unsigned { kErrPollTimeout = 1u, kErrMailboxTimeout = 2u };

// Buffer-resource dword3 for raw buffer access on gfx9 (32-bit data format).
constexpr int kRsrcWord3 = 0x00020000;
// Cache-policy bits for agent-scope coherence (LLVM CPol::SC1) and non-temporal access
// (CPol::NT).
constexpr int kSc1 = 16;
constexpr int kNt = 2;

struct LayerWeights {
  uint32_t norm1, norm2, qkv, out, gateup, down;  // byte offsets into the weight arena
};

// Step arguments, kept in device memory and read through a restrict pointer (~0.6 KB).
struct StepArgs {
  // shape
  int layers, width, heads, ffn, window, features, dim;
  float epsilon;
  int width_p, ffn_p, features_p;  // padded row lengths (elements), multiples of 16 B
  int chunk;                       // attention slots per work item
  int attn_regs;                   // 1: head dim suits the register attention path
  int grid;                        // workgroups in this launch
  // weights (one arena, byte offsets)
  const char* weights;
  uint32_t weight_bytes;
  uint32_t w_input, w_final_norm, w_score;
  LayerWeights layer[kMaxLayers];
  // state
  void* keys;                      // [L][H][W][dh], float or half
  void* values;
  uint32_t cache_bytes;            // bytes of one of keys/values
  float* scratch;                  // fp32 scratch arena (agent-coherent access)
  uint32_t scratch_bytes;
  // scratch offsets (floats): host-staged input, hidden state, score
  uint32_t s_input, s_hidden, s_score;
  // tagged vectors (8-byte elements: epoch << 32 | float bits)
  unsigned long long* tagged;
  uint32_t tagged_bytes;
  uint32_t t_x, t_q, t_k, t_v, t_attn, t_act, t_done;  // element offsets
  uint32_t t_po, t_pm, t_ps;       // attention partials per item: o [items][dh], max, exp sum
  unsigned long long* position;
  unsigned* epoch;                 // epoch of phase 0 of the next step
  unsigned* error;                 // sticky error bits
  const float* rope_freq;          // [dh/2]
  const float* input;              // event source for the INPUT phase (device memory)
  unsigned long long spin_limit;   // poll timeout in wall-clock ticks
  // persistent backend: mailbox words in coherent pinned host memory (device aliases)
  unsigned long long* mb_request;
  unsigned long long* mb_completion;
  unsigned long long* mb_exited;
  int* mb_command;
  float* mb_score;
  unsigned long long* mb_checksum;
  unsigned* mb_error;              // device error bits, copied out with each completion
  const float* mapped_input;       // the host's event buffer
  unsigned char* mapped_snapshot;  // SNAPSHOT destination in host memory (layout: snapshot_owned)
  unsigned long long idle_ticks;   // idle budget before the worker exits
  unsigned long long max_events;   // RUN budget (0 = unlimited)
  unsigned long long initial_sequence;
  int backoff;                     // sleep between mailbox polls
  uint32_t t_cmd, t_in, t_wdone;   // tagged: command word, staged event, per-workgroup done
  unsigned long long* stamps;      // optional per-phase wall-clock stamps (workgroup 0)
};

// ---------------------------------------------------------------------------------------------
// memory helpers

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}

__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
// A 16-byte weight load. NT marks it non-temporal: weights that exceed the Infinity Cache are
// streamed without displacing the data that stays cached across steps (K/V rows, the tagged
// exchange vectors, arguments); weights that fit stay resident in it from step to step.
template <bool NT>
__device__ __forceinline__ uint4 ld16w(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, NT ? kNt : 0));
}
__device__ __forceinline__ float4 ld16_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kSc1));
}
__device__ __forceinline__ float ld4_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kSc1));
}
__device__ __forceinline__ void st4_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), r, (int)off, 0, kSc1);
}
__device__ __forceinline__ void st2_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, unsigned short v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, (int)off, 0, kSc1);
}
__device__ __forceinline__ unsigned short ld2_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, kSc1);
}

__device__ __forceinline__ float half_to_float(unsigned short h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ unsigned short float_to_half(float f) {
  return __builtin_bit_cast(unsigned short, (_Float16)f);  // round to nearest even
}
__device__ __forceinline__ float bf16_to_float(unsigned short b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}
// Round a float to the nearest FP16 value (the reference's cast_value in mixed mode,
// src/cuda/Primitives.cuh:82-84).
template <int P>
__device__ __forceinline__ float cast(float v) {
  if constexpr (P == kMixed) return (float)(_Float16)v;
  return v;
}


// Cross-lane reductions without LDS round trips: DPP within rows of 16 lanes (quad_perm
// [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror, row_ror:8) and the gfx950 permlane
// swaps across rows (permlane16_swap pairs rows 0/1 and 2/3, permlane32_swap the halves).
// Every combining step adds (or maxes) a lane's value with its partner's, so the lanes of a
// group finish with the same bits.
template <int kCtrl>
__device__ __forceinline__ float dpp_get(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}
template <int kCtrl>
__device__ __forceinline__ float dpp_add(float v) { return v + dpp_get<kCtrl>(v); }
template <int kCtrl>
__device__ __forceinline__ float dpp_max(float v) { return fmaxf(v, dpp_get<kCtrl>(v)); }
// Both halves of a swap of v with itself. The vector elements are copied to scalars before
// any bit cast: __builtin_bit_cast applied to r[1] directly reads element 0.
template <bool k32>
__device__ __forceinline__ void swap_halves(float v, float& lo, float& hi) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  unsigned a, b;
  if constexpr (k32) {
    auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    a = r[0];
    b = r[1];
  } else {
    auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    a = r[0];
    b = r[1];
  }
  lo = __builtin_bit_cast(float, a);
  hi = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float pair16_add(float v) {
  float a, b;
  swap_halves<false>(v, a, b);
  return a + b;
}
__device__ __forceinline__ float pair32_add(float v) {
  float a, b;
  swap_halves<true>(v, a, b);
  return a + b;
}
__device__ __forceinline__ float pair16_max(float v) {
  float a, b;
  swap_halves<false>(v, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float pair32_max(float v) {
  float a, b;
  swap_halves<true>(v, a, b);
  return fmaxf(a, b);
}
// Sum over aligned groups of `group` lanes (a power of two up to 64), in every lane.
__device__ __forceinline__ float group_sum(float v, int group) {
  if (group >= 2) v = dpp_add<0xB1>(v);
  if (group >= 4) v = dpp_add<0x4E>(v);
  if (group >= 8) v = dpp_add<0x141>(v);
  if (group >= 16) v = dpp_add<0x140>(v);
  if (group >= 32) v = pair16_add(v);
  if (group >= 64) v = pair32_add(v);
  return v;
}
// Sum over the lanes that share lane % group (group a power of two up to 64).
__device__ __forceinline__ float column_sum(float v, int group) {
  for (int o = group; o < 8; o <<= 1) v += __shfl_xor(v, o);
  if (group <= 8) v = dpp_add<0x128>(v);  // row_ror:8 pairs lane i with lane i ^ 8
  if (group <= 16) v = pair16_add(v);
  if (group <= 32) v = pair32_add(v);
  return v;
}
__device__ __forceinline__ float wave_total(float v) {
  v = dpp_add<0xB1>(v);
  v = dpp_add<0x4E>(v);
  v = dpp_add<0x141>(v);
  v = dpp_add<0x140>(v);
  v = pair16_add(v);
  return pair32_add(v);
}
__device__ __forceinline__ float wave_top(float v) {
  v = dpp_max<0xB1>(v);
  v = dpp_max<0x4E>(v);
  v = dpp_max<0x141>(v);
  v = dpp_max<0x140>(v);
  v = pair16_max(v);
  return pair32_max(v);
}

// LDS-typed pointers: stores through them are ds_write, never flat (a flat access to LDS
// goes through the vector memory pipeline and waits behind outstanding global loads).
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) float lds_float;
typedef __attribute__((address_space(3))) v2f lds_v2f;
typedef __attribute__((address_space(3))) v4f lds_v4f;
__device__ __forceinline__ lds_float* to_lds(float* p) { return (lds_float*)p; }
// Load 16 bytes at byte offset off of buffer r (per lane) straight into LDS, no VGPR round
// trip: dst is the same for every lane of the wave, and lane i's bytes land at dst + 16 i.
__device__ __forceinline__ void ld16_to_lds(__amdgpu_buffer_rsrc_t r, float* dst, uint32_t off) {
  typedef __attribute__((address_space(3))) void lds_void;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)to_lds(dst), 16, (int)off, 0, 0, 1);
}
// Store two (four) consecutive floats to LDS at p (8- or 16-byte aligned).
__device__ __forceinline__ void lds_store2(float* p, float2 v) { *(lds_v2f*)p = v2f{v.x, v.y}; }
__device__ __forceinline__ void lds_store4(float* p, float4 v) { *(lds_v4f*)p = v4f{v.x, v.y, v.z, v.w}; }
// Load 16 bytes from LDS at p (16-byte aligned) as four words.
typedef unsigned v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 lds_load_u4(const float* p) {
  const v4u v = *(const __attribute__((address_space(3))) v4u*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}


__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Elements of the weight type per 16-byte chunk.
template <int P> struct Traits {
  static constexpr int kEpc = (P == kFp32) ? 4 : 8;
  static constexpr int kWBytes = (P == kFp32) ? 4 : 2;
  static constexpr int kKvBytes = (P == kMixed) ? 2 : 4;
};

// Dot product of one 16-byte weight chunk with the matching activations in LDS.
template <int P>
__device__ __forceinline__ float chunk_dot(uint4 w, const float* xs) {
  if constexpr (P == kFp32) {
    float4 x = *reinterpret_cast<const float4*>(xs);
    float s = __builtin_bit_cast(float, w.x) * x.x;
    s += __builtin_bit_cast(float, w.y) * x.y;
    s += __builtin_bit_cast(float, w.z) * x.z;
    s += __builtin_bit_cast(float, w.w) * x.w;
    return s;
  } else {
    float4 x0 = *reinterpret_cast<const float4*>(xs);
    float4 x1 = *reinterpret_cast<const float4*>(xs + 4);
    uint32_t u[4] = {w.x, w.y, w.z, w.w};
    float lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      if constexpr (P == kMixed) {
        lo[k] = half_to_float((unsigned short)(u[k] & 0xffffu));
        hi[k] = half_to_float((unsigned short)(u[k] >> 16));
      } else {
        lo[k] = __builtin_bit_cast(float, u[k] << 16);
        hi[k] = __builtin_bit_cast(float, u[k] & 0xffff0000u);
      }
    }
    float s = lo[0] * x0.x;
    s += hi[0] * x0.y;
    s += lo[1] * x0.z;
    s += hi[1] * x0.w;
    s += lo[2] * x1.x;
    s += hi[2] * x1.y;
    s += lo[3] * x1.z;
    s += hi[3] * x1.w;
    return s;
  }
}

template <int P>
__device__ __forceinline__ float load_weight_scalar(__amdgpu_buffer_rsrc_t wr, uint32_t off, int i) {
  if constexpr (P == kFp32) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wr, (int)(off + 4u * i), 0, 0));
  } else {
    unsigned short h = __builtin_amdgcn_raw_buffer_load_b16(wr, (int)(off + 2u * i), 0, 0);
    return P == kMixed ? half_to_float(h) : bf16_to_float(h);
  }
}

// ---------------------------------------------------------------------------------------------
// shared memory

struct Lds {
  float xs[kXs];                       // phase input vector (normalized where required)
  float qkv[3 * kMaxDim];              // attention: q, current k, current v
  float stage[kStreamWaves][kAttnLds]; // attention K/V chunk staging per stream wave
  float red[kWaves];                   // cross-wave scratch
};

// ---------------------------------------------------------------------------------------------
// phase description (pure arithmetic on the phase index)

struct Phase {
  int kind, layer;
};

__device__ __forceinline__ Phase phase_of(const StepArgs& a, int ph) {
  if (ph == 0) return {kInput, 0};
  int last = 1 + 5 * a.layers;
  if (ph >= last) return {kFinal, a.layers - 1};
  int l = (ph - 1) / 5;
  return {kQkv + (ph - 1) % 5, l};
}

// Matvec geometry of a phase: rows, padded row length, rows per unit, weight offset.
struct Mv {
  int rows, cols_p, unit;
  uint32_t woff;
};

template <int P>
__device__ __forceinline__ Mv matvec_of(const StepArgs& a, Phase p) {
  const LayerWeights& w = a.layer[p.layer];
  switch (p.kind) {
    case kInput: return {a.width, a.features_p, 1, a.w_input};
    case kQkv: return {3 * a.width, a.width_p, 2, w.qkv};
    case kOut: return {a.width, a.width_p, 1, w.out};
    case kGateUp: return {2 * a.ffn, a.width_p, 2, w.gateup};
    case kDown: return {a.width, a.ffn_p, 1, w.down};
    default: return {0, 0, 1, 0};
  }
}

// Work of one stream wave in a matvec phase. Rows are padded to whole slabs (1 KiB), so
// the U rows of a unit form U*S consecutive slabs.
struct WaveWork {
  int slabs_row;        // slabs per row (S)
  int per_unit;         // slabs per unit (U*S)
  int slabs;            // total slabs owned by this wave
  uint32_t base;        // byte offset of the first owned unit
  uint32_t unit_stride; // bytes between consecutive owned units
};

// Incremental cursor over a wave's slab stream (all fields wave-uniform).
struct SlabCursor {
  uint32_t unit_off;  // byte offset of the current unit
  int r;              // slab within the unit
  __device__ __forceinline__ uint32_t offset(int lane) const {
    return unit_off + (uint32_t)r * 1024u + (uint32_t)lane * 16u;
  }
  __device__ __forceinline__ void advance(const WaveWork& w) {
    if (++r == w.per_unit) {
      r = 0;
      unit_off += w.unit_stride;
    }
  }
};

__device__ __forceinline__ SlabCursor cursor_at(const WaveWork& w, int k) {
  int m = k / w.per_unit;
  return {w.base + (uint32_t)m * w.unit_stride, k - m * w.per_unit};
}

}  // namespace stamd
