// Phase bodies, grid barrier and kernels. Included once by runtime.hip.
#pragma once

#include "step_device.hpp"

namespace stamd {

struct LdsAll : Lds {
  float xres[kMaxDim];          // residual input x for OUT/DOWN epilogues
  float probs[kStreamWaves][64];
};

template <int P>
struct Ctx {
  const StepArgs& a;
  LdsAll& lds;
  __amdgpu_buffer_rsrc_t wr, kr, vr, sr;
  int g, lane, wave;
  unsigned long long t;
  int valid, slot;
  const float* input;  // event read by the INPUT phase

  __device__ __forceinline__ Ctx(const StepArgs& args, LdsAll& l, int grid_index)
      : a(args), lds(l), g(grid_index), lane(lane_id()), wave(wave_id()), t(0), valid(0), slot(0),
        input(args.input) {
    wr = make_rsrc(a.weights, a.weight_bytes);
    kr = make_rsrc(a.keys, a.cache_bytes);
    vr = make_rsrc(a.values, a.cache_bytes);
    sr = make_rsrc(a.scratch, a.scratch_bytes);
  }
  __device__ __forceinline__ void set_position(unsigned long long pos) {
    t = pos;
    valid = pos + 1 < (unsigned long long)a.window ? (int)(pos + 1) : a.window;
    slot = (int)(pos % (unsigned long long)a.window);
  }
  __device__ __forceinline__ float sload(uint32_t index) { return ld4_coherent(sr, index * 4u); }
  __device__ __forceinline__ void sstore(uint32_t index, float v) { st4_coherent(sr, index * 4u, v); }
};

__device__ __forceinline__ unsigned long long load_position(const StepArgs& a) {
  return __hip_atomic_load(a.position, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------------
// control wave: stage phase inputs into LDS

// Copy n floats (n padded to a multiple of 4 in scratch) from scratch into LDS.
template <int P>
__device__ __forceinline__ void stage_vector(Ctx<P>& c, uint32_t src, int n_p, float* dst) {
  for (int i = c.lane * 4; i < n_p; i += 256) {
    float4 v = ld16_coherent(c.sr, (src + (uint32_t)i) * 4u);
    *reinterpret_cast<float4*>(dst + i) = v;
  }
}

// RMSNorm of the width-vector in dst (in place), src/cuda/Primitives.cuh:122-135.
template <int P>
__device__ __forceinline__ void norm_in_place(Ctx<P>& c, float* v, uint32_t w_off) {
  const int d = c.a.width;
  float sum = 0.f;
  for (int i = c.lane; i < d; i += 64) sum += v[i] * v[i];
  sum = wave_sum(sum);
  float scale = 1.0f / sqrtf(sum / (float)d + c.a.epsilon);
  for (int i = c.lane; i < d; i += 64) {
    float w = load_weight_scalar<P>(c.wr, w_off, i);
    v[i] = cast<P>(v[i] * scale * w);
  }
}

template <int P>
__device__ __forceinline__ void stage_inputs(Ctx<P>& c, Phase p) {
  const StepArgs& a = c.a;
  switch (p.kind) {
    case kInput: {
      __amdgpu_buffer_rsrc_t ir = make_rsrc(c.input, (uint32_t)a.features_p * 4u);
      for (int i = c.lane * 4; i < a.features_p; i += 256)
        *reinterpret_cast<float4*>(c.lds.xs + i) = ld16_coherent(ir, (uint32_t)i * 4u);
      break;
    }
    case kQkv:
      stage_vector(c, a.s_x, a.width_p, c.lds.xs);
      norm_in_place(c, c.lds.xs, a.layer[p.layer].norm1);
      break;
    case kAttn:
      stage_vector(c, a.s_q, a.width_p, c.lds.qkv);
      stage_vector(c, a.s_kcur, a.width_p, c.lds.qkv + kMaxDim);
      stage_vector(c, a.s_vcur, a.width_p, c.lds.qkv + 2 * kMaxDim);
      break;
    case kOut:
      stage_vector(c, a.s_attn, a.width_p, c.lds.xs);
      stage_vector(c, a.s_x, a.width_p, c.lds.xres);
      break;
    case kGateUp:
      stage_vector(c, a.s_x, a.width_p, c.lds.xs);
      norm_in_place(c, c.lds.xs, a.layer[p.layer].norm2);
      break;
    case kDown:
      stage_vector(c, a.s_act, a.ffn_p, c.lds.xs);
      stage_vector(c, a.s_x, a.width_p, c.lds.xres);
      break;
    case kFinal:
      stage_vector(c, a.s_x, a.width_p, c.lds.xs);
      norm_in_place(c, c.lds.xs, a.w_final_norm);
      break;
  }
}

// ---------------------------------------------------------------------------------------------
// stream waves: matvec phases

template <int P>
__device__ __forceinline__ void prefetch_matvec(Ctx<P>& c, const WaveWork& w, uint4 (&ring)[kPF]) {
  if (w.slabs == 0) return;
  SlabCursor cur = cursor_at(w, 0);
  SlabCursor last = cursor_at(w, w.slabs - 1);
#pragma unroll
  for (int j = 0; j < kPF; j++) {
    ring[j] = ld16(c.wr, (j < w.slabs ? cur : last).offset(c.lane));
    cur.advance(w);
  }
}

// Attention work item geometry.
struct AttnWork {
  int wid, nw, items, nch;  // items owned by this wave; chunks per head
  int kchunks;              // 16-byte chunks of one K (or V) block
};

template <int P>
__device__ __forceinline__ AttnWork attn_work(const StepArgs& a, int grid, int g, int sw) {
  AttnWork w;
  w.nw = grid * kStreamWaves;
  w.wid = g + grid * sw;
  w.nch = (a.window + a.chunk - 1) / a.chunk;
  int total = a.heads * w.nch;
  w.items = total > w.wid ? (total - w.wid + w.nw - 1) / w.nw : 0;
  w.kchunks = (a.chunk * a.dim * Traits<P>::kKvBytes + 15) / 16;
  return w;
}

// Byte offset of the kk-th 16-byte chunk of the K/V block of item (h, ch), clamped.
template <int P>
__device__ __forceinline__ uint32_t attn_chunk_offset(const StepArgs& a, int layer, int h, int ch, int kk,
                                             int kchunks) {
  int k = kk < kchunks ? kk : kchunks - 1;
  uint32_t row0 = ((uint32_t)(layer * a.heads + h) * (uint32_t)a.window + (uint32_t)(ch * a.chunk));
  return row0 * (uint32_t)a.dim * Traits<P>::kKvBytes + (uint32_t)k * 16u;
}

template <int P>
__device__ __forceinline__ void prefetch_attn(Ctx<P>& c, int layer, const AttnWork& w, uint4 (&ring)[kPF]) {
  if (w.items == 0) return;
  int it = w.wid;
  int h = it / w.nch, ch = it - h * w.nch;
  // K block chunks at ring[0..kPF/2), V block at ring[kPF/2..kPF)
#pragma unroll
  for (int j = 0; j < kPF / 2; j++) {
    uint32_t off = attn_chunk_offset<P>(c.a, layer, h, ch, c.lane + 64 * j, w.kchunks);
    ring[j] = ld16(c.kr, off);
    ring[kPF / 2 + j] = ld16(c.vr, off);
  }
}

template <int P>
__device__ __forceinline__ void prefetch(Ctx<P>& c, Phase p, int grid, uint4 (&ring)[kPF]) {
  int sw = c.wave - 1;
  if (p.kind == kAttn) {
    AttnWork w = attn_work<P>(c.a, grid, c.g, sw);
    prefetch_attn(c, p.layer, w, ring);
  } else if (p.kind != kFinal) {
    Mv m = matvec_of<P>(c.a, p);
    WaveWork w = work_of<P>(c.a, m, grid, c.g, sw);
    prefetch_matvec(c, w, ring);
  }
}

// Epilogue of one unit (lane 0 only). s0/s1 are the row sums.
template <int P>
__device__ __forceinline__ void epilogue(Ctx<P>& c, Phase p, int unit, float s0, float s1) {
  const StepArgs& a = c.a;
  switch (p.kind) {
    case kInput:
      c.sstore(a.s_x + unit, cast<P>(s0));
      break;
    case kQkv: {
      int r0 = unit * 2;
      int sec = r0 / a.width;
      int i = r0 - sec * a.width;
      float va = cast<P>(s0), vb = cast<P>(s1);
      int h = i / a.dim;
      int e = i - h * a.dim;
      uint32_t kv = ((uint32_t)(p.layer * a.heads + h) * (uint32_t)a.window + (uint32_t)c.slot) *
                        (uint32_t)a.dim + (uint32_t)e;
      if (sec < 2) {
        // RoPE on the adjacent pair (i, i+1), src/cuda/Primitives.cuh:148-159
        float angle = (float)c.t * a.rope_freq[e >> 1];
        float co = cosf(angle), si = sinf(angle);
        float ra = cast<P>(va * co - vb * si);
        float rb = cast<P>(va * si + vb * co);
        if (sec == 0) {
          c.sstore(a.s_q + i, ra);
          c.sstore(a.s_q + i + 1, rb);
        } else {
          c.sstore(a.s_kcur + i, ra);
          c.sstore(a.s_kcur + i + 1, rb);
          if constexpr (P == kMixed) {
            st2_coherent(c.kr, kv * 2u, float_to_half(ra));
            st2_coherent(c.kr, kv * 2u + 2u, float_to_half(rb));
          } else {
            st4_coherent(c.kr, kv * 4u, ra);
            st4_coherent(c.kr, kv * 4u + 4u, rb);
          }
        }
      } else {
        c.sstore(a.s_vcur + i, va);
        c.sstore(a.s_vcur + i + 1, vb);
        if constexpr (P == kMixed) {
          st2_coherent(c.vr, kv * 2u, float_to_half(va));
          st2_coherent(c.vr, kv * 2u + 2u, float_to_half(vb));
        } else {
          st4_coherent(c.vr, kv * 4u, va);
          st4_coherent(c.vr, kv * 4u + 4u, vb);
        }
      }
      break;
    }
    case kOut: {
      float v = cast<P>(c.lds.xres[unit] + cast<P>(s0));
      c.sstore(a.s_x + unit, v);
      break;
    }
    case kGateUp: {
      float gv = cast<P>(s0), uv = cast<P>(s1);
      c.sstore(a.s_act + unit, cast<P>((gv / (1.0f + expf(-gv))) * uv));
      break;
    }
    case kDown: {
      float v = cast<P>(c.lds.xres[unit] + cast<P>(s0));
      c.sstore(a.s_x + unit, v);
      c.sstore(a.s_hidden + (uint32_t)p.layer * a.width + unit, v);
      break;
    }
    default:
      break;
  }
}

template <int P>
__device__ __forceinline__ void compute_matvec(Ctx<P>& c, Phase p, int grid, uint4 (&ring)[kPF]) {
  Mv m = matvec_of<P>(c.a, p);
  WaveWork w = work_of<P>(c.a, m, grid, c.g, c.wave - 1);
  if (w.slabs == 0) return;
  SlabCursor refill = cursor_at(w, kPF);
  int unit = w.wid;  // global unit index of the unit being reduced
  int ru = 0, s = 0; // row within the unit, slab within the row
  float acc0 = 0.f, acc1 = 0.f;
  const float* xs = c.lds.xs + c.lane * Traits<P>::kEpc;
  for (int base = 0; base < w.slabs; base += kPF) {
#pragma unroll
    for (int j = 0; j < kPF; j++) {
      if (base + j < w.slabs) {
        float d = chunk_dot<P>(ring[j], xs + s * 64 * Traits<P>::kEpc);
        if (ru == 0) acc0 += d; else acc1 += d;
        if (base + j + kPF < w.slabs) {
          ring[j] = ld16(c.wr, refill.offset(c.lane));
          refill.advance(w);
        }
        if (++s == w.slabs_row) {
          s = 0;
          if (++ru == m.unit) {
            ru = 0;
            float s0 = wave_sum(acc0);
            float s1 = m.unit == 2 ? wave_sum(acc1) : 0.f;
            if (c.lane == 0) epilogue(c, p, unit, s0, s1);
            unit += w.nw;
            acc0 = 0.f;
            acc1 = 0.f;
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// stream waves: attention phase (src/cuda/Primitives.cuh:167-219, src/cpu/Cpu.cpp:97-109)

// Write a prefetched K or V block (register ring half) into this wave's LDS stage as
// [chunk rows][dim + 4] floats. Row/column of each element advance incrementally.
template <int P>
__device__ __forceinline__ void block_to_lds(Ctx<P>& c, const uint4* part, int kchunks, float* stage) {
  const int dim = c.a.dim, stride = dim + 4, chunk = c.a.chunk;
  constexpr int kPer = 16 / Traits<P>::kKvBytes;
  const int step_el = 64 * kPer;
  const int step_row = step_el / dim, step_col = step_el - step_row * dim;
  int row = (c.lane * kPer) / dim;
  int col = c.lane * kPer - row * dim;
#pragma unroll
  for (int j = 0; j < kPF / 2; j++) {
    if (c.lane + 64 * j < kchunks) {
      float v[kPer];
      if constexpr (P == kMixed) {
        uint32_t u[4] = {part[j].x, part[j].y, part[j].z, part[j].w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          v[2 * e] = half_to_float((unsigned short)(u[e] & 0xffffu));
          v[2 * e + 1] = half_to_float((unsigned short)(u[e] >> 16));
        }
      } else {
        v[0] = __builtin_bit_cast(float, part[j].x);
        v[1] = __builtin_bit_cast(float, part[j].y);
        v[2] = __builtin_bit_cast(float, part[j].z);
        v[3] = __builtin_bit_cast(float, part[j].w);
      }
      int r = row, cc = col;
#pragma unroll
      for (int e = 0; e < kPer; e++) {
        if (r < chunk) stage[r * stride + cc] = v[e];
        if (++cc == dim) {
          cc = 0;
          r++;
        }
      }
    }
    col += step_col;
    row += step_row;
    if (col >= dim) {
      col -= dim;
      row++;
    }
  }
}

// Load the K or V block of item (h, ch) directly (items beyond the first of a wave).
template <int P>
__device__ __forceinline__ void load_block(Ctx<P>& c, __amdgpu_buffer_rsrc_t r, int layer, int h, int ch,
                                  int kchunks, uint4* part) {
#pragma unroll
  for (int j = 0; j < kPF / 2; j++)
    part[j] = ld16(r, attn_chunk_offset<P>(c.a, layer, h, ch, c.lane + 64 * j, kchunks));
}

template <int P>
__device__ __forceinline__ void compute_attn(Ctx<P>& c, Phase p, int grid, uint4 (&ring)[kPF]) {
  const StepArgs& a = c.a;
  AttnWork w = attn_work<P>(a, grid, c.g, c.wave - 1);
  const int dim = a.dim, stride = dim + 4, chunk = a.chunk;
  float* stage = c.lds.stage[c.wave - 1];
  float* probs = c.lds.probs[c.wave - 1];
  const float* q_all = c.lds.qkv;
  const float* k_cur = c.lds.qkv + kMaxDim;
  const float* v_cur = c.lds.qkv + 2 * kMaxDim;
  const int nactive = (c.valid + chunk - 1) / chunk;
  const float inv_scale_div = sqrtf((float)dim);
  for (int m = 0; m < w.items; m++) {
    int it = w.wid + w.nw * m;
    int h = it / w.nch, ch = it - h * w.nch;
    if (ch >= nactive) continue;
    if (m > 0) {
      load_block<P>(c, c.kr, p.layer, h, ch, w.kchunks, ring);
      load_block<P>(c, c.vr, p.layer, h, ch, w.kchunks, ring + kPF / 2);
    }
    int row0 = ch * chunk;
    int rows = c.valid - row0 < chunk ? c.valid - row0 : chunk;  // valid slots are [0, valid)
    // K block -> LDS, then patch in the slot written this step
    block_to_lds<P>(c, ring, w.kchunks, stage);
    int cur = c.slot - row0;
    if (cur >= 0 && cur < chunk)
      for (int i = c.lane; i < dim; i += 64) stage[cur * stride + i] = k_cur[h * dim + i];
    __builtin_amdgcn_wave_barrier();
    float logit = -INFINITY;
    if (c.lane < rows) {
      const float* kr = stage + c.lane * stride;
      const float* q = q_all + h * dim;
      float dot = 0.f;
      for (int i = 0; i < dim; i++) dot += q[i] * kr[i];
      logit = dot / inv_scale_div;
    }
    float mx = wave_max(logit);
    float pr = c.lane < rows ? expf(logit - mx) : 0.f;
    float total = wave_sum(pr);
    if (c.lane < 64) probs[c.lane] = pr;
    __builtin_amdgcn_wave_barrier();
    // V block -> LDS (overwrites K)
    block_to_lds<P>(c, ring + kPF / 2, w.kchunks, stage);
    if (cur >= 0 && cur < chunk)
      for (int i = c.lane; i < dim; i += 64) stage[cur * stride + i] = v_cur[h * dim + i];
    __builtin_amdgcn_wave_barrier();
    uint32_t pbase = ((uint32_t)(h * w.nch + ch)) * (uint32_t)(dim + 2);
    for (int i = c.lane; i < dim; i += 64) {
      float o = 0.f;
      for (int j = 0; j < rows; j++) o += probs[j] * stage[j * stride + i];
      c.sstore(a.s_partial + pbase + 2 + i, o);
    }
    if (c.lane == 0) {
      c.sstore(a.s_partial + pbase, mx);
      c.sstore(a.s_partial + pbase + 1, total);
    }
    // Publish the partial, then count it; the last chunk of the head combines.
    __builtin_amdgcn_s_waitcnt(0);
    unsigned old = 0;
    if (c.lane == 0)
      old = __hip_atomic_fetch_add(a.head_count + h * 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __shfl(old, 0);
    if ((int)old == nactive - 1) {
      float big = -INFINITY;
      for (int cc = 0; cc < nactive; cc++)
        big = fmaxf(big, c.sload(a.s_partial + (uint32_t)(h * w.nch + cc) * (uint32_t)(dim + 2)));
      float denom = 0.f;
      for (int cc = 0; cc < nactive; cc++) {
        uint32_t b = (uint32_t)(h * w.nch + cc) * (uint32_t)(dim + 2);
        denom += c.sload(a.s_partial + b + 1) * expf(c.sload(a.s_partial + b) - big);
      }
      for (int i = c.lane; i < dim; i += 64) {
        float o = 0.f;
        for (int cc = 0; cc < nactive; cc++) {
          uint32_t b = (uint32_t)(h * w.nch + cc) * (uint32_t)(dim + 2);
          o += c.sload(a.s_partial + b + 2 + i) * expf(c.sload(a.s_partial + b) - big);
        }
        c.sstore(a.s_attn + h * dim + i, cast<P>(o / denom));
      }
      if (c.lane == 0)
        __hip_atomic_store(a.head_count + h * 32, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// Final phase (workgroup 0, control wave): score = W_score . norm(x), not cast; position++.
template <int P>
__device__ __forceinline__ void compute_final(Ctx<P>& c) {
  const StepArgs& a = c.a;
  const int chunks = a.width_p / Traits<P>::kEpc;
  float acc = 0.f;
  for (int s = 0; s * 64 < chunks; s++) {
    int chunk = s * 64 + c.lane;
    bool live = chunk < chunks;
    int cc = live ? chunk : chunks - 1;
    uint4 wv = ld16(c.wr, a.w_score + (uint32_t)cc * 16u);
    float d = chunk_dot<P>(wv, c.lds.xs + cc * Traits<P>::kEpc);
    acc += live ? d : 0.f;
  }
  float score = wave_sum(acc);
  if (c.lane == 0) {
    c.sstore(a.s_score, score);
    __hip_atomic_store(a.position, c.t + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int P>
__device__ __forceinline__ void compute(Ctx<P>& c, Phase p, int grid, uint4 (&ring)[kPF]) {
  if (p.kind == kAttn) compute_attn(c, p, grid, ring);
  else if (p.kind != kFinal) compute_matvec(c, p, grid, ring);
}

// ---------------------------------------------------------------------------------------------
// grid barrier: per-workgroup flags, written through to the device coherence point

__device__ __forceinline__ void grid_arrive(const StepArgs& a, int g, unsigned epoch) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's stores are complete
  __builtin_amdgcn_s_barrier();
  if (threadIdx.x == 0)
    __hip_atomic_store(a.flags + g * kFlagStride, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Control wave only. Returns false on timeout (sets the sticky error bit).
__device__ __forceinline__ bool grid_wait(const StepArgs& a, int grid, unsigned epoch) {
  const int lane = lane_id();
  unsigned long long start = wall_clock64();
  while (true) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < kMaxGrid / 64; k++) {
      int i = lane + 64 * k;
      if (k * 64 < grid) {
        int j = i < grid ? i : grid - 1;
        unsigned f = __hip_atomic_load(a.flags + j * kFlagStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = ok && (int)(f - epoch) >= 0;
      }
    }
    if (__all(ok)) return true;
    if (wall_clock64() - start > a.spin_limit) {
      if (lane == 0) __hip_atomic_fetch_or(a.error, kErrBarrierTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
  __builtin_amdgcn_s_barrier();
}

// ---------------------------------------------------------------------------------------------
// kernels

// One phase per launch (staged and graph backends).
template <int P>
__global__ __launch_bounds__(kThreads) void phase_kernel(const StepArgs* __restrict__ ap, int ph) {
  const StepArgs& a = *ap;
  __shared__ LdsAll lds;
  Ctx<P> c(a, lds, (int)blockIdx.x);
  c.set_position(load_position(a));
  Phase p = phase_of(a, ph);
  if (p.kind == kFinal && blockIdx.x != 0) return;
  uint4 ring[kPF];
  if (c.wave == 0) stage_inputs(c, p);
  else prefetch(c, p, (int)gridDim.x, ring);
  lds_barrier();
  if (p.kind == kFinal) {
    if (c.wave == 0) compute_final(c);
    return;
  }
  if (c.wave != 0) compute(c, p, (int)gridDim.x, ring);
}

// One forward over the device-held state. Used by the fused, persistent and trace kernels.
// The epoch argument counts barriers; returns the next epoch.
template <int P>
__device__ __forceinline__ unsigned forward(Ctx<P>& c, int grid, unsigned epoch, uint4 (&ring)[kPF],
                                   bool barrier_after_final) {
  const StepArgs& a = c.a;
  const int nph = 5 * a.layers + 2;
  if (c.wave == 0) stage_inputs(c, phase_of(a, 0));
  else prefetch(c, phase_of(a, 0), grid, ring);
  lds_barrier();
  for (int ph = 0; ph + 1 < nph; ph++) {
    Phase p = phase_of(a, ph);
    if (c.wave != 0) compute(c, p, grid, ring);
    grid_arrive(a, c.g, ++epoch);
    Phase next = phase_of(a, ph + 1);
    if (next.kind == kFinal && c.g != 0) {
      if (barrier_after_final) {
        // Nothing to publish: arrive at once for the post-FINAL barrier and wait for
        // workgroup 0 to finish the score and the position update.
        grid_arrive(a, c.g, ++epoch);
        if (c.wave == 0) grid_wait(a, grid, epoch);
        __builtin_amdgcn_s_barrier();
      }
      return epoch;
    }
    if (c.wave == 0) {
      grid_wait(a, grid, epoch);
      stage_inputs(c, next);
    } else {
      prefetch(c, next, grid, ring);
    }
    lds_barrier();
  }
  // FINAL (workgroup 0 only)
  if (c.wave == 0) compute_final(c);
  if (barrier_after_final) {
    grid_arrive(a, c.g, ++epoch);
    if (c.wave == 0) grid_wait(a, grid, epoch);
    __builtin_amdgcn_s_barrier();
  }
  return epoch;
}

template <int P>
__global__ __launch_bounds__(kThreads) void fused_kernel(const StepArgs* __restrict__ ap) {
  const StepArgs& a = *ap;
  __shared__ LdsAll lds;
  Ctx<P> c(a, lds, (int)blockIdx.x);
  c.set_position(load_position(a));
  unsigned epoch0 = __hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint4 ring[kPF];
  unsigned end = forward(c, (int)gridDim.x, epoch0, ring, false);
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(a.epoch, end, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Device-only timing loop over a preloaded trace: per-event wall-clock stamps.
template <int P>
__global__ __launch_bounds__(kThreads) void trace_kernel(const StepArgs* __restrict__ ap, const float* events,
                                                         int count, unsigned long long* stamps) {
  const StepArgs& a = *ap;
  __shared__ LdsAll lds;
  Ctx<P> c(a, lds, (int)blockIdx.x);
  unsigned epoch = __hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint4 ring[kPF];
  for (int e = 0; e < count; e++) {
    if (blockIdx.x == 0 && threadIdx.x == 0) stamps[e] = wall_clock64();
    c.set_position(load_position(a));
    c.input = events + (size_t)e * a.features_p;
    epoch = forward(c, (int)gridDim.x, epoch, ring, true);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    stamps[count] = wall_clock64();
    __hip_atomic_store(a.epoch, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Zero K/V, hidden state, attention counters and the position (src/cuda/Primitives.cuh:280-292).
__global__ void reset_kernel(const StepArgs* __restrict__ ap) {
  const StepArgs& a = *ap;
  size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  uint32_t* k = reinterpret_cast<uint32_t*>(a.keys);
  uint32_t* v = reinterpret_cast<uint32_t*>(a.values);
  for (size_t i = tid; i < a.cache_bytes / 4; i += stride) { k[i] = 0; v[i] = 0; }
  for (size_t i = tid; i < (size_t)a.layers * a.width; i += stride) a.scratch[a.s_hidden + i] = 0.f;
  for (size_t i = tid; i < (size_t)a.heads * 32; i += stride) a.head_count[i] = 0;
  if (tid == 0) *a.position = 0;
}

}  // namespace stamd
