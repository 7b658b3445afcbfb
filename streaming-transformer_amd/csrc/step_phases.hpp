// Phase bodies and kernels. Included once by runtime.hip.
//
// Cross-workgroup dataflow uses epoch-tagged vectors: every element of x, q, k, v, attn and
// act is one 8-byte word (epoch << 32 | float bits), written with a single write-through
// store and read with agent-coherent loads. A consumer polls the elements it needs until
// every tag equals the epoch of the producing phase, so there is no grid barrier, no store
// acknowledgement wait before publishing and no separate staging round trip. Each phase p
// of a step has epoch base + p; base advances by phases + 1 per step.
//
// Reuse safety: a tagged vector is overwritten only in a phase whose writers have
// consumed outputs that every reader of the previous value produced after its read
// (x: INPUT/OUT/DOWN, q/k/v: QKV, attn: ATTN, act: GATEUP), so no reader can observe a
// newer epoch than the one it waits for. Workgroups without work in a phase skip its
// reads. The K/V ring row of the current slot is written by the attention item that owns
// the slot, before that item's partial is counted, so the row is complete before anything
// downstream of the attention output runs.
#pragma once

#include "step_device.hpp"

namespace stamd {

// A stream wave's share of one matvec kind. The share depends on the kind, the grid and the
// wave, not on the layer (which only moves the weight base), so a forward computes it once.
struct WaveSplit {
  int slabs, per_unit, slabs_row, unit0, unit;
  uint32_t base_rel, unit_stride;  // first owned unit from the matrix start; stride between units
  uint32_t refill_off, last_off;   // unit offsets (from the matrix start) of slab kPF and the last slab
  int refill_r, last_r;            // slab within that unit
};

struct LdsAll {
  float xs[2][kXs];                      // phase input vector, double buffered by phase parity
  float xres[2][kMaxDim];                // x before this layer (OUT residual) and after OUT (DOWN residual)
  float qkv[3 * kMaxDim];                // attention LDS path: q, k, v of the step
  float stage[kStreamWaves][kAttnLds];   // attention LDS path: per-wave K/V staging
  float probs[kStreamWaves][64];
  float rope_cos[kMaxDim / 2];           // RoPE cos / sin of this step's position per pair
  float rope_sin[kMaxDim / 2];
  WaveSplit split[kStreamWaves][kFinal];  // per stream wave and matvec kind (forward only)
  unsigned done[2];                      // stream waves finished with the phase of this parity
  unsigned refilled[2];                  // waves that have issued all their refills in the phase
  unsigned helped[3];                    // epochs of the wide-vector chunks the helper waves staged
  int cmd;                               // persistent worker: the current mailbox command
  unsigned stamps[kStampPhases][kStamps];  // profiling: low 32 bits of the wall clock
};

// Bit 2 of a kernel's A parameter: the weights are streamed with non-temporal loads.
constexpr int kWeightNt = 4;
constexpr bool weight_nt(int A) { return (A & kWeightNt) != 0; }

template <int P>
struct Ctx {
  const StepArgs& a;
  LdsAll& lds;
  __amdgpu_buffer_rsrc_t wr, kr, vr, sr, tr;
  int g, grid, lane, wave;
  unsigned long long t;  // position of the step
  int valid, slot;
  unsigned base;         // epoch of phase 0 of this step
  bool dead;             // a poll timed out; stop waiting
  const float* input;    // event read by the INPUT phase
  bool tagged_input;     // the event is the tagged vector t_in (persistent worker)
  bool split_wide;       // a stream wave polls the odd 1024-piece chunks of wide vectors
  bool kv_lds;           // K/V of each stream wave's first attention item are in its LDS stage
  bool split_ready;      // lds.split holds this wave's matvec shares
  int phase_parity;      // parity of the phase a stream wave computes (forward)
#if STAMD_POLL_STAMPS
  int pph = -1;  // phase whose staging stamps the polls record (control wave)
#endif

  __device__ __forceinline__ Ctx(const StepArgs& args, LdsAll& l, int grid_index, int grid_size)
      : a(args), lds(l), g(grid_index), grid(grid_size), lane(lane_id()), wave(wave_id()), t(0), valid(0),
        slot(0), base(0), dead(false), input(args.input), tagged_input(false), split_wide(false), kv_lds(false), split_ready(false),
        phase_parity(0) {
    wr = make_rsrc(a.weights, a.weight_bytes);
    kr = make_rsrc(a.keys, a.cache_bytes);
    vr = make_rsrc(a.values, a.cache_bytes);
    sr = make_rsrc(a.scratch, a.scratch_bytes);
    tr = make_rsrc(a.tagged, a.tagged_bytes);
  }
  __device__ __forceinline__ void set_position(unsigned long long pos) {
    t = pos;
    valid = pos + 1 < (unsigned long long)a.window ? (int)(pos + 1) : a.window;
    slot = (int)(pos % (unsigned long long)a.window);
  }
  __device__ __forceinline__ unsigned epoch(int ph) const { return base + (unsigned)ph; }
  __device__ __forceinline__ float sload(uint32_t index) { return ld4_coherent(sr, index * 4u); }
  __device__ __forceinline__ void sstore(uint32_t index, float v) { st4_coherent(sr, index * 4u, v); }
  // Publish one element of a tagged vector.
  __device__ __forceinline__ void tstore(uint32_t index, unsigned ep, float v) {
    typedef int v2i __attribute__((ext_vector_type(2)));
    v2i w = {__builtin_bit_cast(int, v), (int)ep};
    __builtin_amdgcn_raw_buffer_store_b64(w, tr, (int)(index * 8u), 0, kSc1);
  }
  __device__ __forceinline__ uint2 tload(uint32_t index) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(tr, (int)(index * 8u), 0, kSc1));
  }
  __device__ __forceinline__ void timeout() {
    if (lane == 0) __hip_atomic_fetch_or(a.error, kErrPollTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    dead = true;
  }
  // True once a poll started at `start` has run past the spin limit (and records it).
  __device__ __forceinline__ bool expired(unsigned long long start) {
    if (wall_clock64() - start > a.spin_limit) {
      timeout();
      return true;
    }
    return false;
  }
};

// Position and epoch are read by every lane; readfirstlane tells the compiler they are
// wave-uniform, so everything derived from them (attention geometry, offsets) stays in
// scalar registers.
__device__ __forceinline__ unsigned long long load_position(const StepArgs& a) {
  unsigned long long v = __hip_atomic_load(a.position, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v), hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
  return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned load_epoch(const StepArgs& a) {
  return __builtin_amdgcn_readfirstlane(__hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// Phase indices within a step.
__device__ __forceinline__ int ph_index(int kind, int layer) { return kind == kInput ? 0 : 1 + 5 * layer + (kind - kQkv); }
__device__ __forceinline__ int ph_final(const StepArgs& a) { return 1 + 5 * a.layers; }
// Phase that last wrote x before `layer`'s QKV phase.
__device__ __forceinline__ int ph_x_before(int layer) { return layer == 0 ? 0 : ph_index(kDown, layer - 1); }

// Profiling stamp k of phase `ph` for this workgroup, when the launch carries a stamp buffer.
// Slots: 0 phase start, 1 stream wave 1 done, 2 all stream waves done, 3 next phase's inputs
// staged, 4-6 progress of stream wave 1 within the phase, 7 stream wave 1 has issued the
// next phase's prefetch. Stamps go to LDS and are written out once, after the step, so that
// recording them puts no stores into the memory pipeline the step is using.
template <int P>
__device__ __forceinline__ void lstamp(Ctx<P>& c, int ph, int k) {
  if (c.a.stamps && ph < kStampPhases) c.lds.stamps[ph][k] = (unsigned)wall_clock64();
}

template <int P>
__device__ __forceinline__ void stamp(Ctx<P>& c, Phase p, int k) {
  if (c.lane == 0) lstamp(c, ph_index(p.kind, p.layer), k);
}

// A global (not flat) 64-bit store: it counts only against vmcnt.
__device__ __forceinline__ void put_global(unsigned long long* base, size_t index, unsigned long long v) {
  typedef __attribute__((address_space(1))) unsigned long long gu64;
  ((gu64*)base)[index] = v;
}

// ---------------------------------------------------------------------------------------------
// polling tagged vectors

constexpr int kPollSleep = 2;  // s_sleep units (64 clocks each) between failed polls

// Wait until elements [2*p0, 2*(p0+np)) of tagged vector `tv` carry epoch `ep` (elements at or
// beyond `n` are padding and are not checked); the pieces stay in buf. One wave; NP 16-byte
// pieces (2 elements) per lane per pass: lane l holds pieces l, l + 64, ...
template <int P, int NP>
__device__ __forceinline__ void poll_regs(Ctx<P>& c, uint32_t tv, int n, int p0, int np, unsigned ep, uint4 (&buf)[NP]) {
  unsigned long long start = wall_clock64();
#if STAMD_POLL_STAMPS
  bool first_pass = p0 == 0;
#endif
  // One lane offset; piece k adds k * 1 KiB as the scalar offset. Pieces past np read
  // whatever follows in the tagged arena (or 0 past its end) and are ignored.
  const uint32_t voff = (tv + 2u * (uint32_t)(p0 + c.lane)) * 8u;
  while (true) {
#pragma unroll
    for (int k = 0; k < NP; k++)
      buf[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(c.tr, (int)voff, 1024 * k, kSc1));
    // The epoch check. Staging polls (up to 8 pieces per lane) use bitwise operators, which
    // compile to lane-mask arithmetic; a short-circuit check compiled to one divergent branch
    // per piece and kept every pass long. Wide polls (16 pieces per lane: the FFN vector) keep
    // the short-circuit form. Measured Large p50: bitwise everywhere 381 us, short-circuit
    // everywhere 380 us, this split 362 us; why the wide polls prefer it is not pinned down.
    bool ok = true;
#pragma unroll
    for (int k = 0; k < NP; k++) {
      const int pc = c.lane + 64 * k;
      const int e0 = 2 * (p0 + pc);
      if constexpr (NP > 8) {
        ok = ok && (pc >= np || ((e0 >= n || buf[k].y == ep) && (e0 + 1 >= n || buf[k].w == ep)));
      } else {
        const bool cur = ((e0 >= n) | (buf[k].y == ep)) & ((e0 + 1 >= n) | (buf[k].w == ep));
        ok = ok & ((pc >= np) | cur);
      }
    }
#if STAMD_POLL_STAMPS
    if (c.pph >= 0 && c.lane == 0) {
      if (first_pass) lstamp(c, c.pph, 8);
      lstamp(c, c.pph, 9);
    }
    first_pass = false;
#endif
    if (__all(ok) || c.dead) break;
    if (wall_clock64() - start > c.a.spin_limit) {
      c.timeout();
      break;
    }
    __builtin_amdgcn_s_sleep(kPollSleep);
  }
#if STAMD_POLL_STAMPS
  if (c.pph >= 0 && c.lane == 0) lstamp(c, c.pph, 10);
#endif
}

// Value pair of piece k (0 for padding at or beyond n).
__device__ __forceinline__ float2 piece_values(uint4 b, int e0, int n) {
  return make_float2(e0 < n ? __builtin_bit_cast(float, b.x) : 0.f, e0 + 1 < n ? __builtin_bit_cast(float, b.z) : 0.f);
}

// poll_regs, then write the values (0 for padding) to dst[0 ..) in LDS. With kAll every lane
// stores all NP pieces (zeros past np): no divergent branch per piece, for callers whose
// destination has room for 64 NP pieces.
template <int P, int NP, bool kAll = false>
__device__ __forceinline__ void poll_pieces(Ctx<P>& c, uint32_t tv, int n, int p0, int np, unsigned ep, float* dst) {
  uint4 buf[NP];
  poll_regs<P, NP>(c, tv, n, p0, np, ep, buf);
#pragma unroll
  for (int k = 0; k < NP; k++) {
    int pc = c.lane + 64 * k;
    if (kAll || pc < np) lds_store2(dst + 2 * pc, piece_values(buf[k], 2 * (p0 + pc), n));
  }
}

// Chunks first, first + step, ... of CH pieces of a wide vector into the activation buffer
// dst. The FFN width is at most 4096 (Runtime's config check): at most 2048 pieces, so a
// whole-chunk store (1024 or 512 pieces) ends at float 4096 at most, inside the buffer.
template <int P, int CH = 1024>
__device__ __forceinline__ void poll_chunks(Ctx<P>& c, uint32_t tv, int n, int pieces, int first, int step, unsigned ep,
                                            float* dst) {
  static_assert(2048 % CH == 0 && 2 * 2048 <= kXs, "whole chunks of a 2048-piece vector fit the activation buffer");
  for (int p0 = first * CH; p0 < pieces; p0 += step * CH)
    poll_pieces<P, CH / 64, true>(c, tv, n, p0, pieces - p0 < CH ? pieces - p0 : CH, ep, dst + 2 * p0);
}

// Whole vector of n elements padded to n_p (a multiple of 256) into dst[0 .. n_p). With
// `split`, a vector of more than 512 pieces is polled in 512-piece chunks shared with up to
// three helper stream waves (see help_stage): this wave polls chunk 0 and waits for the
// helpers' chunks 1-3. Smaller polls per wave, issued by four waves at once, cut the FFN
// vector's exchange (Large 361 -> 353 us, Main 168 -> 157 us against two 1024-piece chunks).
template <int P>
__device__ __forceinline__ void poll_vector(Ctx<P>& c, uint32_t tv, int n, int n_p, unsigned ep, float* dst,
                                            bool split = false) {
  const int pieces = n_p / 2;
  if (pieces <= 512) {
    poll_pieces<P, 8>(c, tv, n, 0, pieces, ep, dst);
  } else if (!split) {
    poll_chunks(c, tv, n, pieces, 0, 1, ep, dst);
  } else {
    poll_chunks<P, 512>(c, tv, n, pieces, 0, 4, ep, dst);
    const int chunks = (pieces + 511) / 512;
    const unsigned long long start = wall_clock64();
    for (int hi = 0; hi + 1 < chunks && hi < 3; hi++) {
      while (__hip_atomic_load(&c.lds.helped[hi], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != ep && !c.dead) {
        if (c.expired(start)) {
          c.timeout();
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
  }
}

// Elements [first, first + count) of tagged vector `tv` into dst[0 .. count).
template <int P>
__device__ __forceinline__ void poll_range(Ctx<P>& c, uint32_t tv, int first, int count, unsigned ep, float* dst) {
  constexpr int NE = 4;
  for (int e0 = 0; e0 < count; e0 += 64 * NE) {
    uint2 buf[NE];
    unsigned long long start = wall_clock64();
    while (true) {
#pragma unroll
      for (int k = 0; k < NE; k++) {
        int e = e0 + c.lane + 64 * k;
        int el = e < count ? e : count - 1;
        buf[k] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                               c.tr, (int)((tv + (uint32_t)(first + el)) * 8u), 0, kSc1));
      }
      bool ok = true;
#pragma unroll
      for (int k = 0; k < NE; k++) ok = ok && (e0 + c.lane + 64 * k >= count || buf[k].y == ep);
      if (__all(ok) || c.dead) break;
      if (wall_clock64() - start > c.a.spin_limit) {
        c.timeout();
        break;
      }
      __builtin_amdgcn_s_sleep(kPollSleep);
    }
    lds_float* d = to_lds(dst);
#pragma unroll
    for (int k = 0; k < NE; k++) {
      int e = e0 + c.lane + 64 * k;
      if (e < count) d[e] = __builtin_bit_cast(float, buf[k].x);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// control wave: stage phase inputs into LDS

// Pieces per lane of a staged vector of up to kMaxDim elements.
constexpr int kStageNP = kMaxDim / 128;

// Norm weights in the piece layout of poll_regs: lane l, piece k holds elements
// 2(l + 64k) and 2(l + 64k) + 1 (clamped; the padding they multiply is 0).
template <int P>
__device__ __forceinline__ void load_norm(Ctx<P>& c, uint32_t w_off, float2 (&w)[kStageNP]) {
  const int d = c.a.width;
#pragma unroll
  for (int k = 0; k < kStageNP; k++) {
    int e0 = 2 * (c.lane + 64 * k);
    w[k] = make_float2(load_weight_scalar<P>(c.wr, w_off, e0 < d ? e0 : d - 1),
                       load_weight_scalar<P>(c.wr, w_off, e0 + 1 < d ? e0 + 1 : d - 1));
  }
}

// Stage one tagged vector of n elements (np pieces, np <= 64 * kStageNP) from registers:
// the raw values to `raw` (when not null) and to `xs`, RMS-normalized when `norm`
// (src/cuda/Primitives.cuh:122-135: s = 1/sqrt(sum(v^2)/d + eps), v = cast(v * s * w)).
template <int P>
__device__ __forceinline__ void stage_vector(Ctx<P>& c, uint32_t tv, int n, int np, unsigned ep, float* xs, float* raw,
                                             bool norm, const float2 (&w)[kStageNP]) {
  uint4 buf[kStageNP];
  poll_regs<P, kStageNP>(c, tv, n, 0, np, ep, buf);
  float2 x[kStageNP];
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < kStageNP; k++) {
    int pc = c.lane + 64 * k;
    x[k] = pc < np ? piece_values(buf[k], 2 * pc, n) : make_float2(0.f, 0.f);
    sum += x[k].x * x[k].x + x[k].y * x[k].y;
  }
  // Every lane stores all kStageNP pieces (zeros past np): 2 * 64 * kStageNP = kMaxDim floats,
  // within both the raw copy and the activation buffer, and past the vector's padded length,
  // where no matvec reads. A store guarded per piece cost one divergent branch each.
  static_assert(2 * 64 * kStageNP <= kMaxDim && kMaxDim <= kXs, "staged pieces fit the LDS buffers");
  if (raw) {
#pragma unroll
    for (int k = 0; k < kStageNP; k++) lds_store2(raw + 2 * (c.lane + 64 * k), x[k]);
  }
  if (norm) {
    const float scale = 1.0f / sqrtf(wave_total(sum) / (float)c.a.width + c.a.epsilon);
#pragma unroll
    for (int k = 0; k < kStageNP; k++) x[k] = make_float2(cast<P>(x[k].x * scale * w[k].x), cast<P>(x[k].y * scale * w[k].y));
  }
#pragma unroll
  for (int k = 0; k < kStageNP; k++) lds_store2(xs + 2 * (c.lane + 64 * k), x[k]);
}

// Units of a matvec phase owned by workgroup g: [first, first + count).
struct Own {
  int first, count;
};

template <int P>
__device__ __forceinline__ Own own_units(const Mv& m, int grid, int g) {
  int total = m.rows / m.unit;
  int per = (total + grid - 1) / grid;
  int first = g * per;
  int end = first + per < total ? first + per : total;
  return {first, end > first ? end - first : 0};
}

// Stage the inputs of phase p into LDS buffer `buf` (control wave). The OUT and DOWN
// residuals read x as it was staged for this layer's QKV (xres[0]) and GATEUP (xres[1])
// phases: a fused step keeps that raw copy in LDS from the earlier staging (`resident`);
// a one-phase launch polls its own rows of it instead.
template <int P, int A>
__device__ __forceinline__ void stage_inputs(Ctx<P>& c, Phase p, int buf, bool resident) {
  const StepArgs& a = c.a;
  float* xs = c.lds.xs[buf];
  // What to poll: up to three whole vectors and an optional range of own rows; then keep a
  // raw copy and/or normalize.
  uint32_t vec[3];
  float* dst[3];
  int nvec = 0, n = a.width, n_p = a.width_p;
  unsigned ep = 0, ep_own = 0;
  float* raw = nullptr;
  float* own_dst = nullptr;
  bool norm = false;
  float2 nw[kStageNP];
  Own own{0, 0};
  if (p.kind == kAttn) {
    if constexpr ((A & 3) != 0) return;
    ep = c.epoch(ph_index(kQkv, p.layer));
    vec[0] = a.t_q; dst[0] = c.lds.qkv;
    vec[1] = a.t_k; dst[1] = c.lds.qkv + kMaxDim;
    vec[2] = a.t_v; dst[2] = c.lds.qkv + 2 * kMaxDim;
    nvec = 3;
  } else if (p.kind == kFinal) {
    if (c.g != 0) return;
    ep = c.epoch(ph_index(kDown, a.layers - 1));
    vec[0] = a.t_x; dst[0] = xs; nvec = 1;
    norm = true;
    load_norm(c, a.w_final_norm, nw);
  } else {
    Mv m = matvec_of<P>(a, p);
    Own mine = own_units<P>(m, c.grid, c.g);
    if (mine.count == 0 && !resident) return;
    switch (p.kind) {
      case kInput: {
        if (c.tagged_input) {
          poll_vector(c, a.t_in, a.features, a.features_p, c.epoch(0), xs);
          return;
        }
        // The event holds `features` floats (any padding after them is not read): whole
        // 16-byte pieces load at once, a partial last piece element by element, and the
        // padded tail of the row is zero.
        __amdgpu_buffer_rsrc_t ir = make_rsrc(c.input, (uint32_t)a.features * 4u);
        for (int i = c.lane * 4; i < a.features_p; i += 256) {
          float4 v;
          if (i + 4 <= a.features) {
            v = ld16_coherent(ir, (uint32_t)i * 4u);
          } else {
            float e[4];
#pragma unroll
            for (int k = 0; k < 4; k++) e[k] = i + k < a.features ? ld4_coherent(ir, (uint32_t)(i + k) * 4u) : 0.f;
            v = make_float4(e[0], e[1], e[2], e[3]);
          }
          lds_store4(xs + i, v);
        }
        return;
      }
      case kQkv:
        ep = c.epoch(ph_x_before(p.layer));
        vec[0] = a.t_x; dst[0] = xs; nvec = 1;
        norm = true;
        load_norm(c, a.layer[p.layer].norm1, nw);
        if (resident) raw = c.lds.xres[0];
        break;
      case kOut:
        if (mine.count == 0) return;
        ep = c.epoch(ph_index(kAttn, p.layer));
        vec[0] = a.t_attn; dst[0] = xs; nvec = 1;
        if (!resident) {
          own = mine; ep_own = c.epoch(ph_x_before(p.layer));
          own_dst = c.lds.xres[0] + mine.first;
        }
        break;
      case kGateUp:
        ep = c.epoch(ph_index(kOut, p.layer));
        vec[0] = a.t_x; dst[0] = xs; nvec = 1;
        norm = true;
        load_norm(c, a.layer[p.layer].norm2, nw);
        if (resident) raw = c.lds.xres[1];
        break;
      default:  // kDown
        if (mine.count == 0) return;
        ep = c.epoch(ph_index(kGateUp, p.layer));
        vec[0] = a.t_act; dst[0] = xs; nvec = 1;
        n = a.ffn; n_p = a.ffn_p;
        if (!resident) {
          own = mine; ep_own = c.epoch(ph_index(kOut, p.layer));
          own_dst = c.lds.xres[1] + mine.first;
        }
        break;
    }
  }
  if (nvec == 1 && n_p / 2 <= 64 * kStageNP) {
    stage_vector(c, vec[0], n, n_p / 2, ep, dst[0], raw, norm, nw);
  } else {
    // Wider vectors and the attention q/k/v carry no norm or raw copy.
    for (int v = 0; v < nvec; v++) poll_vector(c, vec[v], n, n_p, ep, dst[v], c.split_wide && p.kind == kDown);
  }
#if STAMD_POLL_STAMPS
  if (c.pph >= 0 && c.lane == 0) lstamp(c, c.pph, 11);
#endif
  if (own.count) poll_range(c, a.t_x, own.first, own.count, ep_own, own_dst);
}

// ---------------------------------------------------------------------------------------------
// stream waves: matvec phases

// Work of stream wave sw: units first + sw, first + sw + 7, ... within the workgroup's block.
template <int P>
__device__ __forceinline__ WaveWork work_of(const Mv& m, int grid, int g, int sw, int& unit0) {
  Own own = own_units<P>(m, grid, g);
  WaveWork w;
  w.slabs_row = m.cols_p * Traits<P>::kWBytes / 1024;
  w.per_unit = m.unit * w.slabs_row;
  int units = own.count > sw ? (own.count - sw + kStreamWaves - 1) / kStreamWaves : 0;
  unit0 = own.first + sw;
  w.slabs = units * w.per_unit;
  w.base = m.woff + (uint32_t)unit0 * (uint32_t)w.per_unit * 1024u;
  w.unit_stride = (uint32_t)kStreamWaves * (uint32_t)w.per_unit * 1024u;
  return w;
}

// A stream wave's share of matvec phase p: from the forward's table when it is filled, else
// computed. unit0 is the first owned unit; refill and last are the cursors of slab kPF and of
// the last slab.
template <int P>
__device__ __forceinline__ WaveWork wave_work(Ctx<P>& c, Phase p, int sw, int& unit0, int& unit, SlabCursor& refill,
                                              SlabCursor& last) {
  const Mv m = matvec_of<P>(c.a, p);
  if (c.split_ready) {
    const WaveSplit sp = c.lds.split[sw][p.kind];
    unit0 = sp.unit0;
    unit = sp.unit;
    refill = {m.woff + sp.refill_off, sp.refill_r};
    last = {m.woff + sp.last_off, sp.last_r};
    return {sp.slabs_row, sp.per_unit, sp.slabs, m.woff + sp.base_rel, sp.unit_stride};
  }
  WaveWork w = work_of<P>(m, c.grid, c.g, sw, unit0);
  unit = m.unit;
  refill = cursor_at(w, kPF);
  last = cursor_at(w, w.slabs > 0 ? w.slabs - 1 : 0);
  return w;
}

// Fill lds.split for this stream wave (once per forward; read back only by this wave).
template <int P>
__device__ __forceinline__ void fill_split(Ctx<P>& c) {
  const int sw = c.wave - 1;
  for (int kind = kInput; kind < kFinal; kind++) {
    if (kind == kAttn) continue;
    Mv m = matvec_of<P>(c.a, Phase{kind, 0});
    m.woff = 0;
    int unit0;
    const WaveWork w = work_of<P>(m, c.grid, c.g, sw, unit0);
    const SlabCursor r = cursor_at(w, kPF), l = cursor_at(w, w.slabs > 0 ? w.slabs - 1 : 0);
    if (c.lane == 0)
      c.lds.split[sw][kind] = WaveSplit{w.slabs, w.per_unit, w.slabs_row, unit0, m.unit, w.base, w.unit_stride,
                                        r.unit_off, l.unit_off, r.r, l.r};
  }
  c.split_ready = true;
}

template <bool NT, int P>
__device__ __forceinline__ void prefetch_matvec(Ctx<P>& c, const WaveWork& w, SlabCursor last, uint4 (&ring)[kPF]) {
  if (w.slabs == 0) return;
  SlabCursor cur{w.base, 0};
#pragma unroll
  for (int j = 0; j < kPF; j++) {
    ring[j] = ld16w<NT>(c.wr, (j < w.slabs ? cur : last).offset(c.lane));
    cur.advance(w);
  }
}

// Attention work items (head, chunk of the window) over all stream waves of the grid.
struct AttnWork {
  int wid, nw, items, nch;  // items owned by this wave; chunks per head
  int kchunks;              // 16-byte chunks of one K (or V) block
  int heads;
  // Items are numbered chunk-major: item it covers chunk it / heads of head it % heads. The
  // chunks of one head then fall on workgroups whose indices agree modulo `heads` (with a
  // grid and a head count that are multiples of 8, on one XCD under round-robin dispatch),
  // and the waves that combine heads (chunk 0) sit in different workgroups.
  __device__ __forceinline__ void decode(int it, int& h, int& ch) const {
    ch = it / heads;
    h = it - ch * heads;
  }
  // Index of the (head, chunk) partial in t_po / t_pm / t_ps: head-major, so that a head's
  // partials are contiguous for its combine.
  __device__ __forceinline__ uint32_t partial(int h, int ch) const { return (uint32_t)(h * nch + ch); }
};

// Workgroup that computes attention item `it` (every layer): item it goes to wave wid = it mod
// nw, and wid = g + grid * sw, so the workgroup is it mod grid.
__device__ __forceinline__ int attn_item_workgroup(int it, int grid) { return it % grid; }

template <int P>
__device__ __forceinline__ AttnWork attn_work(const StepArgs& a, int grid, int g, int sw) {
  AttnWork w;
  w.nw = grid * kStreamWaves;
  w.wid = g + grid * sw;
  w.nch = (a.window + a.chunk - 1) / a.chunk;
  int total = a.heads * w.nch;
  w.items = total > w.wid ? (total - w.wid + w.nw - 1) / w.nw : 0;
  w.kchunks = (a.chunk * a.dim * Traits<P>::kKvBytes + 15) / 16;
  w.heads = a.heads;
  return w;
}

// Byte offset of the kk-th 16-byte chunk of the K/V block of item (h, ch), clamped.
template <int P>
__device__ __forceinline__ uint32_t attn_chunk_offset(const StepArgs& a, int layer, int h, int ch, int kk, int kchunks) {
  int k = kk < kchunks ? kk : kchunks - 1;
  uint32_t row0 = ((uint32_t)(layer * a.heads + h) * (uint32_t)a.window + (uint32_t)(ch * a.chunk));
  return row0 * (uint32_t)a.dim * Traits<P>::kKvBytes + (uint32_t)k * 16u;
}

template <int P>
__device__ __forceinline__ void load_block(Ctx<P>& c, __amdgpu_buffer_rsrc_t r, int layer, int h, int ch, int kchunks,
                                           uint4* part) {
#pragma unroll
  for (int j = 0; j < kKB; j++) part[j] = ld16(r, attn_chunk_offset<P>(c.a, layer, h, ch, c.lane + 64 * j, kchunks));
}

template <bool NT, int P>
__device__ __forceinline__ void prefetch(Ctx<P>& c, Phase p, uint4 (&ring)[kPF]) {
  int sw = c.wave - 1;
  if (p.kind == kAttn) {
    AttnWork w = attn_work<P>(c.a, c.grid, c.g, sw);
    if (w.items == 0) return;
    int h, ch;
    w.decode(w.wid, h, ch);
    load_block<P>(c, c.kr, p.layer, h, ch, w.kchunks, ring);
    load_block<P>(c, c.vr, p.layer, h, ch, w.kchunks, ring + kKB);
  } else if (p.kind != kFinal) {
    int unit0, unit;
    SlabCursor refill, last;
    const WaveWork w = wave_work(c, p, sw, unit0, unit, refill, last);
    prefetch_matvec<NT>(c, w, last, ring);
  }
}

// Epilogue of one unit (lane 0 only); s0/s1 are the row sums, xres the x of the residual.
template <int P>
__device__ __forceinline__ void epilogue(Ctx<P>& c, Phase p, int unit, float s0, float s1, const float* xres) {
  const StepArgs& a = c.a;
  const unsigned ep = c.epoch(ph_index(p.kind, p.layer));
  switch (p.kind) {
    case kInput:
      c.tstore(a.t_x + unit, ep, cast<P>(s0));
      break;
    case kQkv: {
      int r0 = unit * 2;
      int sec = (r0 >= a.width) + (r0 >= 2 * a.width);
      int i = r0 - sec * a.width;
      float va = cast<P>(s0), vb = cast<P>(s1);
      if (sec < 2) {
        // RoPE on the adjacent pair (i, i+1), src/cuda/Primitives.cuh:148-159
        int e = (a.dim & (a.dim - 1)) == 0 ? (i & (a.dim - 1)) : i % a.dim;
        float co = c.lds.rope_cos[e >> 1], si = c.lds.rope_sin[e >> 1];
        float ra = cast<P>(va * co - vb * si);
        float rb = cast<P>(va * si + vb * co);
        // Both offsets are read as uniform values and blended (a select of the two fields
        // would become a per-lane load from the argument block, waited for with vmcnt(0)).
        const uint32_t tq = a.t_q, tk = a.t_k;
        uint32_t tv = tk + (uint32_t)(sec == 0) * (tq - tk);
        c.tstore(tv + i, ep, ra);
        c.tstore(tv + i + 1, ep, rb);
      } else {
        c.tstore(a.t_v + i, ep, va);
        c.tstore(a.t_v + i + 1, ep, vb);
      }
      break;
    }
    case kOut:
      c.tstore(a.t_x + unit, ep, cast<P>(xres[unit] + cast<P>(s0)));
      break;
    case kGateUp: {
      float gv = cast<P>(s0), uv = cast<P>(s1);
      c.tstore(a.t_act + unit, ep, cast<P>((gv / (1.0f + expf(-gv))) * uv));
      break;
    }
    case kDown: {
      float v = cast<P>(xres[unit] + cast<P>(s0));
      c.tstore(a.t_x + unit, ep, v);
      c.sstore(a.s_hidden + (uint32_t)p.layer * a.width + unit, v);
      break;
    }
    default:
      break;
  }
}

template <bool NT, int P>
__device__ __forceinline__ void compute_matvec(Ctx<P>& c, Phase p, const float* xs_buf, const float* xres,
                                               uint4 (&ring)[kPF]) {
  int unit, munit;
  SlabCursor refill, last;
  const WaveWork w = wave_work(c, p, c.wave - 1, unit, munit, refill, last);
  if (w.slabs == 0) return;
  int ru = 0, s = 0;  // row within the unit, slab within the row
  float acc0 = 0.f, acc1 = 0.f;
  // Lane k holds the row sums of the k-th unit finished since the last epilogue batch. The
  // epilogues (whose tagged stores are written through to memory) run after the ring loop:
  // stores issued inside it would count against the same vmcnt as the ring's loads, and the
  // ring's waits would then also wait for their write acknowledgements.
  float su0 = 0.f, su1 = 0.f;
  int finished = 0;
  const float* xs = xs_buf + c.lane * Traits<P>::kEpc;
  // One slab: its dot product into the current row's sum, then the row / unit bookkeeping.
  auto consume = [&](const uint4& slab) {
    const float d = chunk_dot<P>(slab, xs + s * 64 * Traits<P>::kEpc);
    if (ru == 0) acc0 += d; else acc1 += d;
    if (++s == w.slabs_row) {
      s = 0;
      if (++ru == munit) {
        ru = 0;
        const float s0 = wave_total(acc0);
        const float s1 = munit == 2 ? wave_total(acc1) : 0.f;
        if (c.lane == finished) {
          su0 = s0;
          su1 = s1;
        }
        finished++;
        acc0 = 0.f;
        acc1 = 0.f;
      }
    }
  };
  if (c.wave == 1) stamp(c, p, 4);
  // Every pass but the last consumes all kPF ring slots and refills each one right after
  // consuming it, unconditionally (past the wave's last slab it reloads that slab, which is
  // cached): every pass then issues exactly kPF loads in ring order, so before slot j the
  // wave waits only for slot j's own load and keeps kPF - 1 loads in flight. With refills
  // under a condition, the compiler could not count the outstanding loads across the back
  // edge and waited for all of them at the start of every pass.
  const int full = (w.slabs - 1) / kPF;
  for (int pass = 0; pass < full; pass++) {
#pragma unroll
    for (int j = 0; j < kPF; j++) {
      consume(ring[j]);
      const bool more = pass * kPF + j + kPF < w.slabs;
      ring[j] = ld16w<NT>(c.wr, (more ? refill : last).offset(c.lane));
      if (more) refill.advance(w);
    }
    // At most kPF units finish in one pass (a unit has at least one slab): flush the batch
    // inside the loop only when the next pass could overflow the 64 lanes (very small grids).
    if (finished > 64 - kPF) {
      if (c.lane < finished) epilogue(c, p, unit + kStreamWaves * c.lane, su0, su1, xres);
      unit += kStreamWaves * finished;
      finished = 0;
    }
  }
  // Every refill of this wave is issued: waves that finished earlier may now queue their
  // next-phase prefetch (streamed weights only; see stream_loop).
  if (NT && full > 0 && c.lane == 0)
    __hip_atomic_fetch_add(&c.lds.refilled[c.phase_parity], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  // The last pass: the remaining 1..kPF slabs, no refills.
#pragma unroll
  for (int j = 0; j < kPF; j++)
    if (full * kPF + j < w.slabs) consume(ring[j]);
  // Epilogues of the finished units, one unit per lane.
  if (c.lane < finished) epilogue(c, p, unit + kStreamWaves * c.lane, su0, su1, xres);
  if (c.wave == 1) stamp(c, p, 6);
}

// ---------------------------------------------------------------------------------------------
// stream waves: attention (src/cuda/Primitives.cuh:167-219, src/cpu/Cpu.cpp:97-109)

// Publish the (max logit, exp sum) of partial `it` as tagged elements t_pm / t_ps[it]; the
// item's o[dim] goes to t_po[it * dim ..].
template <int P>
__device__ __forceinline__ void publish_stats(Ctx<P>& c, unsigned ep, int it, float m, float s) {
  if (c.lane == 0) {
    c.tstore(c.a.t_pm + (uint32_t)it, ep, m);
    c.tstore(c.a.t_ps + (uint32_t)it, ep, s);
  }
}

__device__ __forceinline__ float lane_value(float v, int k) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
}

// Combine the chunk partials of head h (done by the wave that computed chunk 0, after all
// of its own items, so no wave waits on work queued behind its own wait), in chunk order:
//   attn = sum_c o_c exp(m_c - M) / sum_c s_c exp(m_c - M),  M = max_c m_c,
// then publish attn_h. Polls the tagged partials.
constexpr int kCombineOne = 32;  // chunks a head combines in one polling pass

template <int P>
__device__ __forceinline__ void combine_head(Ctx<P>& c, int layer, int h, int nch, int nactive) {
  const StepArgs& a = c.a;
  const int dim = a.dim;
  const unsigned ep = c.epoch(ph_index(kAttn, layer));
  const uint32_t item0 = (uint32_t)(h * nch);
  if (nactive <= kCombineOne && dim <= 64) {
    // One pass: lane c polls (m_c, s_c) and lane i polls o_c[i] of every chunk.
    const int cl = c.lane < nactive ? c.lane : nactive - 1;
    const int il = c.lane < dim ? c.lane : dim - 1;
    uint2 pm, ps, po[kCombineOne];
    unsigned long long start = wall_clock64();
    while (true) {
      pm = c.tload(a.t_pm + item0 + (uint32_t)cl);
      ps = c.tload(a.t_ps + item0 + (uint32_t)cl);
#pragma unroll
      for (int k = 0; k < kCombineOne; k++) {
        int cc = k < nactive ? k : nactive - 1;
        po[k] = c.tload(a.t_po + (item0 + (uint32_t)cc) * (uint32_t)dim + (uint32_t)il);
      }
      bool ok = pm.y == ep && ps.y == ep;
#pragma unroll
      for (int k = 0; k < kCombineOne; k++) ok = ok && po[k].y == ep;
      if (__all(ok) || c.dead || c.expired(start)) break;
      __builtin_amdgcn_s_sleep(kPollSleep);
    }
    const float mc = __builtin_bit_cast(float, pm.x), sc = __builtin_bit_cast(float, ps.x);
    const float big = wave_top(c.lane < nactive ? mc : -INFINITY);
    const float e = c.lane < nactive ? expf(mc - big) : 0.f;
    const float denom = wave_total(sc * e);
    // No per-chunk branch: chunks at or beyond nactive have e = 0 (lanes >= nactive) and
    // hold the clamped, current partial of chunk nactive - 1, so their terms are exact zeros
    // and the chunk-order sum is unchanged. (A branch per chunk made the compiler precompute
    // and spill 32 predicates and serialize the loop on them: about 1.4 us per combine.)
    float o = 0.f;
#pragma unroll
    for (int k = 0; k < kCombineOne; k++) o += __builtin_bit_cast(float, po[k].x) * lane_value(e, k);
    if (c.lane < dim) c.tstore(a.t_attn + h * dim + c.lane, ep, cast<P>(o / denom));
    return;
  }
  if (nactive <= 64 && dim <= 64) {
    // Lane c polls (m_c, s_c); then lane i reads o_c[i] of the chunks in groups of 8.
    const int cl = c.lane < nactive ? c.lane : nactive - 1;
    const int il = c.lane < dim ? c.lane : dim - 1;
    uint2 pm, ps;
    unsigned long long start = wall_clock64();
    while (true) {
      pm = c.tload(a.t_pm + item0 + (uint32_t)cl);
      ps = c.tload(a.t_ps + item0 + (uint32_t)cl);
      if (__all(pm.y == ep && ps.y == ep) || c.dead || c.expired(start)) break;
      __builtin_amdgcn_s_sleep(kPollSleep);
    }
    const float mc = __builtin_bit_cast(float, pm.x), sc = __builtin_bit_cast(float, ps.x);
    const float big = wave_top(c.lane < nactive ? mc : -INFINITY);
    const float e = c.lane < nactive ? expf(mc - big) : 0.f;
    const float denom = wave_total(sc * e);
    float o = 0.f;
    for (int k0 = 0; k0 < nactive; k0 += 8) {
      uint2 po[8];
      start = wall_clock64();
      while (true) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < 8; k++) {
          int cc = k0 + k < nactive ? k0 + k : nactive - 1;
          po[k] = c.tload(a.t_po + (item0 + (uint32_t)cc) * (uint32_t)dim + (uint32_t)il);
        }
#pragma unroll
        for (int k = 0; k < 8; k++) ok = ok && po[k].y == ep;
        if (__all(ok) || c.dead || c.expired(start)) break;
        __builtin_amdgcn_s_sleep(kPollSleep);
      }
      // Chunks at or beyond nactive add exact zeros (e = 0 there), as in the one-pass path.
#pragma unroll
      for (int k = 0; k < 8; k++) o += __builtin_bit_cast(float, po[k].x) * lane_value(e, k0 + k);
    }
    if (c.lane < dim) c.tstore(a.t_attn + h * dim + c.lane, ep, cast<P>(o / denom));
    return;
  }
  // General sizes: wait for every chunk's statistics, then maxima, denominators and outputs
  // in chunk order.
  for (int c0 = 0; c0 < nactive; c0 += 64) {
    const int cc = c0 + c.lane < nactive ? c0 + c.lane : nactive - 1;
    unsigned long long start = wall_clock64();
    while (true) {
      uint2 vm = c.tload(a.t_pm + item0 + (uint32_t)cc);
      uint2 vs = c.tload(a.t_ps + item0 + (uint32_t)cc);
      if (__all(vm.y == ep && vs.y == ep) || c.dead || c.expired(start)) break;
      __builtin_amdgcn_s_sleep(kPollSleep);
    }
  }
  float big = -INFINITY;
  for (int c0 = 0; c0 < nactive; c0 += 64) {
    int cc = c0 + c.lane;
    if (cc < nactive) big = fmaxf(big, __builtin_bit_cast(float, c.tload(a.t_pm + item0 + (uint32_t)cc).x));
  }
  big = wave_top(big);
  float denom = 0.f;
  for (int c0 = 0; c0 < nactive; c0 += 64) {
    int cc = c0 + c.lane;
    if (cc < nactive) {
      float mc = __builtin_bit_cast(float, c.tload(a.t_pm + item0 + (uint32_t)cc).x);
      float sc = __builtin_bit_cast(float, c.tload(a.t_ps + item0 + (uint32_t)cc).x);
      denom += sc * expf(mc - big);
    }
  }
  denom = wave_total(denom);
  for (int i = c.lane; i < dim; i += 64) {
    float o = 0.f;
    for (int cc = 0; cc < nactive; cc++) {
      unsigned long long start = wall_clock64();
      uint2 vo;
      while (true) {
        vo = c.tload(a.t_po + (item0 + (uint32_t)cc) * (uint32_t)dim + (uint32_t)i);
        if (vo.y == ep || c.dead || c.expired(start)) break;
        __builtin_amdgcn_s_sleep(kPollSleep);
      }
      float mc = __builtin_bit_cast(float, c.tload(a.t_pm + item0 + (uint32_t)cc).x);
      o += __builtin_bit_cast(float, vo.x) * expf(mc - big);
    }
    c.tstore(a.t_attn + h * dim + i, ep, cast<P>(o / denom));
  }
}

// Combines owed by this wave: the heads whose chunk 0 it computed in this phase.
template <int P>
__device__ __forceinline__ void combine_owned(Ctx<P>& c, Phase p, const AttnWork& w, int nactive) {
  for (int m = 0; m < w.items; m++) {
    int h, ch;
    w.decode(w.wid + w.nw * m, h, ch);
    if (ch == 0) combine_head(c, p.layer, h, w.nch, nactive);
  }
}

// Store element i of the current K and V rows of (layer, head h) into the ring.
template <int P>
__device__ __forceinline__ void ring_write(Ctx<P>& c, int layer, int h, int i, float kv, float vv) {
  uint32_t idx =
      ((uint32_t)(layer * c.a.heads + h) * (uint32_t)c.a.window + (uint32_t)c.slot) * (uint32_t)c.a.dim + (uint32_t)i;
  if constexpr (P == kMixed) {
    st2_coherent(c.kr, idx * 2u, float_to_half(kv));
    st2_coherent(c.vr, idx * 2u, float_to_half(vv));
  } else {
    st4_coherent(c.kr, idx * 4u, kv);
    st4_coherent(c.vr, idx * 4u, vv);
  }
}

// Decode the 16-byte chunk of a K/V block into E floats.
template <int P>
__device__ __forceinline__ void kv_decode(uint4 u, float* v) {
  if constexpr (P == kMixed) {
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[2 * e] = half_to_float((unsigned short)(w[e] & 0xffffu));
      v[2 * e + 1] = half_to_float((unsigned short)(w[e] >> 16));
    }
  } else {
    v[0] = __builtin_bit_cast(float, u.x);
    v[1] = __builtin_bit_cast(float, u.y);
    v[2] = __builtin_bit_cast(float, u.z);
    v[3] = __builtin_bit_cast(float, u.w);
  }
}

// Attention on the register-held K/V block (power-of-two head dim with E <= dim <= 64E,
// E elements per 16-byte chunk). Lane l's j-th chunk holds row (l*E)/dim + j*(64E/dim),
// columns (l*E)%dim .. +E-1; the dim/E lanes of a row reduce q.k with a butterfly and the
// output columns reduce across rows the same way. Each wave polls the q, k, v elements of
// its own head, so attention waits only on the QKV units of that head.
// G: lanes per row (dim / E) when known at compile time, else 0. A one-wave item is a chain
// of dependent instructions, so the reductions are specialized on G.
template <int P, int G>
__device__ __forceinline__ void compute_attn_regs(Ctx<P>& c, Phase p, uint4 (&ring)[kPF]) {
  const StepArgs& a = c.a;
  AttnWork w = attn_work<P>(a, c.grid, c.g, c.wave - 1);
  constexpr int E = 16 / Traits<P>::kKvBytes;
  const int dim = G ? G * E : a.dim, chunk = a.chunk;
  const int group = G ? G : dim / E;
  const int rows_per_load = 64 / group;
  const int loads = (w.kchunks + 63) / 64;
  const int col0 = (c.lane * E) % dim;
  const int row_lane = (c.lane * E) / dim;
  const int nactive = (c.valid + chunk - 1) / chunk;
  const float div = sqrtf((float)dim);
  const unsigned ep_qkv = c.epoch(ph_index(kQkv, p.layer));
  for (int m = 0; m < w.items; m++) {
    int h, ch;
    w.decode(w.wid + w.nw * m, h, ch);
    if (ch >= nactive) continue;
    const uint32_t pi = w.partial(h, ch);
    // The K and V blocks: the first item's from the LDS stage (loaded by the control wave
    // during the QKV phase) or from the ring (prefetched); later items' from memory.
    uint4 kb[kKB], vb[kKB];
    if (m == 0 && c.kv_lds) {
      const float* st = c.lds.stage[c.wave - 1];
#pragma unroll
      for (int j = 0; j < kKB; j++) {
        kb[j] = lds_load_u4(st + 4 * (c.lane + 64 * j));
        vb[j] = lds_load_u4(st + 256 * kKB + 4 * (c.lane + 64 * j));
      }
    } else if (m == 0) {
#pragma unroll
      for (int j = 0; j < kKB; j++) {
        kb[j] = ring[j];
        vb[j] = ring[kKB + j];
      }
    } else {
      load_block<P>(c, c.kr, p.layer, h, ch, w.kchunks, kb);
      load_block<P>(c, c.vr, p.layer, h, ch, w.kchunks, vb);
    }
    // q, k, v of this lane's columns of head h (E each), polled from the tagged vectors.
    float q[E], kc[E], vc[E];
    {
      uint4 pq[E / 2], pk[E / 2], pv[E / 2];
      const uint32_t e0 = (uint32_t)(h * dim + col0);
      unsigned long long start = wall_clock64();
      while (true) {
#pragma unroll
        for (int k = 0; k < E / 2; k++) {
          uint32_t off = (e0 + 2u * k) * 8u;
          pq[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(c.tr, (int)(a.t_q * 8u + off), 0, kSc1));
          pk[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(c.tr, (int)(a.t_k * 8u + off), 0, kSc1));
          pv[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(c.tr, (int)(a.t_v * 8u + off), 0, kSc1));
        }
        bool ok = true;
#pragma unroll
        for (int k = 0; k < E / 2; k++)
          ok = ok && pq[k].y == ep_qkv && pq[k].w == ep_qkv && pk[k].y == ep_qkv && pk[k].w == ep_qkv &&
               pv[k].y == ep_qkv && pv[k].w == ep_qkv;
        if (__all(ok) || c.dead) break;
        if (wall_clock64() - start > a.spin_limit) {
          c.timeout();
          break;
        }
        __builtin_amdgcn_s_sleep(kPollSleep);
      }
      if (c.wave == 1) stamp(c, p, 4);
#pragma unroll
      for (int k = 0; k < E / 2; k++) {
        q[2 * k] = __builtin_bit_cast(float, pq[k].x);
        q[2 * k + 1] = __builtin_bit_cast(float, pq[k].z);
        kc[2 * k] = __builtin_bit_cast(float, pk[k].x);
        kc[2 * k + 1] = __builtin_bit_cast(float, pk[k].z);
        vc[2 * k] = __builtin_bit_cast(float, pv[k].x);
        vc[2 * k + 1] = __builtin_bit_cast(float, pv[k].z);
      }
    }
    const int row0 = ch * chunk;
    const bool owns_slot = c.slot >= row0 && c.slot < row0 + chunk;
    if (owns_slot && c.lane < group) {
#pragma unroll
      for (int e = 0; e < E; e++) ring_write(c, p.layer, h, col0 + e, kc[e], vc[e]);
    }
    float logit[kKB];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kKB; j++) {
      int row = row_lane + j * rows_per_load;
      bool live = j < loads && (c.lane + 64 * j) < w.kchunks && row < chunk && row0 + row < c.valid;
      bool cur = row0 + row == c.slot;
      float k[E];
      kv_decode<P>(kb[j], k);
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < E; e++) dot += q[e] * (cur ? kc[e] : k[e]);
      dot = group_sum(dot, group);
      logit[j] = live ? dot / div : -INFINITY;
      mx = fmaxf(mx, logit[j]);
    }
    mx = wave_top(mx);
    float psum = 0.f;
    float out[E];
#pragma unroll
    for (int e = 0; e < E; e++) out[e] = 0.f;
#pragma unroll
    for (int j = 0; j < kKB; j++) {
      float pr = logit[j] == -INFINITY ? 0.f : expf(logit[j] - mx);
      psum += pr;
      int row = row_lane + j * rows_per_load;
      bool cur = row0 + row == c.slot;
      float v[E];
      kv_decode<P>(vb[j], v);
#pragma unroll
      for (int e = 0; e < E; e++) out[e] += pr * (cur ? vc[e] : v[e]);
    }
    float total = wave_total((c.lane & (group - 1)) == 0 ? psum : 0.f);
#pragma unroll
    for (int e = 0; e < E; e++)
      out[e] = column_sum(out[e], group);
    const unsigned ep = c.epoch(ph_index(kAttn, p.layer));
    if (c.lane < group) {
      const uint32_t ob = pi * (uint32_t)dim + (uint32_t)col0;
#pragma unroll
      for (int e = 0; e < E; e++) c.tstore(a.t_po + ob + (uint32_t)e, ep, out[e]);
    }
    publish_stats(c, ep, pi, mx, total);
    if (c.wave == 1) stamp(c, p, 5);
  }
  combine_owned(c, p, w, nactive);
  if (c.wave == 1) stamp(c, p, 6);
}

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
  for (int j = 0; j < kKB; j++) {
    if (c.lane + 64 * j < kchunks) {
      float v[kPer];
      kv_decode<P>(part[j], v);
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

// General head dims: K/V block staged through LDS, q/k/v of the step staged by the control
// wave (lds.qkv).
template <int P>
__device__ __forceinline__ void compute_attn_lds(Ctx<P>& c, Phase p, uint4 (&ring)[kPF]) {
  const StepArgs& a = c.a;
  AttnWork w = attn_work<P>(a, c.grid, c.g, c.wave - 1);
  const int dim = a.dim, stride = dim + 4, chunk = a.chunk;
  float* stage = c.lds.stage[c.wave - 1];
  float* probs = c.lds.probs[c.wave - 1];
  const float* q_all = c.lds.qkv;
  const float* k_cur = c.lds.qkv + kMaxDim;
  const float* v_cur = c.lds.qkv + 2 * kMaxDim;
  const int nactive = (c.valid + chunk - 1) / chunk;
  const float div = sqrtf((float)dim);
  for (int m = 0; m < w.items; m++) {
    int h, ch;
    w.decode(w.wid + w.nw * m, h, ch);
    if (ch >= nactive) continue;
    const uint32_t pi = w.partial(h, ch);
    if (m > 0) {
      load_block<P>(c, c.kr, p.layer, h, ch, w.kchunks, ring);
      load_block<P>(c, c.vr, p.layer, h, ch, w.kchunks, ring + kKB);
    }
    int row0 = ch * chunk;
    int rows = c.valid - row0 < chunk ? c.valid - row0 : chunk;  // valid slots are [0, valid)
    int cur = c.slot - row0;
    if (cur >= 0 && cur < chunk)
      for (int i = c.lane; i < dim; i += 64) ring_write(c, p.layer, h, i, k_cur[h * dim + i], v_cur[h * dim + i]);
    block_to_lds<P>(c, ring, w.kchunks, stage);
    if (cur >= 0 && cur < chunk)
      for (int i = c.lane; i < dim; i += 64) stage[cur * stride + i] = k_cur[h * dim + i];
    __builtin_amdgcn_wave_barrier();
    float logit = -INFINITY;
    if (c.lane < rows) {
      const float* krow = stage + c.lane * stride;
      const float* q = q_all + h * dim;
      float dot = 0.f;
      for (int i = 0; i < dim; i++) dot += q[i] * krow[i];
      logit = dot / div;
    }
    float mx = wave_top(logit);
    float pr = c.lane < rows ? expf(logit - mx) : 0.f;
    float total = wave_total(pr);
    probs[c.lane] = pr;
    __builtin_amdgcn_wave_barrier();
    block_to_lds<P>(c, ring + kKB, w.kchunks, stage);
    if (cur >= 0 && cur < chunk)
      for (int i = c.lane; i < dim; i += 64) stage[cur * stride + i] = v_cur[h * dim + i];
    __builtin_amdgcn_wave_barrier();
    const unsigned ep = c.epoch(ph_index(kAttn, p.layer));
    for (int i = c.lane; i < dim; i += 64) {
      float o = 0.f;
      for (int j = 0; j < rows; j++) o += probs[j] * stage[j * stride + i];
      c.tstore(a.t_po + pi * (uint32_t)dim + (uint32_t)i, ep, o);
    }
    publish_stats(c, ep, pi, mx, total);
    __builtin_amdgcn_wave_barrier();
  }
  combine_owned(c, p, w, nactive);
}

// Final phase (workgroup 0, control wave): score = W_score . norm(x), not cast; position++.
template <int P>
__device__ __forceinline__ void compute_final(Ctx<P>& c, const float* xs_buf) {
  const StepArgs& a = c.a;
  const int slabs = a.width_p * Traits<P>::kWBytes / 1024;  // <= 4
  uint4 wv[kMaxDim * 4 / 1024];
#pragma unroll
  for (int s = 0; s < kMaxDim * 4 / 1024; s++) {
    int sc = s < slabs ? s : slabs - 1;
    wv[s] = ld16(c.wr, a.w_score + (uint32_t)sc * 1024u + (uint32_t)c.lane * 16u);
  }
  float acc = 0.f;
#pragma unroll
  for (int s = 0; s < kMaxDim * 4 / 1024; s++)
    if (s < slabs) acc += chunk_dot<P>(wv[s], xs_buf + (s * 64 + c.lane) * Traits<P>::kEpc);
  float score = wave_total(acc);
  if (c.lane == 0) {
    c.sstore(a.s_score, score);
    // System scope: written through to memory, so a host copy sees it while a persistent
    // worker is still running.
    __hip_atomic_store(a.position, c.t + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// A selects, one per instantiation, the attention path in its low two bits: 0 the LDS path
// (general head dims); the register path with a head row of 1, 2, 3: sixteen, eight, any
// other number of 16-byte chunks. Bit 2 (kWeightNt) makes the weight loads non-temporal.
// The host picks A from the head dim and the weight bytes.
template <int P, int A>
__device__ __forceinline__ void compute(Ctx<P>& c, Phase p, int buf, uint4 (&ring)[kPF]) {
  if (p.kind == kAttn) {
    if constexpr ((A & 3) == 1) compute_attn_regs<P, 16>(c, p, ring);
    else if constexpr ((A & 3) == 2) compute_attn_regs<P, 8>(c, p, ring);
    else if constexpr ((A & 3) == 3) compute_attn_regs<P, 0>(c, p, ring);
    else compute_attn_lds(c, p, ring);
  } else if (p.kind != kFinal) {
    compute_matvec<weight_nt(A)>(c, p, c.lds.xs[buf], c.lds.xres[p.kind == kDown ? 1 : 0], ring);
  }
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
  __builtin_amdgcn_s_barrier();
}

// ---------------------------------------------------------------------------------------------
// kernels

// RoPE cos / sin of this step's position for each pair of a head (src/cuda/Primitives.cuh:
// 148-159): angle = position * inverse frequency, computed once per step instead of per unit.
template <int P>
__device__ __forceinline__ void fill_rope(Ctx<P>& c) {
  for (int i = threadIdx.x; i < c.a.dim / 2; i += kThreads) {
    const float angle = (float)c.t * c.a.rope_freq[i];
    c.lds.rope_cos[i] = cosf(angle);
    c.lds.rope_sin[i] = sinf(angle);
  }
}

// One phase per launch (staged and graph backends). The FINAL launch advances the epoch.
template <int P, int A>
__global__ __launch_bounds__(kThreads) void phase_kernel(const StepArgs* __restrict__ ap, int ph) {
  const StepArgs& a = *ap;
  __shared__ LdsAll lds;
  Ctx<P> c(a, lds, (int)blockIdx.x, (int)gridDim.x);
  Phase p = phase_of(a, ph);
  if (p.kind == kFinal && blockIdx.x != 0) return;
  c.base = load_epoch(a);
  c.set_position(load_position(a));
  uint4 ring[kPF];
  fill_rope(c);
  if (c.wave == 0) stage_inputs<P, A>(c, p, 0, false);
  else prefetch<weight_nt(A)>(c, p, ring);
  lds_barrier();
  if (p.kind == kFinal) {
    if (c.wave == 0) {
      compute_final(c, c.lds.xs[0]);
      if (c.lane == 0)
        __hip_atomic_store(a.epoch, c.base + (unsigned)ph_final(a) + 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  if (c.wave != 0) compute<P, A>(c, p, 0, ring);
}

// Control wave, at the start of a layer's QKV phase: load the K and V blocks of each stream
// wave's first attention item of the layer into that wave's LDS stage, with loads that write
// LDS directly (K at stage[0 ..), V at stage[256 * kKB ..), 16-byte chunk i at float 4i).
// The blocks do not depend on this step's q, k, v (attention takes the current slot's row from
// k and v), so they stream while the QKV phase runs, and the stream waves' rings can
// prefetch the OUT weights instead.
template <int P>
__device__ __forceinline__ void load_kv_to_lds(Ctx<P>& c, int layer) {
  const StepArgs& a = c.a;
  const int nactive = (c.valid + a.chunk - 1) / a.chunk;
  for (int sw = 0; sw < kStreamWaves; sw++) {
    const AttnWork w = attn_work<P>(a, c.grid, c.g, sw);
    if (w.items == 0) break;  // items go to waves in order: none for later waves either
    int h, ch;
    w.decode(w.wid, h, ch);
    if (ch >= nactive) continue;
    float* st = c.lds.stage[sw];
#pragma unroll
    for (int j = 0; j < kKB; j++) {
      const uint32_t off = attn_chunk_offset<P>(a, layer, h, ch, c.lane + 64 * j, w.kchunks);
      ld16_to_lds(c.kr, st + 256 * j, off);
      ld16_to_lds(c.vr, st + 256 * (kKB + j), off);
    }
  }
}

// The helper stream waves (the last three: waves 7, 6, 5 as helpers 0, 1, 2) each stage one
// 512-piece chunk (1, 2, 3) of the DOWN phase's activation vector while the control wave
// polls chunk 0, so that the wide vector costs about one polling round trip of a short poll.
// Mirrors the DOWN case of stage_inputs (same workgroups, epoch and LDS buffer); each helper
// signals through lds.helped[helper].
template <int P>
__device__ __forceinline__ void help_stage(Ctx<P>& c, Phase p, int buf) {
  const StepArgs& a = c.a;
  if (p.kind != kDown || a.ffn_p / 2 <= 512) return;
  if (own_units<P>(matvec_of<P>(a, p), c.grid, c.g).count == 0) return;
  const unsigned ep = c.epoch(ph_index(kGateUp, p.layer));
  const int hi = kWaves - 1 - c.wave;  // helper 0, 1, 2: waves 7, 6, 5
  if ((hi + 1) * 512 >= a.ffn_p / 2) return;
  poll_chunks<P, 512>(c, a.t_act, a.ffn, a.ffn_p / 2, hi + 1, 4, ep, c.lds.xs[buf]);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the chunk's LDS writes are done
  if (c.lane == 0) __hip_atomic_store(&c.lds.helped[hi], ep, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Control wave of one forward: stage each phase's inputs once this workgroup's stream
// waves are done with the previous phase. One barrier per phase, matching stream_loop.
template <int P, int A>
__device__ __forceinline__ void control_loop(Ctx<P>& c, int nph) {
  const StepArgs& a = c.a;
  // Optional wall-clock stamps (slots as in lstamp()); the step end follows the last phase.
  const bool stamps = a.stamps && threadIdx.x == 0;
  stage_inputs<P, A>(c, phase_of(a, 0), 0, true);
  for (int ph = 0; ph < nph; ph++) {
    lds_barrier();
    if (stamps) lstamp(c, ph, 0);
    Phase p = phase_of(a, ph);
    // refilled[ph & 1] counts this phase's waves done with their refills; the other parity's
    // counter was last read in the previous phase.
    if (weight_nt(A) && c.lane == 0)
      __hip_atomic_store(&c.lds.refilled[(ph + 1) & 1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (p.kind == kFinal) {
      if (c.g == 0) compute_final(c, c.lds.xs[ph & 1]);
      if (stamps && c.g == 0) put_global(a.stamps, (size_t)kStamps * c.grid * nph, wall_clock64());
      break;
    }
    if constexpr ((A & 3) != 0)
      if (c.kv_lds && p.kind == kQkv) load_kv_to_lds(c, p.layer);
    // Start polling for the next phase's inputs only once this workgroup's own part of
    // the current phase is done: the producers elsewhere finish at about the same time,
    // and polling earlier would only add memory traffic.
    while (__hip_atomic_load(&c.lds.done[ph & 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < (unsigned)kStreamWaves)
      __builtin_amdgcn_s_sleep(1);
    if (c.lane == 0) __hip_atomic_store(&c.lds.done[ph & 1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (stamps) lstamp(c, ph, 2);
#if STAMD_POLL_STAMPS
    c.pph = a.stamps ? ph : -1;
#endif
    stage_inputs<P, A>(c, phase_of(a, ph + 1), (ph + 1) & 1, true);
    // The attention phase reads the K/V blocks loaded above once the barrier is passed.
    if ((A & 3) != 0 && c.kv_lds && p.kind == kQkv) __builtin_amdgcn_s_waitcnt(0);
    if (stamps) lstamp(c, ph, 3);
  }
}

// Stream wave of one forward: compute each phase from the register ring, then prefetch
// the next phase's first slabs while the control wave stages its inputs.
template <int P, int A>
__device__ __forceinline__ void stream_loop(Ctx<P>& c, int nph) {
  const StepArgs& a = c.a;
  const bool stamps = a.stamps && c.wave == 1 && c.lane == 0;
  fill_split(c);
  uint4 ring[kPF];
  prefetch<weight_nt(A)>(c, phase_of(a, 0), ring);
  for (int ph = 0; ph < nph; ph++) {
    lds_barrier();
    Phase p = phase_of(a, ph);
    if (p.kind == kFinal) break;
    if constexpr (weight_nt(A)) c.phase_parity = ph & 1;
    compute<P, A>(c, p, ph & 1, ring);
    if (stamps) lstamp(c, ph, 1);
    // Signal before issuing the next phase's prefetch: the issue itself can stall on a
    // full memory pipeline, and the control wave can stage meanwhile.
    if (c.lane == 0) __hip_atomic_fetch_add(&c.lds.done[ph & 1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    {
      // With the attention K/V in LDS the ring has nothing to prefetch for attention. It
      // stays empty, so that the attention phase's stores and polls find this CU's memory
      // queue empty; OUT is prefetched after attention. (Waves without OUT rows prefetching
      // their GATEUP share here instead was slower: Large 323 -> 329 us, Main 152 -> 161 us.)
      const Phase nxt = phase_of(a, ph + 1);
      if (weight_nt(A) && p.kind != kAttn && c.lds.split[0][p.kind].slabs > kPF) {
        // Streamed weights, shares longer than the ring: a wave that is done with the phase
        // waits (at most 2000 wall-clock ticks, 20 us at 100 MHz; an ordering hint only, on
        // which no result depends) until every wave with refills has issued them, so that its
        // next-phase prefetch does not sit ahead of them in the CU's memory queue: the waves
        // without DOWN rows, and in GATEUP the waves with two units against those with three.
        // Large FP32: 311 -> 303.5 us.
        int rows = 0;
        for (int sw = 0; sw < kStreamWaves; sw++) rows += c.lds.split[sw][p.kind].slabs > kPF;
        const unsigned long long start = wall_clock64();
        while (__hip_atomic_load(&c.lds.refilled[ph & 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) <
                   (unsigned)rows &&
               wall_clock64() - start < 2000u)
          __builtin_amdgcn_s_sleep(1);
      }
      if (!((A & 3) != 0 && c.kv_lds && nxt.kind == kAttn)) prefetch<weight_nt(A)>(c, nxt, ring);
    }
    if (c.wave >= kWaves - 3) help_stage(c, phase_of(a, ph + 1), (ph + 1) & 1);
    if (stamps) lstamp(c, ph, 7);
  }
}

// One forward over the device-held state with the context's position and epoch base.
template <int P, int A>
__device__ __forceinline__ void forward(Ctx<P>& c) {
  const StepArgs& a = c.a;
  const int nph = ph_final(a) + 1;
  if (threadIdx.x == 0) {
    c.lds.refilled[0] = c.lds.refilled[1] = 0;
    c.lds.done[0] = 0;
    c.lds.done[1] = 0;
    c.lds.helped[0] = c.lds.helped[1] = c.lds.helped[2] = ~0u;
  }
  fill_rope(c);
  const int nst = (nph < kStampPhases ? nph : kStampPhases) * kStamps;
  if (a.stamps)
    for (int i = threadIdx.x; i < nst; i += kThreads) (&c.lds.stamps[0][0])[i] = 0u;
  c.split_wide = true;
  c.kv_lds = (A & 3) != 0;
  if (c.wave == 0) control_loop<P, A>(c, nph);
  else stream_loop<P, A>(c, nph);
  if (a.stamps) {
    lds_barrier();
    for (int i = threadIdx.x; i < nst; i += kThreads)
      put_global(a.stamps, (size_t)kStamps * ((size_t)(i / kStamps) * c.grid + c.g) + i % kStamps,
                 (&c.lds.stamps[0][0])[i]);
  }
}

// One step per launch (fused backend). `event` overrides the INPUT source when not null.
template <int P, int A>
__global__ __launch_bounds__(kThreads) void fused_kernel(const StepArgs* __restrict__ ap, const float* event) {
  const StepArgs& a = *ap;
  __shared__ LdsAll lds;
  Ctx<P> c(a, lds, (int)blockIdx.x, (int)gridDim.x);
  if (event) c.input = event;
  c.base = load_epoch(a);
  c.set_position(load_position(a));
  forward<P, A>(c);
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(a.epoch, c.base + (unsigned)ph_final(a) + 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Several independent streams in one launch: workgroups [s * per, (s + 1) * per) run one step
// of stream s with that stream's own arguments args[s] (state, tagged arena, epochs; the
// weight arena may be shared), reading its event at events + s * stride. Every stream runs the
// fused step unchanged on a grid of `per` workgroups, and the step's results do not depend on
// the grid size, so each stream's results are bit-identical to the single-stream runtime's.
// The arguments are one read-only array (a restrict kernel parameter indexed by a uniform
// value), so their fields load through the scalar cache as in fused_kernel; reached through
// a loaded pointer they became vector loads queued behind the weight stream (Main 148 ->
// 251 us). With `per` a multiple of 8, workgroup g of every stream sits on XCD g mod 8
// (round-robin dispatch), so the streams' reads of the same weight rows meet in one XCD's L2.
template <int P, int A>
__global__ __launch_bounds__(kThreads) void fused_streams_kernel(const StepArgs* __restrict__ args, int per,
                                                                 const float* events, int stride) {
  const int s = (int)blockIdx.x / per;
  const StepArgs& a = args[s];
  __shared__ LdsAll lds;
  Ctx<P> c(a, lds, (int)blockIdx.x - s * per, per);
  if (events) c.input = events + (size_t)s * (size_t)stride;
  c.base = load_epoch(a);
  c.set_position(load_position(a));
  forward<P, A>(c);
  if (c.g == 0 && threadIdx.x == 0)
    __hip_atomic_store(a.epoch, c.base + (unsigned)ph_final(a) + 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Device-only loop over a preloaded trace (the reference's trace_kernel): `count` steps in
// one launch (event e at events + e * stride floats), with a wall-clock stamp per
// step from workgroup 0. Workgroup 0 publishes a step-done word after each FINAL; every
// workgroup waits for it before the next step writes x.
template <int P, int A>
__global__ __launch_bounds__(kThreads) void trace_kernel(const StepArgs* __restrict__ ap, const float* events, int count,
                                                         int stride, unsigned long long* stamps) {
  const StepArgs& a = *ap;
  __shared__ LdsAll lds;
  Ctx<P> c(a, lds, (int)blockIdx.x, (int)gridDim.x);
  const unsigned base0 = load_epoch(a);
  const unsigned long long t0 = load_position(a);
  const unsigned per_step = (unsigned)ph_final(a) + 2u;  // phases + the step-done word
  for (int e = 0; e < count; e++) {
    if (blockIdx.x == 0 && threadIdx.x == 0) stamps[e] = wall_clock64();
    c.base = base0 + (unsigned)e * per_step;
    c.set_position(t0 + (unsigned long long)e);
    c.input = events + (size_t)e * (size_t)stride;
    if (e > 0 && c.wave == 0) {
      float done[2];
      poll_pieces<P, 1>(c, a.t_done, 1, 0, 1, c.base - 1u, done);
    }
    forward<P, A>(c);
    if (c.g == 0 && threadIdx.x == 0) c.tstore(a.t_done, c.base + per_step - 1u, 0.f);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    stamps[count] = wall_clock64();
    __hip_atomic_store(a.epoch, base0 + (unsigned)count * per_step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Persistent worker's RESET: this workgroup zeroes, with write-through stores, the K/V rows
// of the attention items it computes (attn_item_workgroup, decoded like AttnWork: chunk-major),
// in every layer, so the only L2 that can hold those rows is its own; a grid-strided share of
// the hidden state; and (workgroup 0) the position.
template <int P>
__device__ __forceinline__ void reset_owned(Ctx<P>& c) {
  const StepArgs& a = c.a;
  const AttnWork w = attn_work<P>(a, c.grid, c.g, 0);
  const int total = a.heads * w.nch;
  for (int it = c.g; it < total; it += c.grid) {
    if (attn_item_workgroup(it, c.grid) != c.g) continue;
    int h, ch;
    w.decode(it, h, ch);
    const int row0 = ch * a.chunk;
    const int rows = a.window - row0 < a.chunk ? a.window - row0 : a.chunk;
    const uint32_t bytes = (uint32_t)rows * (uint32_t)a.dim * Traits<P>::kKvBytes;  // a multiple of 4
    for (int l = 0; l < a.layers; l++) {
      const uint32_t b0 = ((uint32_t)(l * a.heads + h) * (uint32_t)a.window + (uint32_t)row0) * (uint32_t)a.dim *
                          Traits<P>::kKvBytes;
      for (uint32_t off = threadIdx.x * 4u; off < bytes; off += kThreads * 4u) {
        st4_coherent(c.kr, b0 + off, 0.f);
        st4_coherent(c.vr, b0 + off, 0.f);
      }
    }
  }
  for (int i = c.g * kThreads + (int)threadIdx.x; i < a.layers * a.width; i += c.grid * kThreads)
    c.sstore(a.s_hidden + (uint32_t)i, 0.f);
  if (c.g == 0 && threadIdx.x == 0) __hip_atomic_store(a.position, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Byte offsets of the SNAPSHOT copy in host memory: position (8 bytes), then K and V as stored
// in the ring, then the hidden state [L][d] FP32.
constexpr uint32_t kSnapKeys = 256;
__host__ __device__ __forceinline__ uint32_t snapshot_ring_bytes(int layers, int width, int window, int kv_bytes) {
  return (uint32_t)layers * (uint32_t)width * (uint32_t)window * (uint32_t)kv_bytes;
}

// SNAPSHOT (persistent worker): copy the carried state into the host buffer while the worker
// stays resident (copy commands on another queue cannot start while the worker holds every
// CU). Each workgroup copies the ring chunks it computes (as RESET) and a grid-strided share of the
// hidden state, all with coherent loads; workgroup 0 writes the position. The stores go to
// fine-grained host memory; the worker releases them (system scope) before reporting done.
template <int P>
__device__ __forceinline__ void snapshot_owned(Ctx<P>& c, unsigned long long t) {
  const StepArgs& a = c.a;
  unsigned char* out = a.mapped_snapshot;
  const uint32_t ring = snapshot_ring_bytes(a.layers, a.width, a.window, Traits<P>::kKvBytes);
  const AttnWork w = attn_work<P>(a, c.grid, c.g, 0);
  const int total = a.heads * w.nch;
  for (int it = c.g; it < total; it += c.grid) {
    if (attn_item_workgroup(it, c.grid) != c.g) continue;
    int h, ch;
    w.decode(it, h, ch);
    const int row0 = ch * a.chunk;
    const int rows = a.window - row0 < a.chunk ? a.window - row0 : a.chunk;
    const uint32_t bytes = (uint32_t)rows * (uint32_t)a.dim * Traits<P>::kKvBytes;  // a multiple of 4
    for (int l = 0; l < a.layers; l++) {
      const uint32_t b0 = ((uint32_t)(l * a.heads + h) * (uint32_t)a.window + (uint32_t)row0) * (uint32_t)a.dim *
                          Traits<P>::kKvBytes;
      for (uint32_t off = threadIdx.x * 4u; off < bytes; off += kThreads * 4u) {
        *reinterpret_cast<float*>(out + kSnapKeys + b0 + off) = ld4_coherent(c.kr, b0 + off);
        *reinterpret_cast<float*>(out + kSnapKeys + ring + b0 + off) = ld4_coherent(c.vr, b0 + off);
      }
    }
  }
  float* hidden = reinterpret_cast<float*>(out + kSnapKeys + 2u * ring);
  for (int i = c.g * kThreads + (int)threadIdx.x; i < a.layers * a.width; i += c.grid * kThreads)
    hidden[i] = ld4_coherent(c.sr, (a.s_hidden + (uint32_t)i) * 4u);
  if (c.g == 0 && threadIdx.x == 0) *reinterpret_cast<unsigned long long*>(out) = t;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
}

// Persistent worker (Backend::PERSISTENT): one resident launch serves RUN / RESET / PING /
// SNAPSHOT / STOP commands from a host mailbox, following the reference's persistent_kernel
// (src/cuda/Runtime.cu:58-122) and its ordering contract (docs/transport.md:9-16):
//  - workgroup 0's control wave acquires the request word (system scope), stages a RUN's
//    event into the tagged vector t_in and publishes the command as the tagged word t_cmd
//    with the command's epoch base; every workgroup polls t_cmd;
//  - each workgroup reports done (t_wdone[g]) after all of its stores have completed, and
//    workgroup 0 then writes the score and releases the completion word (system scope);
//  - the worker exits on STOP, after max_events RUN commands, or when no request arrives
//    within the idle budget; it then sets the exited word. Every command uses one step's
//    worth of epochs.
template <int P, int A>
__global__ __launch_bounds__(kThreads) void persistent_kernel(const StepArgs* __restrict__ ap) {
  const StepArgs& a = *ap;
  __shared__ LdsAll lds;
  Ctx<P> c(a, lds, (int)blockIdx.x, (int)gridDim.x);
  c.tagged_input = true;
  const unsigned base0 = load_epoch(a);
  const unsigned per_step = (unsigned)ph_final(a) + 2u;
  unsigned long long t = load_position(a);
  unsigned long long previous = a.initial_sequence, processed = 0, seq = 0;
  unsigned k = 0;
  for (;; k++) {
    const unsigned base = base0 + k * per_step;
    c.base = base;
    if (c.wave == 0) {
      int cmd = kCmdExit;
      if (c.g == 0) {
        unsigned long long got = previous;
        if (c.lane == 0) {
          const unsigned long long start = wall_clock64();
          while (true) {
            got = __hip_atomic_load(a.mb_request, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
            if (got != previous) {
              cmd = __hip_atomic_load(a.mb_command, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
              break;
            }
            if (wall_clock64() - start >= a.idle_ticks) break;  // idle budget spent: exit
            if (a.backoff) __builtin_amdgcn_s_sleep(127);
            else __builtin_amdgcn_s_sleep(2);
          }
        }
        cmd = __shfl(cmd, 0);
        seq = ((unsigned long long)(unsigned)__shfl((int)(got >> 32), 0) << 32) | (unsigned)__shfl((int)got, 0);
        if (cmd == kCmdRun) {
          // The event crosses PCIe: issue all of a lane's loads (features_p <= 1024, so at
          // most 16) before any store, one round trip instead of one per element.
          constexpr int kIn = 1024 / 64;
          float v[kIn];
#pragma unroll
          for (int j = 0; j < kIn; j++) {
            const int i = c.lane + 64 * j;
            v[j] = i < a.features ? a.mapped_input[i] : 0.f;
          }
#pragma unroll
          for (int j = 0; j < kIn; j++) {
            const int i = c.lane + 64 * j;
            if (i < a.features_p) c.tstore(a.t_in + (uint32_t)i, base, v[j]);
          }
        }
        if (c.lane == 0) c.tstore(a.t_cmd, base, __builtin_bit_cast(float, cmd));
      }
      // Every workgroup waits for the command (as long as the coordinator may wait, and then
      // the usual poll limit).
      const unsigned long long start = wall_clock64();
      uint2 w;
      while (true) {
        w = c.tload(a.t_cmd);
        if (w.y == base) break;
        if (wall_clock64() - start > a.idle_ticks + a.spin_limit) {
          c.timeout();
          w.x = (unsigned)kCmdExit;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      if (c.lane == 0) c.lds.cmd = (int)w.x;
    }
    lds_barrier();
    const int cmd = __builtin_amdgcn_readfirstlane(c.lds.cmd);
    if (cmd == kCmdExit) break;
    if (cmd == kCmdRun) {
      c.set_position(t);
      forward<P, A>(c);
      t++;
    } else if (cmd == kCmdReset) {
      reset_owned(c);
      t = 0;
    } else if (cmd == kCmdSnapshot) {
      snapshot_owned(c, t);
    } else if (cmd == kCmdPing && c.g == 0 && threadIdx.x == 0) {
      unsigned long long sum = 0;
      for (int i = 0; i < a.features; i++) sum += __builtin_bit_cast(unsigned, a.mapped_input[i]);
      __hip_atomic_store(a.mb_checksum, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    // This workgroup's stores are complete: report done for this command.
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    const unsigned done_ep = base + per_step - 1u;
    if (threadIdx.x == 0) c.tstore(a.t_wdone + (uint32_t)c.g, done_ep, 0.f);
    if (c.g == 0 && c.wave == 0) {
      const unsigned long long start = wall_clock64();
      while (true) {
        bool ok = true;
        for (int i = c.lane; i < c.grid; i += 64) ok = ok && c.tload(a.t_wdone + (uint32_t)i).y == done_ep;
        if (__all(ok) || c.dead || c.expired(start)) break;
        __builtin_amdgcn_s_sleep(2);
      }
      if (c.lane == 0) {
        if (cmd == kCmdRun)
          __hip_atomic_store(a.mb_score, ld4_coherent(c.sr, a.s_score * 4u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(a.mb_error, __hip_atomic_load(a.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(a.mb_completion, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
      }
    }
    previous = seq;
    if (cmd == kCmdRun) processed++;
    if (cmd == kCmdStop || (a.max_events && processed >= a.max_events)) break;
    lds_barrier();  // every wave has read lds.cmd before the next command overwrites it
  }
  if (c.g == 0 && threadIdx.x == 0) {
    __hip_atomic_store(a.epoch, base0 + (k + 1u) * per_step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(a.mb_exited, 1ull, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// Zero K/V, hidden state and the position (src/cuda/Primitives.cuh:280-292). Tagged vectors
// keep their tags: epochs only grow.
__global__ void reset_kernel(const StepArgs* __restrict__ ap) {
  const StepArgs& a = *ap;
  size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  uint32_t* k = reinterpret_cast<uint32_t*>(a.keys);
  uint32_t* v = reinterpret_cast<uint32_t*>(a.values);
  for (size_t i = tid; i < a.cache_bytes / 4; i += stride) {
    k[i] = 0;
    v[i] = 0;
  }
  for (size_t i = tid; i < (size_t)a.layers * a.width; i += stride) a.scratch[a.s_hidden + i] = 0.f;
  if (tid == 0) *a.position = 0;
}

}  // namespace stamd
