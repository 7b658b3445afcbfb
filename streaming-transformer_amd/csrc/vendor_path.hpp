// Vendor GEMV backends (Backend::CUBLAS / CUBLAS_GRAPH of the reference, src/cuda/Runtime.cu:
// 330-385): the step as a staged sequence whose projections are rocBLAS calls, the comparison
// point for the hand-written kernels. FP32 models use rocblas_sgemv (transposed, on the
// row-major weight arena); mixed models cast the GEMV input to FP16 and use rocblas_gemm_ex
// (FP16 in, FP32 out, FP32 compute), then round the output to FP16 at the reference's cast
// points; the input projection uses an FP32 copy of its weights (src/cuda/Runtime.cu:255-256,
// 333). Everything else runs in small HIP kernels over the runtime's own ring, hidden state
// and position, so reset, snapshot and the traces are shared with the other backends.
// Included by runtime.hip inside namespace stamd.
#pragma once

struct VendorArgs {
  int layers, width, heads, dim, ffn, window, features;
  int width_p, ffn_p;
  float epsilon;
  const char* weights;
  void* keys;                     // ring [L][H][W][dh], FP32 or FP16 (mixed)
  void* values;
  float* hidden;                  // [L][d]
  unsigned long long* position;
  const float* rope_freq;         // [dh/2]
  float* score_out;               // the runtime's score word
  float* x;                       // [d] residual stream
  float* xn;                      // [max(d, F)] GEMV input (FP32)
  uint16_t* xh;                   // [max(d, F)] GEMV input as FP16 (mixed)
  float* y;                       // [max(3d, 2F)] GEMV output
  float* q;                       // [d] rotated query
  float* score;                   // [1] score GEMV output
  float* part;                    // attention partials [H][chunks][dh + 2]: o, max, exp sum
};

constexpr int kVendorThreads = 256;

// Round where the mixed model casts (src/cuda/Primitives.cuh:82-84); identity otherwise.
template <bool M>
__device__ __forceinline__ float vcast(float v) {
  if constexpr (M) return (float)(_Float16)v;
  return v;
}
template <bool M>
__device__ __forceinline__ float vweight(const char* w, uint32_t off, int i) {
  if constexpr (M) return half_to_float(reinterpret_cast<const uint16_t*>(w + off)[i]);
  return reinterpret_cast<const float*>(w + off)[i];
}
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_total(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float s = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return s;
}

// RMSNorm of x into the GEMV input (src/cuda/Primitives.cuh:122-135): out = x s g, s =
// 1/sqrt(sum x^2 / d + eps), cast; FP16 copy for the mixed GEMM. kCastIn first rounds x in
// place (the input projection's output cast in mixed mode).
template <bool M, bool kCastIn>
__global__ __launch_bounds__(kVendorThreads) void vnd_norm(const VendorArgs* __restrict__ ap, uint32_t w_norm) {
  const VendorArgs& a = *ap;
  __shared__ float red[kVendorThreads / 64];
  float s = 0.f;
  for (int i = threadIdx.x; i < a.width; i += blockDim.x) {
    float v = a.x[i];
    if constexpr (kCastIn) {
      v = vcast<M>(v);
      a.x[i] = v;
    }
    s += v * v;
  }
  const float scale = 1.0f / sqrtf(block_sum(s, red) / (float)a.width + a.epsilon);
  for (int i = threadIdx.x; i < a.width; i += blockDim.x) {
    const float v = vcast<M>(a.x[i] * scale * vweight<M>(a.weights, w_norm, i));
    a.xn[i] = v;
    if constexpr (M) a.xh[i] = float_to_half(v);
  }
}

// RoPE on adjacent pairs of q and k, then the ring write of k and v at slot t mod W
// (src/cuda/Primitives.cuh:148-166). y holds q; k; v from one GEMV. One thread per pair.
template <bool M>
__global__ __launch_bounds__(kVendorThreads) void vnd_rope_ring(const VendorArgs* __restrict__ ap, int layer) {
  const VendorArgs& a = *ap;
  const int pair = blockIdx.x * blockDim.x + threadIdx.x;
  if (pair >= 3 * a.width / 2) return;
  const int n = 2 * pair, sec = n / a.width, i = n - sec * a.width;
  const unsigned long long t = *a.position;
  float va = vcast<M>(a.y[n]), vb = vcast<M>(a.y[n + 1]);
  if (sec < 2) {
    const int e = i % a.dim;
    const float angle = (float)t * a.rope_freq[e >> 1];
    const float co = cosf(angle), si = sinf(angle);
    const float ra = va * co - vb * si, rb = va * si + vb * co;
    va = vcast<M>(ra);
    vb = vcast<M>(rb);
  }
  if (sec == 0) {
    a.q[i] = va;
    a.q[i + 1] = vb;
    return;
  }
  const int h = i / a.dim, d = i - h * a.dim;
  const size_t idx = (((size_t)layer * a.heads + h) * a.window + (size_t)(t % (unsigned long long)a.window)) * a.dim + d;
  void* ring = sec == 1 ? a.keys : a.values;
  if constexpr (M) {
    reinterpret_cast<uint16_t*>(ring)[idx] = float_to_half(va);
    reinterpret_cast<uint16_t*>(ring)[idx + 1] = float_to_half(vb);
  } else {
    reinterpret_cast<float*>(ring)[idx] = va;
    reinterpret_cast<float*>(ring)[idx + 1] = vb;
  }
}

template <bool M>
__device__ __forceinline__ float ring_at(const void* ring, size_t i) {
  if constexpr (M) return half_to_float(reinterpret_cast<const uint16_t*>(ring)[i]);
  return reinterpret_cast<const float*>(ring)[i];
}

// Attention (src/cuda/Primitives.cuh:167-219) in two kernels, so that the window is read by
// many workgroups: vnd_attn_part computes, for one (head, 64-slot chunk), the chunk's logit
// maximum m, exp sum s and unnormalized output o = sum_j e^(l_j - m) V_j; vnd_attn_combine
// merges a head's chunks in chunk order: out = sum_c o_c e^(m_c - M) / sum_c s_c e^(m_c - M),
// then casts. Chunks past the valid window report m = -inf, s = 0.
// vnd_attn_part: 256 threads = 16 groups of 16 lanes. Logits: a group per K row (lane r
// covers elements 4r .. 4r+3 of each 64-element piece), a 16-lane DPP sum. Values: group g
// sums its slots' V rows, the 16 groups summed in LDS in group order.
constexpr int kAttnChunk = 64;
constexpr int kAttnPartThreads = 256;
template <bool M>
__global__ __launch_bounds__(kAttnPartThreads) void vnd_attn_part(const VendorArgs* __restrict__ ap, int layer) {
  const VendorArgs& a = *ap;
  __shared__ float pr[kAttnChunk];
  __shared__ float red[kAttnPartThreads / 64];
  __shared__ float4 vred[16][17];
  const int nch = (a.window + kAttnChunk - 1) / kAttnChunk;
  const int h = blockIdx.x / nch, ch = blockIdx.x - h * nch;
  const int dim = a.dim, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = tid & 15, grp = tid >> 4;
  const unsigned long long t = *a.position;
  const int valid = t + 1 < (unsigned long long)a.window ? (int)(t + 1) : a.window;
  const int s0 = ch * kAttnChunk, s1 = min(valid, s0 + kAttnChunk);
  float* part = a.part + (size_t)blockIdx.x * (dim + 2);
  if (s0 >= valid) {  // uniform over the workgroup
    for (int d = tid; d < dim; d += blockDim.x) part[d] = 0.f;
    if (tid == 0) {
      part[dim] = -INFINITY;
      part[dim + 1] = 0.f;
    }
    return;
  }
  const size_t base = ((size_t)layer * a.heads + h) * (size_t)a.window * dim;
  const float* q = a.q + h * dim;
  const float div = sqrtf((float)dim);
  float mx = -INFINITY;
  for (int sb = s0; sb < s1; sb += 16) {
    const int s = sb + grp;
    const size_t row = base + (size_t)(s < s1 ? s : s1 - 1) * dim;
    float dot = 0.f;
    for (int d = 4 * r; d < dim; d += 64)
#pragma unroll
      for (int j = 0; j < 4; j++)
        if (d + j < dim) dot += q[d + j] * ring_at<M>(a.keys, row + d + j);
    dot = group_sum(dot, 16);
    if (s < s1) {
      const float lg = dot / div;
      if (r == 0) pr[s - s0] = lg;
      mx = fmaxf(mx, lg);
    }
  }
  mx = wave_top(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.f;
  if (tid < s1 - s0) {
    const float e = expf(pr[tid] - mx);
    pr[tid] = e;
    sum = e;
  }
  sum = wave_total(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  sum = (red[0] + red[1]) + (red[2] + red[3]);
  for (int d0 = 0; d0 < dim; d0 += 64) {
    const int d = d0 + 4 * r;
    float o[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s = s0 + grp; s < s1; s += 16) {
      const float p = pr[s - s0];
      const size_t row = base + (size_t)s * dim;
#pragma unroll
      for (int j = 0; j < 4; j++)
        if (d + j < dim) o[j] += p * ring_at<M>(a.values, row + d + j);
    }
    vred[grp][r] = make_float4(o[0], o[1], o[2], o[3]);
    __syncthreads();
    if (tid < 16) {
      float4 acc = vred[0][tid];
      for (int k = 1; k < 16; k++) {
        const float4 v = vred[k][tid];
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
      }
      const float vals[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
      for (int j = 0; j < 4; j++)
        if (d0 + 4 * tid + j < dim) part[d0 + 4 * tid + j] = vals[j];
    }
    __syncthreads();
  }
  if (tid == 0) {
    part[dim] = mx;
    part[dim + 1] = sum;
  }
}

template <bool M>
__global__ __launch_bounds__(64) void vnd_attn_combine(const VendorArgs* __restrict__ ap) {
  const VendorArgs& a = *ap;
  const int nch = (a.window + kAttnChunk - 1) / kAttnChunk;
  const int h = blockIdx.x, dim = a.dim;
  const float* part = a.part + (size_t)h * nch * (dim + 2);
  float mx = -INFINITY;
  for (int c = 0; c < nch; c++) mx = fmaxf(mx, part[(size_t)c * (dim + 2) + dim]);
  float total = 0.f;
  for (int c = 0; c < nch; c++) {
    const float* p = part + (size_t)c * (dim + 2);
    total += p[dim + 1] * expf(p[dim] - mx);
  }
  for (int d = threadIdx.x; d < dim; d += blockDim.x) {
    float o = 0.f;
    for (int c = 0; c < nch; c++) {
      const float* p = part + (size_t)c * (dim + 2);
      o += p[d] * expf(p[dim] - mx);
    }
    const float v = vcast<M>(o / total);
    a.xn[h * dim + d] = v;
    if constexpr (M) a.xh[h * dim + d] = float_to_half(v);
  }
}

// x += cast(y) then cast (src/cuda/Primitives.cuh:221-229); the DOWN residual also records
// the hidden state of the layer.
template <bool M>
__global__ __launch_bounds__(kVendorThreads) void vnd_residual(const VendorArgs* __restrict__ ap, int layer,
                                                                 int record) {
  const VendorArgs& a = *ap;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.width) return;
  const float v = vcast<M>(a.x[i] + vcast<M>(a.y[i]));
  a.x[i] = v;
  if (record) a.hidden[(size_t)layer * a.width + i] = v;
}

// SwiGLU on the interleaved gate/up GEMV output (src/cuda/Primitives.cuh:231-239).
template <bool M>
__global__ __launch_bounds__(kVendorThreads) void vnd_swiglu(const VendorArgs* __restrict__ ap) {
  const VendorArgs& a = *ap;
  const int u = blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= a.ffn) return;
  const float g = vcast<M>(a.y[2 * u]), up = vcast<M>(a.y[2 * u + 1]);
  const float v = vcast<M>((g / (1.0f + expf(-g))) * up);
  a.xn[u] = v;
  if constexpr (M) a.xh[u] = float_to_half(v);
}

// Publish the score and advance the position (src/cuda/Runtime.cu:380-383).
__global__ void vnd_advance(const VendorArgs* __restrict__ ap) {
  const VendorArgs& a = *ap;
  *a.score_out = *a.score;
  *a.position = *a.position + 1;
}

#define ROCBLAS_CHECK(expr)                                                                        \
  do {                                                                                            \
    rocblas_status rb_status_ = (expr);                                                           \
    if (rb_status_ != rocblas_status_success)                                                     \
      throw Error(ST_ERR_DEVICE, std::string("rocBLAS: ") + rocblas_status_to_string(rb_status_) + " at " #expr); \
  } while (0)

class VendorPath {
 public:
  VendorPath(const st_config& c, bool mixed, const StepArgs& s, const st_tensor* tensors, size_t count,
             hipStream_t stream)
      : c_(c), mixed_(mixed), s_(s), stream_(stream) {
    ROCBLAS_CHECK(rocblas_create_handle(&handle_));
    ROCBLAS_CHECK(rocblas_set_stream(handle_, stream_));
    ROCBLAS_CHECK(rocblas_set_pointer_mode(handle_, rocblas_pointer_mode_host));
    ROCBLAS_CHECK(rocblas_set_atomics_mode(handle_, rocblas_atomics_not_allowed));
    // Library workspace owned here and set before any capture (src/cuda/Runtime.cu:258-261).
    workspace_.alloc(4u << 20);
    ROCBLAS_CHECK(rocblas_set_workspace(handle_, workspace_.ptr, 4u << 20));
    VendorArgs& a = args_;
    a.layers = c.layers;
    a.width = c.width;
    a.heads = c.heads;
    a.dim = c.width / c.heads;
    a.ffn = c.ffn;
    a.window = c.window;
    a.features = c.features;
    a.width_p = s.width_p;
    a.ffn_p = s.ffn_p;
    a.epsilon = c.epsilon;
    a.weights = s.weights;
    a.keys = s.keys;
    a.values = s.values;
    a.hidden = s.scratch + s.s_hidden;
    a.position = s.position;
    a.rope_freq = s.rope_freq;
    a.score_out = s.scratch + s.s_score;
    const size_t wide = (size_t)std::max(c.width, c.ffn), out = (size_t)std::max(3 * c.width, 2 * c.ffn);
    a.x = alloc(x_, c.width);
    a.xn = alloc(xn_, wide);
    xh_.alloc(wide * 2);
    HIP_CHECK(hipMemset(xh_.ptr, 0, wide * 2));
    a.xh = reinterpret_cast<uint16_t*>(xh_.ptr);
    a.y = alloc(y_, out);
    a.q = alloc(q_, c.width);
    a.score = alloc(score_, 1);
    a.part = alloc(part_, (size_t)c.heads * ((c.window + kAttnChunk - 1) / kAttnChunk) * (c.width / c.heads + 2));
    // FP32 view of the input projection (the arena holds FP16 for a mixed model).
    const float* input = nullptr;
    for (size_t i = 0; i < count; i++)
      if (tensors[i].name && std::strcmp(tensors[i].name, "input") == 0) input = tensors[i].data;
    if (!input) throw Error(ST_ERR_INVALID, "Missing tensor: input");
    input_f32_.alloc((size_t)c.width * c.features * 4);
    HIP_CHECK(hipMemcpy(input_f32_.ptr, input, (size_t)c.width * c.features * 4, hipMemcpyHostToDevice));
    args_dev_.alloc(sizeof(VendorArgs));
    HIP_CHECK(hipMemcpy(args_dev_.ptr, &args_, sizeof(VendorArgs), hipMemcpyHostToDevice));
    dargs_ = reinterpret_cast<const VendorArgs*>(args_dev_.ptr);
  }
  ~VendorPath() {
    if (handle_) (void)rocblas_destroy_handle(handle_);
  }
  void launch() {
    if (mixed_) launch_t<true>();
    else launch_t<false>();
  }

 private:
  float* alloc(DeviceBuffer& b, size_t n) {
    b.alloc(n * 4);
    HIP_CHECK(hipMemset(b.ptr, 0, n * 4));
    return reinterpret_cast<float*>(b.ptr);
  }
  // y[0..rows) = W[rows x cols] . input over the arena rows (leading dimension ld elements).
  void gemv(uint32_t woff, int ld, int rows, int cols, bool half_input, const float* input, float* y) {
    const float one = 1.f, zero = 0.f;
    const void* w = s_.weights + woff;
    if (!half_input) {
      ROCBLAS_CHECK(rocblas_sgemv(handle_, rocblas_operation_transpose, cols, rows, &one,
                                  reinterpret_cast<const float*>(w), ld, input, 1, &zero, y, 1));
    } else {
      ROCBLAS_CHECK(rocblas_gemm_ex(handle_, rocblas_operation_transpose, rocblas_operation_none, rows, 1, cols, &one,
                                    w, rocblas_datatype_f16_r, ld, args_.xh, rocblas_datatype_f16_r, cols, &zero, y,
                                    rocblas_datatype_f32_r, rows, y, rocblas_datatype_f32_r, rows,
                                    rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0));
    }
  }
  template <bool M>
  void launch_t() {
    const VendorArgs& a = args_;
    const int d = c_.width, F = c_.ffn, T = kVendorThreads;
    const int chunks = (c_.window + kAttnChunk - 1) / kAttnChunk;
    const float one = 1.f, zero = 0.f;
    // Input projection on the FP32 weights and the FP32 event.
    ROCBLAS_CHECK(rocblas_sgemv(handle_, rocblas_operation_transpose, c_.features, d, &one,
                                reinterpret_cast<const float*>(input_f32_.ptr), c_.features, s_.scratch + s_.s_input, 1,
                                &zero, a.x, 1));
    for (int l = 0; l < c_.layers; l++) {
      const LayerWeights& w = s_.layer[l];
      if (l == 0) hipLaunchKernelGGL((vnd_norm<M, true>), dim3(1), dim3(T), 0, stream_, dargs_, w.norm1);
      else hipLaunchKernelGGL((vnd_norm<M, false>), dim3(1), dim3(T), 0, stream_, dargs_, w.norm1);
      gemv(w.qkv, a.width_p, 3 * d, d, M, a.xn, a.y);
      hipLaunchKernelGGL((vnd_rope_ring<M>), dim3((3 * d / 2 + T - 1) / T), dim3(T), 0, stream_, dargs_, l);
      hipLaunchKernelGGL((vnd_attn_part<M>), dim3(c_.heads * chunks), dim3(kAttnPartThreads), 0, stream_, dargs_, l);
      hipLaunchKernelGGL((vnd_attn_combine<M>), dim3(c_.heads), dim3(64), 0, stream_, dargs_);
      gemv(w.out, a.width_p, d, d, M, a.xn, a.y);
      hipLaunchKernelGGL((vnd_residual<M>), dim3((d + T - 1) / T), dim3(T), 0, stream_, dargs_, l, 0);
      hipLaunchKernelGGL((vnd_norm<M, false>), dim3(1), dim3(T), 0, stream_, dargs_, w.norm2);
      gemv(w.gateup, a.width_p, 2 * F, d, M, a.xn, a.y);
      hipLaunchKernelGGL((vnd_swiglu<M>), dim3((F + T - 1) / T), dim3(T), 0, stream_, dargs_);
      gemv(w.down, a.ffn_p, d, F, M, a.xn, a.y);
      hipLaunchKernelGGL((vnd_residual<M>), dim3((d + T - 1) / T), dim3(T), 0, stream_, dargs_, l, 1);
    }
    hipLaunchKernelGGL((vnd_norm<M, false>), dim3(1), dim3(T), 0, stream_, dargs_, s_.w_final_norm);
    gemv(s_.w_score, a.width_p, 1, d, M, a.xn, a.score);  // final: no cast
    hipLaunchKernelGGL(vnd_advance, dim3(1), dim3(1), 0, stream_, dargs_);
    HIP_CHECK(hipGetLastError());
  }

  st_config c_;
  bool mixed_;
  const StepArgs& s_;
  hipStream_t stream_;
  rocblas_handle handle_ = nullptr;
  DeviceBuffer workspace_, x_, xn_, xh_, y_, q_, score_, part_, input_f32_, args_dev_;
  VendorArgs args_{};
  const VendorArgs* dargs_ = nullptr;
};
