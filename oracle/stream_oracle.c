/*
 * CPU oracle: plain-C restatement of the reference CPU step.
 *
 * TEST INFRASTRUCTURE ONLY (a reference for comparison, never the product): loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 *
 * Follows, function by function:
 *   oracle_linear   <- Cpu::linear      src/cpu/Cpu.cpp:29-41   (row-major GEMV, cast unless final)
 *   oracle_norm     <- Cpu::norm        src/cpu/Cpu.cpp:43-57   (1/sqrt(sum/width + eps), cast)
 *   so_step         <- Cpu::step        src/cpu/Cpu.cpp:59-141  (op order, RoPE :73-83, ring write
 *                                        :91-96, physical-ring attention :97-109, residuals, SwiGLU)
 *   so_step_trace   <- Cpu::step with a CpuTrace  src/cpu/Cpu.cpp:29-57,64-66,86-133 (entry names
 *                                        and capture points of linear, norm and the step)
 *   so_reset        <- Cpu::reset       src/cpu/Cpu.cpp:143-148
 *   so_round_half   <- roundHalf        src/runtime/Model.cpp:59-61 (Eigen::half: RNE, overflow to inf)
 *   mixed cast rule <- reference/model.py:1-5 and Math.cast :57-58
 *
 * Pinning (each check lives in tests/):
 *   - end-to-end against the reference's golden vectors fixtures/small-{fp32,mixed}/expected
 *     (201 events, eviction, several ring revolutions, warm reset): test_oracle_golden.py;
 *   - the float and double accumulation variants against each other at the Small, Main and Large shapes;
 *   - an independent numpy FullSequence local-causal masked forward (reference/model.py:140-160),
 *     which shares no ring/position logic with this file: test_oracle_invariants.py;
 *   - closed forms: adjacent-pair RoPE (tests/test_porting_contract.py:10-21), zero Q/K =>
 *     attention is the mean of the retained V across eviction and reset (:24-51), zero input =>
 *     score exactly 0 (tests/Lifecycle.cu:38), roundHalf KAT (tests/Native.cpp:20-21) and the
 *     half/bfloat16 rounders against numpy/torch conversions.
 * Eigen's exact GEMV reduction tree is not restated (this file uses eight interleaved partial
 * sums), so float results agree with the reference within its FP32 tolerance, not bit for bit.
 */
#include "stream_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

struct so_state {
  so_config c;
  int mixed, dbl, threads;
  int dim;
  uint64_t position;
  float** w;        /* tensors in canonical order, owned copies */
  float *keys, *values, *hidden;
  float *x, *norm, *q, *k, *v, *attention, *temp, *gate, *up, *logits;
  so_trace_fn trace; /* per-operation capture (so_step_trace), else NULL */
  void* trace_user;
};

/* Report one captured vector as "<prefix><name><suffix>" when tracing. */
static void emit(const so_state* s, const char* prefix, const char* name, const char* suffix, const float* v, int n) {
  if (!s->trace) return;
  char full[96];
  snprintf(full, sizeof full, "%s%s%s", prefix, name, suffix);
  s->trace(s->trace_user, full, v, n);
}

/* ---------------- rounding helpers ---------------- */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t so_half_bits(float value) {
  uint32_t u = f2u(value);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t exp = (u >> 23) & 0xffu;
  uint32_t man = u & 0x7fffffu;
  if (exp == 0xffu) { /* inf / nan */
    return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
  }
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
  if (e <= 0) {
    /* subnormal half (or zero): value = man_full * 2^(exp-150); half unit = 2^-24 */
    if (e < -10) return (uint16_t)sign; /* below half of the smallest subnormal */
    uint32_t full = man | 0x800000u;
    int shift = 14 - e; /* 14..24 */
    uint32_t half = full >> shift;
    uint32_t rem = full & ((1u << shift) - 1u);
    uint32_t mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1u))) half++;
    return (uint16_t)(sign | half);
  }
  uint32_t half = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++; /* may carry into exponent/inf */
  return (uint16_t)(sign | half);
}

float so_half_to_float(uint16_t bits) {
  uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
  uint32_t exp = (bits >> 10) & 0x1fu;
  uint32_t man = bits & 0x3ffu;
  if (exp == 0x1fu) return u2f(sign | 0x7f800000u | (man << 13));
  if (exp == 0) {
    if (!man) return u2f(sign);
    float f = (float)man * 5.9604644775390625e-8f; /* 2^-24, exact */
    return sign ? -f : f;
  }
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

float so_round_half(float value) { return so_half_to_float(so_half_bits(value)); }

uint16_t so_bf16_bits(float value) {
  uint32_t u = f2u(value);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

float so_round_bf16(float value) { return u2f((uint32_t)so_bf16_bits(value) << 16); }

/* ---------------- model ---------------- */

enum { T_INPUT = 0, T_FINAL_NORM = 1, T_SCORE = 2, T_LAYER = 3 };
enum { L_NORM1, L_NORM2, L_Q, L_K, L_V, L_OUT, L_GATE, L_UP, L_DOWN, L_COUNT };

static size_t tensor_elems(const so_config* c, int index) {
  size_t d = (size_t)c->width, f = (size_t)c->ffn;
  if (index == T_INPUT) return d * (size_t)c->features;
  if (index == T_FINAL_NORM || index == T_SCORE) return d;
  switch ((index - T_LAYER) % L_COUNT) {
    case L_NORM1: case L_NORM2: return d;
    case L_Q: case L_K: case L_V: case L_OUT: return d * d;
    default: return f * d;
  }
}

/* ModelConfig::validate, src/runtime/Model.cpp:22-29 */
static int valid_config(const so_config* c) {
  return !(c->layers < 1 || c->layers > 16 || c->width < 1 || c->width > 1024 || c->heads < 1 ||
           c->width % c->heads || (c->width / c->heads) % 2 || c->ffn < 1 || c->ffn > 4096 ||
           c->window < 1 || c->window > 4096 || c->features < 1 || c->features > 1024 ||
           !isfinite(c->epsilon) || c->epsilon <= 0);
}

static float* layer_w(so_state* s, int l, int which) { return s->w[T_LAYER + l * L_COUNT + which]; }

static void cast(const so_state* s, float* data, int n) {
  if (s->mixed) for (int i = 0; i < n; i++) data[i] = so_round_half(data[i]);
}

/* Cpu::linear: output[r] = sum_c W[r,c] * input[c], cast unless final. `prefix` + `name`
 * names the projection in a trace. */
static void oracle_linear(so_state* s, const char* prefix, const char* name, const float* weight, const float* input,
                          float* output, int rows, int cols, int final) {
  emit(s, prefix, name, ".operand", input, cols);
  if (s->dbl) {
#pragma omp parallel for num_threads(s->threads) if (s->threads > 1) schedule(static)
    for (int r = 0; r < rows; r++) {
      const float* row = weight + (size_t)r * cols;
      double sum = 0;
      for (int c = 0; c < cols; c++) sum += (double)row[c] * (double)input[c];
      output[r] = (float)sum;
    }
  } else {
#pragma omp parallel for num_threads(s->threads) if (s->threads > 1) schedule(static)
    for (int r = 0; r < rows; r++) {
      /* Eight interleaved FP32 partial sums combined pairwise, like Eigen's packet
       * accumulation in its row-major GEMV; vectorizes without reassociation. */
      const float* row = weight + (size_t)r * cols;
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      int c = 0;
      for (; c + 8 <= cols; c += 8)
        for (int k = 0; k < 8; k++) acc[k] += row[c + k] * input[c + k];
      float sum = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
      for (; c < cols; c++) sum += row[c] * input[c];
      output[r] = sum;
    }
  }
  emit(s, prefix, name, ".pre_cast", output, rows);
  if (!final) cast(s, output, rows);
  emit(s, prefix, name, ".linear", output, rows);
}

/* Cpu::norm */
static void oracle_norm(so_state* s, const char* prefix, const char* name, const float* input, const float* weight,
                        float* output) {
  int d = s->c.width;
  emit(s, prefix, name, ".operand", input, d);
  if (s->dbl) {
    double sum = 0;
    for (int i = 0; i < d; i++) sum += (double)input[i] * input[i];
    double scale = 1.0 / sqrt(sum / d + (double)s->c.epsilon);
    for (int i = 0; i < d; i++) output[i] = (float)((double)input[i] * scale * weight[i]);
  } else {
    float sum = 0;
    for (int i = 0; i < d; i++) sum += input[i] * input[i];
    float scale = 1.0f / sqrtf(sum / d + s->c.epsilon);
    for (int i = 0; i < d; i++) output[i] = input[i] * scale * weight[i];
  }
  emit(s, prefix, name, ".pre_cast", output, d);
  cast(s, output, d);
  emit(s, prefix, name, ".norm", output, d);
}

so_state* so_create(const so_config* config, int mixed, int accumulate_double,
                    const float* const* tensors) {
  if (!config || !tensors || !valid_config(config)) return NULL;
  so_state* s = (so_state*)calloc(1, sizeof(so_state));
  if (!s) return NULL;
  s->c = *config;
  s->mixed = mixed != 0;
  s->dbl = accumulate_double != 0;
  s->threads = 1;
  s->dim = config->width / config->heads;
  int count = T_LAYER + config->layers * L_COUNT;
  s->w = (float**)calloc((size_t)count, sizeof(float*));
  for (int i = 0; i < count; i++) {
    size_t n = tensor_elems(config, i);
    s->w[i] = (float*)malloc(n * sizeof(float));
    memcpy(s->w[i], tensors[i], n * sizeof(float));
  }
  size_t cache = (size_t)config->layers * config->width * config->window;
  int d = config->width;
  s->keys = (float*)calloc(cache, sizeof(float));
  s->values = (float*)calloc(cache, sizeof(float));
  s->hidden = (float*)calloc((size_t)config->layers * d, sizeof(float));
  s->x = (float*)calloc((size_t)d, sizeof(float));
  s->norm = (float*)calloc((size_t)d, sizeof(float));
  s->q = (float*)calloc((size_t)d, sizeof(float));
  s->k = (float*)calloc((size_t)d, sizeof(float));
  s->v = (float*)calloc((size_t)d, sizeof(float));
  s->attention = (float*)calloc((size_t)d, sizeof(float));
  s->temp = (float*)calloc((size_t)d, sizeof(float));
  s->gate = (float*)calloc((size_t)config->ffn, sizeof(float));
  s->up = (float*)calloc((size_t)config->ffn, sizeof(float));
  s->logits = (float*)calloc((size_t)config->window, sizeof(float));
  return s;
}

void so_destroy(so_state* s) {
  if (!s) return;
  int count = T_LAYER + s->c.layers * L_COUNT;
  for (int i = 0; i < count; i++) free(s->w[i]);
  free(s->w);
  free(s->keys); free(s->values); free(s->hidden);
  free(s->x); free(s->norm); free(s->q); free(s->k); free(s->v);
  free(s->attention); free(s->temp); free(s->gate); free(s->up); free(s->logits);
  free(s);
}

void so_set_threads(so_state* s, int threads) { if (s) s->threads = threads < 1 ? 1 : threads; }

/* Per-head attention over the physical ring order, Cpu.cpp:97-109. */
static void oracle_attention(so_state* s, int l, int h, int valid) {
  const so_config* c = &s->c;
  int d = s->dim;
  size_t base = ((size_t)l * c->heads + h) * (size_t)c->window * d;
  const float* keys = s->keys + base;
  const float* values = s->values + base;
  const float* q = s->q + h * d;
  float* out = s->attention + h * d;
  if (s->dbl) {
    double maximum = -INFINITY;
    double* p = (double*)malloc((size_t)valid * sizeof(double));
    for (int j = 0; j < valid; j++) {
      double dot = 0;
      for (int i = 0; i < d; i++) dot += (double)keys[(size_t)j * d + i] * q[i];
      p[j] = dot / sqrt((double)d);
      if (p[j] > maximum) maximum = p[j];
    }
    double total = 0;
    for (int j = 0; j < valid; j++) { p[j] = exp(p[j] - maximum); total += p[j]; }
    for (int j = 0; j < valid; j++) p[j] /= total;
    for (int i = 0; i < d; i++) {
      double sum = 0;
      for (int j = 0; j < valid; j++) sum += (double)values[(size_t)j * d + i] * p[j];
      out[i] = (float)sum;
    }
    free(p);
  } else {
    float* p = s->logits;
    float maximum = -INFINITY;
    for (int j = 0; j < valid; j++) {
      float dot = 0;
      for (int i = 0; i < d; i++) dot += keys[(size_t)j * d + i] * q[i];
      p[j] = dot / sqrtf((float)d);
      if (p[j] > maximum) maximum = p[j];
    }
    float total = 0;
    for (int j = 0; j < valid; j++) { p[j] = expf(p[j] - maximum); total += p[j]; }
    for (int j = 0; j < valid; j++) p[j] /= total;
    for (int i = 0; i < d; i++) {
      float sum = 0;
      for (int j = 0; j < valid; j++) sum += values[(size_t)j * d + i] * p[j];
      out[i] = sum;
    }
  }
}

float so_step(so_state* s, const float* input) {
  const so_config* c = &s->c;
  int d = s->dim, width = c->width;
  int slot = (int)(s->position % (uint64_t)c->window);
  int valid = s->position + 1 < (uint64_t)c->window ? (int)(s->position + 1) : c->window;
  oracle_linear(s, "", "input", s->w[T_INPUT], input, s->x, width, c->features, 0);
  emit(s, "", "input", "", s->x, width);
  for (int l = 0; l < c->layers; l++) {
    char p[32];
    snprintf(p, sizeof p, "layers.%d.", l);
    oracle_norm(s, p, "norm1", s->x, layer_w(s, l, L_NORM1), s->norm);
    oracle_linear(s, p, "q", layer_w(s, l, L_Q), s->norm, s->q, width, width, 0);
    oracle_linear(s, p, "k", layer_w(s, l, L_K), s->norm, s->k, width, width, 0);
    oracle_linear(s, p, "v", layer_w(s, l, L_V), s->norm, s->v, width, width, 0);
    /* RoPE on adjacent pairs inside each head, Cpu.cpp:73-83 */
    for (int h = 0; h < c->heads; h++) {
      for (int i = 0; i < d; i += 2) {
        float angle = (float)s->position * powf(10000.0f, -(float)i / (float)d);
        float co = cosf(angle), si = sinf(angle);
        float* vectors[2] = {s->q, s->k};
        for (int m = 0; m < 2; m++) {
          float a = vectors[m][h * d + i], b = vectors[m][h * d + i + 1];
          vectors[m][h * d + i] = a * co - b * si;
          vectors[m][h * d + i + 1] = a * si + b * co;
        }
      }
    }
    cast(s, s->q, width);
    cast(s, s->k, width);
    emit(s, p, "q", "", s->q, width);
    emit(s, p, "k", "", s->k, width);
    emit(s, p, "v", "", s->v, width);
    for (int h = 0; h < c->heads; h++) {
      size_t base = ((size_t)l * c->heads + h) * (size_t)c->window * d;
      for (int i = 0; i < d; i++) {
        s->keys[base + (size_t)slot * d + i] = s->k[h * d + i];
        s->values[base + (size_t)slot * d + i] = s->v[h * d + i];
      }
      oracle_attention(s, l, h, valid);
    }
    cast(s, s->attention, width);
    emit(s, p, "attention", "", s->attention, width);
    oracle_linear(s, p, "out", layer_w(s, l, L_OUT), s->attention, s->temp, width, width, 0);
    for (int i = 0; i < width; i++) s->x[i] += s->temp[i];
    cast(s, s->x, width);
    emit(s, p, "attention_residual", "", s->x, width);
    oracle_norm(s, p, "norm2", s->x, layer_w(s, l, L_NORM2), s->norm);
    oracle_linear(s, p, "gate", layer_w(s, l, L_GATE), s->norm, s->gate, c->ffn, width, 0);
    oracle_linear(s, p, "up", layer_w(s, l, L_UP), s->norm, s->up, c->ffn, width, 0);
    for (int i = 0; i < c->ffn; i++) {
      if (s->dbl) {
        double g = s->gate[i];
        s->gate[i] = (float)((g / (1.0 + exp(-g))) * s->up[i]);
      } else {
        s->gate[i] = (s->gate[i] / (1.0f + expf(-s->gate[i]))) * s->up[i];
      }
    }
    cast(s, s->gate, c->ffn);
    emit(s, p, "activation", "", s->gate, c->ffn);
    oracle_linear(s, p, "down", layer_w(s, l, L_DOWN), s->gate, s->temp, width, c->ffn, 0);
    for (int i = 0; i < width; i++) s->x[i] += s->temp[i];
    cast(s, s->x, width);
    emit(s, p, "hidden", "", s->x, width);
    memcpy(s->hidden + (size_t)l * width, s->x, (size_t)width * sizeof(float));
  }
  oracle_norm(s, "", "final_norm", s->x, s->w[T_FINAL_NORM], s->norm);
  float score;
  oracle_linear(s, "", "score", s->w[T_SCORE], s->norm, &score, 1, width, 1);
  s->position++;
  return score;
}

float so_step_trace(so_state* s, const float* input, so_trace_fn fn, void* user) {
  s->trace = fn;
  s->trace_user = user;
  const float score = so_step(s, input);
  s->trace = NULL;
  s->trace_user = NULL;
  return score;
}

void so_reset(so_state* s) {
  size_t cache = (size_t)s->c.layers * s->c.width * s->c.window;
  s->position = 0;
  memset(s->keys, 0, cache * sizeof(float));
  memset(s->values, 0, cache * sizeof(float));
  memset(s->hidden, 0, (size_t)s->c.layers * s->c.width * sizeof(float));
}

uint64_t so_position(const so_state* s) { return s->position; }

void so_snapshot(const so_state* s, float* keys, float* values, float* hidden) {
  size_t cache = (size_t)s->c.layers * s->c.width * s->c.window;
  if (keys) memcpy(keys, s->keys, cache * sizeof(float));
  if (values) memcpy(values, s->values, cache * sizeof(float));
  if (hidden) memcpy(hidden, s->hidden, (size_t)s->c.layers * s->c.width * sizeof(float));
}
