/*
 * CPU oracle for the streaming local-causal transformer step.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the reference for comparison: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product path (libstamd.so) never links or calls it.
 *
 * It restates the reference CPU backend `Stream::Cpu` (src/cpu/Cpu.cpp:59-141)
 * with plain loops instead of Eigen (Eigen is not installed here), keeping the
 * reference's operation order and FP16 cast points (reference/model.py:1-5).
 * Two accumulation types are offered: float (the reference's own arithmetic)
 * and double (an FP64-accumulating referee, the method of
 * docs/NumericalDiagnosis.md:23).
 *
 * Pinning: see the header of stream_oracle.c.
 */
#ifndef STREAM_ORACLE_H
#define STREAM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same seven fields as ModelConfig (include/Model.hpp:12-18). */
typedef struct {
  int32_t layers, width, heads, ffn, window, features;
  float epsilon;
} so_config;

typedef struct so_state so_state;

/* Canonical tensor order for `tensors` (row-major [out, in] matrices):
 *   0 input [width, features]   1 final_norm [width]   2 score [1, width]
 *   then per layer l, base 3 + 9*l:
 *   norm1 [width], norm2 [width], q, k, v, out [width, width],
 *   gate, up [ffn, width], down [width, ffn]
 * Values are FP32. In mixed mode they must already be FP16-representable
 * (the reference decodes its FP16 file to FP32: src/runtime/Model.cpp:103-109).
 * The oracle copies the tensors. Returns NULL on invalid configuration. */
so_state* so_create(const so_config* config, int mixed, int accumulate_double,
                    const float* const* tensors);
void so_destroy(so_state* state);
/* One event of `features` floats; returns the score (Cpu::step). */
float so_step(so_state* state, const float* input);
/* Per-operation trace (the reference's CpuTrace, src/cpu/Cpu.cpp:29-57,64-66,86-133): one
 * step that also reports every operation and cast boundary to `fn`, in execution order, under
 * the reference's names: for each projection N ("input", "layers.{l}.q|k|v|out|gate|up|down",
 * "score") N.operand, N.pre_cast and N.linear; for each norm N ("layers.{l}.norm1|norm2",
 * "final_norm") N.operand, N.pre_cast and N.norm; and "input", "layers.{l}.q|k|v" (after RoPE
 * and the cast), "layers.{l}.attention", ".attention_residual", ".activation", ".hidden".
 * The values pointer is valid only during the call. The step's results are those of so_step. */
typedef void (*so_trace_fn)(void* user, const char* name, const float* values, int count);
float so_step_trace(so_state* state, const float* input, so_trace_fn fn, void* user);
/* Zero K/V/hidden and the position (Cpu::reset, src/cpu/Cpu.cpp:143-148). */
void so_reset(so_state* state);
uint64_t so_position(const so_state* state);
/* keys/values: layers*heads*window*dim floats ([L][H][W][dh]); hidden: layers*width. */
void so_snapshot(const so_state* state, float* keys, float* values, float* hidden);
/* Row-parallel matvecs over `threads` OpenMP threads (1 = the reference default). */
void so_set_threads(so_state* state, int threads);
/* Rounding helpers: float -> IEEE half (round to nearest even, overflow to inf)
 * -> float, and float -> bfloat16 (round to nearest even) -> float. */
float so_round_half(float value);
uint16_t so_half_bits(float value);
float so_half_to_float(uint16_t bits);
float so_round_bf16(float value);
uint16_t so_bf16_bits(float value);

#ifdef __cplusplus
}
#endif
#endif
