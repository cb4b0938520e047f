/* ORACLE (test infrastructure only).
 *
 * CPU restatement of the reference Qwen3-0.6B forward pass, engine/core.cpp.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library; the product never links or calls it.
 *
 * Arithmetic followed, function by function:
 *   cpuref_dot        engine/core.cpp:119-127 (and dot4 131-147, identical per row)
 *   cpuref_gemv       engine/core.cpp:292-326 (B1 project / project_group)
 *   cpuref_norm       engine/core.cpp:207-215 (FP32 squares, FP64 sum)
 *   cpuref_rope       engine/core.cpp:216-218, tables 287-288
 *   cpuref_attention  engine/core.cpp:606-624 (decode; prefill 407-605 is the
 *                     same arithmetic per output row)
 *   cpuref_swiglu     engine/core.cpp:636-639
 *   cpuref_argmax     engine/main.cpp:51-59 (greedy Sampler::select)
 *   model functions   engine/core.cpp:353-414, 625-646, 707-758
 * Deviations (documented where they occur): batched prefill projections use
 * the B1 dot order per row instead of Accelerate's cblas_sgemm (closed
 * source, order unknown); vvexpf/vvtanhf become glibc expf/tanhf; expressions
 * are evaluated as written with FP contraction off.
 */
#ifndef QWEN_ORACLE_CPU_REF_H
#define QWEN_ORACLE_CPU_REF_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cpuref_model cpuref_model;

/* Model API (mirrors qwen_cpu::Model, engine/core.hpp:25-56). All functions
 * return 0 on success, nonzero on error; cpuref_error() gives the message. */
cpuref_model* cpuref_create(const char* weights, int decode_threads, int prefill_threads, int context,
                            char* error, size_t error_len);
void cpuref_destroy(cpuref_model* m);
const char* cpuref_error(const cpuref_model* m);
int cpuref_reset(cpuref_model* m);
int cpuref_truncate(cpuref_model* m, int position);
int cpuref_prefill(cpuref_model* m, const int* ids, size_t count);
int cpuref_step(cpuref_model* m, int token);
int cpuref_position(const cpuref_model* m);
/* Borrowed [151936] logits and [1024] hidden; NULL when no current logits. */
const float* cpuref_logits(const cpuref_model* m);
const float* cpuref_hidden(const cpuref_model* m);

/* Single operations on caller buffers (FP16 passed as raw uint16 bits). */
float cpuref_dot(const float* x, const uint16_t* w, int n);
void cpuref_gemv(const float* x, const uint16_t* w, float* y, int rows, int n, int threads);
void cpuref_norm(const float* x, const float* w, float* out, int n);
void cpuref_rope_tables(int context, float* cosines, float* sines);
void cpuref_rope(float* x, const float* cs, const float* sn);
/* One query head over n canonical [n][128] FP16 key/value rows. */
void cpuref_attention(const float* q, const uint16_t* keys, const uint16_t* values, int n, float* out);
void cpuref_swiglu(const float* gate, const float* up, float* out, int n);
/* Greedy select: lowest id among maxima; returns -1 on any nonfinite logit. */
int cpuref_argmax(const float* logits, int n);
uint16_t cpuref_f32_to_f16(float x);
float cpuref_f16_to_f32(uint16_t h);

#ifdef __cplusplus
}
#endif
#endif
