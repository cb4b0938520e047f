/* qwen_gpu: C ABI of the MI355X (gfx950) Qwen3-0.6B FP16 engine.
 *
 * Drop-in boundary for the reference's native engine API, qwen_cpu::Model
 * (engine/core.hpp:8-56), exported as plain C: opaque handle, plain pointers
 * and sizes, integer status codes, no exceptions and no C++/torch types.
 * Every function returns QWEN_GPU_OK (0) on success; on failure it returns
 * QWEN_GPU_ERROR and qwen_gpu_last_error() (per calling thread) holds the
 * message, using the reference's wording (engine/core.cpp:235-276, 707-752).
 * One caller at a time per model (engine/core.hpp:23).
 *
 * Decode kernels hand values between the workgroups of one launch, so a
 * launch needs the whole GPU (all 256 CUs) to itself. Calls that run them on
 * models stepped from different threads of one process take a process-wide
 * lock and run one after another; another process decoding on the same GPU
 * at the same time can make a step fail with "Decode step stalled" (a
 * bounded wait that gave up, never a hang).
 *
 * A prefill, step or batched step that fails after validation (a stalled
 * exchange, a HIP error) returns each model to its position before the call,
 * without current logits; K/V rows from that position on are rewritten by
 * the next call. A failed verification resets the model
 * (engine/core.cpp:740).
 */
#ifndef QWEN_GPU_H
#define QWEN_GPU_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWEN_GPU_OK 0
#define QWEN_GPU_ERROR 1
#define QWEN_GPU_VOCABULARY 151936          /* qwen_cpu::vocabulary, engine/core.hpp:9 */
#define QWEN_GPU_HIDDEN 1024
#define QWEN_GPU_PREFIX_REUSE_CHUNK 512     /* qwen_cpu::prefix_reuse_chunk, engine/core.hpp:10 */

typedef struct qwen_gpu_model qwen_gpu_model;

/* qwen_cpu::Options (engine/core.hpp:11-15). Thread counts are validated
 * (1..64) and echoed; context is 1..4096. */
typedef struct qwen_gpu_options {
    int decode_threads;
    int prefill_threads;
    int context;
} qwen_gpu_options;

/* Message of the last failed call on this thread ("" if none). */
const char* qwen_gpu_last_error(void);

/* qwen_cpu::Model::Model(weights_file, Options), engine/core.hpp:28 and
 * engine/core.cpp:235-290: maps and validates the QWCPU01 pack, then uploads
 * it to GPU 0. options == NULL means {12, 6, 4096}. */
int qwen_gpu_create(const char* weights, const qwen_gpu_options* options, qwen_gpu_model** out);
/* qwen_cpu::Model::~Model, engine/core.hpp:29. NULL is ignored. */
void qwen_gpu_destroy(qwen_gpu_model* model);

/* A further model on the device weights already uploaded for `owner` (no
 * second upload): its own K/V cache, position and buffers. options == NULL
 * copies owner's. The weights stay until the last model using them is
 * destroyed. No reference counterpart (the reference is single-stream): it
 * backs the batched decode below for callers serving several sequences. */
int qwen_gpu_create_sharing(const qwen_gpu_model* owner, const qwen_gpu_options* options, qwen_gpu_model** out);
/* dst becomes src truncated to `positions`: K/V rows 0..positions-1 copied on
 * the device as src computed them, no current logits. The canonical
 * prefix-reuse rewind (engine/INTERFACE.md:94-103; Model::truncate,
 * engine/core.cpp:722-727) applied to a copy; both models share weights.
 * Fails with "Rewind position out of range" unless 0 <= positions <= src's
 * position. */
int qwen_gpu_copy_prefix(qwen_gpu_model* dst, const qwen_gpu_model* src, int positions);
/* One decode step for each of `count` (1..8) distinct models that share
 * weights: models[i] consumes tokens[i] (Model::step, engine/core.hpp:38),
 * with every projection reading each weight matrix once for all rows (FP16
 * matrix cores, FP32 activations split into FP16 hi + lo, FP32 sums) and an
 * online-softmax attention over position pieces (held to the reference's
 * tolerance gate, not bit-equal to a batch-1 step). Rows that models hold as
 * copies of the same prefix (qwen_gpu_copy_prefix) are read from one of
 * them. Every model is validated (pending verification, capacity, token
 * range) before any runs. Afterwards each model has current logits and
 * qwen_gpu_greedy works as after a step. No reference counterpart. */
int qwen_gpu_step_batch(qwen_gpu_model* const* models, const int* tokens, int count);
/* qwen_gpu_step_batch, then next[i] = qwen_gpu_greedy(models[i]) in the same
 * call (one host round trip per step for a greedy decode loop). Fails as
 * either would; on failure next is unspecified. No reference counterpart. */
int qwen_gpu_step_batch_greedy(qwen_gpu_model* const* models, const int* tokens, int count, int* next);

/* Model::reset, engine/core.hpp:32; engine/core.cpp:718-721. */
int qwen_gpu_reset(qwen_gpu_model* model);
/* Model::truncate(position), engine/core.hpp:35; engine/core.cpp:722-727. */
int qwen_gpu_truncate(qwen_gpu_model* model, int position);
/* Model::prefill(ids), engine/core.hpp:37; engine/core.cpp:727,707-714. */
int qwen_gpu_prefill(qwen_gpu_model* model, const int* ids, size_t count);
/* Model::step(token), engine/core.hpp:38; engine/core.cpp:728. */
int qwen_gpu_step(qwen_gpu_model* model, int token);
/* Model::verify_two(first, second) -> VerificationRows, engine/core.hpp:17-22,43;
 * engine/core.cpp:729-741. Borrowed row-major [2 x 151936] logits and
 * [2 x 1024] hidden, valid until commit/reset/truncate or another mutation. */
int qwen_gpu_verify_two(qwen_gpu_model* model, int first, int second, const float** logits,
                        const float** hidden, int* base_position);
/* Model::commit_verified(count), engine/core.hpp:46; engine/core.cpp:742-752. */
int qwen_gpu_commit_verified(qwen_gpu_model* model, int count);
/* Model::logits(), engine/core.hpp:47; engine/core.cpp:753. Borrowed FP32
 * [151936] valid until the next mutation; *count is 0 when there are none. */
int qwen_gpu_logits(qwen_gpu_model* model, const float** data, size_t* count);
/* Model::hidden(), engine/core.hpp:48-50; engine/core.cpp:754-757. Fails with
 * "No current hidden state" when there are no current logits. */
int qwen_gpu_hidden(qwen_gpu_model* model, const float** data, size_t* count);
/* Model::position(), engine/core.hpp:51. Returns the position (not a status). */
int qwen_gpu_position(const qwen_gpu_model* model);
/* Model::lossless_bf16_cache_bytes(), engine/core.hpp:53; always 0 (engine/core.cpp:759). */
size_t qwen_gpu_lossless_bf16_cache_bytes(const qwen_gpu_model* model);
/* Which batch-1 decode kernels the model runs (no reference counterpart;
 * for tests and benchmarks): 2 one persistent launch per token, 1 two fused
 * launches per layer, 0 separate kernels (no exchanges inside a launch, as
 * when the device does not deal workgroups round-robin over 8 XCDs). */
int qwen_gpu_decode_kernels(const qwen_gpu_model* model);
/* Options actually in effect (echoed by the protocol handshake, engine/main.cpp:71-79). */
int qwen_gpu_get_options(const qwen_gpu_model* model, qwen_gpu_options* options);

/* Greedy Sampler::select of the current logits (engine/main.cpp:51-59):
 * lowest id among maxima, computed on the GPU without copying the logits.
 * Fails with "Nonfinite model logits" or "No current full-vocabulary logits". */
int qwen_gpu_greedy(qwen_gpu_model* model, int* token);
/* Greedy selections of both pending verification rows (engine/main.cpp:138,142). */
int qwen_gpu_verify_greedy(qwen_gpu_model* model, int* first, int* second);
/* verify_two followed by verify_greedy, without copying the rows to host
 * memory: what the protocol's verify-greedy command needs (engine/main.cpp:
 * 128-147 calls verify_two and selects from the returned rows). The rows stay
 * pending for qwen_gpu_commit_verified. No counterpart in the reference class. */
int qwen_gpu_verify_two_greedy(qwen_gpu_model* model, int first, int second, int* first_choice,
                               int* second_choice);

/* Chat-mode candidates of the current logits on the GPU (engine/main.cpp:
 * 51-62: score = (logit - (seen ? 1.5 : 0)) / 0.7, partial sort of the 20
 * best by value descending, id ascending): the k (1..32) best scores
 * (logit - (penalized ? penalty : 0)) / temperature in that order, with their
 * ids. Only these leave the device; the caller draws from them. Fails with
 * "No current full-vocabulary logits" or "Nonfinite model logits" like the
 * reference's select. */
int qwen_gpu_top_scores(qwen_gpu_model* model, float penalty, float temperature, int k, float* values,
                        int* ids);
/* The model's penalized-token flags, the device copy of the sampler's seen
 * set (engine/main.cpp:42,47-49): cleared when `clear` is nonzero, then
 * ids[0..count) set. All flags start clear; reset/truncate leave them as
 * they are (the sampler owns them, as in the reference). */
int qwen_gpu_update_penalized(qwen_gpu_model* model, int clear, const int* ids, size_t count);

/* Synthetic QWCPU01 pack (format: engine/INTERFACE.md:8-21; tensor order of
 * tools/export_native_cpu_weights.py:29-39): matrices N(0, stddev) rounded to
 * FP16 from a counter-based splitmix64 Box-Muller stream, norm gains 1.0.
 * Writes PATH, PATH.index and PATH.manifest.json; refuses existing outputs. */
int qwen_gpu_write_random_pack(const char* path, uint64_t seed, double stddev, int threads);
/* The pack checks of Model::Model without a device: maps PATH and runs the
 * header, index, shape, range, overlap and finiteness checks of
 * engine/core.cpp:235-276 with the same messages (what qwen_gpu_create runs
 * before touching the GPU). For exporters and tools on hosts without one. */
int qwen_gpu_validate_pack(const char* path);

/* Device memory plumbing for callers that hold no other GPU runtime (the
 * op-level entry points below take device pointers). No reference counterpart:
 * they exist so tests and C callers need not load a second HIP runtime. */
int qwen_gpu_device_malloc(size_t bytes, void** pointer);
int qwen_gpu_device_free(void* pointer);
int qwen_gpu_memcpy_to_device(void* device, const void* host, size_t bytes);
int qwen_gpu_memcpy_to_host(void* host, const void* device, size_t bytes);
int qwen_gpu_device_synchronize(void);

/* Kernel-level entry points on caller-owned device memory (stream may be
 * NULL for the default stream); used by parity tests and the GEMV microbench.
 * Converts natural row-major FP16 [rows x cols] to the engine's chain-tiled
 * GEMV layout; second != NULL interleaves two equal-shape matrices by 4 rows. */
int qwen_gpu_op_tile_matrix(const uint16_t* first, const uint16_t* second, uint16_t* dst, int rows, int cols,
                            void* stream);
/* y[r] = dot(x, W[r]) with the reference dot's chain order (engine/core.cpp:119-147),
 * W chain-tiled; cols in {1024, 2048, 3072}; rows a multiple of 16. */
int qwen_gpu_op_gemv(const uint16_t* tiled, const float* x, float* y, int rows, int cols, void* stream);
/* Batched projection of the prefill path (engine/core.cpp:292-294, the
 * cblas_sgemm branch): C[M x N] = A[M x K] . W[N x K]^T, or C += when
 * accumulate != 0. A is FP32 (split exactly into FP16 hi + lo on the matrix
 * cores), W natural row-major FP16; N and K multiples of 64, M >= 1. */
int qwen_gpu_op_gemm(const float* a, const uint16_t* w, float* c, int m, int n, int k, int accumulate,
                     void* stream);
/* qwen_gpu_op_gemm without any device allocation, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). No counterpart in the reference. The FP16 operand
 * planes live in a static device array of the library (4 MiB per device,
 * held until the process ends), so m * k may be at most 1048576; larger
 * inputs fail with an error and launch nothing. The call only enqueues work
 * on `stream` (NULL: the default stream) and returns; the caller synchronizes
 * before reading c. Every call on one device shares that array: calls that
 * may overlap on a device (other streams, other threads) race and must be
 * serialized by the caller. Results are bit-identical to qwen_gpu_op_gemm. */
int qwen_gpu_op_gemm_static(const float* a, const uint16_t* w, float* c, int m, int n, int k, int accumulate,
                            void* stream);
/* Gate/up projection of the prefill path with its SwiGLU epilogue
 * (engine/core.cpp:630-639 with batch > 1: the gate and up projections, then
 * gate * (0.5 + 0.5 tanh(gate / 2)) * up): w natural FP16 [n x k] holding
 * n / 2 gate rows then n / 2 up rows, a FP32 [m x k]; act[m][i] is written
 * as FP16 hi and lo planes [m x n / 2] and exponents act_exp [m x n / 16]
 * (one byte per group of 8 activations), with
 * act = (hi + lo) * 2^act_exp[m][i / 8] (the FP32 result to 2^-22; the
 * exponent is 0 unless the group's largest magnitude reaches 65504, the
 * FP16 limit). n a multiple of 256, k of 64. Parity-test entry for the
 * kernel the prefill runs between the post-attention norm and the down
 * GEMM. */
int qwen_gpu_op_gemm_swiglu(const float* a, const uint16_t* w, uint16_t* act_hi, uint16_t* act_lo, uint8_t* act_exp,
                            int m, int n, int k, void* stream);
/* The batch-1 decode projections as a step runs them (parity-test entries;
 * all weights in the chain-tiled layout of qwen_gpu_op_tile_matrix):
 * qkv[4096] = W_qkv . RMSNorm(x, norm_weight) with W_qkv = q, k, v rows
 * stacked [4096 x 1024] (engine/core.cpp:384-386: norm, then project_group<3>
 * over q/k/v). */
int qwen_gpu_op_norm_qkv(const uint16_t* tiled, const float* norm_weight, const float* x, float* qkv, void* stream);
/* act[3072] = SwiGLU(W_gate . h, W_up . h), h = RMSNorm(x + the 16 pending
 * per-query-head O partials parts[16][1024], added in the engine's fixed
 * tree order; parts NULL means none), the tiled matrix interleaving gate and
 * up rows 4 by 4 (qwen_gpu_op_tile_matrix with second = up)
 * (engine/core.cpp:625-639: residual, norm, project_group<2>, SwiGLU).
 * raw (NULL to skip, else [6144]) receives the gate and up dot products in
 * that interleaved row order: 8t + i is gate row 4t + i, 8t + 4 + i up row
 * 4t + i (i < 4). */
int qwen_gpu_op_norm_gate_up(const uint16_t* tiled, const float* norm_weight, const float* x, const float* parts,
                             float* act, float* raw, void* stream);
/* x[r] = (x[r] + the pending O partials of row r, NULL for none) +
 * W_down[r] . act, W_down [1024 x 3072] (engine/core.cpp:640-641: project,
 * then the residual add). */
int qwen_gpu_op_down_residual(const uint16_t* tiled, const float* act, const float* parts, float* x, void* stream);
/* The FFN of one layer as the fused decode kernel runs it
 * (engine/core.cpp:625-641, with the down projection split into 8 column
 * slices): xm = x + the 16 O partials parts[16][1024] (fixed tree order);
 * act = SwiGLU(W_gate . h, W_up . h), h = RMSNorm(xm), posted to
 * exchange[3072] as (tag << 32 | FP32 bits); dparts[g][r] = W_down[r][384 g
 * .. 384 g + 383] . act[384 g .. 384 g + 383] (the reference's 8-chain dot
 * over that slice), g < 8. The next layer adds xm + the 8 slices (see
 * qwen_gpu_op_norm_qkv_folded). exchange must hold no word carrying tag
 * (zero it once; tag != 0 and different from the previous call's); *stall
 * is set nonzero if a workgroup gave up waiting for the slice's
 * activations. Parity-test entry. */
int qwen_gpu_op_fused_ffn(const uint16_t* gateup_tiled, const uint16_t* down_tiled, const float* norm_weight,
                          const float* x, const float* parts, float* xm, float* dparts, uint64_t* exchange, int* stall,
                          uint32_t tag, void* stream);
/* qkv[4096] = W_qkv . RMSNorm(x) where x = xm + the 8 down slices
 * dparts[8][1024] added in the fixed tree order ((d0+d1)+(d2+d3)) +
 * ((d4+d5)+(d6+d7)); x[1024] is written out (engine/core.cpp:641 then
 * 384-386). Parity-test entry. */
int qwen_gpu_op_norm_qkv_folded(const uint16_t* tiled, const float* norm_weight, const float* xm,
                                const float* dparts, float* x, float* qkv, void* stream);
/* Causal GQA attention of a prefill chunk (engine/core.cpp:407-605, the
 * batched rows' attention): rows queries at positions pos0 .. pos0 + rows - 1
 * from qkv FP32 [rows x 4096] (columns 0..2047: 16 query heads of 128),
 * against FP16 keys / values [8 KV heads][context][128] holding positions
 * 0 .. pos0 + rows - 1 (query head h reads KV head h / 2; q and k channels in
 * one common order), scale 1/sqrt(128). Output [rows x 2048] as FP16 hi and
 * lo planes (hi + lo is the FP32 result to 2^-22). rows 1..4096, pos0 + rows
 * <= context. Parity-test entry for the kernel the prefill runs between its
 * QKV and O GEMMs. */
int qwen_gpu_op_attention_prefill(const float* qkv, const uint16_t* keys, const uint16_t* values, uint16_t* att_hi,
                                  uint16_t* att_lo, int rows, int pos0, int context, void* stream);
/* Batched projection of the multi-sequence decode: y[b] = W x[b] for b <
 * batch (1..8) on the matrix cores; W natural row-major FP16 [rows x cols],
 * x FP32 [batch x cols], y FP32 [batch x rows]; rows a multiple of 16, cols
 * in {1024, 2048, 3072}. No reference counterpart (parity-test entry). */
int qwen_gpu_op_bgemv(const uint16_t* w, const float* x, float* y, int batch, int rows, int cols, void* stream);
/* Isolated GEMV microbenchmark: average milliseconds of one op_gemv launch
 * over `iterations` back-to-back launches on the default stream, timed with
 * HIP events, cycling through `copies` chain-tiled weight copies laid
 * `copy_stride` bytes apart (enough copies keep the weights streaming from
 * HBM rather than the 256 MB Infinity Cache). No reference counterpart. */
int qwen_gpu_op_gemv_time(const uint16_t* tiled, size_t copy_stride, int copies, const float* x, float* y, int rows,
                          int cols, int iterations, float* milliseconds);
/* Plain 16-byte-per-thread device copy (bytes a multiple of 16). No reference
 * counterpart: a kernel of known traffic for calibrating HBM byte counters. */
int qwen_gpu_op_copy(const void* src, void* dst, size_t bytes, void* stream);
/* Average milliseconds of one standalone launch of a decode kernel on the
 * model's stream, timed with HIP events (which: 0 norm+QKV, 1 attention,
 * 2 O, 3 norm+gate/up, 4 down, 5 lm_head, 6 the fused FFN kernel and 7 the
 * fused norm + QKV + attention + O kernel of the two-kernel step, 8 the
 * token kernel that runs all 28 layers of a step in one launch). Needs
 * position() > 0. The O projection runs with the attention (timed as 1: one
 * kernel up to 512 positions, split attention + merge/O beyond) and 2
 * reports 0. Kernels 0-7 replay layer by layer over all 28 layers, 8 replays
 * whole steps. Afterwards the current logits are invalid; timing the
 * attention or the token kernel (1, 7 or 8) also resets the model, so time
 * them last. */
int qwen_gpu_time_kernel(qwen_gpu_model* model, int which, int iterations, float* milliseconds);

#ifdef __cplusplus
}
#endif
#endif
