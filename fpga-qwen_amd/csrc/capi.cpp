// extern "C" boundary: exceptions become status codes + a thread-local message.
#include "qwen_gpu.h"

#include <string>

#include "batch.hpp"
#include "engine.hpp"
#include "pack.hpp"
#include "prefill.hpp"

struct qwen_gpu_model {
    qwen_hip::Engine engine;
    qwen_gpu_model(const std::string& path, const qwen_hip::Options& o) : engine(path, o) {}
    qwen_gpu_model(std::shared_ptr<qwen_hip::Weights> w, const qwen_hip::Options& o) : engine(std::move(w), o) {}
};

namespace {
thread_local std::string last_error;

template <class Fn>
int guarded(Fn&& fn) {
    try {
        fn();
        last_error.clear();
        return QWEN_GPU_OK;
    } catch (const std::exception& e) {
        last_error = e.what();
    } catch (...) {
        last_error = "Unknown error";
    }
    return QWEN_GPU_ERROR;
}

void need(const void* p, const char* what) {
    if (!p) throw std::runtime_error(std::string("Null argument: ") + what);
}
}  // namespace

extern "C" {

const char* qwen_gpu_last_error(void) { return last_error.c_str(); }

int qwen_gpu_create(const char* weights, const qwen_gpu_options* options, qwen_gpu_model** out) {
    return guarded([&] {
        need(weights, "weights");
        need(out, "out");
        *out = nullptr;
        qwen_hip::Options o;
        if (options) {
            o.decode_threads = options->decode_threads;
            o.prefill_threads = options->prefill_threads;
            o.context = options->context;
        }
        *out = new qwen_gpu_model(weights, o);
    });
}

void qwen_gpu_destroy(qwen_gpu_model* model) { delete model; }

int qwen_gpu_create_sharing(const qwen_gpu_model* owner, const qwen_gpu_options* options, qwen_gpu_model** out) {
    return guarded([&] {
        need(owner, "owner");
        need(out, "out");
        *out = nullptr;
        qwen_hip::Options o = owner->engine.options();
        if (options) {
            o.decode_threads = options->decode_threads;
            o.prefill_threads = options->prefill_threads;
            o.context = options->context;
        }
        *out = new qwen_gpu_model(owner->engine.weights(), o);
    });
}

int qwen_gpu_copy_prefix(qwen_gpu_model* dst, const qwen_gpu_model* src, int positions) {
    return guarded([&] {
        need(dst, "dst");
        need(src, "src");
        dst->engine.copy_prefix(src->engine, positions);
    });
}

int qwen_gpu_step_batch(qwen_gpu_model* const* models, const int* tokens, int count) {
    return guarded([&] {
        need(models, "models");
        need(tokens, "tokens");
        if (count < 1 || count > 8) throw std::runtime_error("Batch must hold 1..8 sequences");
        qwen_hip::Engine* engines[8];
        for (int i = 0; i < count; ++i) {
            need(models[i], "model");
            engines[i] = &models[i]->engine;
        }
        qwen_hip::Engine::step_batch(engines, tokens, count);
    });
}

int qwen_gpu_step_batch_greedy(qwen_gpu_model* const* models, const int* tokens, int count, int* next) {
    return guarded([&] {
        need(models, "models");
        need(tokens, "tokens");
        need(next, "next");
        if (count < 1 || count > 8) throw std::runtime_error("Batch must hold 1..8 sequences");
        qwen_hip::Engine* engines[8];
        for (int i = 0; i < count; ++i) {
            need(models[i], "model");
            engines[i] = &models[i]->engine;
        }
        qwen_hip::Engine::step_batch(engines, tokens, count);
        for (int i = 0; i < count; ++i) next[i] = engines[i]->greedy();
    });
}

int qwen_gpu_reset(qwen_gpu_model* m) {
    return guarded([&] {
        need(m, "model");
        m->engine.reset();
    });
}

int qwen_gpu_truncate(qwen_gpu_model* m, int position) {
    return guarded([&] {
        need(m, "model");
        m->engine.truncate(position);
    });
}

int qwen_gpu_prefill(qwen_gpu_model* m, const int* ids, size_t count) {
    return guarded([&] {
        need(m, "model");
        if (count) need(ids, "ids");
        m->engine.prefill(ids, count);
    });
}

int qwen_gpu_step(qwen_gpu_model* m, int token) {
    return guarded([&] {
        need(m, "model");
        m->engine.step(token);
    });
}

int qwen_gpu_verify_two(qwen_gpu_model* m, int first, int second, const float** logits, const float** hidden,
                        int* base_position) {
    return guarded([&] {
        need(m, "model");
        need(logits, "logits");
        need(hidden, "hidden");
        need(base_position, "base_position");
        m->engine.verify_two(first, second);
        m->engine.verification_rows(logits, hidden, base_position);
    });
}

int qwen_gpu_verify_two_greedy(qwen_gpu_model* m, int first, int second, int* first_choice, int* second_choice) {
    return guarded([&] {
        need(m, "model");
        need(first_choice, "first_choice");
        need(second_choice, "second_choice");
        m->engine.verify_two(first, second);
        m->engine.verify_greedy(first_choice, second_choice);
    });
}

int qwen_gpu_commit_verified(qwen_gpu_model* m, int count) {
    return guarded([&] {
        need(m, "model");
        m->engine.commit_verified(count);
    });
}

int qwen_gpu_logits(qwen_gpu_model* m, const float** data, size_t* count) {
    return guarded([&] {
        need(m, "model");
        need(data, "data");
        need(count, "count");
        *data = m->engine.logits();
        *count = *data ? size_t(qwen_hip::kVocab) : 0;
    });
}

int qwen_gpu_hidden(qwen_gpu_model* m, const float** data, size_t* count) {
    return guarded([&] {
        need(m, "model");
        need(data, "data");
        need(count, "count");
        const float* h = m->engine.hidden();
        qwen_hip::require(h != nullptr, "No current hidden state");
        *data = h;
        *count = size_t(qwen_hip::kHidden);
    });
}

int qwen_gpu_decode_kernels(const qwen_gpu_model* model) {
    return model ? model->engine.decode_kernels() : -1;
}

int qwen_gpu_position(const qwen_gpu_model* m) { return m ? m->engine.position() : 0; }

size_t qwen_gpu_lossless_bf16_cache_bytes(const qwen_gpu_model*) { return 0; }

int qwen_gpu_get_options(const qwen_gpu_model* m, qwen_gpu_options* options) {
    return guarded([&] {
        need(m, "model");
        need(options, "options");
        const auto& o = m->engine.options();
        options->decode_threads = o.decode_threads;
        options->prefill_threads = o.prefill_threads;
        options->context = o.context;
    });
}

int qwen_gpu_greedy(qwen_gpu_model* m, int* token) {
    return guarded([&] {
        need(m, "model");
        need(token, "token");
        *token = m->engine.greedy();
    });
}

int qwen_gpu_verify_greedy(qwen_gpu_model* m, int* first, int* second) {
    return guarded([&] {
        need(m, "model");
        need(first, "first");
        need(second, "second");
        m->engine.verify_greedy(first, second);
    });
}

int qwen_gpu_top_scores(qwen_gpu_model* m, float penalty, float temperature, int k, float* values, int* ids) {
    return guarded([&] {
        need(m, "model");
        need(values, "values");
        need(ids, "ids");
        m->engine.top_scores(penalty, temperature, k, values, ids);
    });
}

int qwen_gpu_update_penalized(qwen_gpu_model* m, int clear, const int* ids, size_t count) {
    return guarded([&] {
        need(m, "model");
        if (count) need(ids, "ids");
        m->engine.update_penalized(clear != 0, ids, count);
    });
}

int qwen_gpu_write_random_pack(const char* path, uint64_t seed, double stddev, int threads) {
    return guarded([&] {
        need(path, "path");
        qwen_hip::write_random_pack(path, seed, stddev, threads);
    });
}

int qwen_gpu_validate_pack(const char* path) {
    return guarded([&] {
        need(path, "path");
        qwen_hip::Pack pack(path);
        pack.validate();
    });
}

static void hip_ok(hipError_t e) {
    if (e != hipSuccess) throw std::runtime_error(std::string("HIP error: ") + hipGetErrorString(e));
}

int qwen_gpu_device_malloc(size_t bytes, void** pointer) {
    return guarded([&] {
        need(pointer, "pointer");
        *pointer = nullptr;
        hip_ok(hipMalloc(pointer, bytes));
    });
}

int qwen_gpu_device_free(void* pointer) { return guarded([&] { hip_ok(hipFree(pointer)); }); }

int qwen_gpu_memcpy_to_device(void* device, const void* host, size_t bytes) {
    return guarded([&] { hip_ok(hipMemcpy(device, host, bytes, hipMemcpyHostToDevice)); });
}

int qwen_gpu_memcpy_to_host(void* host, const void* device, size_t bytes) {
    return guarded([&] { hip_ok(hipMemcpy(host, device, bytes, hipMemcpyDeviceToHost)); });
}

int qwen_gpu_device_synchronize(void) { return guarded([&] { hip_ok(hipDeviceSynchronize()); }); }

int qwen_gpu_op_tile_matrix(const uint16_t* first, const uint16_t* second, uint16_t* dst, int rows, int cols,
                            void* stream) {
    return guarded([&] {
        need(first, "first");
        need(dst, "dst");
        qwen_hip::launch_tile_matrix(first, second, dst, rows, cols, static_cast<hipStream_t>(stream));
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) throw std::runtime_error(std::string("HIP error: ") + hipGetErrorString(e));
    });
}

int qwen_gpu_op_gemv(const uint16_t* tiled, const float* x, float* y, int rows, int cols, void* stream) {
    return guarded([&] {
        need(tiled, "tiled");
        need(x, "x");
        need(y, "y");
        qwen_hip::launch_gemv_plain(tiled, x, y, rows, cols, static_cast<hipStream_t>(stream));
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) throw std::runtime_error(std::string("HIP error: ") + hipGetErrorString(e));
    });
}

int qwen_gpu_op_gemm(const float* a, const uint16_t* w, float* c, int m, int n, int k, int accumulate,
                     void* stream) {
    return guarded([&] {
        need(a, "a");
        need(w, "w");
        need(c, "c");
        qwen_hip::launch_gemm(a, w, c, m, n, k, accumulate != 0, static_cast<hipStream_t>(stream));
        hip_ok(hipGetLastError());
    });
}

int qwen_gpu_op_gemm_static(const float* a, const uint16_t* w, float* c, int m, int n, int k, int accumulate,
                            void* stream) {
    return guarded([&] {
        need(a, "a");
        need(w, "w");
        need(c, "c");
        qwen_hip::launch_gemm_static(a, w, c, m, n, k, accumulate != 0, static_cast<hipStream_t>(stream));
        hip_ok(hipGetLastError());
    });
}

int qwen_gpu_op_gemm_swiglu(const float* a, const uint16_t* w, uint16_t* act_hi, uint16_t* act_lo, uint8_t* act_exp,
                            int m, int n, int k, void* stream) {
    return guarded([&] {
        need(a, "a");
        need(w, "w");
        need(act_hi, "act_hi");
        need(act_lo, "act_lo");
        need(act_exp, "act_exp");
        qwen_hip::launch_gemm_swiglu(a, w, act_hi, act_lo, act_exp, m, n, k, static_cast<hipStream_t>(stream));
        hip_ok(hipGetLastError());
    });
}

int qwen_gpu_op_norm_qkv(const uint16_t* tiled, const float* norm_weight, const float* x, float* qkv, void* stream) {
    return guarded([&] {
        need(tiled, "tiled");
        need(norm_weight, "norm_weight");
        need(x, "x");
        need(qkv, "qkv");
        qwen_hip::launch_norm_qkv(tiled, norm_weight, x, qkv, static_cast<hipStream_t>(stream));
        hip_ok(hipGetLastError());
    });
}

int qwen_gpu_op_norm_gate_up(const uint16_t* tiled, const float* norm_weight, const float* x, const float* parts,
                             float* act, float* raw, void* stream) {
    return guarded([&] {
        need(tiled, "tiled");
        need(norm_weight, "norm_weight");
        need(x, "x");
        need(act, "act");
        qwen_hip::launch_norm_gate_up(tiled, norm_weight, x, parts, act, raw, static_cast<hipStream_t>(stream));
        hip_ok(hipGetLastError());
    });
}

int qwen_gpu_op_down_residual(const uint16_t* tiled, const float* act, const float* parts, float* x, void* stream) {
    return guarded([&] {
        need(tiled, "tiled");
        need(act, "act");
        need(x, "x");
        qwen_hip::launch_down_residual(tiled, act, parts, x, static_cast<hipStream_t>(stream));
        hip_ok(hipGetLastError());
    });
}

int qwen_gpu_op_fused_ffn(const uint16_t* gateup_tiled, const uint16_t* down_tiled, const float* norm_weight,
                          const float* x, const float* parts, float* xm, float* dparts, uint64_t* exchange, int* stall,
                          uint32_t tag, void* stream) {
    return guarded([&] {
        need(gateup_tiled, "gateup_tiled");
        need(down_tiled, "down_tiled");
        need(norm_weight, "norm_weight");
        need(x, "x");
        need(parts, "parts");
        need(xm, "xm");
        need(dparts, "dparts");
        need(exchange, "exchange");
        need(stall, "stall");
        qwen_hip::launch_fused_ffn(gateup_tiled, down_tiled, norm_weight, x, parts, xm, dparts, exchange, stall, tag,
                                   static_cast<hipStream_t>(stream));
        hip_ok(hipGetLastError());
    });
}

int qwen_gpu_op_norm_qkv_folded(const uint16_t* tiled, const float* norm_weight, const float* xm,
                                const float* dparts, float* x, float* qkv, void* stream) {
    return guarded([&] {
        need(tiled, "tiled");
        need(norm_weight, "norm_weight");
        need(xm, "xm");
        need(dparts, "dparts");
        need(x, "x");
        need(qkv, "qkv");
        qwen_hip::launch_norm_qkv_folded(tiled, norm_weight, xm, dparts, x, qkv, static_cast<hipStream_t>(stream));
        hip_ok(hipGetLastError());
    });
}

int qwen_gpu_op_attention_prefill(const float* qkv, const uint16_t* keys, const uint16_t* values, uint16_t* att_hi,
                                  uint16_t* att_lo, int rows, int pos0, int context, void* stream) {
    return guarded([&] {
        need(qkv, "qkv");
        need(keys, "keys");
        need(values, "values");
        need(att_hi, "att_hi");
        need(att_lo, "att_lo");
        qwen_hip::launch_attention_prefill(qkv, keys, values, att_hi, att_lo, rows, pos0, context,
                                           static_cast<hipStream_t>(stream));
        hip_ok(hipGetLastError());
    });
}

int qwen_gpu_op_bgemv(const uint16_t* w, const float* x, float* y, int batch, int rows, int cols, void* stream) {
    return guarded([&] {
        need(w, "w");
        need(x, "x");
        need(y, "y");
        qwen_hip::launch_bgemv_plain(w, x, y, batch, rows, cols, static_cast<hipStream_t>(stream));
        hip_ok(hipGetLastError());
    });
}

int qwen_gpu_op_gemv_time(const uint16_t* tiled, size_t copy_stride, int copies, const float* x, float* y, int rows,
                          int cols, int iterations, float* milliseconds) {
    return guarded([&] {
        need(tiled, "tiled");
        need(x, "x");
        need(y, "y");
        need(milliseconds, "milliseconds");
        if (copies < 1 || iterations < 1) throw std::runtime_error("gemv_time: copies and iterations must be positive");
        if (copy_stride < size_t(rows) * size_t(cols) * 2 && copies > 1)
            throw std::runtime_error("gemv_time: copy_stride smaller than one matrix");
        auto launch = [&](int i) {
            const auto* w = reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(tiled) +
                                                              size_t(i % copies) * copy_stride);
            qwen_hip::launch_gemv_plain(w, x, y, rows, cols, nullptr);
        };
        for (int i = 0; i < copies; ++i) launch(i);  // warm: code, TLB
        hipEvent_t start, stop;
        hip_ok(hipEventCreate(&start));
        hip_ok(hipEventCreate(&stop));
        hip_ok(hipEventRecord(start, nullptr));
        for (int i = 0; i < iterations; ++i) launch(i);
        hip_ok(hipEventRecord(stop, nullptr));
        hip_ok(hipEventSynchronize(stop));
        float ms = 0.f;
        hip_ok(hipEventElapsedTime(&ms, start, stop));
        (void)hipEventDestroy(start);
        (void)hipEventDestroy(stop);
        hip_ok(hipGetLastError());
        *milliseconds = ms / float(iterations);
    });
}

int qwen_gpu_op_copy(const void* src, void* dst, size_t bytes, void* stream) {
    return guarded([&] {
        need(src, "src");
        need(dst, "dst");
        qwen_hip::launch_copy(src, dst, bytes, static_cast<hipStream_t>(stream));
        hip_ok(hipGetLastError());
    });
}

int qwen_gpu_time_kernel(qwen_gpu_model* m, int which, int iterations, float* milliseconds) {
    return guarded([&] {
        need(m, "model");
        need(milliseconds, "milliseconds");
        *milliseconds = m->engine.time_kernel(which, iterations);
    });
}

}  // extern "C"
