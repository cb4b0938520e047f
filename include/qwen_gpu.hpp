// C++ facade over the qwen_gpu C ABI with the reference API's shape:
// qwen_gpu::Model mirrors qwen_cpu::Model (engine/core.hpp:8-56) member for
// member, and throws std::runtime_error with the engine's message on failure.
// Header-only; link against libqwen_gpu.so.
#pragma once
#include <cstddef>
#include <memory>
#include <span>
#include <stdexcept>
#include <string>
#include <vector>

#include "qwen_gpu.h"

namespace qwen_gpu {
inline constexpr int vocabulary = QWEN_GPU_VOCABULARY;
inline constexpr int prefix_reuse_chunk = QWEN_GPU_PREFIX_REUSE_CHUNK;
struct Options {
    int decode_threads = 12;
    int prefill_threads = 6;
    int context = 4096;
};
struct VerificationRows {
    // Borrowed row-major [2, vocabulary] and [2, 1024] outputs, valid until
    // commit/reset/truncate/another successful model mutation.
    std::span<const float> logits;
    std::span<const float> hidden;
    int base_position;
};

namespace detail {
inline void check(int status) {
    if (status != QWEN_GPU_OK) throw std::runtime_error(qwen_gpu_last_error());
}
}  // namespace detail

// One caller at a time. FP16 stored matrices, FP32 norms/math, FP16 KV.
class Model {
public:
    Model(const std::string& weights_file, Options options) {
        const qwen_gpu_options o{options.decode_threads, options.prefill_threads, options.context};
        qwen_gpu_model* m = nullptr;
        detail::check(qwen_gpu_create(weights_file.c_str(), &o, &m));
        handle_.reset(m);
    }
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;
    void reset() { detail::check(qwen_gpu_reset(handle_.get())); logits_.clear(); }
    void truncate(int position) { detail::check(qwen_gpu_truncate(handle_.get(), position)); logits_.clear(); }
    void prefill(const std::vector<int>& ids) {
        logits_.clear();
        detail::check(qwen_gpu_prefill(handle_.get(), ids.data(), ids.size()));
    }
    void step(int token) {
        logits_.clear();
        detail::check(qwen_gpu_step(handle_.get(), token));
    }
    VerificationRows verify_two(int first, int second) {
        const float* l = nullptr;
        const float* h = nullptr;
        int base = 0;
        detail::check(qwen_gpu_verify_two(handle_.get(), first, second, &l, &h, &base));
        return {std::span<const float>(l, size_t(2) * vocabulary), std::span<const float>(h, size_t(2) * QWEN_GPU_HIDDEN),
                base};
    }
    void commit_verified(int count) {
        detail::check(qwen_gpu_commit_verified(handle_.get(), count));
        logits_.clear();
    }
    // Current full-vocabulary logits (empty when there are none). Copied from
    // the device on first access after each mutation.
    const std::vector<float>& logits() const {
        if (logits_.empty()) {
            const float* data = nullptr;
            size_t count = 0;
            detail::check(qwen_gpu_logits(handle_.get(), &data, &count));
            if (count) logits_.assign(data, data + count);
        }
        return logits_;
    }
    std::span<const float> hidden() const {
        const float* data = nullptr;
        size_t count = 0;
        detail::check(qwen_gpu_hidden(handle_.get(), &data, &count));
        return std::span<const float>(data, count);
    }
    int position() const { return qwen_gpu_position(handle_.get()); }
    std::size_t lossless_bf16_cache_bytes() const { return qwen_gpu_lossless_bf16_cache_bytes(handle_.get()); }

    // Extensions of the GPU engine: device-side greedy selection.
    int greedy() const {
        int token = 0;
        detail::check(qwen_gpu_greedy(handle_.get(), &token));
        return token;
    }
    std::pair<int, int> verify_greedy() const {
        int a = 0, b = 0;
        detail::check(qwen_gpu_verify_greedy(handle_.get(), &a, &b));
        return {a, b};
    }
    // Chat-mode candidates (qwen_gpu_top_scores): fills values/ids[0..k).
    void top_scores(float penalty, float temperature, int k, float* values, int* ids) const {
        detail::check(qwen_gpu_top_scores(handle_.get(), penalty, temperature, k, values, ids));
    }
    void update_penalized(bool clear, const std::vector<int>& ids) {
        detail::check(qwen_gpu_update_penalized(handle_.get(), clear ? 1 : 0, ids.data(), ids.size()));
    }
    // verify_two + verify_greedy without copying the rows to the host.
    std::pair<int, int> verify_two_greedy(int first, int second) {
        int a = 0, b = 0;
        logits_.clear();
        detail::check(qwen_gpu_verify_two_greedy(handle_.get(), first, second, &a, &b));
        return {a, b};
    }

private:
    struct Deleter {
        void operator()(qwen_gpu_model* m) const { qwen_gpu_destroy(m); }
    };
    std::unique_ptr<qwen_gpu_model, Deleter> handle_;
    mutable std::vector<float> logits_;
};
}  // namespace qwen_gpu
