// HIP engine for the Qwen3-0.6B FP16 path: the device-side replacement of
// qwen_cpu::Model::Impl (engine/core.cpp:220-758).
#pragma once
#include <hip/hip_runtime.h>

#include <memory>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "prefill.hpp"
#include "sampler.hpp"
#include "token.hpp"

namespace qwen_hip {

struct Options {
    int decode_threads = 12;   // accepted and echoed (engine/core.hpp:11-15)
    int prefill_threads = 6;
    int context = 4096;
};

// Device weights of one pack, shared by every sequence created from it
// (freed when the last one goes).
struct Weights {
    Weights() = default;
    Weights(const Weights&) = delete;
    Weights& operator=(const Weights&) = delete;
    ~Weights();
    std::vector<void*> allocations;
    std::vector<LayerDevice> layers;    // keys/values unset
    std::vector<PrefillLayer> prefill;  // keys/values unset
    uint16_t* embed = nullptr;          // natural [vocab x 1024]
    uint16_t* lm_t = nullptr;           // chain-tiled embedding
    uint16_t* embed_mfma = nullptr;     // embedding in matrix-core order (batched head)
    float* final_norm = nullptr;
    float* cosines = nullptr;           // [4096][64]
    float* sines = nullptr;
};

// True when the dispatcher deals a launch's workgroups round-robin over the
// 8 XCDs of a 256-CU device (probed once per process), which the decode
// kernels that exchange values inside a launch rely on.
bool placement_ok();

class Engine {
public:
    Engine(const std::string& weights, Options options);
    // A further sequence on already uploaded weights: own KV cache and state.
    Engine(std::shared_ptr<Weights> weights, Options options);
    const std::shared_ptr<Weights>& weights() const { return weights_; }
    ~Engine();
    Engine(const Engine&) = delete;
    Engine& operator=(const Engine&) = delete;

    void reset();
    void truncate(int position);
    void prefill(const int* ids, size_t count);
    void step(int token);
    // Two consumed ids with B1 arithmetic; rows stay pending until commit.
    // Both rows run as one launch that reads every weight once for both
    // (the token kernel's two-row form) unless the two positions take
    // different attention forms or the token kernel is off; then as two
    // single steps.
    void verify_two(int first, int second);
    // Host copies of the pending rows ([2 x vocab] logits, [2 x 1024]
    // hidden), copied on first access, and the base position.
    void verification_rows(const float** logits, const float** hidden, int* base);
    void commit_verified(int count);
    // Host copies of the current logits/hidden (nullptr when none).
    const float* logits();
    const float* hidden();
    int position() const { return pos_; }
    // 2: one persistent launch per token, 1: two fused launches per layer,
    // 0: separate kernels.
    int decode_kernels() const { return token_kernel_ ? 2 : (fused_ffn_ && fused_attn_) ? 1 : 0; }
    // Device greedy selection of the current logits (engine/main.cpp:51-59).
    int greedy();
    // Greedy selections of the pending verification rows.
    void verify_greedy(int* first, int* second);
    // Chat-mode candidates of the current logits (engine/main.cpp:51-62):
    // the k best (logit - (penalized ? penalty : 0)) / temperature, value
    // descending then id ascending; k in 1..kTopMax.
    void top_scores(float penalty, float temperature, int k, float* values, int* ids);
    // The penalized-token flags (the sampler's consumed ids): cleared first
    // when `clear`, then ids[0..count) set.
    void update_penalized(bool clear, const int* ids, size_t count);
    const Options& options() const { return options_; }

    // Average duration (ms) of one standalone launch of a decode kernel,
    // timed with HIP events on the engine stream. which: 0 qkv, 1 attention,
    // 2 o, 3 gate/up, 4 down, 5 lm_head, 6 fused FFN, 7 fused QKV +
    // attention + O, 8 token kernel (all layers). Requires position() > 0.
    float time_kernel(int which, int iterations);
    hipStream_t stream() const { return stream_; }

    // This sequence becomes `src` truncated to `positions`: K/V rows
    // 0..positions-1 copied on the device, no current logits.
    void copy_prefix(const Engine& src, int positions);
    // One decode step for each of `count` sequences sharing weights, from one
    // read of every weight matrix (tokens[i] is consumed by seqs[i]).
    static void step_batch(Engine* const* seqs, const int* tokens, int count);

private:
    void init_state();
    void append(const int* ids, size_t count);
    void run_append(const int* ids, size_t count);
    void roll_back(int position);
    void run_token(int token, bool head, int result_slot);
    void run_pair(int first, int second);
    TokenLaunch token_launch(int rows, int pos, int first, int second, float* x_out);
    LayerFlow layer_flow(int layer);
    uint32_t next_tag();
    // `count` consecutive tags (none of them 0) for one launch.
    uint32_t reserve_tags(int count);
    void clear_exchanges();
    void check_stall(int slot) const;
    void release();
    void sync();
    void settle();
    void await_result(int slot);
    void invalidate();

    Options options_;
    std::shared_ptr<Weights> weights_;
    hipStream_t stream_ = nullptr;
    std::vector<void*> allocations_;
    std::vector<LayerDevice> layers_;
    std::vector<PrefillLayer> prefill_layers_;
    PrefillScratch prefill_{};
    int* ids_dev_ = nullptr;    // prompt ids of the current call
    int* ids_host_ = nullptr;   // pinned staging for them
    uint16_t* embed_ = nullptr;     // the shared weights' pointers, for brevity
    uint16_t* lm_t_ = nullptr;
    float* final_norm_ = nullptr;
    float* cosines_ = nullptr;
    float* sines_ = nullptr;
    DecodeScratch scratch_{};
    ArgmaxResult* result_host_ = nullptr;  // pinned [3]: current, verify row 0, verify row 1
    uint8_t* penalized_ = nullptr;         // device [vocab] flags of the chat sampler
    void* top_scratch_ = nullptr;          // device candidates of top_scores
    TopScores* top_device_ = nullptr;
    TopScores* top_host_ = nullptr;        // pinned
    float* ver_logits_ = nullptr;   // device [2 x vocab]
    float* ver_hidden_ = nullptr;   // device [2 x 1024]
    float* base_logits_ = nullptr;  // public logits saved across a two-step verification
    float* base_hidden_ = nullptr;
    PairScratch pair_{};            // one-pass verification buffers (logits/hidden = ver_*)
    float* ver_host_ = nullptr;     // pinned [2 x vocab] logits then [2 x 1024] hidden
    bool ver_host_valid_ = false;
    int pos_ = 0;
    // Layers 0-26 run the fused FFN kernel (norm + gate/up + SwiGLU + down
    // slices in one launch) unless QWEN_HIP_FUSED_FFN=0; every fused launch
    // takes the next tag (never 0, the cleared exchange).
    bool fused_ffn_ = true;
    // Norm + QKV + attention + O run as one kernel per layer unless
    // QWEN_HIP_FUSED_ATTENTION=0; its launches take tags from the same counter.
    bool fused_attn_ = true;
    uint32_t ffn_tag_ = 0;
    uint32_t result_seq_ = 0;  // sequence number of the last single-row head launch
    bool unsynced_ = false;    // a step returned on its result word; the stream may still be finishing
    // A single-row step runs its 28 layers as one persistent launch
    // (launch_token_layers) unless QWEN_HIP_TOKEN_KERNEL=0 (or either fused
    // kernel is switched off): exchange words, poll limit and the test-only
    // withheld post of the next launch (QWEN_HIP_TEST_WITHHOLD / _SPINS).
    bool token_kernel_ = true;
    uint64_t* token_words_ = nullptr;
    unsigned token_spins_ = kTokenSpins;
    int token_withhold_ = -1;
    bool token_prefetch_ = true;
    // Identity of this sequence's K/V rows [0, pos_): a new process-unique
    // id whenever rows below pos_ may be rewritten (construction, reset,
    // rewind, copy_prefix). A copy records its source's id and length: rows
    // [0, prefix_len_) are that content, so sequences of one batched step
    // with the same prefix_id_ read those rows from one cache (unless
    // QWEN_HIP_SHARED_PREFIX=0).
    uint64_t content_id_ = 0;
    uint64_t prefix_id_ = 0;
    int prefix_len_ = 0;
    bool share_prefix_ = true;
    void renew_content();
    bool has_logits_ = false;
    bool pending_ = false;
    std::vector<float> host_logits_, host_hidden_;
    bool host_logits_valid_ = false, host_hidden_valid_ = false;

    template <class T>
    T* device_alloc(size_t count);
};

}  // namespace qwen_hip
