// Engine: device state, weight upload, the per-token kernel sequence and the
// qwen_cpu::Model semantics (engine/core.cpp:707-758) on top of them.
#include "engine.hpp"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "batch.hpp"
#include "pack.hpp"
#include "prefill.hpp"

#define HIP_CHECK(expr)                                                                                  \
    do {                                                                                                 \
        const hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess) throw std::runtime_error(std::string("HIP error: ") + hipGetErrorString(e_) + \
                                                       " (" #expr ")");                                  \
    } while (0)

namespace qwen_hip {

// The fused decode kernels and the batched step hand values between the
// workgroups of one launch, so each launch needs all of its 256 workgroups
// resident at once (one per CU). Two such launches in flight together, from
// engines stepped on different host threads, could split the CUs between
// them and both give up polling ("Decode step stalled"). Every call that
// launches them holds this process-wide lock (the engine runs on device 0)
// until its stream has drained, so such calls from several threads run one
// after another.
static std::mutex& launch_lock() {
    static std::mutex lock;
    return lock;
}

// The decode kernels that exchange values between the workgroups of one
// launch assume what the dispatcher does on this chip: 256 CUs, and the
// workgroups of a launch dealt round-robin to the 8 XCDs, so that all
// workgroups w with the same w % 8 share one XCD (and its L2) and the 8
// residues sit on 8 different XCDs. A probe launch records each workgroup's
// XCD (HW_REG_XCC_ID) once per process; if the mapping or the CU count
// differs, the engine runs the separate kernels (no exchanges inside a
// launch) and refuses the batched step.
__global__ void placement_probe_kernel(unsigned* xcc) {
    if (threadIdx.x == 0) {
        unsigned v;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
        xcc[blockIdx.x] = v & 15u;
    }
}

static bool probe_placement() {
    hipDeviceProp_t prop{};
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess || prop.multiProcessorCount != 256) return false;
    unsigned* d = nullptr;
    if (hipMalloc(&d, 256 * sizeof(unsigned)) != hipSuccess) return false;
    unsigned h[256] = {};
    placement_probe_kernel<<<256, 64>>>(d);
    const bool ran = hipGetLastError() == hipSuccess && hipDeviceSynchronize() == hipSuccess &&
                     hipMemcpy(h, d, sizeof(h), hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(d);
    if (!ran) return false;
    unsigned seen = 0;
    for (int r = 0; r < 8; ++r) {
        for (int w = r; w < 256; w += 8)
            if (h[w] != h[r]) return false;
        if (seen & (1u << h[r])) return false;
        seen |= 1u << h[r];
    }
    return true;
}

bool placement_ok() {
    static const bool ok = [] {
        const char* env = std::getenv("QWEN_HIP_ASSUME_NO_PLACEMENT");  // tests: act as if the probe failed
        return !(env && std::string(env) != "0") && probe_placement();
    }();
    return ok;
}

template <class T>
T* Engine::device_alloc(size_t count) {
    void* p = nullptr;
    HIP_CHECK(hipMalloc(&p, count * sizeof(T)));
    allocations_.push_back(p);
    return static_cast<T*>(p);
}

Weights::~Weights() {
    for (void* p : allocations) (void)hipFree(p);
}

// Uploads a validated pack: natural copies of every matrix (gather, prefill
// GEMMs, batched decode), chain-tiled copies (batch-1 GEMVs), the embedding
// in matrix-core order (batched head), norms and the RoPE tables for the
// full 4096-position range.
static std::shared_ptr<Weights> load_weights(const Pack& pack, hipStream_t stream) {
    auto w = std::make_shared<Weights>();
    auto alloc = [&](size_t bytes) {
        void* p = nullptr;
        HIP_CHECK(hipMalloc(&p, bytes));
        w->allocations.push_back(p);
        return p;
    };
    auto alloc_half = [&](size_t count) { return static_cast<uint16_t*>(alloc(count * 2)); };
    auto upload = [&](uint16_t* dst, const PackTensor& t) {
        HIP_CHECK(hipMemcpy(dst, t.half, size_t(t.rows) * t.cols * 2, hipMemcpyHostToDevice));
    };
    auto upload_norm = [&](const PackTensor& t) {
        float* d = static_cast<float*>(alloc(size_t(t.rows) * 4));
        HIP_CHECK(hipMemcpy(d, t.norm, size_t(t.rows) * 4, hipMemcpyHostToDevice));
        return d;
    };

    // Embedding: natural copy (gather) and chain-tiled copy (tied head).
    const PackTensor& emb = pack.tensor("model.embed_tokens.weight");
    w->embed = alloc_half(size_t(kVocab) * kHidden);
    HIP_CHECK(hipMemcpy(w->embed, emb.half, size_t(kVocab) * kHidden * 2, hipMemcpyHostToDevice));
    w->lm_t = alloc_half(size_t(kVocab) * kHidden);
    launch_tile_matrix(w->embed, nullptr, w->lm_t, kVocab, kHidden, stream);
    w->embed_mfma = alloc_half(size_t(kVocab) * kHidden);
    launch_mfma_order(w->embed, w->embed_mfma, kVocab, kHidden, 128, stream);
    w->final_norm = upload_norm(pack.tensor("model.norm.weight"));

    w->layers.resize(kLayers);
    w->prefill.resize(kLayers);
    for (int l = 0; l < kLayers; ++l) {
        LayerDevice& L = w->layers[l];
        uint16_t* qkv_n = alloc_half(size_t(kQKVRows) * kHidden);
        upload(qkv_n, pack.layer(l, "self_attn.q_proj.weight"));
        upload(qkv_n + size_t(kQDim) * kHidden, pack.layer(l, "self_attn.k_proj.weight"));
        upload(qkv_n + size_t(kQDim + kKVDim) * kHidden, pack.layer(l, "self_attn.v_proj.weight"));
        uint16_t* o_n = alloc_half(size_t(kHidden) * kQDim);
        upload(o_n, pack.layer(l, "self_attn.o_proj.weight"));
        uint16_t* gu_n = alloc_half(size_t(2 * kFFN) * kHidden);
        upload(gu_n, pack.layer(l, "mlp.gate_proj.weight"));
        upload(gu_n + size_t(kFFN) * kHidden, pack.layer(l, "mlp.up_proj.weight"));
        uint16_t* down_n = alloc_half(size_t(kHidden) * kFFN);
        upload(down_n, pack.layer(l, "mlp.down_proj.weight"));
        uint16_t* qkv_t = alloc_half(size_t(kQKVRows) * kHidden);
        launch_tile_matrix(qkv_n, nullptr, qkv_t, kQKVRows, kHidden, stream);
        uint16_t* gu_t = alloc_half(size_t(2 * kFFN) * kHidden);
        launch_tile_matrix(gu_n, gu_n + size_t(kFFN) * kHidden, gu_t, kFFN, kHidden, stream);
        uint16_t* down_t = alloc_half(size_t(kHidden) * kFFN);
        launch_tile_matrix(down_n, nullptr, down_t, kHidden, kFFN, stream);
        // Matrix-core order for the batched step: QKV tiles and the lm_head
        // take 128-column blocks per wave, O 64, down 96; gate / up tiles
        // of 12 rows.
        L.qkv_m = alloc_half(size_t(kQKVRows) * kHidden);
        launch_mfma_order(qkv_n, L.qkv_m, kQKVRows, kHidden, 128, stream);
        L.o_m = alloc_half(size_t(kHidden) * kQDim);
        launch_mfma_order(o_n, L.o_m, kHidden, kQDim, 64, stream);
        L.down_m = alloc_half(size_t(kHidden) * kFFN);
        launch_mfma_order(down_n, L.down_m, kHidden, kFFN, 96, stream);
        L.gateup_m = alloc_half(kGateupOrderHalves);
        launch_gateup_order(gu_n, L.gateup_m, stream);
        L.qkv_t = qkv_t;
        L.o_n = o_n;
        L.qkv_n = qkv_n;
        L.gateup_n = gu_n;
        L.down_n = down_n;
        L.gateup_t = gu_t;
        L.down_t = down_t;
        L.in_norm = upload_norm(pack.layer(l, "input_layernorm.weight"));
        L.post_norm = upload_norm(pack.layer(l, "post_attention_layernorm.weight"));
        L.q_norm = upload_norm(pack.layer(l, "self_attn.q_norm.weight"));
        L.k_norm = upload_norm(pack.layer(l, "self_attn.k_norm.weight"));
        {
            float* qk = static_cast<float*>(alloc(2 * kHeadDim * 4));
            HIP_CHECK(hipMemcpy(qk, L.q_norm, kHeadDim * 4, hipMemcpyDeviceToDevice));
            HIP_CHECK(hipMemcpy(qk + kHeadDim, L.k_norm, kHeadDim * 4, hipMemcpyDeviceToDevice));
            L.qk_norm = qk;
        }
        w->prefill[l] = PrefillLayer{qkv_n, o_n, gu_n, down_n, L.in_norm, L.post_norm, L.q_norm, L.k_norm,
                                     nullptr, nullptr};
    }
    HIP_CHECK(hipStreamSynchronize(stream));

    // RoPE tables in double, stored as FP32 (engine/core.cpp:287-288).
    std::vector<float> cs(size_t(kMaxContext) * 64), sn(cs.size());
    for (int p = 0; p < kMaxContext; ++p)
        for (int j = 0; j < 64; ++j) {
            const double angle = p / std::pow(1000000.0, 2.0 * j / kHeadDim);
            cs[size_t(p) * 64 + j] = float(std::cos(angle));
            sn[size_t(p) * 64 + j] = float(std::sin(angle));
        }
    w->cosines = static_cast<float*>(alloc(cs.size() * 4));
    w->sines = static_cast<float*>(alloc(sn.size() * 4));
    HIP_CHECK(hipMemcpy(w->cosines, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(w->sines, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    HIP_CHECK(hipGetLastError());
    return w;
}

static void check_options(const Options& opt) {
    require(opt.decode_threads >= 1 && opt.decode_threads <= 64 && opt.prefill_threads >= 1 &&
                opt.prefill_threads <= 64,
            "Threads must be in 1..64");
    require(opt.context >= 1 && opt.context <= kMaxContext, "Context must be in 1..4096");
}

Engine::Engine(const std::string& weights, Options opt) : options_(opt) {
    // Same check order as the reference constructor: map, option ranges,
    // header/index (engine/core.cpp:235-276).
    Pack pack(weights);
    check_options(opt);
    pack.validate();

    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices < 1)
        throw std::runtime_error("No HIP device available");
    try {
        HIP_CHECK(hipSetDevice(0));
        HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
        weights_ = load_weights(pack, stream_);
        init_state();
    } catch (...) {
        release();
        throw;
    }
}

Engine::Engine(std::shared_ptr<Weights> weights, Options opt) : options_(opt) {
    check_options(opt);
    require(weights != nullptr, "No weights to share");
    try {
        HIP_CHECK(hipSetDevice(0));
        HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
        weights_ = std::move(weights);
        init_state();
    } catch (...) {
        release();
        throw;
    }
}

// Per-sequence state: KV cache, decode and prefill scratch, pinned staging.
void Engine::init_state() {
    const int ctx = options_.context;
    const Weights& w = *weights_;
    embed_ = w.embed;
    lm_t_ = w.lm_t;
    final_norm_ = w.final_norm;
    cosines_ = w.cosines;
    sines_ = w.sines;
    layers_ = w.layers;
    prefill_layers_ = w.prefill;
    for (int l = 0; l < kLayers; ++l) {
        // Keys then values of a layer in one allocation (the token kernel
        // addresses both from the keys).
        layers_[l].keys = device_alloc<uint16_t>(2 * size_t(kKVHeads) * ctx * kHeadDim);
        layers_[l].values = layers_[l].keys + size_t(kKVHeads) * ctx * kHeadDim;
        prefill_layers_[l].keys = layers_[l].keys;
        prefill_layers_[l].values = layers_[l].values;
    }

    DecodeScratch& s = scratch_;
    s.x = device_alloc<float>(kHidden);
    s.qkv = device_alloc<float>(kQKVRows);
    s.attended = device_alloc<float>(kQDim);
    s.act = device_alloc<float>(kFFN);
    s.logits = device_alloc<float>(kVocab);
    s.hidden = device_alloc<float>(kHidden);
    s.attn_partial = device_alloc<float>(size_t(kKVHeads) * kAttnSplits * kAttnPartial);
    s.o_part = device_alloc<float>(size_t(kOParts) * kHidden);
    s.lm_value = device_alloc<float>(kLmPartials);
    s.lm_index = device_alloc<int>(kLmPartials);
    s.lm_bad = device_alloc<int>(kLmPartials);
    s.result = device_alloc<ArgmaxResult>(1);
    s.xm = device_alloc<float>(kHidden);
    s.dparts = device_alloc<float>(size_t(kFfnSlices) * kHidden);
    s.exchange = device_alloc<uint64_t>(kFFN);
    s.stall = device_alloc<int>(1);
    s.xqkv = device_alloc<uint64_t>(kXqkvWords);
    s.xpart = device_alloc<uint64_t>(kXPartWords);
    s.bexchange = device_alloc<uint64_t>(kBatchExchangeWords);
    s.lm_words = device_alloc<uint64_t>(4 * kLmStreamGroups);

    ver_logits_ = device_alloc<float>(size_t(2) * kVocab);
    ver_hidden_ = device_alloc<float>(size_t(2) * kHidden);
    base_logits_ = device_alloc<float>(kVocab);
    base_hidden_ = device_alloc<float>(kHidden);
    pair_.x = device_alloc<float>(2 * kHidden);
    pair_.logits = ver_logits_;
    pair_.hidden = ver_hidden_;
    pair_.result = device_alloc<ArgmaxResult>(2);
    token_words_ = device_alloc<uint64_t>(2 * size_t(kTokWords));  // a block per verification row
    HIP_CHECK(hipMemsetAsync(s.stall, 0, sizeof(int), stream_));
    clear_exchanges();

    if (const char* env = std::getenv("QWEN_HIP_FUSED_FFN")) fused_ffn_ = std::string(env) != "0";
    if (const char* env = std::getenv("QWEN_HIP_FUSED_ATTENTION")) fused_attn_ = std::string(env) != "0";
    if (const char* env = std::getenv("QWEN_HIP_SHARED_PREFIX")) share_prefix_ = std::string(env) != "0";
    if (const char* env = std::getenv("QWEN_HIP_TOKEN_KERNEL")) token_kernel_ = std::string(env) != "0";
    if (const char* env = std::getenv("QWEN_HIP_TOKEN_PREFETCH")) token_prefetch_ = std::string(env) != "0";
    if (const char* env = std::getenv("QWEN_HIP_TEST_WITHHOLD")) token_withhold_ = std::atoi(env);
    if (const char* env = std::getenv("QWEN_HIP_TEST_SPINS")) token_spins_ = unsigned(std::max(1, std::atoi(env)));
    if (!placement_ok()) fused_ffn_ = fused_attn_ = false;
    token_kernel_ = token_kernel_ && fused_ffn_ && fused_attn_;
    renew_content();

    penalized_ = device_alloc<uint8_t>(kVocab);
    top_scratch_ = device_alloc<uint8_t>(top_scores_scratch_bytes());
    top_device_ = device_alloc<TopScores>(1);
    void* pinned = nullptr;
    HIP_CHECK(hipHostMalloc(&pinned, sizeof(TopScores), hipHostMallocDefault));
    top_host_ = static_cast<TopScores*>(pinned);
    HIP_CHECK(hipHostMalloc(&pinned, sizeof(float) * 2 * (size_t(kVocab) + kHidden), hipHostMallocDefault));
    ver_host_ = static_cast<float*>(pinned);
    HIP_CHECK(hipHostMalloc(&pinned, sizeof(ArgmaxResult) * 3, hipHostMallocDefault));
    result_host_ = static_cast<ArgmaxResult*>(pinned);
    std::memset(result_host_, 0, sizeof(ArgmaxResult) * 3);
    PrefillScratch& ps = prefill_;
    const size_t prows = size_t(std::max(2, std::min(ctx, kPrefillRows)));  // a call never exceeds the context
    ps.x = device_alloc<float>(prows * kHidden);
    ps.h_hi = device_alloc<uint16_t>(prows * kHidden);
    ps.h_lo = device_alloc<uint16_t>(prows * kHidden);
    ps.qkv = device_alloc<float>(prows * kQKVRows);
    ps.att_hi = device_alloc<uint16_t>(prows * kQDim);
    ps.att_lo = device_alloc<uint16_t>(prows * kQDim);
    ps.act_hi = device_alloc<uint16_t>(prows * kFFN);
    ps.act_lo = device_alloc<uint16_t>(prows * kFFN);
    ps.part = device_alloc<float>(4 * prows * kHidden);
    ps.row_exp = device_alloc<int>(prows);
    ps.act_flag = device_alloc<int>(4 * prows);
    ps.act_exp = device_alloc<uint8_t>(prows * (kFFN / 8));
    ids_dev_ = device_alloc<int>(size_t(ctx));
    HIP_CHECK(hipHostMalloc(&pinned, sizeof(int) * size_t(ctx), hipHostMallocDefault));
    ids_host_ = static_cast<int*>(pinned);
    launch_mark_penalized(penalized_, true, nullptr, 0, stream_);
    HIP_CHECK(hipStreamSynchronize(stream_));
    HIP_CHECK(hipGetLastError());
}

void Engine::release() {
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (void* p : allocations_) (void)hipFree(p);
    if (result_host_) (void)hipHostFree(result_host_);
    if (ver_host_) (void)hipHostFree(ver_host_);
    ver_host_ = nullptr;
    if (top_host_) (void)hipHostFree(top_host_);
    top_host_ = nullptr;
    if (ids_host_) (void)hipHostFree(ids_host_);
    ids_host_ = nullptr;
    if (stream_) (void)hipStreamDestroy(stream_);
    allocations_.clear();
    result_host_ = nullptr;
    stream_ = nullptr;
}

Engine::~Engine() { release(); }

void Engine::sync() {
    HIP_CHECK(hipStreamSynchronize(stream_));
    unsynced_ = false;
}

// Host reads of device memory and launches that read another engine's
// buffers first let a step that returned early drain.
void Engine::settle() {
    if (unsynced_) sync();
}

// A decode step returns as soon as its argmax kernel has stored the result
// word of this launch in pinned memory (the last store of the step's last
// kernel), instead of waiting for the stream's completion signal. Bounded:
// after ~20 ms it waits for the stream, which also reports a failed launch.
void Engine::await_result(int slot) {
    const unsigned long long* word = &result_host_[slot].done;
    const auto start = std::chrono::steady_clock::now();
    for (unsigned spin = 1;; ++spin) {
        const unsigned long long w = __atomic_load_n(word, __ATOMIC_ACQUIRE);
        if (uint32_t(w >> 32) == result_seq_) {
            result_host_[slot].token = int(w & 0x3fffffffu);
            result_host_[slot].nonfinite = int((w >> 30) & 1u);
            result_host_[slot].stalled = int((w >> 31) & 1u);
            unsynced_ = true;
            return;
        }
        if ((spin & 1023u) == 0 && std::chrono::steady_clock::now() - start > std::chrono::milliseconds(20)) break;
    }
    sync();
}

void Engine::invalidate() {
    has_logits_ = false;
    host_logits_valid_ = host_hidden_valid_ = false;
}

void Engine::renew_content() {
    static std::atomic<uint64_t> next_id{1};
    content_id_ = next_id.fetch_add(1);
}

// engine/core.cpp:718-721
void Engine::reset() {
    pos_ = 0;
    pending_ = false;
    prefix_len_ = 0;
    renew_content();
    invalidate();
}

// engine/core.cpp:722-727
void Engine::truncate(int position) {
    require(position >= 0 && position <= pos_, "Rewind position out of range");
    if (position < pos_) renew_content();  // rows from position on will be rewritten
    pos_ = position;
    prefix_len_ = std::min(prefix_len_, position);
    pending_ = false;
    invalidate();
}

// A call that fails after launching its kernels (an exchange that gave up,
// a HIP error) leaves the K/V rows from its start position on written from
// garbage or not at all: the sequence returns to that position without
// current logits, and its content identity is renewed since those rows will
// be rewritten.
void Engine::roll_back(int position) {
    pos_ = position;
    prefix_len_ = std::min(prefix_len_, position);
    pending_ = false;
    renew_content();
    invalidate();
}

// One token through the 28 layers (5 kernels each) and, when `head`, the
// final norm, tied lm_head and greedy argmax into host result slot
// `result_slot`. The step scalars are kernel arguments.
// Exchange tags: every launch of a fused kernel takes the next one (never 0,
// the cleared exchange), so no launch reads a word an earlier one wrote.
// When the counter wraps, the exchanges are cleared again (on the engine's
// stream, ahead of any launch that uses the new tags), so a word written
// 2^32 launches earlier can never carry a reused tag.
uint32_t Engine::next_tag() {
    if (++ffn_tag_ == 0) {
        clear_exchanges();
        ffn_tag_ = 1;
    }
    return ffn_tag_;
}

// Exchange words start with tag 0, which no launch uses.
void Engine::clear_exchanges() {
    HIP_CHECK(hipMemsetAsync(scratch_.exchange, 0, kFFN * sizeof(uint64_t), stream_));
    HIP_CHECK(hipMemsetAsync(scratch_.xqkv, 0, kXqkvWords * sizeof(uint64_t), stream_));
    HIP_CHECK(hipMemsetAsync(scratch_.xpart, 0, kXPartWords * sizeof(uint64_t), stream_));
    HIP_CHECK(hipMemsetAsync(scratch_.bexchange, 0, kBatchExchangeWords * sizeof(uint64_t), stream_));
    HIP_CHECK(hipMemsetAsync(token_words_, 0, 2 * kTokWords * sizeof(uint64_t), stream_));
    HIP_CHECK(hipMemsetAsync(scratch_.lm_words, 0, 4 * kLmStreamGroups * sizeof(uint64_t), stream_));
}

uint32_t Engine::reserve_tags(int count) {
    if (ffn_tag_ > 0xFFFFFFFFu - uint32_t(count)) {
        clear_exchanges();
        ffn_tag_ = 0;
    }
    const uint32_t first = ffn_tag_ + 1;
    ffn_tag_ += uint32_t(count);
    return first;
}

LayerFlow Engine::layer_flow(int layer) {
    LayerFlow f{};
    f.fold_input = fused_ffn_ && layer > 0;
    if (fused_attn_) f.attn_tag = next_tag();
    if (fused_ffn_) f.ffn_tag = next_tag();
    return f;
}

// A launch whose exchange poll gave up leaves garbage in the residual
// stream; the argmax of the step reports it.
void Engine::check_stall(int slot) const {
    if (result_host_[slot].stalled)
        throw std::runtime_error("Decode step stalled: an exchange between workgroups did not complete");
}

void Engine::run_token(int token, bool head, int result_slot) {
    if (token_kernel_) {
        TokenLaunch t = token_launch(1, pos_, token, 0, scratch_.x);
        t.withhold = token_withhold_;
        token_withhold_ = -1;  // the test knob withholds one post, once
        launch_token_layers(t, stream_);
        if (head) launch_lm_head(lm_t_, final_norm_, scratch_, result_host_ + result_slot, next_tag(), stream_, ++result_seq_);
        HIP_CHECK(hipGetLastError());
        ++pos_;
        return;
    }
    for (int l = 0; l < kLayers; ++l)
        launch_decode_layer(layers_[l], l == 0 ? embed_ : nullptr, pos_, token, cosines_, sines_, options_.context,
                            scratch_, layer_flow(l), stream_);
    if (fused_ffn_) launch_fold_residual(scratch_.xm, scratch_.dparts, scratch_.x, 1, stream_);
    if (head) launch_lm_head(lm_t_, final_norm_, scratch_, result_host_ + result_slot, next_tag(), stream_, ++result_seq_);
    HIP_CHECK(hipGetLastError());
    ++pos_;
}

// engine/core.cpp:707-714: validate everything before mutating, then run.
void Engine::append(const int* ids, size_t count) {
    require(!pending_, "Commit or discard pending verification before inference");
    require(count > 0, "Empty token input");
    require(count <= size_t(options_.context - pos_), "Context capacity exceeded");
    for (size_t i = 0; i < count; ++i) require(ids[i] >= 0 && ids[i] < kVocab, "Token ID out of range");
    const int start = pos_;
    std::lock_guard<std::mutex> hold(launch_lock());
    try {
        run_append(ids, count);
    } catch (...) {
        roll_back(start);
        throw;
    }
}

void Engine::run_append(const int* ids, size_t count) {
    invalidate();
    // The reference splits a call into 512-row chunks counted from its start
    // and runs a one-row chunk on the batch-1 path (engine/core.cpp:712). Every
    // row of the batched path is computed independently of the rows grouped
    // with it (GEMM rows, row kernels, and causal attention whose key split
    // follows absolute positions), so consecutive 512-row chunks run as one
    // batched pass; only a trailing one-row chunk takes the batch-1 path.
    const size_t batched = count % kChunk == 1 ? count - 1 : count;
    require(batched <= size_t(kPrefillRows), "prefill: call longer than the batched pass");
    if (batched > 0) {
        // Only the batched pass reads the ids from the device; a one-row
        // chunk takes its token as a kernel argument.
        std::copy(ids, ids + batched, ids_host_);
        HIP_CHECK(hipMemcpyAsync(ids_dev_, ids_host_, batched * sizeof(int), hipMemcpyHostToDevice, stream_));
        const int rows = int(batched);
        launch_prefill_chunk(prefill_layers_.data(), embed_, ids_dev_, rows, pos_, cosines_, sines_,
                             options_.context, prefill_, stream_);
        pos_ += rows;
        if (batched == count) {
            HIP_CHECK(hipMemcpyAsync(scratch_.x, prefill_.x + size_t(rows - 1) * kHidden, kHidden * sizeof(float),
                                     hipMemcpyDeviceToDevice, stream_));
            launch_lm_head(lm_t_, final_norm_, scratch_, result_host_, next_tag(), stream_);
        }
    }
    if (batched < count) run_token(ids[count - 1], true, 0);
    HIP_CHECK(hipGetLastError());
    if (batched == 0) await_result(0);  // one row: its argmax is the call's last kernel
    else sync();
    check_stall(0);
    has_logits_ = true;
}

void Engine::prefill(const int* ids, size_t count) { append(ids, count); }
void Engine::step(int token) { append(&token, 1); }

const float* Engine::logits() {
    if (!has_logits_) return nullptr;
    if (!host_logits_valid_) {
        settle();
        host_logits_.resize(kVocab);
        HIP_CHECK(hipMemcpy(host_logits_.data(), scratch_.logits, size_t(kVocab) * 4, hipMemcpyDeviceToHost));
        host_logits_valid_ = true;
    }
    return host_logits_.data();
}

const float* Engine::hidden() {
    if (!has_logits_ || pos_ <= 0) return nullptr;
    if (!host_hidden_valid_) {
        settle();
        host_hidden_.resize(kHidden);
        HIP_CHECK(hipMemcpy(host_hidden_.data(), scratch_.hidden, size_t(kHidden) * 4, hipMemcpyDeviceToHost));
        host_hidden_valid_ = true;
    }
    return host_hidden_.data();
}

// The reference rewinds one model to a 512-token boundary and prefills a new
// suffix (engine/INTERFACE.md:94-103); for several sequences that share a
// prefix the same rewind is applied to a copy: src's K/V rows
// 0..positions-1 on the device, as computed by src.
void Engine::copy_prefix(const Engine& src, int positions) {
    require(!pending_, "Commit or discard pending verification before inference");
    require(src.weights_ == weights_, "Sequences do not share weights");
    require(positions >= 0 && positions <= src.pos_, "Rewind position out of range");
    require(positions <= options_.context, "Context capacity exceeded");
    invalidate();
    if (&src == this) {  // a rewind of this sequence
        truncate(positions);
        return;
    }
    pos_ = 0;
    prefix_len_ = 0;
    renew_content();
    const size_t row = size_t(kHeadDim) * sizeof(uint16_t);
    if (positions > 0) {
        HIP_CHECK(hipStreamSynchronize(src.stream_));
        for (int l = 0; l < kLayers; ++l) {
            HIP_CHECK(hipMemcpy2DAsync(layers_[l].keys, row * options_.context, src.layers_[l].keys,
                                       row * src.options_.context, row * positions, kKVHeads,
                                       hipMemcpyDeviceToDevice, stream_));
            HIP_CHECK(hipMemcpy2DAsync(layers_[l].values, row * options_.context, src.layers_[l].values,
                                       row * src.options_.context, row * positions, kKVHeads,
                                       hipMemcpyDeviceToDevice, stream_));
        }
        sync();
    }
    pos_ = positions;
    // The copied rows are src's content; rows src itself copied are that
    // copy's source's content, so a copy of a copy joins the first copies.
    if (positions <= src.prefix_len_) {
        prefix_id_ = src.prefix_id_;
    } else {
        prefix_id_ = src.content_id_;
    }
    prefix_len_ = positions;
}

// Validates every sequence before running any (as append does for one).
void Engine::step_batch(Engine* const* seqs, const int* tokens, int count) {
    require(count >= 1 && count <= kMaxBatch, "Batch must hold 1..8 sequences");
    require(placement_ok(), "Batched decode needs 256 CUs with workgroups dealt round-robin over 8 XCDs");
    for (int i = 0; i < count; ++i) {
        require(seqs[i] != nullptr, "Null sequence in batch");
        for (int j = 0; j < i; ++j) require(seqs[j] != seqs[i], "Sequence repeated in batch");
        require(seqs[i]->weights_ == seqs[0]->weights_, "Sequences do not share weights");
        require(!seqs[i]->pending_, "Commit or discard pending verification before inference");
        require(seqs[i]->pos_ < seqs[i]->options_.context, "Context capacity exceeded");
        require(tokens[i] >= 0 && tokens[i] < kVocab, "Token ID out of range");
    }
    BatchSeq bs[kMaxBatch];
    Engine& lead = *seqs[0];
    // Sequences holding copies of the same rows read them from the first
    // such sequence of the batch, up to the shorter of the two copies (whole
    // 64-row blocks).
    int shared_seq[kMaxBatch], shared[kMaxBatch];
    for (int i = 0; i < count; ++i) {
        const Engine& e = *seqs[i];
        shared_seq[i] = i;
        shared[i] = 0;
        if (!e.share_prefix_ || e.prefix_len_ < 64) continue;
        for (int j = 0; j < i; ++j) {
            const Engine& f = *seqs[j];
            if (f.share_prefix_ && f.prefix_id_ == e.prefix_id_ && f.prefix_len_ >= 64 && shared_seq[j] == j) {
                shared_seq[i] = j;
                break;
            }
        }
    }
    for (int i = 0; i < count; ++i) {
        if (shared_seq[i] == i) continue;
        shared[i] = std::min(seqs[i]->prefix_len_, seqs[shared_seq[i]]->prefix_len_) / 64 * 64;
    }
    // The batched launches exchange through the first sequence's buffers,
    // which its single-sequence launches use too: tags from its counter.
    int starts[kMaxBatch];
    for (int i = 0; i < count; ++i) starts[i] = seqs[i]->pos_;
    std::lock_guard<std::mutex> hold(launch_lock());
    try {
        uint32_t tags[kBatchTagsPerLayer * kLayers];
        for (uint32_t& t : tags) t = lead.next_tag();
        for (int i = 0; i < count; ++i) {
            Engine& e = *seqs[i];
            e.invalidate();
            bs[i] = BatchSeq{e.layers_.data(), e.scratch_, e.pos_, tokens[i], e.options_.context, e.result_host_,
                             shared_seq[i], shared[i]};
            HIP_CHECK(hipStreamSynchronize(e.stream_));
        }
        launch_decode_batch(bs, count, lead.embed_, lead.weights_->embed_mfma, lead.final_norm_, lead.cosines_,
                            lead.sines_, tags, lead.stream_);
        HIP_CHECK(hipGetLastError());
        lead.sync();
        for (int i = 0; i < count; ++i) ++seqs[i]->pos_;
        for (int i = 0; i < count; ++i) seqs[i]->check_stall(0);  // as append: no logits after a stall
    } catch (...) {
        // Every sequence of the batch wrote its K/V rows at its position.
        for (int i = 0; i < count; ++i) seqs[i]->roll_back(starts[i]);
        throw;
    }
    for (int i = 0; i < count; ++i) seqs[i]->has_logits_ = true;
}

int Engine::greedy() {
    require(has_logits_, "No current full-vocabulary logits");
    if (result_host_[0].nonfinite) throw std::runtime_error("Nonfinite model logits");
    return result_host_[0].token;
}

// Both verification rows through the 28 layers in one launch that reads
// every weight once for both (the token kernel's two-row form: row 1 attends
// to row 0's new K/V, each row with a single step's arithmetic), then the
// head for both; K/V rows written at pos_ and pos_ + 1, pos_ unchanged.
// The token kernel's launch record: every layer, `rows` rows from position
// pos, fresh tags.
TokenLaunch Engine::token_launch(int rows, int pos, int first, int second, float* x_out) {
    TokenLaunch t{};
    for (int l = 0; l < kLayers; ++l) {
        const LayerDevice& L = layers_[l];
        t.layers[l] = TokenLayer{L.qkv_t, L.o_n, L.gateup_t, L.down_t, L.in_norm, L.post_norm, L.qk_norm, L.keys};
    }
    t.layer_count = kLayers;
    t.embed = embed_;
    t.token[0] = first;
    t.token[1] = second;
    t.rows = rows;
    t.pos = pos;
    t.context = options_.context;
    t.cosines = cosines_;
    t.sines = sines_;
    t.x_out = x_out;
    t.words = token_words_;
    t.stall = scratch_.stall;
    t.scale = 1.0f / std::sqrt(128.0f);
    t.tag = reserve_tags(kLayers);
    t.spins = token_spins_;
    t.withhold = -1;
    t.prefetch = token_prefetch_ ? 1 : 0;
    return t;
}

void Engine::run_pair(int first, int second) {
    launch_token_layers(token_launch(2, pos_, first, second, pair_.x), stream_);
    launch_lm_head_pair(lm_t_, final_norm_, scratch_, pair_, result_host_ + 1, next_tag(), stream_, ++result_seq_);
    HIP_CHECK(hipGetLastError());
}

// engine/core.cpp:729-741: the rows of two B1 steps; public state stays at
// the base.
void Engine::verify_two(int first, int second) {
    require(!pending_, "Verification already pending");
    require(first >= 0 && first < kVocab && second >= 0 && second < kVocab, "Token ID out of range");
    require(pos_ <= options_.context - 2, "Context capacity exceeded");
    const int start = pos_;
    std::lock_guard<std::mutex> hold(launch_lock());
    try {
        const bool pair = token_kernel_ && token_pair_supported(start);
        if (pair) {
            run_pair(first, second);
        } else {
            // Without the token kernel, or where the two rows would take
            // different attention forms (256 and 257 cached positions): two
            // single steps, with the public logits saved and restored around
            // them.
            if (has_logits_) {
                HIP_CHECK(hipMemcpyAsync(base_logits_, scratch_.logits, size_t(kVocab) * 4,
                                         hipMemcpyDeviceToDevice, stream_));
                HIP_CHECK(hipMemcpyAsync(base_hidden_, scratch_.hidden, size_t(kHidden) * 4,
                                         hipMemcpyDeviceToDevice, stream_));
            }
            const int ids[2] = {first, second};
            for (int row = 0; row < 2; ++row) {
                run_token(ids[row], true, 1 + row);
                HIP_CHECK(hipMemcpyAsync(ver_logits_ + size_t(row) * kVocab, scratch_.logits, size_t(kVocab) * 4,
                                         hipMemcpyDeviceToDevice, stream_));
                HIP_CHECK(hipMemcpyAsync(ver_hidden_ + size_t(row) * kHidden, scratch_.hidden,
                                         size_t(kHidden) * 4, hipMemcpyDeviceToDevice, stream_));
            }
            if (has_logits_) {
                HIP_CHECK(hipMemcpyAsync(scratch_.logits, base_logits_, size_t(kVocab) * 4,
                                         hipMemcpyDeviceToDevice, stream_));
                HIP_CHECK(hipMemcpyAsync(scratch_.hidden, base_hidden_, size_t(kHidden) * 4,
                                         hipMemcpyDeviceToDevice, stream_));
            }
        }
        if (pair) {  // both rows' result words, stored last by the one head launch
            await_result(1);
            await_result(2);
        } else {
            sync();
        }
        check_stall(1);
        check_stall(2);
        pos_ = start;
        pending_ = true;
        ver_host_valid_ = false;
    } catch (...) {
        reset();
        throw;
    }
}

void Engine::verification_rows(const float** logits, const float** hidden, int* base) {
    require(pending_, "No verification pending");
    if (!ver_host_valid_) {
        HIP_CHECK(hipMemcpyAsync(ver_host_, ver_logits_, size_t(2) * kVocab * 4, hipMemcpyDeviceToHost, stream_));
        HIP_CHECK(hipMemcpyAsync(ver_host_ + size_t(2) * kVocab, ver_hidden_, size_t(2) * kHidden * 4,
                                 hipMemcpyDeviceToHost, stream_));
        sync();
        ver_host_valid_ = true;
    }
    *logits = ver_host_;
    *hidden = ver_host_ + size_t(2) * kVocab;
    *base = pos_;
}

void Engine::verify_greedy(int* first, int* second) {
    require(pending_, "No verification pending");
    for (int row = 0; row < 2; ++row)
        if (result_host_[1 + row].nonfinite) throw std::runtime_error("Nonfinite model logits");
    *first = result_host_[1].token;
    *second = result_host_[2].token;
}

void Engine::top_scores(float penalty, float temperature, int k, float* values, int* ids) {
    require(k >= 1 && k <= kTopMax, "top scores: k must be 1..32");
    require(std::isfinite(penalty) && std::isfinite(temperature) && temperature > 0.f,
            "top scores: penalty and temperature must be finite, temperature positive");
    require(has_logits_, "No current full-vocabulary logits");
    if (result_host_[0].nonfinite) throw std::runtime_error("Nonfinite model logits");
    launch_top_scores(scratch_.logits, penalized_, penalty, temperature, k, top_scratch_, top_device_, top_host_,
                      stream_);
    HIP_CHECK(hipGetLastError());
    sync();
    std::copy(top_host_->value, top_host_->value + k, values);
    std::copy(top_host_->id, top_host_->id + k, ids);
}

void Engine::update_penalized(bool clear, const int* ids, size_t count) {
    for (size_t i = 0; i < count; ++i) require(ids[i] >= 0 && ids[i] < kVocab, "Token ID out of range");
    if (clear) launch_mark_penalized(penalized_, true, nullptr, 0, stream_);
    // Staged through the prompt-id buffers, one context-sized piece at a time.
    const size_t piece = size_t(options_.context);
    for (size_t done = 0; done < count; done += piece) {
        const size_t n = std::min(piece, count - done);
        std::copy(ids + done, ids + done + n, ids_host_);
        HIP_CHECK(hipMemcpyAsync(ids_dev_, ids_host_, n * sizeof(int), hipMemcpyHostToDevice, stream_));
        launch_mark_penalized(penalized_, false, ids_dev_, int(n), stream_);
        sync();
    }
    HIP_CHECK(hipGetLastError());
    sync();
}

// engine/core.cpp:742-752
void Engine::commit_verified(int count) {
    require(pending_, "No verification pending");
    require(count == 1 || count == 2, "Commit count must be one or two");
    try {
        const int row = count - 1;
        HIP_CHECK(hipMemcpyAsync(scratch_.logits, ver_logits_ + size_t(row) * kVocab, size_t(kVocab) * 4,
                                 hipMemcpyDeviceToDevice, stream_));
        HIP_CHECK(hipMemcpyAsync(scratch_.hidden, ver_hidden_ + size_t(row) * kHidden, size_t(kHidden) * 4,
                                 hipMemcpyDeviceToDevice, stream_));
        sync();
        result_host_[0] = result_host_[1 + row];
        invalidate();
        has_logits_ = true;
        pos_ += count;
        pending_ = false;
    } catch (...) {
        reset();
        throw;
    }
}

float Engine::time_kernel(int which, int iterations) {
    require(pos_ > 0 && !pending_, "time_kernel needs a current position");
    std::lock_guard<std::mutex> hold(launch_lock());
    HIP_CHECK(hipStreamSynchronize(stream_));
    require(which >= 0 && which <= 8 && iterations > 0, "time_kernel: bad arguments");
    if (which == 2) return 0.f;  // O runs with the attention (1)
    require(which != 6 || fused_ffn_, "time_kernel: the fused FFN kernel is switched off");
    require(which != 7 || fused_attn_, "time_kernel: the fused QKV + attention kernel is switched off");
    require(which != 8 || token_kernel_, "time_kernel: the token kernel is switched off");
    // Replays kernels of the last processed position; the state is reset
    // afterwards. Layer kernels rotate over all 28 layers so that, as in a
    // real step, their weights (about 880 MB in total) stream from HBM rather
    // than from the 256 MB Infinity Cache.
    // 0, 1, 3 and 4 time the separate norm+QKV, attention, norm+gate/up and
    // down kernels (with the fused kernels on, a step runs none of them), 6
    // the fused FFN kernel, 7 the fused QKV + attention + O kernel, 8 the
    // token kernel (all 28 layers in one launch).
    const int layers = kLayers;
    int layer = 0;
    auto launch = [&] {
        LayerFlow flow = layer_flow(layer);
        if (which == 3 || which == 4) flow.ffn_tag = 0;
        if (which == 0 || which == 1) flow.attn_tag = 0;
        if (which == 8)
            launch_token_layers(token_launch(1, pos_ - 1, 0, 0, scratch_.x), stream_);
        else if (which == 5)
            launch_lm_head(lm_t_, final_norm_, scratch_, result_host_, next_tag(), stream_);
        else
            launch_layer_kernel(which == 6 ? 3 : which == 7 ? 0 : which, layers_[layer], nullptr, pos_ - 1, 0,
                                cosines_, sines_, options_.context, scratch_, flow, stream_);
        layer = (layer + 1) % layers;
    };
    for (int i = 0; i < (which == 8 ? 2 : layers); ++i) launch();
    hipEvent_t start, stop;
    HIP_CHECK(hipEventCreate(&start));
    HIP_CHECK(hipEventCreate(&stop));
    HIP_CHECK(hipEventRecord(start, stream_));
    for (int i = 0; i < iterations; ++i) launch();
    HIP_CHECK(hipEventRecord(stop, stream_));
    HIP_CHECK(hipEventSynchronize(stop));
    float ms = 0.f;
    HIP_CHECK(hipEventElapsedTime(&ms, start, stop));
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
    // The replayed kernels overwrite the residual stream and logits; the
    // attention and token kernels also rewrite cached K/V, so they reset the
    // model.
    if (which == 1 || which == 7 || which == 8)
        reset();
    else
        invalidate();
    return ms / float(iterations);
}

}  // namespace qwen_hip
