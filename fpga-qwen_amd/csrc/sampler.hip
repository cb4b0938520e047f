// Chat-mode candidate selection on the device (engine/main.cpp:51-62).
//
// The reference sampler scores every id as (logit - (seen ? 1.5 : 0)) / 0.7
// and keeps the 20 best under the order (value descending, id ascending);
// only those 20 scores enter its top-p draw. Here the scores and the
// selection run on the GPU and just the k winners travel to the host, which
// draws from them exactly as the reference does. Scores use IEEE single
// precision subtraction and correctly rounded division, as on the host.
//
// Selection: each (score, id) becomes one 64-bit key whose unsigned order is
// the sampler's order (high word: the score's bits mapped to an unsigned
// order with -0 folded onto +0, so equal floats compare equal; low word:
// ~id, so lower ids win ties). A first kernel sorts chunks of 1024 keys in
// LDS (bitonic) and keeps each chunk's best kTopMax; one workgroup sorts
// those candidates and decodes the k best.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "sampler.hpp"

namespace qwen_hip {
namespace {

constexpr int kScoreChunk = 1024;
constexpr int kScoreChunks = (kVocab + kScoreChunk - 1) / kScoreChunk;  // 149
constexpr int kMergeKeys = 8192;  // kScoreChunks * kTopMax rounded up to a power of two
static_assert(kScoreChunks * kTopMax <= kMergeKeys, "merge buffer too small");

__device__ __forceinline__ uint64_t score_key(float score, int id) {
    uint32_t bits = __builtin_bit_cast(uint32_t, score);
    if ((bits & 0x7fffffffu) == 0) bits = 0;  // -0 == +0
    const uint32_t ordered = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
    return (uint64_t(ordered) << 32) | uint64_t(~uint32_t(id));
}

__device__ __forceinline__ float key_score(uint64_t key) {
    const uint32_t ordered = uint32_t(key >> 32);
    const uint32_t bits = (ordered & 0x80000000u) ? (ordered & 0x7fffffffu) : ~ordered;
    return __builtin_bit_cast(float, bits);
}

// Bitonic sort of N keys in LDS, descending, by THREADS threads.
template <int N, int THREADS>
__device__ __forceinline__ void sort_desc(uint64_t* keys) {
    for (int size = 2; size <= N; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int t = threadIdx.x; t < N / 2; t += THREADS) {
                const int lo = 2 * t - (t & (stride - 1));
                const int hi = lo + stride;
                const bool descending = (lo & size) == 0;
                const uint64_t a = keys[lo], b = keys[hi];
                if ((a < b) == descending) {
                    keys[lo] = b;
                    keys[hi] = a;
                }
            }
        }
    }
    __syncthreads();
}

__global__ __launch_bounds__(256) void top_chunk_kernel(const float* __restrict__ logits,
                                                        const uint8_t* __restrict__ penalized, float penalty,
                                                        float temperature, uint64_t* __restrict__ best) {
    __shared__ uint64_t keys[kScoreChunk];
    const int base = blockIdx.x * kScoreChunk;
#pragma unroll
    for (int k = 0; k < kScoreChunk / 256; ++k) {
        const int i = threadIdx.x + 256 * k, id = base + i;
        uint64_t key = 0;  // below every real key (their high word is at least 0x00800000)
        if (id < kVocab) {
            const float score = (logits[id] - (penalized[id] ? penalty : 0.f)) / temperature;
            key = score_key(score, id);
        }
        keys[i] = key;
    }
    sort_desc<kScoreChunk, 256>(keys);
    if (threadIdx.x < kTopMax) best[blockIdx.x * kTopMax + threadIdx.x] = keys[threadIdx.x];
}

__global__ __launch_bounds__(1024) void top_merge_kernel(const uint64_t* __restrict__ best, int k,
                                                         TopScores* __restrict__ out, TopScores* host_out) {
    __shared__ uint64_t keys[kMergeKeys];
    for (int i = threadIdx.x; i < kMergeKeys; i += 1024) keys[i] = i < kScoreChunks * kTopMax ? best[i] : 0;
    sort_desc<kMergeKeys, 1024>(keys);
    if (threadIdx.x < k) {
        const uint64_t key = keys[threadIdx.x];
        const float value = key_score(key);
        const int id = int(~uint32_t(key));
        out->value[threadIdx.x] = value;
        out->id[threadIdx.x] = id;
        host_out->value[threadIdx.x] = value;
        host_out->id[threadIdx.x] = id;
    }
}

__global__ void mark_kernel(uint8_t* __restrict__ penalized, const int* __restrict__ ids, int count) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) penalized[ids[i]] = 1;
}

__global__ void clear_kernel(uint32_t* __restrict__ words, int count) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) words[i] = 0;
}

}  // namespace

size_t top_scores_scratch_bytes() { return sizeof(uint64_t) * kScoreChunks * kTopMax; }

void launch_top_scores(const float* logits, const uint8_t* penalized, float penalty, float temperature, int k,
                       void* scratch, TopScores* device_out, TopScores* host_out, hipStream_t stream) {
    require(k >= 1 && k <= kTopMax, "top scores: k must be 1..32");
    uint64_t* best = static_cast<uint64_t*>(scratch);
    top_chunk_kernel<<<kScoreChunks, 256, 0, stream>>>(logits, penalized, penalty, temperature, best);
    top_merge_kernel<<<1, 1024, 0, stream>>>(best, k, device_out, host_out);
}

void launch_mark_penalized(uint8_t* penalized, bool clear, const int* ids, int count, hipStream_t stream) {
    static_assert(kVocab % 4 == 0, "the penalized flags are cleared as 32-bit words");
    if (clear) clear_kernel<<<(kVocab / 4 + 255) / 256, 256, 0, stream>>>(reinterpret_cast<uint32_t*>(penalized),
                                                                         kVocab / 4);
    if (count > 0) mark_kernel<<<(count + 255) / 256, 256, 0, stream>>>(penalized, ids, count);
}

}  // namespace qwen_hip
