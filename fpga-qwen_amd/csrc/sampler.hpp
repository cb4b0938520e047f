// Device side of the chat-mode sampler (engine/main.cpp:40-69): candidate
// scores and the penalized-token flags.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "qwen_common.hpp"

namespace qwen_hip {

inline constexpr int kTopMax = 32;  // most candidates one selection returns

// The k best scores, value descending then id ascending.
struct TopScores {
    float value[kTopMax];
    int id[kTopMax];
};

// Device scratch the selection needs (the per-chunk candidates).
size_t top_scores_scratch_bytes();

// Scores (logits[id] - (penalized[id] ? penalty : 0)) / temperature of all
// kVocab ids; the k (1..kTopMax) best go to device_out and host_out (pinned).
void launch_top_scores(const float* logits, const uint8_t* penalized, float penalty, float temperature, int k,
                       void* scratch, TopScores* device_out, TopScores* host_out, hipStream_t stream);

// penalized[ids[i]] = 1 for i < count (ids on the device, each in range),
// after zeroing all kVocab flags when `clear`.
void launch_mark_penalized(uint8_t* penalized, bool clear, const int* ids, int count, hipStream_t stream);

}  // namespace qwen_hip
