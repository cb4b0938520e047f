// Model constants and small host helpers shared by the engine sources.
// Shapes follow engine/core.cpp:28 and engine/core.hpp:9-10 (Qwen3-0.6B).
#pragma once
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace qwen_hip {

inline constexpr int kHidden = 1024;      // H
inline constexpr int kHeadDim = 128;      // D
inline constexpr int kQHeads = 16;        // Q
inline constexpr int kKVHeads = 8;        // K
inline constexpr int kFFN = 3072;         // F
inline constexpr int kLayers = 28;        // L
inline constexpr int kVocab = 151936;     // vocabulary
inline constexpr int kChunk = 512;        // prefix_reuse_chunk / the reference's prefill chunk
inline constexpr int kPrefillRows = 4096; // rows of one batched prefill launch sequence
inline constexpr int kMaxContext = 4096;  // Options::context upper bound
inline constexpr int kQDim = kQHeads * kHeadDim;    // 2048
inline constexpr int kKVDim = kKVHeads * kHeadDim;  // 1024
inline constexpr int kQKVRows = kQDim + 2 * kKVDim; // 4096
inline constexpr int kEosA = 151643, kEosB = 151645;

inline void require(bool ok, const std::string& message) {
    if (!ok) throw std::runtime_error(message);
}

}  // namespace qwen_hip
