// One launch per decode token: the 28 layers of a batch-1 step
// (engine/core.cpp:353-646 for one row) in a single persistent kernel.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.hpp"

namespace qwen_hip {

// The per-layer pointers the token kernel reads (per sequence: the weights
// are shared, the K/V cache is the sequence's own).
struct TokenLayer {
    const uint16_t* qkv_t;     // chain-tiled [4096 x 1024]
    const uint16_t* o_n;       // natural [1024 x 2048]
    const uint16_t* gateup_t;  // chain-tiled, gate / up interleaved 4 rows each
    const uint16_t* down_t;    // chain-tiled [1024 x 3072]
    const float* in_norm;      // [1024]
    const float* post_norm;    // [1024]
    const float* qk_norm;      // [256]: q norm, k norm
    uint16_t* keys;            // [8][context][128] chain-permuted key rows, then [8][context][128] value rows
};

// Exchange words of the token kernel (uint64: tag << 32 | FP32 bits): q/k/v
// rows [8][512], the split form's attention partials as plain FP32
// [8][32][2][130] (two per word) with one tagged flag per posting wave
// [8][32][4] (posted once the wave's partial floats are in the XCD's L2),
// O partials posted across
// XCDs [16 heads][1024 rows], the post-attention residual broadcast in each
// XCD [8][1024], activations [3072], down slices posted across XCDs
// [8 slices][1024 rows], the next layer's residual broadcast in each XCD
// [8][1024]. Posts across XCDs are laid out so that each workgroup writes
// whole contiguous lines (write-through stores of partial lines cost far
// more).
inline constexpr int kTokQkvOffset = 0;
inline constexpr int kTokPartOffset = kTokQkvOffset + kKVHeads * 512;
inline constexpr int kTokPartFlagOffset = kTokPartOffset + kKVHeads * 32 * 2 * (kHeadDim + 2) / 2;
inline constexpr int kTokOCrossOffset = kTokPartFlagOffset + kKVHeads * 32 * 4;
inline constexpr int kTokXmOffset = kTokOCrossOffset + kHidden * kQHeads;
inline constexpr int kTokActOffset = kTokXmOffset + 8 * kHidden;
inline constexpr int kTokDCrossOffset = kTokActOffset + kFFN;
inline constexpr int kTokXOffset = kTokDCrossOffset + kHidden * 8;
inline constexpr int kTokWords = kTokXOffset + 8 * kHidden;

// Poll limit of the token kernel's exchanges: ~0.1 s, far beyond the
// microseconds an exchange takes.
inline constexpr unsigned kTokenSpins = 1u << 18;

struct TokenLaunch {
    TokenLayer layers[kLayers];  // layers 0 .. layer_count - 1 (kernel arguments: read with scalar loads)
    int layer_count;
    const uint16_t* embed;     // natural embedding (layer 0 of row q starts from row token[q])
    int token[2];
    int rows;                  // 1, or 2: the rows of a verification at pos and pos + 1
    int pos;                   // position written by row 0 (n = pos + 1 cached positions)
    int context;
    const float* cosines;      // [4096][64]
    const float* sines;
    float* x_out;              // [rows][1024] residual after the last layer
    uint64_t* words;           // [rows][kTokWords] exchange words
    int* stall;                // raised when a poll gave up (cleared by the argmax kernel)
    float scale;               // 1 / sqrt(128), the attention score scale
    uint32_t tag;              // layer l uses tag + l (never 0, unique since the words were cleared)
    unsigned spins;            // poll limit (kTokenSpins)
    int withhold;              // workgroup that does not post its q/k/v rows in layer 0 (-1: none; tests)
    int prefetch;              // nonzero: load waves pull the next layer's K/V rows into L2
};

// True when the verification rows at pos and pos + 1 take the same
// attention form (which one launch of two rows requires).
bool token_pair_supported(int pos);

// Runs layers 0 .. layer_count - 1 of one decode row at position pos (or of
// the two verification rows at pos and pos + 1):
// 256 workgroups, one per CU (all resident together: the caller holds the
// GPU), workgroup w on XCD w % 8. Compute waves 0-7 keep the arithmetic of
// the fused QKV + attention and FFN kernels (bit-identical results); waves
// 8-11 stream each layer's weight tiles into LDS a layer ahead.
void launch_token_layers(const TokenLaunch& t, hipStream_t stream);

}  // namespace qwen_hip
