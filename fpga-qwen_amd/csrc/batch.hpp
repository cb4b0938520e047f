// Batched decode of up to 8 sequences sharing the weights (no reference
// counterpart: the reference is single-stream; see batch.hip).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.hpp"

namespace qwen_hip {

// One sequence of a batched step.
struct BatchSeq {
    const LayerDevice* layers;  // [28]: shared weights, this sequence's K/V cache
    DecodeScratch s;            // this sequence's decode buffers
    int pos;                    // position being written
    int token;                  // id consumed at pos
    int context;                // K/V cache capacity
    ArgmaxResult* host_out;     // pinned slot for the greedy selection
    int shared_seq;             // batch index of the sequence whose K/V rows [0, shared) equal this one's
    int shared;                 // multiple of 64, at most pos (0: none)
};

// Exchange tags a batched step takes per layer (attention + O, FFN).
inline constexpr int kBatchTagsPerLayer = 2;

// One decode step for each sequence: 28 x (norm + QKV + attention + piece
// merge + O + residual in one launch, norm + gate/up + SwiGLU + down +
// residual in another), final norm + tied lm_head + per-sequence argmax.
// Logits, hidden and selections land in each sequence's buffers.
// tags[2 l], tags[2 l + 1] (nonzero, unique per launch) tag layer l's
// exchanges between workgroups, which use the first sequence's buffers.
// embed_mfma: the embedding in matrix-core order (launch_mfma_order).
void launch_decode_batch(const BatchSeq* seqs, int count, const uint16_t* embed, const uint16_t* embed_mfma,
                         const float* final_norm, const float* cosines, const float* sines, const uint32_t* tags,
                         hipStream_t stream);

// dst = W (natural [rows x K] FP16, rows % 16 == 0, K % BW == 0) in the
// order the batched kernels' matrix-core loads read it: each 16-row tile, per
// BW-column block and 32-column step, as 64 lanes x 16 bytes (one load of
// 1 KiB contiguous per wave).
void launch_mfma_order(const uint16_t* src, uint16_t* dst, int rows, int K, int BW, hipStream_t stream);
// The same for the batched FFN's gate / up tiles (12 rows each, 48 pieces
// per wave and step; natural [6144 x 1024] gate rows then up rows in).
void launch_gateup_order(const uint16_t* gateup, uint16_t* dst, hipStream_t stream);
inline constexpr size_t kGateupOrderHalves = size_t(256) * 2 * 8 * 4 * 48 * 8;

// Y[b] = W X[b] for b < batch on the matrix cores (W natural row-major
// [rows x cols] FP16, X [batch x cols] FP32, Y [batch x rows] FP32); rows a
// multiple of 16, cols in {1024, 2048, 3072}.
void launch_bgemv_plain(const uint16_t* w, const float* x, float* y, int batch, int rows, int cols,
                        hipStream_t stream);

}  // namespace qwen_hip
