// Device-side data layout and kernel launchers of the decode engine.
//
// Chain-tiled matrix layout (for batch-1 GEMV). The reference dot product
// (engine/core.cpp:119-127) accumulates column j of a row into FP32 chain
// c = j % 8 with fused multiply-adds in ascending j, then combines
// ((c0+c4)+(c1+c5)) + ((c2+c6)+(c3+c7)). A GEMV thread owns one chain of one
// row. Rows are grouped in tiles of 8; within a tile, block b holds, for each
// thread t = 8*r + c, the 8 halves {W[8T+r][64b + 8i + c] : i = 0..7}
// contiguously (16 bytes). One wavefront therefore reads 1 KiB contiguous per
// 16-byte load, and each thread's halves arrive in its chain order.
//   tiled[(((T * NB) + b) * 64 + t) * 8 + i],  NB = cols / 64.
//
// KV cache: [layer][kv head][position][128] FP16 (engine/core.cpp:350-352).
// Key rows are stored chain-permuted: element j = 8s + c (chain c, step s of
// the reference dot) sits at kperm(j) = 64 (s / 8) + 8c + s % 8, so 16-byte
// piece c of the row holds steps 0..7 of chain c and piece c + 8 steps
// 8..15. The 8 threads scoring one position (thread c = chain c) read pieces
// c and c + 8: 128 contiguous bytes per load instruction and group. Value
// rows are stored in natural channel order.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "qwen_common.hpp"

namespace qwen_hip {

__host__ __device__ constexpr int kperm(int j) { return (j & ~63) | ((j & 7) << 3) | ((j >> 3) & 7); }

// Greedy selection result of the lm_head kernel.
struct ArgmaxResult {
    int token;
    int nonfinite;
    int stalled;  // a fused FFN launch of this step gave up waiting for an exchange
    int pad;
    // The step's result in one word, stored last by the argmax kernel at
    // system scope (host memory): seq << 32 | stalled << 31 | nonfinite << 30
    // | token. A host that sees its step's seq has the whole result.
    unsigned long long done;
};

inline constexpr int kAttnSplits = 32;          // max position splits per KV head
inline constexpr int kAttnTile = 128;           // positions per split
inline constexpr int kAttnPartial = 2 * 132;    // per split: 2 heads x (128 o + m + l + pad)

// Position splitting of decode attention over n = pos + 1 cached positions:
// 128 positions per split, up to 32 splits for a 4096 context.
__host__ __device__ inline void attn_split(int n, int& chunk, int& splits) {
    chunk = kAttnTile;
    splits = (n + kAttnTile - 1) / kAttnTile;
}

// Contexts of up to 512 positions take the fused attention + O-projection
// kernel: one workgroup per (query head, block of kAttnORows O rows) attends
// over all positions of the head (K/V rows are re-read from L2 by the 32
// workgroups of a KV head, which share an XCD), then multiplies the head's
// 128 attention outputs into its rows of O. Longer contexts split the
// positions (128 per split) and a merge kernel with the same workgroup
// layout combines the splits of its head and applies the same O rows. Either
// way the kOParts per-head partial sums of O.att land in o_part and are added
// to the residual stream by the gate/up prologue and the down epilogue, in a
// fixed order.
inline constexpr int kFusedMaxPositions = 512;
inline constexpr int kAttnORows = 64;
inline constexpr int kOParts = kQHeads;                                // 16 partial O projections
inline constexpr int kAttnOGroups = kQHeads * (kHidden / kAttnORows);  // 256 workgroups
__host__ __device__ inline bool attn_fused(int n) { return n <= kFusedMaxPositions; }

inline constexpr int kMaxBatch = 8;             // sequences per batched decode step
inline constexpr int kBatchRows = 16;           // output rows of one batched-GEMV MFMA tile
inline constexpr int kBatchLmGroups = 256;       // batched lm_head workgroups (one per CU)

inline constexpr int kLmStreamGroups = 256;     // single-sequence lm_head: one workgroup per CU
// Entries of the lm_head partial buffers: the batched head's groups x sequences.
inline constexpr int kLmPartials = kBatchLmGroups * kMaxBatch;
static_assert(kVocab % 8 == 0, "lm_head tiles of 8 rows must cover the vocabulary");

struct LayerDevice {
    const uint16_t* qkv_t;     // tiled [4096 x 1024]: q rows, k rows, v rows
    const uint16_t* o_n;       // natural [1024 x 2048] (attention + O kernels, batched decode)
    const uint16_t* qkv_n;     // natural [4096 x 1024] (batched decode)
    const uint16_t* gateup_n;  // natural [6144 x 1024]: gate rows then up rows (batched decode)
    const uint16_t* down_n;    // natural [1024 x 3072] (batched decode)
    const uint16_t* gateup_t;  // tiled [6144 x 1024]: tile T = gate rows 4T..4T+3, up rows 4T..4T+3
    const uint16_t* down_t;    // tiled [1024 x 3072]
    uint16_t* qkv_m;           // matrix-core orders (launch_mfma_order) for the batched step
    uint16_t* o_m;
    uint16_t* gateup_m;
    uint16_t* down_m;
    const float* in_norm;      // [1024]
    const float* post_norm;    // [1024]
    const float* q_norm;       // [128]
    const float* k_norm;       // [128]
    const float* qk_norm;      // [256]: q_norm then k_norm in one allocation (token kernel)
    uint16_t* keys;            // [8][context][128], chain-permuted rows
    uint16_t* values;          // [8][context][128]
};

struct DecodeScratch {
    float* x;             // [1024] residual stream
    float* qkv;           // [4096] raw projections
    float* attended;      // [2048] normalized attention output (split attention with one split)
    float* act;           // [3072]
    float* logits;        // [151936]
    float* hidden;        // [1024] final normalized hidden
    float* attn_partial;  // [8][kAttnSplits][kAttnPartial]: unnormalized o, max, sum per split
    float* o_part;        // [16][1024]: per-query-head partial O projections
    float* lm_value;      // [kLmPartials] argmax partials of the batched head: [kBatchLmGroups][kMaxBatch]
    int* lm_index;
    int* lm_bad;
    ArgmaxResult* result; // [1] device copy of the selection
    float* xm;            // [1024] residual after the O partials (written by the fused FFN kernel)
    float* dparts;        // [8][1024] down products of the 8 activation slices (fused FFN kernel)
    uint64_t* exchange;   // [3072] activations with their launch tag, exchanged inside each XCD
    int* stall;           // nonzero once an exchange poll gave up (cleared by the argmax kernel)
    uint64_t* xqkv;       // [8][512] q/k/v rows of each KV head group (fused QKV + attention kernel)
    uint64_t* xpart;      // [kXPartWords] attention partials of its workgroups
    uint64_t* bexchange;  // [kBatchExchangeWords] batched step exchanges (when this sequence leads a batch)
    uint64_t* lm_words;   // [2 rows][kLmStreamGroups][2] lm_head candidates (value, id | nonfinite) with the launch tag
};

// Exchange words of a batched step, in the first sequence's buffers. The
// attention launch uses q/k/v rows [8 KV heads][kMaxBatch][512], piece
// partials [8][32 workgroups][2 heads][130], merged rows [8][kMaxBatch][256]
// and O shares [1024][kMaxBatch][8 XCDs]; the FFN launch activations
// [8 XCDs][kMaxBatch][384] (over the q/k/v rows: another launch, another
// tag) and down shares (over the O shares).
inline constexpr int kBatchQkvWords = kKVHeads * kMaxBatch * 512;
inline constexpr int kBatchPieceWords = kKVHeads * 32 * 2 * (kHeadDim + 2);
inline constexpr int kBatchAttWords = kKVHeads * kMaxBatch * 256;
inline constexpr int kBatchShareWords = kHidden * kMaxBatch * 8;
inline constexpr int kBatchActWords = 8 * kMaxBatch * (kFFN / 8);
inline constexpr int kBatchPieceOffset = kBatchQkvWords;
inline constexpr int kBatchAttOffset = kBatchPieceOffset + kBatchPieceWords;
inline constexpr int kBatchShareOffset = kBatchAttOffset + kBatchAttWords;
inline constexpr int kBatchActOffset = 0;
static_assert(kBatchActWords <= kBatchQkvWords, "the FFN activations fit the q/k/v words");
inline constexpr int kBatchExchangeWords = kBatchShareOffset + kBatchShareWords;

// The fused FFN kernel (norm + gate/up + SwiGLU + down in one launch): XCD
// g computes activations 384 g .. 384 g + 383 and their share of the down
// product; the 8 shares are added by the next layer's QKV prologue.
inline constexpr int kFfnSlices = 8;
inline constexpr int kFfnSlice = kFFN / kFfnSlices;  // 384 activations per XCD
inline constexpr int kFfnGroups = 256;               // workgroups (32 per XCD)
// The fused QKV + attention + O kernel: exchange words for the q/k/v rows and
// for the (128 outputs, max, sum) partials of 2 heads x 32 workgroups x 8 KV heads.
inline constexpr int kXqkvWords = kKVHeads * 512;
inline constexpr int kXPartWords = kKVHeads * 32 * 2 * (kHeadDim + 2);

// Layout conversion: natural row-major FP16 [rows x cols] -> chain-tiled.
// When `second` is non-null the tiles interleave two matrices of equal shape:
// tile T holds rows 4T..4T+3 of `first` then rows 4T..4T+3 of `second`.
void launch_tile_matrix(const uint16_t* first, const uint16_t* second, uint16_t* dst, int rows, int cols,
                        hipStream_t stream);

// y[r] = dot(x, W[r]) with the reference chain order; W chain-tiled, cols in
// {1024, 2048, 3072}, rows a multiple of 8 * waves (waves = 2).
void launch_gemv_plain(const uint16_t* w_t, const float* x, float* y, int rows, int cols, hipStream_t stream);

// One decode layer: norm+QKV, attention (+q/k norm, RoPE, KV write) with the
// per-head O partials, norm+gate/up (+O partials, +SwiGLU), down (+O
// partials, +residual). With n = pos + 1 <= kFusedMaxPositions attention is
// one kernel (four kernels per layer), beyond it split attention + merge/O
// (five).
// pos is the position being written (n = pos + 1 cached positions after
// it); when `embed` is non-null (first layer) x is first loaded from
// embed[token]. Step scalars travel as kernel arguments.
// How a layer hands its residual stream on. fold_input: the previous layer
// ran the fused FFN kernel, so QKV reads s.xm plus the 8 down slices and
// writes their sum to s.x. ffn_tag != 0: this layer runs the fused FFN kernel
// (that tag must differ from the previous fused launch's on these buffers;
// after the last layer the caller folds s.xm and the slices into s.x);
// 0: the norm+gate/up and down kernels.
// attn_tag != 0: norm + QKV + attention + O run as one kernel with that
// tag; 0: the QKV and attention kernels.
struct LayerFlow {
    bool fold_input;
    uint32_t ffn_tag;
    uint32_t attn_tag;
};

void launch_decode_layer(const LayerDevice& layer, const uint16_t* embed, int pos, int token,
                         const float* cosines, const float* sines, int context, const DecodeScratch& s,
                         LayerFlow flow, hipStream_t stream);

// One stage of a decode layer: 0 norm+QKV (the fused QKV + attention + O
// kernel when flow.attn_tag != 0), 1 attention with the O partials (one
// kernel up to kFusedMaxPositions, split + merge/O beyond; nothing after a
// fused launch), 2 nothing (O runs with the attention), 3 norm+gate/up (the
// fused FFN kernel when flow.ffn_tag != 0), 4 down (nothing after a fused FFN
// launch).
void launch_layer_kernel(int which, const LayerDevice& layer, const uint16_t* embed, int pos, int token,
                         const float* cosines, const float* sines, int context, const DecodeScratch& s,
                         LayerFlow flow, hipStream_t stream);

// Buffers of a two-token verification (rows at positions pos and pos + 1).
struct PairScratch {
    float* x;             // [2][1024] residual streams after the last layer
    float* logits;        // [2][151936]
    float* hidden;        // [2][1024]
    ArgmaxResult* result; // [2] device copies of the selections
};

// Final norm + lm_head + greedy selection of both verification rows in one
// launch (each weight block read once for both; candidate words of s);
// selections to pair.result and host_out[0..1], each with its result word.
void launch_lm_head_pair(const uint16_t* lm_t, const float* final_norm, const DecodeScratch& s,
                         const PairScratch& pair, ArgmaxResult* host_out, uint32_t tag, hipStream_t stream,
                         unsigned seq);

// One sequence of a batched norm + QKV + attention + O launch.
struct AttnSeq {
    const float* x;          // residual stream the layer starts from
    const uint16_t* embed;   // first layer: the token's embedding row (the residual is then fp32 of it), else null
    float* x_out;            // residual after the O projection (a buffer other than x)
    uint16_t* keys;          // this layer's cache [8][context][128]
    uint16_t* values;
    int pos;                 // position being written
    int context;
    // Rows [0, shared) hold the same values in this cache and in the cache at
    // shared_keys / shared_values (capacity shared_context), which the other
    // sequences of the batch with that copy read too, so the rows come from
    // HBM once per batch. shared is a multiple of 64 and at most pos.
    const uint16_t* shared_keys;
    const uint16_t* shared_values;
    int shared_context;
    int shared;
};

// Pieces per (sequence, KV head) of a batched attention launch over
// sequences with `positions` cached rows (the one being written included):
// returns the grid's pieces per sequence (one workgroup per CU), sets `per`
// (the most 64-position blocks a piece holds; each sequence's blocks are
// shared evenly by the pieces) and pieces_out[i] (pieces of sequence i that
// hold positions; the partials the merge reads).
int attn_batch_pieces(const int* positions, int count, int* pieces_out, int& per);

// RMSNorm + QKV projection + decode attention + O projection + residual of
// one layer for up to kMaxBatch sequences in one launch (256 workgroups).
// words: the batched exchange buffer (kBatchExchangeWords), used under `tag`
// (nonzero, unique per launch); stall is set if a workgroup gave up waiting.
void launch_attention_o_batch(const AttnSeq* seqs, int count, const uint16_t* w_qkv, const uint16_t* w_o,
                              const float* in_norm, const float* q_norm, const float* k_norm, const float* cosines,
                              const float* sines, uint64_t* words, int* stall, uint32_t tag, hipStream_t stream);

// The batch-1 decode projections of one layer as the step runs them, on
// caller buffers (parity-test entries):
// qkv[4096] = W_qkv . RMSNorm(x) (norm prologue, one chain-ordered dot per row);
void launch_norm_qkv(const uint16_t* qkv_t, const float* norm_w, const float* x, float* qkv, hipStream_t stream);
// act[3072] = SwiGLU(W_gate . h, W_up . h) with h = RMSNorm(x + the 16 pending
// O partials folded in their fixed tree order; none when parts is null),
// W chain-tiled with gate / up rows interleaved 4 by 4; raw (optional,
// [6144]) receives the dot products in that interleaved row order;
void launch_norm_gate_up(const uint16_t* gateup_t, const float* norm_w, const float* x, const float* parts,
                         float* act, float* raw, hipStream_t stream);
// x[r] = (x[r] + folded O partials of row r) + W_down[r] . act (two-segment chains).
void launch_down_residual(const uint16_t* down_t, const float* act, const float* parts, float* x,
                          hipStream_t stream);
// The fused FFN kernel of one layer: xm = x + folded O partials (parts
// [16][1024]), act = SwiGLU(gate/up . RMSNorm(xm)) posted to exchange[3072]
// with `tag`, dparts[g][r] = W_down[r][384 g .. 384 g + 383] . act[same]
// (8-chain dot over the slice). The exchange must hold no word with `tag`
// (zeroed, or last written with another tag); stall is set if a poll gave up.
void launch_fused_ffn(const uint16_t* gateup_t, const uint16_t* down_t, const float* norm_w, const float* x,
                      const float* parts, float* xm, float* dparts, uint64_t* exchange, int* stall, uint32_t tag,
                      hipStream_t stream);
// x[q] = xm[q] + the 8 down slices dparts[q][8][1024] (fixed tree order), q < rows (1 or 2).
void launch_fold_residual(const float* xm, const float* dparts, float* x, int rows, hipStream_t stream);
// qkv = W_qkv . RMSNorm(x) with x = xm + the 8 down slices dparts[8][1024]
// added in the fixed tree order; x is also written out.
void launch_norm_qkv_folded(const uint16_t* qkv_t, const float* norm_w, const float* xm, const float* dparts,
                            float* x, float* qkv, hipStream_t stream);

// Plain device copy (bytes a multiple of 16), for counter calibration.
void launch_copy(const void* src, void* dst, size_t bytes, hipStream_t stream);

// Final norm + tied lm_head GEMV + greedy argmax (lowest id on ties,
// nonfinite flagged). Also writes the final hidden vector; the selection
// goes to s.result and to `host_out` (pinned host memory).
void launch_lm_head(const uint16_t* lm_t, const float* final_norm, const DecodeScratch& s, ArgmaxResult* host_out,
                    uint32_t tag, hipStream_t stream, unsigned seq = 0);

}  // namespace qwen_hip
