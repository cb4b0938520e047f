// Batch-1 decode kernels for gfx950 (CDNA4, wave64).
//
// GEMV: each thread owns one FP32 chain of one row (see kernels.hpp for the
// chain-tiled layout), so every projection output is bit-identical to the
// reference dot (engine/core.cpp:119-147). Weights stream from HBM as
// 16-byte loads, 1 KiB contiguous per wave instruction; the input vector sits
// in LDS, permuted so each thread reads its 8 activations as two float4.
// Prologues fuse the RMSNorm (engine/core.cpp:207-215: FP32 squares summed in
// FP64), epilogues fuse the residual add (626, 641), SwiGLU (636-639) and the
// greedy argmax (engine/main.cpp:51-59).
//
// Attention: up to 512 cached positions, one kernel fuses attention with the
// O projection (attn_o_kernel); beyond that, flash-decoding over splits of
// 128 positions (attn_split_body) whose (max, sum, output) partials a small
// merge kernel combines in fixed split order, so results do not depend on
// scheduling. Each workgroup owns one KV head (both GQA query heads 2g, 2g+1
// share every K/V row it loads); the one holding the current position also
// applies QK-norm + RoPE to k and writes K/V (FP16, round-to-nearest-even)
// into the cache (engine/core.cpp:395-406), and all use them from LDS.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <climits>
#include <type_traits>

#include "decode_dev.hpp"
#include "kernels.hpp"

namespace qwen_hip {
namespace {

using namespace dev;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Residual stream entry x + the 16 per-query-head partial O projections of
// the fused attention kernel, summed in a fixed tree order (every kernel
// that reads the entry gets the same value).
__device__ __forceinline__ float fold_parts(float x, const float (&p)[kOParts]) {
    const float lo = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    const float hi = ((p[8] + p[9]) + (p[10] + p[11])) + ((p[12] + p[13]) + (p[14] + p[15]));
    return x + (lo + hi);
}

// Residual stream entry xm + the 8 per-slice down products of the fused FFN
// kernel, summed in a fixed tree order.
__device__ __forceinline__ float fold_slices(float xm, const float (&d)[kFfnSlices]) {
    return xm + (((d[0] + d[1]) + (d[2] + d[3])) + ((d[4] + d[5]) + (d[6] + d[7])));
}

// Weights of one 8-row tile for this lane: NB 16-byte blocks. Issued right
// after the (small) prologue inputs, so the HBM round trip overlaps the
// prologue.
template <int N>
__device__ __forceinline__ void load_tile(const uint16_t* __restrict__ w_t, size_t tile, int lane, u32x4 (&wv)[N / 64]) {
    constexpr int NB = N / 64;
    const u32x4* wp = reinterpret_cast<const u32x4*>(w_t) + tile * (NB * 64) + lane;
#pragma unroll
    for (int b = 0; b < NB; ++b) wv[b] = __builtin_nontemporal_load(wp + b * 64);
}

// Chain dot of the loaded tile against the permuted LDS vector.
template <int N>
__device__ __forceinline__ float tile_dot(const u32x4 (&wv)[N / 64], const float* xs, int lane) {
    constexpr int NB = N / 64;
    const float4* xs4 = reinterpret_cast<const float4*>(xs);
    const int c = lane & 7;
    float acc = 0.f;
#pragma unroll
    for (int b = 0; b < NB; ++b) acc = chain8(acc, wv[b], xs4[16 * b + 2 * c], xs4[16 * b + 2 * c + 1]);
    return combine_chains(acc);
}

enum GemvMode { kPlain, kQKV, kGateUp, kDown };

// With ROWS input vectors (two-token verification), row q of each per-row
// buffer starts q strides in: in + q N, x / hidden + q 1024, parts +
// q 16384, out + q out_stride.
struct GemvArgs {
    const uint16_t* w;        // chain-tiled weights
    const float* in;          // input vector (plain; O: attention output; down), residual x (norm modes)
    const float* norm_w;      // RMSNorm weights (QKV, gate/up, lm_head)
    const uint16_t* embed;    // natural embedding, first layer only (QKV)
    const float* parts;       // gate/up, down: pending [16][1024] per-head O partials, or null
    int token[2];             // first-layer QKV: embedding row of each input row
    int out_stride;           // ROWS > 1: distance between the rows' outputs
    float* out;               // plain/QKV: y; gate/up: activation; lm_head: logits
    float* x;                 // residual stream (O/down add, first-layer QKV store)
    float* hidden;            // lm_head: final normalized hidden
    float* lm_value;
    int* lm_index;
    int* lm_bad;
    float* raw;               // gate/up, optional: the dot products in tile row order (parity tests)
};

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

// PARTS (gate/up, down): the residual stream still has the fused attention
// kernel's 16 partial O projections pending in a.parts. PARTS with QKV: the
// input is the previous layer's s.xm and a.parts holds its 8 down slices;
// the folded residual is the norm's input and is written to a.x (workgroup
// b writes entries 4b .. 4b + 3, so a grid of 256 covers all 1024).
// ROWS input vectors share every weight load: lane (row, chain) keeps one
// chain per input with the same FMA order, so each row's result is the one
// a single-row launch gives.
template <int N, int WAVES, int MODE, bool PARTS = false, int ROWS = 1>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(const GemvArgs a) {
    constexpr int THREADS = WAVES * 64, PER = N / THREADS;
    constexpr bool kNorm = MODE == kQKV || MODE == kGateUp;
    __shared__ float4 xs4[ROWS][N / 4];
    __shared__ double red[ROWS][WAVES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t tile = size_t(blockIdx.x) * WAVES + wave;
    const int c = lane & 7, r = lane >> 3;
    const int row = int(tile) * 8 + r;

    // Every load of the prologue and epilogue is issued before the weights:
    // loads complete in issue order, so one issued after the weight tile
    // would wait for all of it. The normalized inputs (QKV, gate/up,
    // lm_head) are held PER consecutive values per thread (j = PER tid + k)
    // and loaded 16 bytes at a time; the others as j = tid + k THREADS.
    constexpr bool kContig = kNorm && PER % 4 == 0;
    static_assert(MODE != kQKV || kContig, "the embedding row is read as consecutive pairs");
    const int jbase = kContig ? PER * tid : tid;
    constexpr int kStride = kContig ? 1 : THREADS;
    auto load_f = [&](const float* src, float (&dst)[PER]) {
        if constexpr (kContig) {
#pragma unroll
            for (int k = 0; k < PER; k += 4) {
                const float4 f = *reinterpret_cast<const float4*>(src + jbase + k);
                dst[k] = f.x; dst[k + 1] = f.y; dst[k + 2] = f.z; dst[k + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < PER; ++k) dst[k] = src[jbase + k * kStride];
        }
    };
    float v[ROWS][PER], wn[PER];
#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        if constexpr (MODE == kQKV) {
            if (a.embed) {  // first layer: x = fp32(E[token]) (engine/core.cpp:382-383)
                const uint16_t* erow = a.embed + size_t(a.token[q]) * N + jbase;
#pragma unroll
                for (int k = 0; k < PER; k += 2) {
                    const uint32_t pair = *reinterpret_cast<const uint32_t*>(erow + k);
                    v[q][k] = h2f(pair & 0xffffu);
                    v[q][k + 1] = h2f(pair >> 16);
                }
            } else {
                load_f(a.in + q * N, v[q]);
            }
        } else {
            load_f(a.in + q * N, v[q]);
        }
    }
    if constexpr (kNorm) load_f(a.norm_w, wn);
    // Pending O partials: of this thread's inputs (gate/up) or of this
    // lane's output row (down).
    float pin[ROWS][kOParts][PARTS && MODE == kGateUp ? PER : 1], prow[ROWS][kOParts];
    if constexpr (PARTS && MODE == kGateUp) {
#pragma unroll
        for (int q = 0; q < ROWS; ++q)
#pragma unroll
            for (int g = 0; g < kOParts; ++g) load_f(a.parts + (q * kOParts + g) * kHidden, pin[q][g]);
    }
    float dsl[ROWS][kFfnSlices][PARTS && MODE == kQKV ? PER : 1];
    if constexpr (PARTS && MODE == kQKV) {
        static_assert(PER == 8 && kContig, "QKV folds 8 consecutive entries per thread");
#pragma unroll
        for (int q = 0; q < ROWS; ++q)
#pragma unroll
            for (int g = 0; g < kFfnSlices; ++g) load_f(a.parts + (q * kFfnSlices + g) * kHidden, dsl[q][g]);
    }
    float xres[ROWS];  // residual entry of this lane's row (O, down)
#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        xres[q] = 0.f;
        if constexpr (MODE == kDown) xres[q] = a.x[q * kHidden + row];
        if constexpr (PARTS && MODE == kDown) {
#pragma unroll
            for (int g = 0; g < kOParts; ++g) prow[q][g] = a.parts[(q * kOParts + g) * kHidden + row];
        }
    }

    // The scheduling barriers keep the weight loads after the prologue loads
    // and ahead of every instruction that waits for those.
    u32x4 wv[N / 64];
    __builtin_amdgcn_sched_barrier(0);
    load_tile<N>(a.w, tile, lane, wv);
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        float* xs = reinterpret_cast<float*>(xs4[q]);
        if constexpr (PARTS && MODE == kGateUp) {
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                float pk[kOParts];
#pragma unroll
                for (int g = 0; g < kOParts; ++g) pk[g] = pin[q][g][k];
                v[q][k] = fold_parts(v[q][k], pk);
            }
        }
        if constexpr (PARTS && MODE == kDown) xres[q] = fold_parts(xres[q], prow[q]);
        if constexpr (PARTS && MODE == kQKV) {
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                float dk[kFfnSlices];
#pragma unroll
                for (int g = 0; g < kFfnSlices; ++g) dk[g] = dsl[q][g][k];
                v[q][k] = fold_slices(v[q][k], dk);
            }
            if (tid == int(blockIdx.x >> 1)) {
                const int h = 4 * (blockIdx.x & 1);
                *reinterpret_cast<float4*>(a.x + q * kHidden + jbase + h) =
                    make_float4(v[q][h], v[q][h + 1], v[q][h + 2], v[q][h + 3]);
            }
        }
        if constexpr (kNorm) {
            if constexpr (MODE == kQKV) {
                if (a.embed && blockIdx.x == 0) {  // kept as the residual stream
#pragma unroll
                    for (int k = 0; k < PER; ++k) a.x[q * kHidden + jbase + k * kStride] = v[q][k];
                }
            }
            norm_to_lds<N, THREADS, kContig>(v[q], wn, xs, red[q],
                                             nullptr);
        } else {
#pragma unroll
            for (int k = 0; k < PER; ++k) xs[xperm(jbase + k * kStride)] = v[q][k];
        }
    }
    __syncthreads();

    float y[ROWS];
#pragma unroll
    for (int q = 0; q < ROWS; ++q) y[q] = tile_dot<N>(wv, reinterpret_cast<const float*>(xs4[q]), lane);

#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        float* out = a.out + size_t(q) * a.out_stride;
        if constexpr (MODE == kPlain || MODE == kQKV) {
            if (c == 0) out[row] = y[q];
        } else if constexpr (MODE == kDown) {
            if (c == 0) a.x[q * kHidden + row] = xres[q] + y[q];
        } else if constexpr (MODE == kGateUp) {
            // Tile rows 0-3 are gate rows 4T..4T+3, rows 4-7 the matching up rows.
            if (a.raw && c == 0) a.raw[size_t(q) * a.out_stride * 2 + row] = y[q];
            const float up = __shfl(y[q], (lane + 32) & 63);
            if (lane < 32 && c == 0) {
                const float gate = y[q];
                const float half_gate = gate * 0.5f;
                const float t = tanhf(half_gate);
                out[int(tile) * 4 + r] = gate * (0.5f + 0.5f * t) * up;
            }
        }
    }
}

// Long-row GEMV (O: 2048 columns, down: 3072) with each chain split into
// SEG consecutive segments of its blocks. A workgroup covers half a tile
// (4 rows x 8 chains = 32 lanes per segment); segment s sits in wave s / 2,
// lanes 32 (s % 2) .. +31. Every lane loads only its segment's blocks, so
// twice (SEG = 2) or four times (SEG = 4, two waves) as many lanes stream
// the matrix as in gemv_kernel, spread over twice the workgroups. The
// running sum moves from segment to segment (lane l -> l + 32 inside a
// wave, through LDS between waves), so each chain performs exactly the
// reference's FMA sequence and the result equals gemv_kernel's bit for bit.
template <int N, int SEG, int MODE, bool PARTS = false>
__global__ __launch_bounds__(SEG * 32) void gemv_seg_kernel(const GemvArgs a) {
    static_assert(SEG == 2 || SEG == 4, "segments: 2 or 4");
    static_assert(MODE == kPlain || MODE == kDown, "long-row modes only");
    constexpr int THREADS = SEG * 32, WAVES = SEG / 2, PER = N / THREADS, NB = N / 64, NBS = NB / SEG;
    static_assert(NB % SEG == 0, "segments must split the blocks evenly");
    __shared__ float4 xs4[N / 4];
    __shared__ float hand[32];
    float* xs = reinterpret_cast<float*>(xs4);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = blockIdx.x >> 1, half = blockIdx.x & 1;
    const int l32 = lane & 31, c = l32 & 7, r = l32 >> 3;
    const int seg = 2 * wave + (lane >> 5);
    const int row = tile * 8 + 4 * half + r;

    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) v[k] = a.in[tid + k * THREADS];
    float xres = 0.f, prow[kOParts];
    if constexpr (MODE == kDown) xres = a.x[row];
    if constexpr (PARTS) {
#pragma unroll
        for (int g = 0; g < kOParts; ++g) prow[g] = a.parts[g * kHidden + row];
    }
    u32x4 wv[NBS];
    __builtin_amdgcn_sched_barrier(0);
    {
        const u32x4* wp = reinterpret_cast<const u32x4*>(a.w) + (size_t(tile) * NB + size_t(seg) * NBS) * 64 +
                          32 * half + l32;
#pragma unroll
        for (int b = 0; b < NBS; ++b) wv[b] = __builtin_nontemporal_load(wp + b * 64);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PARTS) xres = fold_parts(xres, prow);
#pragma unroll
    for (int k = 0; k < PER; ++k) xs[xperm(tid + k * THREADS)] = v[k];
    __syncthreads();

    // Phase p of wave w runs segment 2w + p: the lanes of that segment hold
    // the true running sum, the other half of the wave computes a discarded
    // value with the same instructions.
    const float4* x4 = xs4 + 16 * (seg * NBS) + 2 * c;
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
        if (wave == w) {
            if (w > 0) acc = hand[l32];
#pragma unroll
            for (int b = 0; b < NBS; ++b) acc = chain8(acc, wv[b], x4[16 * b], x4[16 * b + 1]);
            acc = __shfl_xor(acc, 32);  // lower half's sum to the upper half
#pragma unroll
            for (int b = 0; b < NBS; ++b) acc = chain8(acc, wv[b], x4[16 * b], x4[16 * b + 1]);
            if (w + 1 < WAVES && lane >= 32) hand[l32] = acc;
        }
        if (w + 1 < WAVES) __syncthreads();
    }
    if (wave == WAVES - 1) {
        const float y = combine_chains(acc);
        if (lane >= 32 && c == 0) {
            if constexpr (MODE == kPlain) a.out[row] = y;
            else a.x[row] = xres + y;
        }
    }
}

struct FfnArgs {
    const uint16_t* gateup_t;  // chain-tiled gate/up, rows interleaved 4 by 4
    const uint16_t* down_t;    // chain-tiled down [1024 x 3072]
    const float* x;            // residual stream before the O partials [ROWS][1024]
    const float* norm_w;       // post-attention RMSNorm weights
    const float* parts;        // [ROWS][16][1024] per-query-head O partials
    float* xm;                 // out: x + folded O partials [ROWS][1024]
    float* dparts;             // out: [ROWS][8][1024] down products of the 8 activation slices
    uint64_t* exchange;        // [ROWS][3072] tagged activations
    int* stall;
    uint32_t tag;
};

// Norm + gate/up + SwiGLU + down of one layer in one launch (batch-1
// decode, engine/core.cpp:627-641). 256 workgroups x 4 waves. Slice g =
// blockIdx % 8 (one XCD) owns activations 384 g .. 384 g + 383; its 32
// workgroups (slot s = blockIdx / 8)
// compute gate/up tiles 96 g + 3 s + w (waves w = 0..2; tile T yields
// activations 4T..4T+3, wave 3 repeats wave 2's tile and discards it), post
// the activations to the exchange, and each then multiplies down tiles
// 4 s + w (rows 32 s + 8 w .. + 7, every wave) over the slice's 384
// columns. Every gate/up row is the reference's chain-ordered dot
// (bit-identical to the norm+gate/up kernel); the down row r of slice g is
// the 8-chain dot over those 384 columns, and the next layer's QKV prologue
// adds the 8 slices in a fixed tree order. Workgroup b also writes entries
// 4b .. 4b + 3 of x + O partials to xm (the residual the slices are added
// to). The down weights are issued before the exchange is polled, so their
// round trip overlaps the wait.
template <int ROWS>
__global__ __launch_bounds__(256) void ffn_kernel(const FfnArgs a) {
    constexpr int THREADS = 256, PER = kHidden / THREADS;
    constexpr int kSliceBlocks = kFfnSlice / 64, kDownBlocks = kFFN / 64;
    static_assert(PER == 4 && kSliceBlocks == 6 && kFfnGroups == 256, "fused FFN shape");
    __shared__ float4 xs4[ROWS][kHidden / 4];
    __shared__ float4 as4[ROWS][kFfnSlice / 4];
    __shared__ double red[ROWS][THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 7, r = lane >> 3;
    // Slice g = blockIdx % 8: the 32 workgroups of a slice share an XCD.
    const int g = int(blockIdx.x & 7), slot = int(blockIdx.x >> 3);
    const int gu_tile = 96 * g + 3 * slot + min(wave, 2);
    const int down_tile = 4 * slot + wave;
    const int jbase = PER * tid;

    float v[ROWS][PER], wn[PER], pin[ROWS][kOParts][PER];
    auto load4 = [&](const float* src, float (&dst)[PER]) {
        const float4 f = *reinterpret_cast<const float4*>(src + jbase);
        dst[0] = f.x; dst[1] = f.y; dst[2] = f.z; dst[3] = f.w;
    };
#pragma unroll
    for (int q = 0; q < ROWS; ++q) load4(a.x + q * kHidden, v[q]);
    load4(a.norm_w, wn);
#pragma unroll
    for (int q = 0; q < ROWS; ++q)
#pragma unroll
        for (int h = 0; h < kOParts; ++h) load4(a.parts + (q * kOParts + h) * kHidden, pin[q][h]);

    u32x4 wv[kHidden / 64];
    __builtin_amdgcn_sched_barrier(0);
    load_tile<kHidden>(a.gateup_t, size_t(gu_tile), lane, wv);
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            float pk[kOParts];
#pragma unroll
            for (int h = 0; h < kOParts; ++h) pk[h] = pin[q][h][k];
            v[q][k] = fold_parts(v[q][k], pk);
        }
        if (tid == int(blockIdx.x))
            *reinterpret_cast<float4*>(a.xm + q * kHidden + jbase) = make_float4(v[q][0], v[q][1], v[q][2], v[q][3]);
        norm_to_lds<kHidden, THREADS, true>(v[q], wn, reinterpret_cast<float*>(xs4[q]), red[q], nullptr);
    }
    __syncthreads();

    // The down weights of this wave's tile over the slice's 6 column blocks.
    u32x4 dw[kSliceBlocks];
    __builtin_amdgcn_sched_barrier(0);
    {
        const u32x4* dp = reinterpret_cast<const u32x4*>(a.down_t) +
                          (size_t(down_tile) * kDownBlocks + size_t(kSliceBlocks) * g) * 64 + lane;
#pragma unroll
        for (int b = 0; b < kSliceBlocks; ++b) dw[b] = __builtin_nontemporal_load(dp + b * 64);
    }
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        const float y = tile_dot<kHidden>(wv, reinterpret_cast<const float*>(xs4[q]), lane);
        // Tile rows 0-3 are gate rows 4T..4T+3, rows 4-7 the matching up rows.
        const float up = __shfl(y, (lane + 32) & 63);
        if (wave < 3 && lane < 32 && c == 0) {
            const float gate = y;
            const float half_gate = gate * 0.5f;
            const float t = tanhf(half_gate);
            exchange_put(a.exchange + q * kFFN + 4 * gu_tile + r, gate * (0.5f + 0.5f * t) * up, a.tag);
        }
    }

    // This XCD's 384 activations (two per thread of waves 0-2), permuted for
    // the chain reads like the GEMV inputs.
    bool ok = true;
    if (tid < kFfnSlice / 2) {
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            float a0 = 0.f, a1 = 0.f;
            if (ok) ok = exchange_get2(a.exchange + q * kFFN + kFfnSlice * g + 2 * tid, a.tag, a0, a1);
            float* as = reinterpret_cast<float*>(as4[q]);
            as[xperm(2 * tid)] = a0;
            as[xperm(2 * tid + 1)] = a1;
        }
    }
    if (!ok) *a.stall = 1;
    __syncthreads();

#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        const float4* as = as4[q];
        float acc = 0.f;
#pragma unroll
        for (int b = 0; b < kSliceBlocks; ++b) acc = chain8(acc, dw[b], as[16 * b + 2 * c], as[16 * b + 2 * c + 1]);
        const float y = combine_chains(acc);
        if (c == 0) a.dparts[(q * kFfnSlices + g) * kHidden + 8 * down_tile + r] = y;
    }
}

struct AttnArgs {
    const float* qkv;      // raw projections [4096]
    const float* q_norm;   // [128]
    const float* k_norm;   // [128]
    const float* cosines;  // [context][64]
    const float* sines;
    uint16_t* keys;        // layer base [8][context][128]
    uint16_t* values;
    int pos;               // position being written
    float* partial;        // [8][kAttnSplits][kAttnPartial]
    float* attended;       // [2048], written instead when there is one split
    const uint16_t* o_n;   // fused: natural O weights [1024 x 2048]
    float* o_part;         // fused: [16][1024] partial O projections
    int context;
    float scale;           // 1.0f / sqrt(128.0f)
};

// One workgroup = one KV head g (GQA query heads 2g, 2g+1) x one split of
// up to kAttnTile = 128 positions (2 passes of 64), with the lane layout of
// the fused kernel: the 8 lanes of position t score it (lane c = chain c of
// the reference dot, engine/core.cpp:612) and multiply its V row by both
// probabilities. The split's maximum (per head, over the 8 waves' maxima)
// is shared through LDS first, so every probability is exp(s - max of the
// split); each wave sums its positions' probabilities and P.V products
// (the four position groups of a wave folded in registers), and the 8
// waves' sums are added in LDS in a fixed tree. A single split writes the normalized output; several write (output, max,
// sum) partials that the merge kernels combine. Every load is issued up
// front and unconditionally (positions outside the split read row 0 and are
// masked), in the order the phases need them.
__device__ __forceinline__ void attn_split_body(const AttnArgs& a, int s, int g) {
    constexpr int kPasses = kAttnTile / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos = a.pos, n = pos + 1;
    int chunk, ns;
    attn_split(n, chunk, ns);
    if (s >= ns) return;  // the grid covers the largest split count of a batch
    const int t_begin = s * chunk, t_end = min(n, t_begin + chunk);
    const size_t head_base = size_t(g) * a.context;
    const int quarter = tid >> 7, j = tid & 127, c = tid & 7, grp = tid >> 3;
    const int vsub = lane >> 4, vcg = lane & 15;

    const float raw = quarter < 2 ? a.qkv[(2 * g + quarter) * 128 + j] : a.qkv[2048 + g * 128 + j];
    const float raw_v = a.qkv[3072 + g * 128 + j];
    // quarter is uniform per wave; selecting the pointer on a scalar keeps it
    // out of vector registers (no per-lane load of the kernel argument).
    const float nw = (__builtin_amdgcn_readfirstlane(quarter) < 2 ? a.q_norm : a.k_norm)[j];
    const float rc = a.cosines[size_t(pos) * 64 + (j & 63)], rs = a.sines[size_t(pos) * 64 + (j & 63)];
    u32x4 kreg[kPasses][2], vreg[kPasses][2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        const int t = t_begin + p * 64 + grp;
        const int tl = t < t_end && t != pos ? t : 0;
        key_pieces(a.keys + (head_base + tl) * 128, c, kreg[p][0], kreg[p][1]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < kPasses; ++p)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const int t = t_begin + p * 64 + 8 * wave + 4 * hf + vsub;
            const int tl = t < t_end && t != pos ? t : 0;
            vreg[p][hf] = reinterpret_cast<const u32x4*>(a.values + (head_base + tl) * 128)[vcg];
        }
    __builtin_amdgcn_sched_barrier(0);

    __shared__ float qp[2][128];
    __shared__ float buf[4][128];
    __shared__ float prob[2][kAttnTile];
    __shared__ __align__(16) float opart[8][2][128];
    __shared__ uint16_t kcur[128], vcur[128];
    __shared__ double red[4][2];
    __shared__ float wmax[8][2], wsum[8][2];

    // QK-norm + RoPE (engine/core.cpp:395-402); the split holding pos writes
    // the new K/V row (403-406) and every split reads only rows t != pos.
    {
        const float r = head_norm_rope(raw, nw, rc, rs, red[quarter], buf[quarter], j);
        const bool owner = s == ns - 1;
        if (quarter < 2) {
            qp[quarter][kperm(j)] = r;
        } else if (quarter == 2) {
            const uint16_t bits = f2h(r);
            kcur[kperm(j)] = bits;
            if (owner) a.keys[(head_base + pos) * 128 + kperm(j)] = bits;
        } else {
            const uint16_t bits = f2h(raw_v);
            vcur[j] = bits;
            if (owner) a.values[(head_base + pos) * 128 + j] = bits;
        }
    }
    __syncthreads();

    float s0[kPasses], s1[kPasses];
    float m0 = -INFINITY, m1 = -INFINITY;
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        const int t = t_begin + p * 64 + grp;
        uint32_t kw[8];
        if (t == pos) {
            key_pieces_lds(kcur, c, kw);
        } else {
            kw[0] = kreg[p][0].x; kw[1] = kreg[p][0].y; kw[2] = kreg[p][0].z; kw[3] = kreg[p][0].w;
            kw[4] = kreg[p][1].x; kw[5] = kreg[p][1].y; kw[6] = kreg[p][1].z; kw[7] = kreg[p][1].w;
        }
        const float d0 = combine_chains(key_chain(qp[0], c, kw, 0.f)) * a.scale;
        const float d1 = combine_chains(key_chain(qp[1], c, kw, 0.f)) * a.scale;
        s0[p] = t < t_end ? d0 : -INFINITY;
        s1[p] = t < t_end ? d1 : -INFINITY;
        m0 = fmaxf(m0, s0[p]);
        m1 = fmaxf(m1, s1[p]);
    }
    m0 = fmaxf(m0, xor_lanes<8>(m0));
    m1 = fmaxf(m1, xor_lanes<8>(m1));
    m0 = fmaxf(m0, xor_lanes<16>(m0));
    m1 = fmaxf(m1, xor_lanes<16>(m1));
    m0 = fmaxf(m0, xor_lanes<32>(m0));
    m1 = fmaxf(m1, xor_lanes<32>(m1));
    // One maximum per head for the whole split: every probability is taken
    // relative to it, so the waves' partial sums add without rescaling.
    if (lane == 0) {
        wmax[wave][0] = m0;
        wmax[wave][1] = m1;
    }
    __syncthreads();
    m0 = wmax[0][0];
    m1 = wmax[0][1];
#pragma unroll
    for (int w = 1; w < 8; ++w) {
        m0 = fmaxf(m0, wmax[w][0]);
        m1 = fmaxf(m1, wmax[w][1]);
    }
    float l0 = 0.f, l1 = 0.f;
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        const int t = t_begin + p * 64 + grp;
        const float p0 = t < t_end ? expf(s0[p] - m0) : 0.f;
        const float p1 = t < t_end ? expf(s1[p] - m1) : 0.f;
        l0 += p0;
        l1 += p1;
        if (c == 0) {
            prob[0][p * 64 + grp] = p0;
            prob[1][p * 64 + grp] = p1;
        }
    }
    l0 += xor_lanes<8>(l0);
    l1 += xor_lanes<8>(l1);
    l0 += xor_lanes<16>(l0);
    l1 += xor_lanes<16>(l1);
    l0 += xor_lanes<32>(l0);
    l1 += xor_lanes<32>(l1);
    // prob[][] of this wave's positions is written and read by this wave only.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    float acc[2][8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[0][i] = acc[1][i] = 0.f;
#pragma unroll
    for (int p = 0; p < kPasses; ++p)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const int tl = p * 64 + 8 * wave + 4 * hf + vsub, t = t_begin + tl;
            if (t < t_end) {
                const float p0 = prob[0][tl], p1 = prob[1][tl];
                uint32_t vw[4];
                if (t == pos) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        vw[i] = uint32_t(vcur[vcg * 8 + 2 * i]) | (uint32_t(vcur[vcg * 8 + 2 * i + 1]) << 16);
                } else {
                    vw[0] = vreg[p][hf].x; vw[1] = vreg[p][hf].y; vw[2] = vreg[p][hf].z; vw[3] = vreg[p][hf].w;
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float v0 = h2f(vw[i] & 0xffffu), v1 = h2f(vw[i] >> 16);
                    acc[0][2 * i] = __builtin_fmaf(v0, p0, acc[0][2 * i]);
                    acc[0][2 * i + 1] = __builtin_fmaf(v1, p0, acc[0][2 * i + 1]);
                    acc[1][2 * i] = __builtin_fmaf(v0, p1, acc[1][2 * i]);
                    acc[1][2 * i + 1] = __builtin_fmaf(v1, p1, acc[1][2 * i + 1]);
                }
            }
        }
    // The wave's four position groups (lanes vcg + 16 vsub) hold partial sums
    // of the same channels: fold them in registers, then one group writes the
    // wave's 2 x 128 outputs.
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            acc[h][i] += xor_lanes<16>(acc[h][i]);
            acc[h][i] += xor_lanes<32>(acc[h][i]);
        }
    if (vsub == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 8; i += 4)
                *reinterpret_cast<float4*>(&opart[wave][h][vcg * 8 + i]) =
                    make_float4(acc[h][i], acc[h][i + 1], acc[h][i + 2], acc[h][i + 3]);
    }
    if (lane == 0) {
        wsum[wave][0] = l0;
        wsum[wave][1] = l1;
    }
    __syncthreads();
    if (tid < 256) {
        const int h = tid >> 7;
        const float o = ((opart[0][h][j] + opart[1][h][j]) + (opart[2][h][j] + opart[3][h][j])) +
                        ((opart[4][h][j] + opart[5][h][j]) + (opart[6][h][j] + opart[7][h][j]));
        const float l = ((wsum[0][h] + wsum[1][h]) + (wsum[2][h] + wsum[3][h])) +
                        ((wsum[4][h] + wsum[5][h]) + (wsum[6][h] + wsum[7][h]));
        const float mx = h ? m1 : m0;
        if (ns == 1) {  // nothing to merge: normalize here
            a.attended[(2 * g + h) * 128 + j] = o / l;
            return;
        }
        float* part = a.partial + (size_t(g) * kAttnSplits + s) * kAttnPartial + h * 132;
        part[j] = o;
        if (j == 0) {
            part[128] = mx;
            part[129] = l;
        }
    }
}

__global__ __launch_bounds__(512) void attn_decode_kernel(const AttnArgs a) {
    attn_split_body(a, blockIdx.x, blockIdx.y);
}

// Merge of the position splits of one query head (flash-decoding, fixed
// split order): o = sum_s w_s o_s / sum_s w_s l_s with w_s = exp(m_s - max).
// One split: attention already wrote the normalized output.
// 512 threads: group q = tid / 128 merges splits 8q .. 8q + 7 against its own
// maximum (thread j = channel j), then the 4 group results are combined with
// weights exp(m_q - max): the same sums, reassociated in a fixed order. Each
// wave loads 8 splits' entries (a wave retires only about 10 GB/s of loads,
// so they are spread over 8 waves), all issued up front (entries past ns
// read split 0 and are skipped).
constexpr int kMergeGroups = 4, kMergePer = kAttnSplits / kMergeGroups;
static_assert(kAttnSplits % kMergeGroups == 0, "merge groups split the splits evenly");
// The merged row goes to out[0..127]; after_loads() runs right after the
// split entries are issued (the fused O kernel issues its weights there).
template <class AfterLoads>
__device__ __forceinline__ void attn_merge_body(const AttnArgs& a, int head, float* out, AfterLoads&& after_loads) {
    const int tid = threadIdx.x, j = tid & 127, grp = tid >> 7;
    int chunk, ns;
    attn_split(a.pos + 1, chunk, ns);
    if (ns == 1) return;
    const float* base = a.partial + size_t(head >> 1) * kAttnSplits * kAttnPartial + (head & 1) * 132;
    float mv[kMergePer], lv[kMergePer], ov[kMergePer];
#pragma unroll
    for (int k = 0; k < kMergePer; ++k) {
        const int sidx = grp * kMergePer + k;
        const float* e = base + (sidx < ns ? sidx : 0) * kAttnPartial;
        mv[k] = e[128];
        lv[k] = e[129];
        ov[k] = e[j];
    }
    after_loads();
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < kMergePer; ++k)
        if (grp * kMergePer + k < ns) mx = fmaxf(mx, mv[k]);
    float l = 0.f, o = 0.f;
#pragma unroll
    for (int k = 0; k < kMergePer; ++k)
        if (grp * kMergePer + k < ns) {
            const float w = expf(mv[k] - mx);
            l += w * lv[k];
            o += w * ov[k];
        }
    __shared__ float gm[kMergeGroups], gl[kMergeGroups], go[kMergeGroups][128];
    if (j == 0) {
        gm[grp] = mx;
        gl[grp] = l;
    }
    go[grp][j] = o;
    __syncthreads();
    if (grp == 0) {
        float m2 = gm[0];
#pragma unroll
        for (int q = 1; q < kMergeGroups; ++q) m2 = fmaxf(m2, gm[q]);
        float lt = 0.f, ot = 0.f;
#pragma unroll
        for (int q = 0; q < kMergeGroups; ++q)
            if (gm[q] != -INFINITY) {  // a group without splits adds nothing
                const float w = expf(gm[q] - m2);
                lt += w * gl[q];
                ot += w * go[q][j];
            }
        out[j] = ot / lt;
    }
}

// Past kFusedMaxPositions: the merge of query head h's position splits fused
// with that head's share of the O projection, laid out as the tail of
// attn_o_kernel. Workgroup blockIdx = 8m + g: h = 2g + m % 2, O rows
// kAttnORows (m / 2) .. + kAttnORows - 1; o_part[h][row] = sum_i
// O[row][128h + i] att[i], folded into the residual stream by the gate/up
// prologue and the down epilogue like the fused kernel's partials.
__global__ __launch_bounds__(512) void attn_merge_o_kernel(const AttnArgs a) {
    const int g = blockIdx.x % kKVHeads, m = blockIdx.x / kKVHeads;
    const int h = 2 * g + (m & 1), rb = m >> 1;
    const int tid = threadIdx.x;
    constexpr int kThreadsPerRow = 512 / kAttnORows, kLoads = 128 / 8 / kThreadsPerRow;
    const int orow = rb * kAttnORows + tid / kThreadsPerRow, opart_id = tid % kThreadsPerRow;
    __shared__ __align__(16) float att[128];
    u32x4 ow[kLoads];
    attn_merge_body(a, h, att, [&] {
        __builtin_amdgcn_sched_barrier(0);
        const u32x4* op = reinterpret_cast<const u32x4*>(a.o_n + size_t(orow) * kQDim + 128 * h) + opart_id;
#pragma unroll
        for (int i = 0; i < kLoads; ++i) ow[i] = __builtin_nontemporal_load(op + kThreadsPerRow * i);
        __builtin_amdgcn_sched_barrier(0);
    });
    __syncthreads();
    float y = 0.f;
    const float4* at4 = reinterpret_cast<const float4*>(att) + 2 * opart_id;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) y = chain8(y, ow[i], at4[2 * kThreadsPerRow * i], at4[2 * kThreadsPerRow * i + 1]);
    static_assert(kThreadsPerRow == 8, "three lane exchanges");
    y += xor_lanes<1>(y);
    y += xor_lanes<2>(y);
    y += xor_lanes<4>(y);
    if (opart_id == 0) a.o_part[h * kHidden + orow] = y;
}

// Fused attention + O projection for n <= kFusedMaxPositions. Workgroup
// blockIdx = 8m + g: KV head g (so the 32 workgroups reading one head's K/V
// rows share an XCD and its L2 copy of them), query head h = 2g + m % 2,
// block rb = m / 2 of kAttnORows O rows. Every workgroup computes its query
// head's attention over all n positions (scores in the reference dot's chain
// order, engine/core.cpp:612; softmax and P.V as in 613-620), then its rows
// of O against the head's 128 attention outputs:
// o_part[h][row] = sum_i O[row][128h + i] * att[i].
// 512 threads, PASSES = ceil(n / 64) passes of 64 positions (a template
// parameter so that every load is unconditional and the compiler waits for
// exactly the loads each phase needs). Wave w owns positions 64p + 8w + i,
// i < 8: its lanes 8i..8i+7 score position i (lane c = chain c); the head's
// maximum over all positions is shared through LDS, then each wave sums the
// probabilities exp(s - max) and P.V products of its positions (4 positions
// x 16 channel groups per load, the 4 position groups folded in registers),
// and the 8 waves' sums are added in LDS in a fixed tree.
// ROWS = 2 (two-token verification): row q is the step at position pos + q
// and attends over its pos + q + 1 positions; both rows share every K/V and
// O load, row 1 takes position pos (row 0's new K/V) from LDS, and each
// row's arithmetic is the single-row kernel's (extra masked positions add
// exact zeros), so its output equals a single-row launch at its position.
template <int PASSES, int ROWS = 1>
__global__ __launch_bounds__(512) void attn_o_kernel(const AttnArgs a) {
    const int g = blockIdx.x % kKVHeads, m = blockIdx.x / kKVHeads;
    const int h = 2 * g + (m & 1), rb = m >> 1;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos = a.pos;
    const size_t head_base = size_t(g) * a.context;
    // Threads 0-127: q of head h, 128-255: k, 256-383: v (384-511 repeat v
    // and write nothing).
    const int quarter = tid >> 7, j = tid & 127, c = tid & 7, grp = tid >> 3;
    const int vsub = lane >> 4, vcg = lane & 15;  // P.V: position within a group of 4, channel group

    // Loads complete in issue order per wave, so they are issued in the
    // order they are needed: this step's q/k/v with their norm weights and
    // rotation, cached K rows, V rows, then this workgroup's O weights. Rows
    // from pos on (taken from LDS) or past them load row 0 instead and are
    // not used.
    float raw[ROWS], rc[ROWS], rs[ROWS];
    const int src = quarter == 0 ? h * 128 + j : (quarter == 1 ? 2048 : 3072) + g * 128 + j;
#pragma unroll
    for (int q = 0; q < ROWS; ++q) raw[q] = a.qkv[q * kQKVRows + src];
    // quarter is uniform per wave; selecting the pointer on a scalar keeps it
    // out of vector registers (no per-lane load of the kernel argument).
    const float nw = (__builtin_amdgcn_readfirstlane(quarter) == 0 ? a.q_norm : a.k_norm)[j];
#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        rc[q] = a.cosines[size_t(pos + q) * 64 + (j & 63)];
        rs[q] = a.sines[size_t(pos + q) * 64 + (j & 63)];
    }
    u32x4 kreg[PASSES][2], vreg[PASSES][2];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int t = p * 64 + grp;
        const int tl = t < pos ? t : 0;
        key_pieces(a.keys + (head_base + tl) * 128, c, kreg[p][0], kreg[p][1]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const int t = p * 64 + 8 * wave + 4 * hf + vsub;
            const int tl = t < pos ? t : 0;
            vreg[p][hf] = reinterpret_cast<const u32x4*>(a.values + (head_base + tl) * 128)[vcg];
        }
    __builtin_amdgcn_sched_barrier(0);
    // O rows: kThreadsPerRow threads per row; load i of thread part q holds
    // the 8 columns 8 (q + kThreadsPerRow i) .. +7 of the head's 128, so the
    // lanes of one row read consecutive 16-byte pieces.
    constexpr int kThreadsPerRow = 512 / kAttnORows, kLoads = 128 / 8 / kThreadsPerRow;
    const int orow = rb * kAttnORows + tid / kThreadsPerRow, opart_id = tid % kThreadsPerRow;
    u32x4 ow[kLoads];
    {
        const u32x4* op = reinterpret_cast<const u32x4*>(a.o_n + size_t(orow) * kQDim + 128 * h) + opart_id;
#pragma unroll
        for (int i = 0; i < kLoads; ++i) ow[i] = __builtin_nontemporal_load(op + kThreadsPerRow * i);
    }
    __builtin_amdgcn_sched_barrier(0);

    __shared__ float qp[ROWS][128];
    __shared__ float buf[ROWS][4][128];
    __shared__ float prob[ROWS][kFusedMaxPositions];
    __shared__ __align__(16) float opart[ROWS][8][128];
    __shared__ __align__(16) float att[ROWS][128];
    __shared__ uint16_t kcur[ROWS][128], vcur[ROWS][128];
    __shared__ double red[ROWS][4][2];
    __shared__ float wmax[ROWS][8], wsum[ROWS][8];

    // QK-norm + RoPE (engine/core.cpp:395-402); one workgroup per KV head
    // (m == 0) writes the new K/V rows (403-406). The others only read rows
    // t < pos.
    const bool owner = m == 0;
#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        const float r = head_norm_rope(raw[q], nw, rc[q], rs[q], red[q][quarter], buf[q][quarter], j);
        if (quarter == 0) {
            qp[q][kperm(j)] = r;
        } else if (quarter == 1) {
            const uint16_t bits = f2h(r);
            kcur[q][kperm(j)] = bits;
            if (owner) a.keys[(head_base + pos + q) * 128 + kperm(j)] = bits;
        } else if (quarter == 2) {
            const uint16_t bits = f2h(raw[q]);
            vcur[q][j] = bits;
            if (owner) a.values[(head_base + pos + q) * 128 + j] = bits;
        }
    }
    __syncthreads();

#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        const int n = pos + q + 1;
        // Scores of this wave's positions (every lane of a position's group
        // of 8 holds the combined value) and the wave's running maximum.
        float s0[PASSES];
        float m0 = -INFINITY;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int t = p * 64 + grp, cur = t - pos;
            uint32_t kw[8];
            if (cur >= 0 && cur <= q) {
                key_pieces_lds(kcur[cur], c, kw);
            } else {
                kw[0] = kreg[p][0].x; kw[1] = kreg[p][0].y; kw[2] = kreg[p][0].z; kw[3] = kreg[p][0].w;
                kw[4] = kreg[p][1].x; kw[5] = kreg[p][1].y; kw[6] = kreg[p][1].z; kw[7] = kreg[p][1].w;
            }
            const float d0 = combine_chains(key_chain(qp[q], c, kw, 0.f)) * a.scale;
            s0[p] = t < n ? d0 : -INFINITY;
            m0 = fmaxf(m0, s0[p]);
        }
        m0 = fmaxf(m0, xor_lanes<8>(m0));
        m0 = fmaxf(m0, xor_lanes<16>(m0));
        m0 = fmaxf(m0, xor_lanes<32>(m0));
        // The head's maximum over all positions (the 8 waves' maxima through
        // LDS): every probability is exp(s - max), so the waves' partial sums
        // add without rescaling.
        if (lane == 0) wmax[q][wave] = m0;
        __syncthreads();
        m0 = wmax[q][0];
#pragma unroll
        for (int w = 1; w < 8; ++w) m0 = fmaxf(m0, wmax[q][w]);
        float l0 = 0.f;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int t = p * 64 + grp;
            const float p0 = t < n ? expf(s0[p] - m0) : 0.f;
            l0 += p0;
            if (c == 0) prob[q][t] = p0;
        }
        l0 += xor_lanes<8>(l0);
        l0 += xor_lanes<16>(l0);
        l0 += xor_lanes<32>(l0);
        // prob[q][t] of this wave's positions is written and read by this
        // wave only.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.f;
#pragma unroll
        for (int p = 0; p < PASSES; ++p)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const int t = p * 64 + 8 * wave + 4 * hf + vsub, cur = t - pos;
                if (t < n) {
                    const float p0 = prob[q][t];
                    uint32_t vw[4];
                    if (cur >= 0) {  // cur <= q here since t < n
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            vw[i] = uint32_t(vcur[cur][vcg * 8 + 2 * i]) |
                                    (uint32_t(vcur[cur][vcg * 8 + 2 * i + 1]) << 16);
                    } else {
                        vw[0] = vreg[p][hf].x; vw[1] = vreg[p][hf].y; vw[2] = vreg[p][hf].z; vw[3] = vreg[p][hf].w;
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        acc[2 * i] = __builtin_fmaf(h2f(vw[i] & 0xffffu), p0, acc[2 * i]);
                        acc[2 * i + 1] = __builtin_fmaf(h2f(vw[i] >> 16), p0, acc[2 * i + 1]);
                    }
                }
            }
        // The wave's four position groups (lanes vcg + 16 vsub) hold partial
        // sums of the same channels: fold them in registers; one group writes.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            acc[i] += xor_lanes<16>(acc[i]);
            acc[i] += xor_lanes<32>(acc[i]);
        }
        if (vsub == 0) {
            *reinterpret_cast<float4*>(&opart[q][wave][vcg * 8]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
            *reinterpret_cast<float4*>(&opart[q][wave][vcg * 8 + 4]) = make_float4(acc[4], acc[5], acc[6], acc[7]);
        }
        if (lane == 0) wsum[q][wave] = l0;
    }
    __syncthreads();
    if (tid < 128 * ROWS) {  // the 8 waves' sums in a fixed tree
        const int q = tid >> 7, ch = tid & 127;
        const float o = ((opart[q][0][ch] + opart[q][1][ch]) + (opart[q][2][ch] + opart[q][3][ch])) +
                        ((opart[q][4][ch] + opart[q][5][ch]) + (opart[q][6][ch] + opart[q][7][ch]));
        const float l = ((wsum[q][0] + wsum[q][1]) + (wsum[q][2] + wsum[q][3])) +
                        ((wsum[q][4] + wsum[q][5]) + (wsum[q][6] + wsum[q][7]));
        att[q][ch] = o / l;
    }
    __syncthreads();

    // This workgroup's rows of O against the head's 128 attention outputs.
#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        float y = 0.f;
        const float4* at4 = reinterpret_cast<const float4*>(att[q]) + 2 * opart_id;
#pragma unroll
        for (int i = 0; i < kLoads; ++i)
            y = chain8(y, ow[i], at4[2 * kThreadsPerRow * i], at4[2 * kThreadsPerRow * i + 1]);
        static_assert(kThreadsPerRow == 8, "three lane exchanges");
        y += xor_lanes<1>(y);
        y += xor_lanes<2>(y);
        y += xor_lanes<4>(y);
        if (opart_id == 0) a.o_part[(q * kOParts + h) * kHidden + orow] = y;
    }
}

// Contexts of up to this many 64-position passes take the fused kernel's
// FULL form (every workgroup attends its head over all positions).
constexpr int kFullAttnPasses = 4;

// Words per attention partial in the exchange: 128 outputs, max, sum.
constexpr int kXPart = kHeadDim + 2;

struct QkvAttnArgs {
    const uint16_t* qkv_t;   // chain-tiled [4096 x 1024]: q rows, k rows, v rows
    const float* in_norm;    // input RMSNorm weights
    const float* x;          // residual the layer starts from (when neither embed nor dparts)
    const float* xm;         // with dparts: the previous fused FFN's residual
    const float* dparts;     // [8][1024] down slices of the previous layer, or null
    const uint16_t* embed;   // first layer: natural embedding, or null
    int token;
    float* x_out;            // with embed or dparts: the residual, written here
    const float* q_norm;
    const float* k_norm;
    const float* cosines;
    const float* sines;
    uint16_t* keys;          // layer base [8][context][128] (keys chain-permuted)
    uint16_t* values;
    int pos;
    int context;
    float scale;
    const uint16_t* o_n;     // natural O weights [1024 x 2048]
    float* o_part;           // [16][1024] per-query-head partial O projections
    uint64_t* xqkv;          // [8][512] tagged q/k/v rows of each KV head group
    uint64_t* xpart;         // [8][32][2][kXPart] tagged attention partials
    int* stall;
    uint32_t tag;
};

// Norm + QKV + attention + O of one decode layer in one launch, for every
// context length. 256 workgroups x 8 waves; KV head g = blockIdx % 8 (one
// XCD) with slot s = blockIdx / 8:
// 1. RMSNorm of the residual (engine/core.cpp:384; the previous layer's 8
//    down slices added first when it ran the fused FFN), then waves 0-1 run
//    QKV tiles 2s and 2s + 1 of head group g (its 512 rows: q heads 2g and
//    2g + 1, k head g, v head g; the reference's chain-ordered dot per row)
//    and post the rows to the XCD's exchange.
// 2. Every workgroup takes the 512 rows, applies QK-norm and RoPE
//    (395-402) and attends (606-624) over its 64-position passes s and
//    s + 32 with the lane layout of the split kernel (one maximum per head
//    over the workgroup, the 8 waves' sums added in a fixed tree); the pass
//    holding pos writes the new K/V row (403-406). Each active workgroup
//    posts its (output, max, sum) partials for both query heads.
// 3. Workgroup (g, s) merges query head h = 2g + s % 2 over the partials of
//    workgroups 0 .. min(32, passes) - 1 in a fixed order (4 groups of 8
//    against their own maximum, then combined) and multiplies the result
//    into O rows 64 (s / 2) .. + 63: o_part[h][row] = O[row][128h ..] . att.
// Every wave issues the same loads (QKV weights, K/V rows of its passes,
// O weights) at the start, so their round trips overlap the norm, the QKV
// dots and both exchanges, and the compiler's waits stay exact. QKV tile
// t = wave % 2 is split into 4 segments of 4 column blocks (wave / 2): the
// segments run in turn, each continuing the chains of the previous one
// (handed over through LDS), so each row is the reference's FMA sequence.
// PASSES = 2 once a context needs more than 32 passes (n > 2048); SRC:
// 0 residual x, 1 embedding row (first layer), 2 xm + down slices.
// FULL (short contexts, PASSES = passes of the whole context): instead of
// steps 2-3, workgroup (g, s) attends query head h = 2g + s % 2 over all n
// positions itself (K/V rows re-read from the XCD's L2 by its 16
// workgroups) and multiplies the result into its O rows: no partials to
// exchange.
template <int PASSES, int SRC, bool FULL>
__global__ __launch_bounds__(512) void qkv_attn_kernel(const QkvAttnArgs a) {
    constexpr int PER = 4, kSegBlocks = kHidden / 64 / 4;  // waves 0-3 hold 4 residual entries per thread
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = int(blockIdx.x & 7), s = int(blockIdx.x >> 3);
    const int pos = a.pos, n = pos + 1, npasses = (n + 63) >> 6;
    const int active = min(npasses, 32);  // workgroups with positions (split form)
    const bool mine = FULL || s < active;
    const int j = tid & 127, c = tid & 7, grp = tid >> 3;
    const int vsub = lane >> 4, vcg = lane & 15;
    const size_t head_base = size_t(g) * a.context;
    // Local QKV tile li of the head group: q tiles 32g + li (li < 32), k
    // tiles 256 + 16g + li - 32, v tiles 384 + 16g + li - 48.
    const int ti = wave & 1, seg = wave >> 1;
    const int li = 2 * s + ti;
    const int qkv_tile = li < 32 ? 32 * g + li : li < 48 ? 256 + 16 * g + (li - 32) : 384 + 16 * g + (li - 48);
    // O rows of phase 3.
    const int hq = s & 1, h = 2 * g + hq, rb = s >> 1;
    constexpr int kThreadsPerRow = 512 / kAttnORows, kOLoads = kHeadDim / 8 / kThreadsPerRow;
    const int orow = rb * kAttnORows + tid / kThreadsPerRow, opart_id = tid % kThreadsPerRow;
    const int jbase = PER * tid;
    const bool holds = wave < 4;  // wave-uniform: waves 0-3 load and normalize the residual

    // Loads in the order they are needed.
    float v[PER], wn[PER], dsl[kFfnSlices][PER];
    if (holds) {
        auto load4 = [&](const float* src, float (&dst)[PER]) {
            const float4 f = *reinterpret_cast<const float4*>(src + jbase);
            dst[0] = f.x; dst[1] = f.y; dst[2] = f.z; dst[3] = f.w;
        };
        if constexpr (SRC == 1) {
            const uint2 e = *reinterpret_cast<const uint2*>(a.embed + size_t(a.token) * kHidden + jbase);
            v[0] = h2f(e.x & 0xffffu);
            v[1] = h2f(e.x >> 16);
            v[2] = h2f(e.y & 0xffffu);
            v[3] = h2f(e.y >> 16);
        } else {
            load4(SRC == 2 ? a.xm : a.x, v);
            if constexpr (SRC == 2) {
#pragma unroll
                for (int k = 0; k < kFfnSlices; ++k) load4(a.dparts + k * kHidden, dsl[k]);
            }
        }
        load4(a.in_norm, wn);
    }
    // QK-norm weights and rotation of this lane's channel pair (lane, lane +
    // 64): waves 0-1 the query heads, wave 2 the key head.
    const float* hw = __builtin_amdgcn_readfirstlane(wave) == 2 ? a.k_norm : a.q_norm;
    const float nw0 = hw[lane], nw1 = hw[lane + 64];
    const float rc = a.cosines[size_t(pos) * 64 + lane], rs = a.sines[size_t(pos) * 64 + lane];
    u32x4 wv[kSegBlocks];
    __builtin_amdgcn_sched_barrier(0);
    {
        const u32x4* wp = reinterpret_cast<const u32x4*>(a.qkv_t) + (size_t(qkv_tile) * (kHidden / 64) +
                                                                     size_t(kSegBlocks) * seg) * 64 + lane;
#pragma unroll
        for (int b = 0; b < kSegBlocks; ++b) wv[b] = __builtin_nontemporal_load(wp + b * 64);
    }
    __builtin_amdgcn_sched_barrier(0);
    // K/V rows of this workgroup's passes (positions past n, the current
    // one, and all of an inactive workgroup's read row 0 and are unused).
    // Pass p covers positions 64 (s + 32 p) .. + 63 (split form) or
    // 64 p .. + 63 (FULL).
    auto pass_base = [&](int p) { return FULL ? 64 * p : 64 * (s + 32 * p); };
    u32x4 kreg[PASSES][2], vreg[PASSES][2];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int t = pass_base(p) + grp;
        const int tl = mine && t < n && t != pos ? t : 0;
        key_pieces(a.keys + (head_base + tl) * 128, c, kreg[p][0], kreg[p][1]);
    }
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const int t = pass_base(p) + 8 * wave + 4 * hf + vsub;
            const int tl = mine && t < n && t != pos ? t : 0;
            vreg[p][hf] = reinterpret_cast<const u32x4*>(a.values + (head_base + tl) * 128)[vcg];
        }
    __builtin_amdgcn_sched_barrier(0);
    u32x4 ow[kOLoads];
    {
        const u32x4* op = reinterpret_cast<const u32x4*>(a.o_n + size_t(orow) * kQDim + 128 * h) + opart_id;
#pragma unroll
        for (int i = 0; i < kOLoads; ++i) ow[i] = __builtin_nontemporal_load(op + kThreadsPerRow * i);
    }
    __builtin_amdgcn_sched_barrier(0);

    __shared__ float4 xs4[kHidden / 4];
    __shared__ double red4[4];
    __shared__ float qp[2][128];
    __shared__ float prob[FULL ? 1 : 2][64 * PASSES];
    __shared__ __align__(16) float opart[8][FULL ? 1 : 2][128];
    __shared__ uint16_t kcur[128], vcur[128];
    __shared__ float wmax[8][2], wsum[8][2];
    __shared__ float gm[4], gl[4], go[4][128];
    __shared__ __align__(16) float att[128];
    __shared__ float hand[2][64];

    // 1. Residual (engine/core.cpp:207-215: FP32 squares summed in FP64),
    // then the QKV rows of the head group.
    if (holds) {
        if constexpr (SRC == 2) {
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                float dk[kFfnSlices];
#pragma unroll
                for (int z = 0; z < kFfnSlices; ++z) dk[z] = dsl[z][k];
                v[k] = fold_slices(v[k], dk);
            }
        }
        if (SRC != 0 && tid == int(blockIdx.x))  // workgroup b writes entries 4b .. 4b + 3
            *reinterpret_cast<float4*>(a.x_out + jbase) = make_float4(v[0], v[1], v[2], v[3]);
        double part = 0.0;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const float square = v[k] * v[k];
            part += static_cast<double>(square);
        }
        part = wave_sum(part);
        if (lane == 0) red4[wave] = part;
    }
    __syncthreads();
    if (holds) {
        const float sum = static_cast<float>(((red4[0] + red4[1]) + red4[2]) + red4[3]);
        const float inv = 1.0f / __builtin_sqrtf(sum / static_cast<float>(kHidden) + 1e-6f);
        float* xs = reinterpret_cast<float*>(xs4);
#pragma unroll
        for (int k = 0; k < PER; ++k) xs[xperm(jbase + k)] = (v[k] * inv) * wn[k];
    }
    __syncthreads();
    {
        float acc = 0.f;
        const float4* x4 = xs4 + 16 * (kSegBlocks * seg) + 2 * c;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (seg == k) {
                if (k > 0) acc = hand[ti][lane];
#pragma unroll
                for (int b = 0; b < kSegBlocks; ++b) acc = chain8(acc, wv[b], x4[16 * b], x4[16 * b + 1]);
                if (k < 3) {
                    hand[ti][lane] = acc;
                } else {
                    const float y = combine_chains(acc);
                    if (c == 0) exchange_put(a.xqkv + g * 512 + 8 * li + (lane >> 3), y, a.tag);
                }
            }
            if (k < 3) __syncthreads();
        }
    }
    // 2. Wave w < 4 takes head-group rows 128 w + lane and 128 w + 64 + lane
    // (q0, q1, k, v): QK-norm (engine/core.cpp:397-398) and rotate-half RoPE
    // (216-218) of the pair inside the wave; the pass holding pos writes the
    // new K/V row (403-406).
    bool ok = true;
    if (holds) {
        const uint64_t* const words[2] = {a.xqkv + g * 512 + 128 * wave + lane, a.xqkv + g * 512 + 128 * wave + 64 + lane};
        float got[2] = {0.f, 0.f};
        ok = exchange_gather<2>(words, a.tag, got, 3u);
        const float x0 = got[0], x1 = got[1];
        const bool owner = ((pos >> 6) & 31) == s;
        if (wave < 3) {
            const float sq0 = x0 * x0, sq1 = x1 * x1;
            const double lo = wave_sum(static_cast<double>(sq0)), hi = wave_sum(static_cast<double>(sq1));
            const float sum = static_cast<float>(lo + hi);
            const float inv = 1.0f / __builtin_sqrtf(sum / 128.0f + 1e-6f);
            const float n0 = (x0 * inv) * nw0, n1 = (x1 * inv) * nw1;
            const float r0 = n0 * rc - n1 * rs, r1 = n1 * rc + n0 * rs;
            if (wave < 2) {
                qp[wave][kperm(lane)] = r0;
                qp[wave][kperm(lane + 64)] = r1;
            } else {
                const uint16_t b0 = f2h(r0), b1 = f2h(r1);
                kcur[kperm(lane)] = b0;
                kcur[kperm(lane + 64)] = b1;
                if (owner) {
                    a.keys[(head_base + pos) * 128 + kperm(lane)] = b0;
                    a.keys[(head_base + pos) * 128 + kperm(lane + 64)] = b1;
                }
            }
        } else {
            const uint16_t b0 = f2h(x0), b1 = f2h(x1);
            vcur[lane] = b0;
            vcur[lane + 64] = b1;
            if (owner) {
                a.values[(head_base + pos) * 128 + lane] = b0;
                a.values[(head_base + pos) * 128 + lane + 64] = b1;
            }
        }
    }
    __syncthreads();

    if constexpr (FULL) {
        // Query head hq over all positions (engine/core.cpp:606-624): one
        // maximum for the head through LDS, then each wave's probabilities and
        // P.V of its positions, the 8 waves' sums added in a fixed tree.
        float s0[PASSES];
        float m0 = -INFINITY;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int t = 64 * p + grp;
            uint32_t kw[8];
            if (t == pos) {
                key_pieces_lds(kcur, c, kw);
            } else {
                kw[0] = kreg[p][0].x; kw[1] = kreg[p][0].y; kw[2] = kreg[p][0].z; kw[3] = kreg[p][0].w;
                kw[4] = kreg[p][1].x; kw[5] = kreg[p][1].y; kw[6] = kreg[p][1].z; kw[7] = kreg[p][1].w;
            }
            const float d0 = combine_chains(key_chain(qp[hq], c, kw, 0.f)) * a.scale;
            s0[p] = t < n ? d0 : -INFINITY;
            m0 = fmaxf(m0, s0[p]);
        }
        m0 = fmaxf(m0, xor_lanes<8>(m0));
        m0 = fmaxf(m0, xor_lanes<16>(m0));
        m0 = fmaxf(m0, xor_lanes<32>(m0));
        if (lane == 0) wmax[wave][0] = m0;
        __syncthreads();
        m0 = wmax[0][0];
#pragma unroll
        for (int w = 1; w < 8; ++w) m0 = fmaxf(m0, wmax[w][0]);
        float l0 = 0.f;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int t = 64 * p + grp;
            const float p0 = t < n ? expf(s0[p] - m0) : 0.f;
            l0 += p0;
            if (c == 0) prob[0][t] = p0;
        }
        l0 += xor_lanes<8>(l0);
        l0 += xor_lanes<16>(l0);
        l0 += xor_lanes<32>(l0);
        // prob[0][t] of this wave's positions is written and read by this wave only.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.f;
#pragma unroll
        for (int p = 0; p < PASSES; ++p)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const int t = 64 * p + 8 * wave + 4 * hf + vsub;
                if (t < n) {
                    const float p0 = prob[0][t];
                    uint32_t vw[4];
                    if (t == pos) {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            vw[i] = uint32_t(vcur[vcg * 8 + 2 * i]) | (uint32_t(vcur[vcg * 8 + 2 * i + 1]) << 16);
                    } else {
                        vw[0] = vreg[p][hf].x; vw[1] = vreg[p][hf].y; vw[2] = vreg[p][hf].z; vw[3] = vreg[p][hf].w;
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        acc[2 * i] = __builtin_fmaf(h2f(vw[i] & 0xffffu), p0, acc[2 * i]);
                        acc[2 * i + 1] = __builtin_fmaf(h2f(vw[i] >> 16), p0, acc[2 * i + 1]);
                    }
                }
            }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            acc[i] += xor_lanes<16>(acc[i]);
            acc[i] += xor_lanes<32>(acc[i]);
        }
        if (vsub == 0) {
            *reinterpret_cast<float4*>(&opart[wave][0][vcg * 8]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
            *reinterpret_cast<float4*>(&opart[wave][0][vcg * 8 + 4]) = make_float4(acc[4], acc[5], acc[6], acc[7]);
        }
        if (lane == 0) wsum[wave][0] = l0;
        if (!ok) *a.stall = 1;
        __syncthreads();
        if (tid < 128) {
            const float o = ((opart[0][0][tid] + opart[1][0][tid]) + (opart[2][0][tid] + opart[3][0][tid])) +
                            ((opart[4][0][tid] + opart[5][0][tid]) + (opart[6][0][tid] + opart[7][0][tid]));
            const float l = ((wsum[0][0] + wsum[1][0]) + (wsum[2][0] + wsum[3][0])) +
                            ((wsum[4][0] + wsum[5][0]) + (wsum[6][0] + wsum[7][0]));
            att[tid] = o / l;
        }
    } else {
    if (mine) {
        float s0[PASSES], s1[PASSES];
        float m0 = -INFINITY, m1 = -INFINITY;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int t = 64 * (s + 32 * p) + grp;
            uint32_t kw[8];
            if (t == pos) {
                key_pieces_lds(kcur, c, kw);
            } else {
                kw[0] = kreg[p][0].x; kw[1] = kreg[p][0].y; kw[2] = kreg[p][0].z; kw[3] = kreg[p][0].w;
                kw[4] = kreg[p][1].x; kw[5] = kreg[p][1].y; kw[6] = kreg[p][1].z; kw[7] = kreg[p][1].w;
            }
            const float d0 = combine_chains(key_chain(qp[0], c, kw, 0.f)) * a.scale;
            const float d1 = combine_chains(key_chain(qp[1], c, kw, 0.f)) * a.scale;
            s0[p] = t < n ? d0 : -INFINITY;
            s1[p] = t < n ? d1 : -INFINITY;
            m0 = fmaxf(m0, s0[p]);
            m1 = fmaxf(m1, s1[p]);
        }
        m0 = fmaxf(m0, xor_lanes<8>(m0));
        m1 = fmaxf(m1, xor_lanes<8>(m1));
        m0 = fmaxf(m0, xor_lanes<16>(m0));
        m1 = fmaxf(m1, xor_lanes<16>(m1));
        m0 = fmaxf(m0, xor_lanes<32>(m0));
        m1 = fmaxf(m1, xor_lanes<32>(m1));
        if (lane == 0) {
            wmax[wave][0] = m0;
            wmax[wave][1] = m1;
        }
        __syncthreads();
        m0 = wmax[0][0];
        m1 = wmax[0][1];
#pragma unroll
        for (int w = 1; w < 8; ++w) {
            m0 = fmaxf(m0, wmax[w][0]);
            m1 = fmaxf(m1, wmax[w][1]);
        }
        float l0 = 0.f, l1 = 0.f;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int t = 64 * (s + 32 * p) + grp;
            const float p0 = t < n ? expf(s0[p] - m0) : 0.f;
            const float p1 = t < n ? expf(s1[p] - m1) : 0.f;
            l0 += p0;
            l1 += p1;
            if (c == 0) {
                prob[0][p * 64 + grp] = p0;
                prob[1][p * 64 + grp] = p1;
            }
        }
        l0 += xor_lanes<8>(l0);
        l1 += xor_lanes<8>(l1);
        l0 += xor_lanes<16>(l0);
        l1 += xor_lanes<16>(l1);
        l0 += xor_lanes<32>(l0);
        l1 += xor_lanes<32>(l1);
        // prob[][] of this wave's positions is written and read by this wave only.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float acc[2][8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[0][i] = acc[1][i] = 0.f;
#pragma unroll
        for (int p = 0; p < PASSES; ++p)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const int tl = p * 64 + 8 * wave + 4 * hf + vsub, t = 64 * (s + 32 * p) + 8 * wave + 4 * hf + vsub;
                if (t < n) {
                    const float p0 = prob[0][tl], p1 = prob[1][tl];
                    uint32_t vw[4];
                    if (t == pos) {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            vw[i] = uint32_t(vcur[vcg * 8 + 2 * i]) | (uint32_t(vcur[vcg * 8 + 2 * i + 1]) << 16);
                    } else {
                        vw[0] = vreg[p][hf].x; vw[1] = vreg[p][hf].y; vw[2] = vreg[p][hf].z; vw[3] = vreg[p][hf].w;
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float v0 = h2f(vw[i] & 0xffffu), v1 = h2f(vw[i] >> 16);
                        acc[0][2 * i] = __builtin_fmaf(v0, p0, acc[0][2 * i]);
                        acc[0][2 * i + 1] = __builtin_fmaf(v1, p0, acc[0][2 * i + 1]);
                        acc[1][2 * i] = __builtin_fmaf(v0, p1, acc[1][2 * i]);
                        acc[1][2 * i + 1] = __builtin_fmaf(v1, p1, acc[1][2 * i + 1]);
                    }
                }
            }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                acc[hh][i] += xor_lanes<16>(acc[hh][i]);
                acc[hh][i] += xor_lanes<32>(acc[hh][i]);
            }
        if (vsub == 0) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int i = 0; i < 8; i += 4)
                    *reinterpret_cast<float4*>(&opart[wave][hh][vcg * 8 + i]) =
                        make_float4(acc[hh][i], acc[hh][i + 1], acc[hh][i + 2], acc[hh][i + 3]);
        }
        if (lane == 0) {
            wsum[wave][0] = l0;
            wsum[wave][1] = l1;
        }
        __syncthreads();
        if (tid < 256) {
            const int hh = tid >> 7;
            const float o = ((opart[0][hh][j] + opart[1][hh][j]) + (opart[2][hh][j] + opart[3][hh][j])) +
                            ((opart[4][hh][j] + opart[5][hh][j]) + (opart[6][hh][j] + opart[7][hh][j]));
            const float l = ((wsum[0][hh] + wsum[1][hh]) + (wsum[2][hh] + wsum[3][hh])) +
                            ((wsum[4][hh] + wsum[5][hh]) + (wsum[6][hh] + wsum[7][hh]));
            uint64_t* part = a.xpart + ((size_t(g) * 32 + s) * 2 + hh) * kXPart;
            exchange_put(part + j, o, a.tag);
            if (j == 0) {
                exchange_put(part + 128, hh ? m1 : m0, a.tag);
                exchange_put(part + 129, l, a.tag);
            }
        }
    }

    // 3. Merge query head h over the active workgroups' partials (group q of
    // 128 threads: workgroups 8q .. 8q + 7), then its O rows.
    {
        const int q = tid >> 7;
        float mv[8], lv[8], ovl[8];
        {
            // The partials of workgroups 8q .. 8q + 7 that have positions:
            // output j, max and sum of each, gathered in one poll.
            const uint64_t* words[24];
            float got[24];
            unsigned want = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint64_t* part = a.xpart + ((size_t(g) * 32 + 8 * q + k) * 2 + hq) * kXPart;
                words[k] = part + j;
                words[8 + k] = part + 128;
                words[16 + k] = part + 129;
                got[k] = got[8 + k] = got[16 + k] = 0.f;
                if (8 * q + k < active) want |= 0x10101u << k;
            }
            // After a give-up, stop polling (the step is reported as stalled).
            if (ok) ok = exchange_gather<24>(words, a.tag, got, want);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                ovl[k] = got[k];
                mv[k] = 8 * q + k < active ? got[8 + k] : -INFINITY;
                lv[k] = got[16 + k];
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (8 * q + k < active) mx = fmaxf(mx, mv[k]);
        float l = 0.f, o = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (8 * q + k < active) {
                const float w = expf(mv[k] - mx);
                l += w * lv[k];
                o += w * ovl[k];
            }
        if (j == 0) {
            gm[q] = mx;
            gl[q] = l;
        }
        go[q][j] = o;
    }
    if (!ok) *a.stall = 1;
    __syncthreads();
    if (tid < 128) {
        float m2 = gm[0];
#pragma unroll
        for (int q = 1; q < 4; ++q) m2 = fmaxf(m2, gm[q]);
        float lt = 0.f, ot = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (gm[q] != -INFINITY) {  // a group without partials adds nothing
                const float w = expf(gm[q] - m2);
                lt += w * gl[q];
                ot += w * go[q][tid];
            }
        att[tid] = ot / lt;
    }
    }  // split form
    __syncthreads();
    float y = 0.f;
    const float4* at4 = reinterpret_cast<const float4*>(att) + 2 * opart_id;
#pragma unroll
    for (int i = 0; i < kOLoads; ++i) y = chain8(y, ow[i], at4[2 * kThreadsPerRow * i], at4[2 * kThreadsPerRow * i + 1]);
    static_assert(kThreadsPerRow == 8, "three lane exchanges");
    y += xor_lanes<1>(y);
    y += xor_lanes<2>(y);
    y += xor_lanes<4>(y);
    if (opart_id == 0) a.o_part[h * kHidden + orow] = y;
}

// Batched decode: norm + QKV projection + attention of one layer for up to
// kMaxBatch sequences, each with its own position and cache. Workgroup w =
// g + 8 (b + B p): KV head g of sequence b, piece p of its positions; the
// W = B x pieces workgroups of KV head g share XCD g.
//
// QKV: every workgroup forms RMSNorm(x) of all sequences (engine/core.cpp
// 207-215, 390; FP32 squares summed in FP64; x is the embedding row in the
// first layer) as FP16 hi + lo in LDS, and computes 16 of the 512 q/k/v rows of KV head g (query
// heads 2g and 2g + 1, key g, value g) on the matrix cores
// (v_mfma_f32_16x16x32_f16, A = weight rows, B = the sequences, the 8 waves
// splitting K, summed in a fixed tree); the rows travel as tagged words
// through the XCD's L2 to the workgroups that attend with them.
//
// Attention: one workgroup per CU. A CU serves its loads in order, so a
// single workgroup per CU that keeps its own stream of K/V rows in flight
// (kInFlight 64-position blocks, the loads of block i + kInFlight issued
// once block i is consumed) overlaps the projection, the q/k/v exchange and
// its arithmetic with the stream. Block layout as in the single-sequence
// split kernel: the 8 lanes of position t score it (lane c = chain c of the
// reference dot, engine/core.cpp:612, key values converted once for both
// heads), and the wave that scored 8 positions multiplies their V rows (4
// positions x 16 channel groups per load). Softmax (613-620) runs online per
// wave: each wave keeps its own running maximum, rescaling its sums when it
// rises, and the 8 waves' sums are combined with weights exp(m_w - max) in a
// fixed tree; the exponentials are the hardware exp2 of x log2(e) (the
// batched path is held to the reference's tolerance gate). Every piece writes (unnormalized output, max, sum) of both
// query heads to the sequence's partial buffer; the batched O projection
// merges the pieces in its prologue. The last piece writes the new K/V row.
struct AttnBatchSeq {
    const float* x;          // residual stream the layer starts from [1024]
    const uint16_t* embed;   // first layer: the token's embedding row (the residual is fp32 of it), else null
    uint16_t* keys;          // layer base [8][context][128]
    uint16_t* values;
    float* x_out;            // residual after the O projection
    int pos;
    int context;
    const uint16_t* shared_keys;    // layer base of a cache whose rows [0, shared) equal these
    const uint16_t* shared_values;
    int shared_context;
    int shared;                     // multiple of 64, at most pos
};

struct AttnBatchArgs {
    AttnBatchSeq seq[kMaxBatch];
    const uint16_t* w_qkv;   // [4096 x 1024] (q rows, k rows, v rows) in matrix-core order, 128-column blocks
    const uint16_t* w_o;     // [1024 x 2048] in matrix-core order, 64-column blocks
    const float* in_norm;    // input RMSNorm weights
    const float* q_norm;
    const float* k_norm;
    const float* cosines;
    const float* sines;
    uint64_t* exchange;      // [8 KV heads][kMaxBatch][512] tagged q/k/v rows
    uint64_t* piece_words;   // [8 KV heads][32 workgroups][2][kXPart] tagged piece partials
    uint64_t* att_words;     // [8 KV heads][kMaxBatch][256] tagged merged attention rows
    uint64_t* share_words;   // [32 row blocks][8 XCDs][kMaxBatch][32 rows] tagged O shares
    int* stall;
    float scale;
    int batch;
    int pieces;  // pieces per (sequence, head)
    uint32_t tag;
};

// Third descriptor word of a raw buffer (gfx9 family: 32-bit data format),
// and the non-temporal cache policy for rows that are read once.
constexpr int kBufferWord3 = 0x00020000;
constexpr int kLoadNT = 2;
constexpr int kInFlight = 4;

// NB = the largest number of 64-position blocks a piece of this launch
// holds; EMBED: the first layer (the residual is the embedding row).
template <int NB, bool EMBED>
__global__ __launch_bounds__(512) void attn_batch_kernel(const AttnBatchArgs args) {
    const int w = blockIdx.x, g = w & 7, r = w >> 3, B = args.batch, b = r % B, p = r / B;
    const int W = B * args.pieces;  // attention workgroups of this XCD (the grid holds 32 per XCD)
    const AttnBatchSeq a = args.seq[b];  // by value: loaded once, ahead of the cache rows
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, quad = lane >> 4;
    const int pos = a.pos, n = pos + 1;
    const int blocks = (n + 63) / 64, per = (blocks + args.pieces - 1) / args.pieces;
    const int ns = (blocks + per - 1) / per;  // pieces with positions
    // A piece past ns has t_end < t_begin: its buffer loads are all out of range.
    const int t_begin = p * per * 64, t_end = min(n, t_begin + per * 64);
    // The block holding row pos (the last piece's last block), or -1.
    const int i_pos = p == ns - 1 ? (pos - t_begin) >> 6 : -1;
    const size_t head_base = size_t(g) * a.context;
    const int quarter = tid >> 7, j = tid & 127, c = tid & 7, grp = tid >> 3;
    const int vsub = lane >> 4, vcg = lane & 15;

    // Loads complete in issue order per wave, so they are issued in the order
    // the phases need them: the residual inputs (elements 2 tid, 2 tid + 1 of
    // every sequence; rows past the batch repeat row B - 1), norm weights,
    // this workgroup's QKV weight tile, rotation.
    // The first layer (EMBED) reads every sequence's embedding row instead.
    float2 xv[kMaxBatch];
    uint32_t ev[kMaxBatch];
#pragma unroll
    for (int bb = 0; bb < kMaxBatch; ++bb) {
        const AttnBatchSeq& s2 = args.seq[min(bb, B - 1)];
        if constexpr (EMBED)
            ev[bb] = reinterpret_cast<const uint32_t*>(s2.embed)[tid];
        else
            xv[bb] = reinterpret_cast<const float2*>(s2.x)[tid];
    }
    const float2 wn = reinterpret_cast<const float2*>(args.in_norm)[tid];
    // QKV tile tr (16 of the 512 rows of KV head g): query rows 256 g + 16 tr
    // for tr < 16, key rows 2048 + 128 g + 16 (tr - 16) for tr < 24, value
    // rows 3072 + 128 g + 16 (tr - 24) after.
    auto tile_row = [&](int tr) {
        return tr < 16 ? 256 * g + 16 * tr : (tr < 24 ? 2048 + 128 * g + 16 * (tr - 16) : 3072 + 128 * g + 16 * (tr - 24));
    };
    auto load_tile = [&](u32x4 (&wt)[4], int tr) {
        // 16-row tile tile_row(tr) / 16, wave's 128-column block, step st:
        // 1 KiB contiguous per load.
        const u32x4* wp = reinterpret_cast<const u32x4*>(args.w_qkv) + (size_t(tile_row(tr) / 16) * 8 + wave) * 256 + lane;
#pragma unroll
        for (int st = 0; st < 4; ++st) wt[st] = __builtin_nontemporal_load(wp + 64 * st);
    };
    u32x4 wq[4];
    __builtin_amdgcn_sched_barrier(0);
    load_tile(wq, r);
    __builtin_amdgcn_sched_barrier(0);
    const float nw = (__builtin_amdgcn_readfirstlane(quarter) < 2 ? args.q_norm : args.k_norm)[j];
    const float rc = args.cosines[size_t(pos) * 64 + (j & 63)], rs = args.sines[size_t(pos) * 64 + (j & 63)];
    // K/V rows through buffer loads: one descriptor per matrix covering this
    // piece's rows (reads past them return zeros without touching memory),
    // per-lane offsets fixed for the piece, the block in the scalar offset.
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(a.keys + head_base * 128, 0, t_end * 256, kBufferWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(a.values + head_base * 128, 0, t_end * 256, kBufferWord3);
    // Blocks below a.shared come from the shared copy, whose descriptors
    // cover the rows of this piece below a.shared; every sequence of the
    // batch with that copy reads the same addresses, on this XCD (KV head g),
    // so all but the first reads hit in its L2.
    const size_t shared_base = size_t(g) * a.shared_context;
    const int shared_end = min(a.shared, t_end);
    const __amdgpu_buffer_rsrc_t skrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.shared_keys) + shared_base * 128, 0, max(shared_end, 0) * 256, kBufferWord3);
    const __amdgpu_buffer_rsrc_t svrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.shared_values) + shared_base * 128, 0, max(shared_end, 0) * 256, kBufferWord3);
    const int koff = (t_begin + grp) * 256 + 16 * c;
    const int voff = (t_begin + 8 * wave + vsub) * 256 + 16 * vcg;
    auto load_block = [&](u32x4 (&k)[2], u32x4 (&v)[2], int i) {
        const bool shared = t_begin + 64 * i < a.shared;  // uniform; a.shared is a multiple of 64
        const __amdgpu_buffer_rsrc_t kb = shared ? skrs : krs, vb = shared ? svrs : vrs;
        // The block offset goes into the per-lane offset, which the range
        // check covers, so rows past the piece are never read.
        k[0] = __builtin_amdgcn_raw_buffer_load_b128(kb, koff + 16384 * i, 0, kLoadNT);
        k[1] = __builtin_amdgcn_raw_buffer_load_b128(kb, koff + 128 + 16384 * i, 0, kLoadNT);
        v[0] = __builtin_amdgcn_raw_buffer_load_b128(vb, voff + 16384 * i, 0, kLoadNT);
        v[1] = __builtin_amdgcn_raw_buffer_load_b128(vb, voff + 1024 + 16384 * i, 0, kLoadNT);
    };
    u32x4 kr[kInFlight][2], vr[kInFlight][2];

    __shared__ __align__(16) _Float16 xh[kMaxBatch][kHidden + 8];
    __shared__ __align__(16) _Float16 xl[kMaxBatch][kHidden + 8];
    __shared__ double nred[8][kMaxBatch];
    __shared__ float inv_row[kMaxBatch];
    __shared__ float qpart[8][64][4];
    __shared__ float qp[2][128];
    __shared__ float buf[4][128];
    __shared__ float prob[2][64];
    __shared__ __align__(16) float opart[8][2][128];
    __shared__ uint16_t kcur[128], vcur[128];
    __shared__ double red[4][2];
    __shared__ float wm[8][2], wl[8][2];
    __shared__ dev::SplitGuard guard;
    guard.init(tid);

    if constexpr (EMBED) {
#pragma unroll
        for (int bb = 0; bb < kMaxBatch; ++bb) xv[bb] = make_float2(h2f(ev[bb] & 0xffffu), h2f(ev[bb] >> 16));
    }

    // RMSNorm of every sequence's row: per-thread FP64 sums of the FP32
    // squares, a reduce-scatter inside each wave (exchanges over lane bits
    // 5, 4 and 3 halve the rows a lane carries, then bits 2..0 are summed, so
    // lane l ends with its wave's total of row (l >> 3) & 7), then the 8 wave
    // totals of a row in fixed order.
    {
        double sq[kMaxBatch];
#pragma unroll
        for (int bb = 0; bb < kMaxBatch; ++bb) {
            const float q0 = xv[bb].x * xv[bb].x, q1 = xv[bb].y * xv[bb].y;
            sq[bb] = static_cast<double>(q0) + static_cast<double>(q1);
        }
        const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
        double r4[4], r2[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const double keep = b5 ? sq[4 + i] : sq[i], send = b5 ? sq[i] : sq[4 + i];
            r4[i] = keep + xor_lanes<32>(send);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const double keep = b4 ? r4[2 + i] : r4[i], send = b4 ? r4[i] : r4[2 + i];
            r2[i] = keep + xor_lanes<16>(send);
        }
        double r1 = (b3 ? r2[1] : r2[0]) + xor_lanes<8>(b3 ? r2[0] : r2[1]);
        r1 += xor_lanes<4>(r1);
        r1 += xor_lanes<2>(r1);
        r1 += xor_lanes<1>(r1);
        if ((lane & 7) == 0) nred[wave][lane >> 3] = r1;
        __syncthreads();
        if (tid < kMaxBatch) {
            const double total = ((nred[0][tid] + nred[1][tid]) + (nred[2][tid] + nred[3][tid])) +
                                 ((nred[4][tid] + nred[5][tid]) + (nred[6][tid] + nred[7][tid]));
            inv_row[tid] = 1.0f / __builtin_sqrtf(static_cast<float>(total) / static_cast<float>(kHidden) + 1e-6f);
        }
        __syncthreads();
        // Normalized rows as FP16 hi / lo, scaled by 2^-e per sequence only
        // when a row reaches the FP16 limit (the guard's slow path).
        auto split_rows = [&](bool scaled) {
            float big = 0.f;
#pragma unroll
            for (int bb = 0; bb < kMaxBatch; ++bb) {
                const float inv = inv_row[bb];
                float n0 = (xv[bb].x * inv) * wn.x, n1 = (xv[bb].y * inv) * wn.y;
                big = fmaxf(big, fmaxf(fabsf(n0), fabsf(n1)));
                if (scaled) {
                    const float down = pow2(-guard.seq_e[bb]);
                    n0 = n0 * down;
                    n1 = n1 * down;
                }
                _Float16 h0, l0, h1, l1;
                split_half(n0, h0, l0);
                split_half(n1, h1, l1);
                *reinterpret_cast<half2_t*>(&xh[bb][2 * tid]) = half2_t{h0, h1};
                *reinterpret_cast<half2_t*>(&xl[bb][2 * tid]) = half2_t{l0, l1};
            }
            return big;
        };
        guard.post(split_rows(false), lane, wave);
        __syncthreads();
        if (guard.needed(8)) {
#pragma unroll
            for (int bb = 0; bb < kMaxBatch; ++bb) {
                const float inv = inv_row[bb];
                guard.offer(bb, fmaxf(fabsf((xv[bb].x * inv) * wn.x), fabsf((xv[bb].y * inv) * wn.y)));
            }
            __syncthreads();
            if (tid < kMaxBatch) guard.seq_e[tid] = guard.exponent(tid);
            __syncthreads();
            split_rows(true);
            __syncthreads();
        }
    }

    // QKV tiles of this workgroup: r, then r + W, ... when W < 32 (the first
    // outside the loop, so that its weights are waited for without the K/V
    // loads issued after them).
    auto project_tile = [&](int tr) {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            // k slot (quad, e) of step st holds column 128 wave + 32 st + 8 quad + e.
            const int k = 128 * wave + 32 * st + 8 * quad;
            const half8 bh = masked_b<half8>(&xh[col & 7][k], col < kMaxBatch);
            const half8 bl = masked_b<half8>(&xl[col & 7][k], col < kMaxBatch);
            const half8 w8 = __builtin_bit_cast(half8, wq[st]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w8, bh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w8, bl, acc, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) qpart[wave][lane][e] = acc[e];
        __syncthreads();
        if (wave < 4) {  // element (row 4 (lane / 16) + wave, sequence lane % 16)
            const auto f = [&](int v8) { return qpart[v8][lane][wave]; };
            const int seq = lane & 15, row = 16 * tr + 4 * (lane >> 4) + wave;
            const float y = (((f(0) + f(1)) + (f(2) + f(3))) + ((f(4) + f(5)) + (f(6) + f(7)))) * guard.up(seq & 7);
            if (seq < B) exchange_put(args.exchange + (size_t(g) * kMaxBatch + seq) * 512 + row, y, args.tag);
        }
        __syncthreads();
    };
    project_tile(r);
    // O weights of this workgroup (rows 32 r + 16 (wave & 1) + col, columns
    // 256 g + 64 (wave >> 1) + 32 st + 8 quad .. + 7), issued ahead of the
    // K/V stream and used after it.
    u32x4 wo[2];
    {
        // Tile 2 r + (wave & 1), 64-column block 4 g + (wave >> 1), steps 0, 1.
        const u32x4* op = reinterpret_cast<const u32x4*>(args.w_o) +
                          ((size_t(2 * r + (wave & 1)) * 32 + 4 * g + (wave >> 1)) * 2) * 64 + lane;
        wo[0] = __builtin_nontemporal_load(op);
        wo[1] = __builtin_nontemporal_load(op + 64);
    }
    // Workgroups past the batch's pieces, or whose piece holds no position,
    // only project.
    if (r < W && p < ns) {

    // This workgroup's q/k/v rows (query heads 2g, 2g + 1, key, value) are
    // gathered by wave 0 into LDS before it issues any K/V load; the other
    // waves start the stream right away. (A CU returns loads in the order it
    // received them, and the memory system serves a flood of stream misses
    // ahead of later ones: issued before the projection, the stream would
    // hold up its inputs; issued before the poll, it holds up the poll. Wave
    // 0's poll still waits behind the other waves' first blocks.)
    __shared__ float rawq[512];
    if (wave == 0) {
        const uint64_t* base = args.exchange + (size_t(g) * kMaxBatch + b) * 512 + lane;
        const uint64_t* const words[8] = {base, base + 64, base + 128, base + 192,
                                          base + 256, base + 320, base + 384, base + 448};
        float got[8] = {};
        if (!exchange_gather_pipe<8, 2>(words, args.tag, got, 0xffu)) *args.stall = 1;
#pragma unroll
        for (int k = 0; k < 8; ++k) rawq[lane + 64 * k] = got[k];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kInFlight && i < NB; ++i) load_block(kr[i], vr[i], i);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    // Thread tid's row: quarter 0/1 query heads, 2 key, 3 value.
    const float raw = rawq[tid];
    const float raw_v = raw;

    // QK-norm + RoPE (engine/core.cpp:395-402); the last piece writes the
    // new K/V row (403-406).
    {
        const float r = head_norm_rope(raw, nw, rc, rs, red[quarter], buf[quarter], j);
        const bool owner = p == ns - 1;
        if (quarter < 2) {
            qp[quarter][kperm(j)] = r;
        } else if (quarter == 2) {
            const uint16_t bits = f2h(r);
            kcur[kperm(j)] = bits;
            if (owner) a.keys[(head_base + pos) * 128 + kperm(j)] = bits;
        } else {
            const uint16_t bits = f2h(raw_v);
            vcur[j] = bits;
            if (owner) a.values[(head_base + pos) * 128 + j] = bits;
        }
    }
    __syncthreads();
    // Lane c's query values in chain order: q[h][2i + e] multiplies half e
    // of key word i (see key_chain).
    float q[2][16];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int base = (i < 4 ? 8 * c : 64 + 8 * c) + 2 * (i & 3);
            q[h][2 * i] = qp[h][base];
            q[h][2 * i + 1] = qp[h][base + 1];
        }

    // Per-wave online softmax over the blocks: running maxima m (uniform in
    // the wave), per-lane probability sums l (one position per block) and
    // P.V sums acc, all rescaled by exp(m_old - m_new) when the maximum rises.
    float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.f, l1 = 0.f;
    float acc[2][8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[0][e] = acc[1][e] = 0.f;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        u32x4(&k)[2] = kr[i % kInFlight];
        u32x4(&v)[2] = vr[i % kInFlight];
        if (64 * i < t_end - t_begin) {  // uniform: blocks past the piece hold no position
            const int t = t_begin + 64 * i + grp;
            uint32_t kw[8] = {k[0].x, k[0].y, k[0].z, k[0].w, k[1].x, k[1].y, k[1].z, k[1].w};
            if (i == i_pos && t == pos) key_pieces_lds(kcur, c, kw);  // i == i_pos is uniform
            float kf[16];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                kf[2 * e] = h2f(kw[e] & 0xffffu);
                kf[2 * e + 1] = h2f(kw[e] >> 16);
            }
            float d[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float chain = 0.f;
#pragma unroll
                for (int e = 0; e < 16; ++e) chain = __builtin_fmaf(q[h][e], kf[e], chain);
                d[h] = combine_chains(chain) * args.scale;
            }
            const bool valid = t < t_end;
            const float s0 = valid ? d[0] : -INFINITY, s1 = valid ? d[1] : -INFINITY;
            float b0 = fmaxf(s0, xor_lanes<8>(s0)), b1 = fmaxf(s1, xor_lanes<8>(s1));
            b0 = fmaxf(b0, xor_lanes<16>(b0));
            b1 = fmaxf(b1, xor_lanes<16>(b1));
            b0 = fmaxf(b0, xor_lanes<32>(b0));
            b1 = fmaxf(b1, xor_lanes<32>(b1));
            const float n0 = fmaxf(m0, b0), n1 = fmaxf(m1, b1);
            // The sums are rescaled only when the wave's running maximum rises
            // (uniform in the wave; from -inf the scale is 0, on empty sums).
            if (n0 != m0 || n1 != m1) {
                const float a0 = n0 == m0 ? 1.f : __expf(m0 - n0);
                const float a1 = n1 == m1 ? 1.f : __expf(m1 - n1);
                l0 *= a0;
                l1 *= a1;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    acc[0][e] *= a0;
                    acc[1][e] *= a1;
                }
                m0 = n0;
                m1 = n1;
            }
            const float p0 = valid ? __expf(s0 - n0) : 0.f;
            const float p1 = valid ? __expf(s1 - n1) : 0.f;
            l0 += p0;
            l1 += p1;
            if (c == 0) {
                prob[0][grp] = p0;
                prob[1][grp] = p1;
            }
            // prob[][] of this wave's positions is written and read by this wave only.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const int tl = 8 * wave + 4 * hf + vsub, tv = t_begin + 64 * i + tl;
                if (tv < t_end) {
                    const float q0 = prob[0][tl], q1 = prob[1][tl];
                    uint32_t vw[4] = {v[hf].x, v[hf].y, v[hf].z, v[hf].w};
                    if (i == i_pos && tv == pos) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            vw[e] = uint32_t(vcur[vcg * 8 + 2 * e]) | (uint32_t(vcur[vcg * 8 + 2 * e + 1]) << 16);
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float v0 = h2f(vw[e] & 0xffffu), v1 = h2f(vw[e] >> 16);
                        acc[0][2 * e] = __builtin_fmaf(v0, q0, acc[0][2 * e]);
                        acc[0][2 * e + 1] = __builtin_fmaf(v1, q0, acc[0][2 * e + 1]);
                        acc[1][2 * e] = __builtin_fmaf(v0, q1, acc[1][2 * e]);
                        acc[1][2 * e + 1] = __builtin_fmaf(v1, q1, acc[1][2 * e + 1]);
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        if (i + kInFlight < NB) {
            __builtin_amdgcn_sched_barrier(0);
            load_block(k, v, i + kInFlight);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // Wave sums: the 8 position lanes of l, the 4 position groups of acc.
    l0 += xor_lanes<8>(l0);
    l1 += xor_lanes<8>(l1);
    l0 += xor_lanes<16>(l0);
    l1 += xor_lanes<16>(l1);
    l0 += xor_lanes<32>(l0);
    l1 += xor_lanes<32>(l1);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            acc[h][e] += xor_lanes<16>(acc[h][e]);
            acc[h][e] += xor_lanes<32>(acc[h][e]);
        }
    if (vsub == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 8; e += 4)
                *reinterpret_cast<float4*>(&opart[wave][h][vcg * 8 + e]) =
                    make_float4(acc[h][e], acc[h][e + 1], acc[h][e + 2], acc[h][e + 3]);
    }
    if (lane == 0) {
        wm[wave][0] = m0;
        wm[wave][1] = m1;
        wl[wave][0] = l0;
        wl[wave][1] = l1;
    }
    __syncthreads();
    // Thread (half, j) of the first 256: output j of query head 2g + half,
    // the 8 waves combined with weights exp(m_w - max) (0 for a wave that
    // saw no position) in a fixed tree.
    const int half = (tid >> 7) & 1;
    float mx = wm[0][half];
#pragma unroll
    for (int v8 = 1; v8 < 8; ++v8) mx = fmaxf(mx, wm[v8][half]);
    float wt[8];
#pragma unroll
    for (int v8 = 0; v8 < 8; ++v8) wt[v8] = wm[v8][half] == -INFINITY ? 0.f : expf(wm[v8][half] - mx);
    auto tree = [&](auto f) {
        return ((f(0) + f(1)) + (f(2) + f(3))) + ((f(4) + f(5)) + (f(6) + f(7)));
    };
    const float o = tree([&](int v8) { return wt[v8] * opart[v8][half][j]; });
    const float l = tree([&](int v8) { return wt[v8] * wl[v8][half]; });
    // Pieces p > 0 post (output, max, sum); piece 0 merges its sequence's
    // pieces in order (out = sum_p e_p o_p / sum_p e_p l_p, e_p =
    // exp(m_p - max)) and posts the merged rows of both query heads.
    uint64_t* const my_piece = args.piece_words + ((size_t(g) * 32 + r) * 2 + half) * kXPart;
    if (p > 0) {
        if (tid < 256) {
            exchange_put(my_piece + j, o, args.tag);
            if (j == 0) {
                exchange_put(my_piece + 128, mx, args.tag);
                exchange_put(my_piece + 129, l, args.tag);
            }
        }
    } else if (tid < 256) {
        float run_m = mx, run_l = l, run_o = o;
        bool ok = true;
        for (int p0 = 1; p0 < ns; p0 += 4) {
            const uint64_t* words[12];
            float got[12];
            unsigned want = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int pk = min(p0 + k, ns - 1);
                const uint64_t* e = args.piece_words + ((size_t(g) * 32 + b + B * pk) * 2 + half) * kXPart;
                words[k] = e + j;
                words[4 + k] = e + 128;
                words[8 + k] = e + 129;
                got[k] = got[4 + k] = got[8 + k] = 0.f;
                if (p0 + k < ns) want |= 0x111u << k;
            }
            if (ok) ok = exchange_gather_pipe<12, 2>(words, args.tag, got, want);
            float cm = -INFINITY;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (p0 + k < ns) cm = fmaxf(cm, got[4 + k]);
            const float nm = fmaxf(run_m, cm), sc = expf(run_m - nm);
            run_l *= sc;
            run_o *= sc;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (p0 + k < ns) {
                    const float e = expf(got[4 + k] - nm);
                    run_l += e * got[8 + k];
                    run_o += e * got[k];
                }
            run_m = nm;
        }
        if (!ok) *args.stall = 1;
        exchange_put(args.att_words + (size_t(g) * kMaxBatch + b) * 256 + half * 128 + j, run_o / run_l, args.tag);
    }
    }  // attention workgroups

    // O projection of this XCD's two query heads (columns 256 g .. + 255)
    // for rows 32 r .. 32 r + 31: the merged rows of every sequence, staged
    // as FP16 hi + lo.
    bool ok = true;
    {
        const uint64_t* words[4];
        float got[4];
        unsigned want = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int idx = tid + 512 * k;  // sequence idx / 256, column idx % 256
            words[k] = args.att_words + size_t(g) * kMaxBatch * 256 + idx;
            got[k] = 0.f;
            if ((idx >> 8) < B) want |= 1u << k;
        }
        ok = exchange_gather_pipe<4, 2>(words, args.tag, got, want);
        // Attention rows are convex combinations of FP16 values: they fit
        // FP16 without the range guard.
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int idx = tid + 512 * k;
            _Float16 h, lo;
            split_half(got[k], h, lo);
            xh[idx >> 8][idx & 255] = h;
            xl[idx >> 8][idx & 255] = lo;
        }
        __syncthreads();
    }
    {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const int k = 64 * (wave >> 1) + 32 * st + 8 * quad;
            const half8 bh = masked_b<half8>(&xh[col & 7][k], col < kMaxBatch);
            const half8 bl = masked_b<half8>(&xl[col & 7][k], col < kMaxBatch);
            const half8 w8 = __builtin_bit_cast(half8, wo[st]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w8, bh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w8, bl, acc, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) qpart[wave][lane][e] = acc[e];
        __syncthreads();
        // Thread (wave w < 4, lane): sequence 2 w + lane / 32, row
        // 32 r + rl (rl = lane % 32: tile rl / 16, element rl % 16 held by
        // MFMA lane 16 (rl / 4 % 4) + sequence, register rl % 4), the tile's
        // 4 column ranges (waves tt, tt + 2, tt + 4, tt + 6) in fixed order;
        // the share goes through memory to the XCD that adds the row. A wave
        // posts 64 consecutive words: the XCD's shares fill whole lines
        // (write-through stores of parts of a line cost far more).
        if (wave < 4) {
            const int seq = 2 * wave + (lane >> 5), rl = lane & 31;
            const int tt = rl >> 4, e4 = rl & 3, el = 16 * ((rl >> 2) & 3) + seq;
            const float y = (qpart[tt][el][e4] + qpart[tt + 2][el][e4]) + (qpart[tt + 4][el][e4] + qpart[tt + 6][el][e4]);
            if (seq < B)
                exchange_put_through(args.share_words + ((size_t(r) * 8 + g) * kMaxBatch + seq) * 32 + rl, y, args.tag);
        }
    }
    // Rows 32 r .. 32 r + 31 of sequence g (threads 0..31, one row each: a
    // whole line of the residual) add the 8 XCD shares in fixed order, into
    // the second residual buffer (every workgroup read the first one).
    if (tid < 32) {
        const int row = 32 * r + tid, seq = g;
        const bool live = seq < B;
        const uint64_t* words[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) words[k] = args.share_words + ((size_t(r) * 8 + k) * kMaxBatch + seq) * 32 + tid;
        float s8[8] = {};
        if (ok) ok = exchange_gather_pipe<8, 6>(words, args.tag, s8, live ? 0xffu : 0u);
        if (live) {
            const float y = ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
            const AttnBatchSeq& sq = args.seq[seq];
            sq.x_out[row] = (EMBED ? h2f(sq.embed[row]) : sq.x[row]) + y;
        }
    }
    if (!ok) *args.stall = 1;
}


__global__ void tile_kernel(const uint16_t* __restrict__ first, const uint16_t* __restrict__ second,
                            uint16_t* __restrict__ dst, int rows, int cols) {
    const int nb = cols / 64;
    const size_t tiles = second ? size_t(rows) / 4 : size_t(rows) / 8;
    const size_t total = tiles * nb * 64;
    const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int t = int(idx & 63), r = t >> 3, c = t & 7;
    const size_t tb = idx >> 6, tileid = tb / nb;
    const int b = int(tb % nb);
    const uint16_t* src;
    if (second)
        src = r < 4 ? first + (4 * tileid + r) * size_t(cols) : second + (4 * tileid + r - 4) * size_t(cols);
    else
        src = first + (8 * tileid + r) * size_t(cols);
    uint32_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        v[i] = uint32_t(src[64 * b + 8 * (2 * i) + c]) | (uint32_t(src[64 * b + 8 * (2 * i + 1) + c]) << 16);
    u32x4 out = {v[0], v[1], v[2], v[3]};
    *reinterpret_cast<u32x4*>(dst + idx * 8) = out;
}

// Waves (8-row tiles) per workgroup of each layer GEMV (measured best).
constexpr int kLayerWaves = 2;
template <int MODE>
constexpr int gemv_waves() {
    if constexpr (MODE == kQKV) return 2;
    else if constexpr (MODE == kGateUp) return 4;
    else return kLayerWaves;
}

template <int N, int MODE>
void launch_gemv(const GemvArgs& a, int rows, hipStream_t stream) {
    if constexpr (N > kHidden) {  // long rows (O, down, plain 2048/3072): two-segment chains
        if constexpr (MODE == kDown) {
            if (a.parts) {
                gemv_seg_kernel<N, 2, MODE, true><<<rows / 4, 64, 0, stream>>>(a);
                return;
            }
        }
        gemv_seg_kernel<N, 2, MODE><<<rows / 4, 64, 0, stream>>>(a);
        return;
    }
    constexpr int W = gemv_waves<MODE>();
    if constexpr (MODE == kGateUp || MODE == kDown || MODE == kQKV) {
        if (a.parts) {
            gemv_kernel<N, W, MODE, true><<<rows / (8 * W), 64 * W, 0, stream>>>(a);
            return;
        }
    }
    gemv_kernel<N, W, MODE><<<rows / (8 * W), 64 * W, 0, stream>>>(a);
}

// Two-row launches (verification pairs): waves per workgroup of each mode.
template <int MODE>
constexpr int gemv_pair_waves() {
    if constexpr (MODE == kGateUp) return 4;
    else if constexpr (MODE == kDown) return 1;
    else return 2;
}

template <int N, int MODE>
void launch_gemv_pair(const GemvArgs& a, int rows, hipStream_t stream) {
    constexpr int W = gemv_pair_waves<MODE>();
    if constexpr (MODE == kGateUp || MODE == kDown || MODE == kQKV) {
        if (a.parts) {
            gemv_kernel<N, W, MODE, true, 2><<<rows / (8 * W), 64 * W, 0, stream>>>(a);
            return;
        }
    }
    gemv_kernel<N, W, MODE, false, 2><<<rows / (8 * W), 64 * W, 0, stream>>>(a);
}

template <int ROWS>
void launch_ffn_rows(const uint16_t* gateup_t, const uint16_t* down_t, const float* norm_w, const float* x,
                     const float* parts, float* xm, float* dparts, uint64_t* exchange, int* stall, uint32_t tag,
                     hipStream_t stream) {
    require(tag != 0, "fused FFN: tag 0 is the cleared exchange");
    FfnArgs f{};
    f.gateup_t = gateup_t;
    f.down_t = down_t;
    f.x = x;
    f.norm_w = norm_w;
    f.parts = parts;
    f.xm = xm;
    f.dparts = dparts;
    f.exchange = exchange;
    f.stall = stall;
    f.tag = tag;
    ffn_kernel<ROWS><<<kFfnGroups, 256, 0, stream>>>(f);
}

// The attention form and pass count for n = pos + 1 cached positions.
template <class F>
void with_attention_form(int pos, F&& go) {
    const int passes = (pos + 1 + 63) / 64;
    using std::integral_constant;
    switch (passes <= kFullAttnPasses ? passes : 0) {
        case 1: go(integral_constant<int, 1>{}, std::true_type{}); break;
        case 2: go(integral_constant<int, 2>{}, std::true_type{}); break;
        case 3: go(integral_constant<int, 3>{}, std::true_type{}); break;
        case 4: go(integral_constant<int, 4>{}, std::true_type{}); break;
        default:
            if (passes > 32) go(integral_constant<int, 2>{}, std::false_type{});
            else go(integral_constant<int, 1>{}, std::false_type{});
    }
}

// The fused QKV + attention + O kernel of one row at position pos. x: the
// residual the layer starts from (written there with embed or dparts); xm
// and dparts: the previous fused FFN's output when dparts is non-null.
void launch_qkv_attn(const LayerDevice& L, const uint16_t* embed, int token, int pos, const float* cosines,
                     const float* sines, int context, float* x, const float* xm, const float* dparts, float* o_part,
                     const DecodeScratch& s, uint32_t tag, hipStream_t stream) {
    require(tag != 0, "fused attention: tag 0 is the cleared exchange");
    require(pos >= 0 && pos < context && pos < 64 * 64, "fused attention: position outside the cache");
    static_assert(kXPartWords == kKVHeads * 32 * 2 * kXPart, "exchange size");
    QkvAttnArgs q{};
    q.qkv_t = L.qkv_t;
    q.in_norm = L.in_norm;
    q.x = x;
    q.xm = xm;
    q.dparts = dparts;
    q.embed = embed;
    q.token = token;
    q.x_out = x;
    q.q_norm = L.q_norm;
    q.k_norm = L.k_norm;
    q.cosines = cosines;
    q.sines = sines;
    q.keys = L.keys;
    q.values = L.values;
    q.pos = pos;
    q.context = context;
    q.scale = 1.0f / std::sqrt(128.0f);
    q.o_n = L.o_n;
    q.o_part = o_part;
    q.xqkv = s.xqkv;
    q.xpart = s.xpart;
    q.stall = s.stall;
    q.tag = tag;
    const int src = embed ? 1 : dparts ? 2 : 0;
    with_attention_form(pos, [&](auto tag_passes, auto tag_full) {
        constexpr int P = decltype(tag_passes)::value;
        constexpr bool F = decltype(tag_full)::value;
        if (src == 0) qkv_attn_kernel<P, 0, F><<<256, 512, 0, stream>>>(q);
        else if (src == 1) qkv_attn_kernel<P, 1, F><<<256, 512, 0, stream>>>(q);
        else qkv_attn_kernel<P, 2, F><<<256, 512, 0, stream>>>(q);
    });
}

template <int ROWS>
void launch_ffn(const LayerDevice& L, const float* x, const float* parts, float* xm, float* dparts,
                uint64_t* exchange, int* stall, uint32_t tag, hipStream_t stream) {
    launch_ffn_rows<ROWS>(L.gateup_t, L.down_t, L.post_norm, x, parts, xm, dparts, exchange, stall, tag, stream);
}

}  // namespace

void launch_tile_matrix(const uint16_t* first, const uint16_t* second, uint16_t* dst, int rows, int cols,
                        hipStream_t stream) {
    require(cols % 64 == 0 && rows % (second ? 4 : 8) == 0, "tile_matrix: unsupported shape");
    const size_t tiles = second ? size_t(rows) / 4 : size_t(rows) / 8;
    const size_t total = tiles * (cols / 64) * 64;
    tile_kernel<<<unsigned((total + 255) / 256), 256, 0, stream>>>(first, second, dst, rows, cols);
}

void launch_gemv_plain(const uint16_t* w_t, const float* x, float* y, int rows, int cols, hipStream_t stream) {
    require(rows > 0 && rows % (8 * kLayerWaves) == 0, "gemv: rows must be a positive multiple of 16");
    GemvArgs a{};
    a.w = w_t;
    a.in = x;
    a.out = y;
    switch (cols) {
        case 1024: launch_gemv<1024, kPlain>(a, rows, stream); break;
        case 2048: launch_gemv<2048, kPlain>(a, rows, stream); break;
        case 3072: launch_gemv<3072, kPlain>(a, rows, stream); break;
        default: throw std::runtime_error("gemv: cols must be 1024, 2048 or 3072");
    }
}

void launch_layer_kernel(int which, const LayerDevice& L, const uint16_t* embed, int pos, int token,
                         const float* cosines, const float* sines, int context, const DecodeScratch& s,
                         LayerFlow flow, hipStream_t stream) {
    switch (which) {
        case 0: {
            if (flow.attn_tag) {
                const bool fold = flow.fold_input && !embed;
                launch_qkv_attn(L, embed, token, pos, cosines, sines, context, s.x, s.xm, fold ? s.dparts : nullptr,
                                s.o_part, s, flow.attn_tag, stream);
                break;
            }
            GemvArgs q{};
            q.w = L.qkv_t;
            q.in = s.x;
            q.norm_w = L.in_norm;
            q.embed = embed;
            q.token[0] = token;
            q.out = s.qkv;
            q.x = s.x;
            if (flow.fold_input && !embed) {
                q.in = s.xm;
                q.parts = s.dparts;
            }
            launch_gemv<kHidden, kQKV>(q, kQKVRows, stream);
            break;
        }
        case 1: {
            if (flow.attn_tag) break;  // the fused kernel ran the attention
            AttnArgs at{};
            at.qkv = s.qkv;
            at.q_norm = L.q_norm;
            at.k_norm = L.k_norm;
            at.cosines = cosines;
            at.sines = sines;
            at.keys = L.keys;
            at.values = L.values;
            at.pos = pos;
            at.partial = s.attn_partial;
            at.attended = s.attended;
            at.context = context;
            at.scale = 1.0f / std::sqrt(128.0f);
            at.o_n = L.o_n;
            at.o_part = s.o_part;
            if (attn_fused(pos + 1)) {
                switch ((pos + 64) / 64) {  // passes of 64 positions over n = pos + 1
                    case 1: attn_o_kernel<1><<<kAttnOGroups, 512, 0, stream>>>(at); break;
                    case 2: attn_o_kernel<2><<<kAttnOGroups, 512, 0, stream>>>(at); break;
                    case 3: attn_o_kernel<3><<<kAttnOGroups, 512, 0, stream>>>(at); break;
                    case 4: attn_o_kernel<4><<<kAttnOGroups, 512, 0, stream>>>(at); break;
                    case 5: attn_o_kernel<5><<<kAttnOGroups, 512, 0, stream>>>(at); break;
                    case 6: attn_o_kernel<6><<<kAttnOGroups, 512, 0, stream>>>(at); break;
                    case 7: attn_o_kernel<7><<<kAttnOGroups, 512, 0, stream>>>(at); break;
                    case 8: attn_o_kernel<8><<<kAttnOGroups, 512, 0, stream>>>(at); break;
                    default: throw std::runtime_error("fused attention: context beyond 512 positions");
                }
                break;
            }
            int chunk, splits;
            attn_split(pos + 1, chunk, splits);
            require(splits > 1, "split attention: a single split takes the fused kernel");
            attn_decode_kernel<<<dim3(splits, kKVHeads), 512, 0, stream>>>(at);
            attn_merge_o_kernel<<<kAttnOGroups, 512, 0, stream>>>(at);
            break;
        }
        case 2:  // O runs with the attention (its per-head partials go to o_part)
            break;
        case 3: {
            if (flow.ffn_tag) {
                launch_ffn<1>(L, s.x, s.o_part, s.xm, s.dparts, s.exchange, s.stall, flow.ffn_tag, stream);
                break;
            }
            GemvArgs gu{};
            gu.w = L.gateup_t;
            gu.in = s.x;
            gu.norm_w = L.post_norm;
            gu.parts = s.o_part;
            gu.out = s.act;
            launch_gemv<kHidden, kGateUp>(gu, 2 * kFFN, stream);
            break;
        }
        case 4: {
            if (flow.ffn_tag) break;  // the fused FFN kernel ran the down projection
            GemvArgs d{};
            d.w = L.down_t;
            d.in = s.act;
            d.parts = s.o_part;
            d.x = s.x;
            launch_gemv<kFFN, kDown>(d, kHidden, stream);
            break;
        }
        default: throw std::runtime_error("unknown decode kernel");
    }
}


int attn_batch_pieces(const int* positions, int count, int* pieces_out, int& per) {
    require(count >= 1 && count <= kMaxBatch, "attention batch: 1..8 sequences");
    int longest = 1;
    for (int i = 0; i < count; ++i) longest = std::max(longest, positions[i]);
    const int pieces = std::min(kAttnSplits, std::max(1, 256 / (kKVHeads * count)));
    per = ((longest + 63) / 64 + pieces - 1) / pieces;
    require(per <= 16, "attention batch: more than 16 blocks per piece");
    for (int i = 0; i < count; ++i) {  // as the kernel splits each sequence
        const int blocks = (positions[i] + 63) / 64, own = (blocks + pieces - 1) / pieces;
        pieces_out[i] = (blocks + own - 1) / own;
    }
    return pieces;
}

void launch_attention_o_batch(const AttnSeq* seqs, int count, const uint16_t* w_qkv, const uint16_t* w_o,
                              const float* in_norm, const float* q_norm, const float* k_norm, const float* cosines,
                              const float* sines, uint64_t* words, int* stall, uint32_t tag, hipStream_t stream) {
    require(count >= 1 && count <= kMaxBatch, "attention batch: 1..8 sequences");
    require(tag != 0, "attention batch: exchange tags are nonzero");
    AttnBatchArgs b{};
    int positions[kMaxBatch];
    for (int i = 0; i < count; ++i) {
        AttnBatchSeq& a = b.seq[i];
        a.x = seqs[i].x;
        a.embed = seqs[i].embed;
        a.x_out = seqs[i].x_out;
        a.keys = seqs[i].keys;
        a.values = seqs[i].values;
        a.pos = seqs[i].pos;
        a.context = seqs[i].context;
        a.shared_keys = seqs[i].shared_keys;
        a.shared_values = seqs[i].shared_values;
        a.shared_context = seqs[i].shared_context;
        a.shared = seqs[i].shared;
        require(a.pos >= 0 && a.pos < a.context, "attention batch: position outside the cache");
        require(a.shared >= 0 && a.shared % 64 == 0 && a.shared <= a.pos && a.shared <= a.shared_context &&
                    (a.shared == 0 || (a.shared_keys != nullptr && a.shared_values != nullptr)),
                "attention batch: shared rows outside the caches");
        require(a.x != nullptr && a.x_out != nullptr && a.x_out != a.x, "attention batch: two residual buffers per sequence");
        positions[i] = a.pos + 1;
    }
    b.w_qkv = w_qkv;
    b.w_o = w_o;
    b.in_norm = in_norm;
    b.q_norm = q_norm;
    b.k_norm = k_norm;
    b.cosines = cosines;
    b.sines = sines;
    b.exchange = words;
    b.piece_words = words + kBatchPieceOffset;
    b.att_words = words + kBatchAttOffset;
    b.share_words = words + kBatchShareOffset;
    b.stall = stall;
    b.scale = 1.0f / std::sqrt(128.0f);
    b.batch = count;
    b.tag = tag;
    int pieces[kMaxBatch], per;
    b.pieces = attn_batch_pieces(positions, count, pieces, per);
    require(count * b.pieces <= 32, "attention batch: at most 32 attention workgroups per XCD");
    constexpr int kGrid = 256;  // 32 workgroups per XCD: one per QKV tile and per 32 O rows
    bool embed = b.seq[0].embed != nullptr;
    for (int i = 1; i < count; ++i)
        require((b.seq[i].embed != nullptr) == embed, "attention batch: embedding rows for all sequences or none");
    auto launch = [&](auto kernel) { kernel<<<kGrid, 512, 0, stream>>>(b); };
    if (embed) {
        if (per <= 2) launch(attn_batch_kernel<2, true>);
        else if (per <= 4) launch(attn_batch_kernel<4, true>);
        else if (per <= 6) launch(attn_batch_kernel<6, true>);
        else if (per <= 9) launch(attn_batch_kernel<9, true>);
        else if (per <= 12) launch(attn_batch_kernel<12, true>);
        else launch(attn_batch_kernel<16, true>);
    } else {
        if (per <= 2) launch(attn_batch_kernel<2, false>);
        else if (per <= 4) launch(attn_batch_kernel<4, false>);
        else if (per <= 6) launch(attn_batch_kernel<6, false>);
        else if (per <= 9) launch(attn_batch_kernel<9, false>);
        else if (per <= 12) launch(attn_batch_kernel<12, false>);
        else launch(attn_batch_kernel<16, false>);
    }
}

void launch_decode_layer(const LayerDevice& L, const uint16_t* embed, int pos, int token, const float* cosines,
                         const float* sines, int context, const DecodeScratch& s, LayerFlow flow, hipStream_t stream) {
    for (int which = 0; which < 5; ++which)
        launch_layer_kernel(which, L, which == 0 ? embed : nullptr, pos, token, cosines, sines, context, s, flow,
                            stream);
}

namespace {
// Final RMSNorm + tied lm_head + greedy selection in one launch: one
// workgroup per CU, 8 waves; wave v of workgroup w streams the chain-tiled
// 8-row tiles 8 w + v + 2048 k, the next tile's loads in flight while it
// forms the current tile's dots (the reference's chain order, the GEMV
// path's arithmetic: logits bit-identical to it). Every workgroup forms the
// norm itself and posts its best (value, lowest id, nonfinite) as two tagged
// words; workgroup 0 gathers the 256 candidates (through memory: they come
// from every XCD), selects, takes and clears the step's stall word and
// writes the result (the argmax kernel's outputs). The selection does not
// depend on the reduction order (greatest value, lowest id among equals).
// ROWS = 2: the two verification rows, every weight block read once for
// both (each row with a single row's arithmetic).
struct LmStreamArgs {
    GemvArgs g;       // in / hidden: row q at + q * 1024; out: row q at + q * out_stride
    uint64_t* words;  // [ROWS][kLmStreamGroups][2]
    uint32_t tag;
    ArgmaxResult* result;    // [ROWS]
    ArgmaxResult* host_out;  // [ROWS]
    int* stall;
    unsigned seq;
};

constexpr int kLmStreamWaves = 8, kLmTiles = kVocab / 8, kLmWaveCount = kLmStreamGroups * kLmStreamWaves;
static_assert(kLmTiles > kLmWaveCount, "every wave streams at least one tile");

template <int ROWS>
__global__ __launch_bounds__(64 * kLmStreamWaves) void lm_head_stream_kernel(const LmStreamArgs a) {
    static_assert(ROWS == 1 || ROWS == 2, "one or two rows");
    constexpr int N = kHidden, THREADS = 64 * kLmStreamWaves, PER = N / THREADS;
    __shared__ float4 xs4[ROWS][N / 4];
    __shared__ double red[ROWS][kLmStreamWaves];
    __shared__ float wbest[ROWS][kLmStreamWaves];
    __shared__ int wi[ROWS][kLmStreamWaves], wb[ROWS][kLmStreamWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 7, r = lane >> 3;
    float v[ROWS][PER], wn[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
#pragma unroll
        for (int q = 0; q < ROWS; ++q) v[q][k] = a.g.in[q * N + tid + k * THREADS];
        wn[k] = a.g.norm_w[tid + k * THREADS];
    }
    // This wave's tiles first, first + 2048, ...; the first one's loads go
    // out behind the norm inputs (loads complete in issue order). A rolling
    // stream: as soon as block b of a tile has entered its dots, block b of
    // the next tile is loaded into the same registers, so a whole tile stays
    // in flight per wave and each dot step waits for exactly the oldest block.
    constexpr int NB = N / 64;
    const int first = kLmStreamWaves * int(blockIdx.x) + wave;
    const int count = (kLmTiles - 1 - first) / kLmWaveCount + 1;
    u32x4 wv[NB];
    __builtin_amdgcn_sched_barrier(0);
    {
        // In block order, as the loop reloads them (the waits count on it).
        const u32x4* wp = reinterpret_cast<const u32x4*>(a.g.w) + size_t(first) * (NB * 64) + lane;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            wv[b] = __builtin_nontemporal_load(wp + b * 64);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int q = 0; q < ROWS; ++q)
        norm_to_lds<N, THREADS, false>(v[q], wn, reinterpret_cast<float*>(xs4[q]), red[q],
                                       blockIdx.x == 0 ? a.g.hidden + q * N : nullptr);
    __syncthreads();
    float bv[ROWS];
    int bi[ROWS], bad[ROWS];
#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        bv[q] = -INFINITY;
        bi[q] = INT_MAX;
        bad[q] = 0;
    }
    // Every lane of a row holds its sum (combine_chains), so all 8 store it
    // and take it into the selection: no divergent store, which keeps the
    // compiler's load waits exact.
    auto finish = [&](const float (&acc)[ROWS], int tile) {
        const int row = tile * 8 + r;
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            const float y = combine_chains(acc[q]);
            a.g.out[size_t(q) * a.g.out_stride + row] = y;
            bad[q] |= !__builtin_isfinite(y);
            if (better(y, row, bv[q], bi[q])) { bv[q] = y; bi[q] = row; }
        }
    };
    auto dot_step = [&](float (&acc)[ROWS], int b) {
#pragma unroll
        for (int q = 0; q < ROWS; ++q)
            acc[q] = chain8(acc[q], wv[b], xs4[q][16 * b + 2 * c], xs4[q][16 * b + 2 * c + 1]);
    };
    int tile = first;
    for (int k = 0; k + 1 < count; ++k, tile += kLmWaveCount) {
        const u32x4* wp = reinterpret_cast<const u32x4*>(a.g.w) + size_t(tile + kLmWaveCount) * (NB * 64) + lane;
        float acc[ROWS] = {};
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            dot_step(acc, b);
            wv[b] = __builtin_nontemporal_load(wp + b * 64);
            __builtin_amdgcn_sched_barrier(0);  // each reload right behind its block's dot steps
        }
        finish(acc, tile);
    }
    {
        float acc[ROWS] = {};
#pragma unroll
        for (int b = 0; b < NB; ++b) dot_step(acc, b);
        finish(acc, tile);
    }
#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        auto step = [&](auto off) {
            constexpr int kOff = decltype(off)::value;
            const float ov = xor_lanes<kOff>(bv[q]);
            const int oi = xor_lanes<kOff>(bi[q]);
            bad[q] |= xor_lanes<kOff>(bad[q]);
            if (better(ov, oi, bv[q], bi[q])) { bv[q] = ov; bi[q] = oi; }
        };
        step(std::integral_constant<int, 8>{});
        step(std::integral_constant<int, 16>{});
        step(std::integral_constant<int, 32>{});
        if (lane == 0) { wbest[q][wave] = bv[q]; wi[q][wave] = bi[q]; wb[q][wave] = bad[q]; }
    }
    __syncthreads();
    if (tid < ROWS) {
        const int q = tid;
        float cv = wbest[q][0];
        int ci = wi[q][0], cb = wb[q][0];
        for (int k = 1; k < kLmStreamWaves; ++k) {
            cb |= wb[q][k];
            if (better(wbest[q][k], wi[q][k], cv, ci)) { cv = wbest[q][k]; ci = wi[q][k]; }
        }
        uint64_t* mine = a.words + 2 * (size_t(q) * kLmStreamGroups + blockIdx.x);
        exchange_put_through(mine, cv, a.tag);
        exchange_put_through(mine + 1, __int_as_float((ci & 0x7fffffff) | (cb ? int(0x80000000u) : 0)), a.tag);
    }
    if (blockIdx.x != 0) return;

    // Workgroup 0: thread t < ROWS x 256 gathers row t / 256's candidate of
    // workgroup t % 256 (waves 0-3: row 0, waves 4-7: row 1).
    static_assert(ROWS * kLmStreamGroups <= THREADS, "one candidate per thread");
    float cv = -INFINITY;
    int ci = INT_MAX, cb = 0, lost = 0;
    if (tid < ROWS * kLmStreamGroups) {
        const uint64_t* const words[2] = {a.words + 2 * tid, a.words + 2 * tid + 1};
        float got[2] = {0.f, 0.f};
        if (exchange_gather_pipe<2, 6>(words, a.tag, got, 3u)) {
            const int packed = __float_as_int(got[1]);
            cv = got[0];
            ci = packed & 0x7fffffff;
            cb = packed < 0;
        } else {
            lost = 1;
        }
    }
    auto step2 = [&](auto off) {
        constexpr int kOff = decltype(off)::value;
        const float ov = xor_lanes<kOff>(cv);
        const int oi = xor_lanes<kOff>(ci);
        cb |= xor_lanes<kOff>(cb);
        lost |= xor_lanes<kOff>(lost);
        if (better(ov, oi, cv, ci)) { cv = ov; ci = oi; }
    };
    step2(std::integral_constant<int, 1>{});
    step2(std::integral_constant<int, 2>{});
    step2(std::integral_constant<int, 4>{});
    step2(std::integral_constant<int, 8>{});
    step2(std::integral_constant<int, 16>{});
    step2(std::integral_constant<int, 32>{});
    __syncthreads();  // wbest / wi / wb are reused
    if (lane == 0) { wbest[0][wave] = cv; wi[0][wave] = ci; wb[0][wave] = cb | (lost << 1); }
    __syncthreads();
    if (tid == 0) {
        // The step's stall word covers both rows (one launch wrote them).
        int flags_all = 0;
        for (int k = 0; k < kLmStreamWaves; ++k) flags_all |= wb[0][k] & 2;
        const int stalled = *a.stall | (flags_all >> 1);
        *a.stall = 0;
        for (int q = 0; q < ROWS; ++q) {
            constexpr int kWavesPerRow = kLmStreamGroups / 64;
            float qv = wbest[0][q * kWavesPerRow];
            int qi = wi[0][q * kWavesPerRow], flags = wb[0][q * kWavesPerRow];
            for (int k = 1; k < kWavesPerRow; ++k) {
                const int w = q * kWavesPerRow + k;
                flags |= wb[0][w];
                if (better(wbest[0][w], wi[0][w], qv, qi)) { qv = wbest[0][w]; qi = wi[0][w]; }
            }
            const int nonfinite = flags & 1;
            a.result[q].token = qi;
            a.result[q].nonfinite = nonfinite;
            a.result[q].stalled = stalled;
            a.host_out[q].token = qi;
            a.host_out[q].nonfinite = nonfinite;
            a.host_out[q].stalled = stalled;
            const unsigned long long word = (static_cast<unsigned long long>(a.seq) << 32) |
                                            (stalled ? 1ull << 31 : 0ull) | (nonfinite ? 1ull << 30 : 0ull) |
                                            (static_cast<unsigned>(qi) & 0x3fffffffu);
            __hip_atomic_store(&a.host_out[q].done, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}
}  // namespace

void launch_lm_head(const uint16_t* lm_t, const float* final_norm, const DecodeScratch& s, ArgmaxResult* host_out,
                    uint32_t tag, hipStream_t stream, unsigned seq) {
    LmStreamArgs a{};
    a.g.w = lm_t;
    a.g.in = s.x;
    a.g.norm_w = final_norm;
    a.g.out = s.logits;
    a.g.out_stride = kVocab;
    a.g.hidden = s.hidden;
    a.words = s.lm_words;
    a.tag = tag;
    a.result = s.result;
    a.host_out = host_out;
    a.stall = s.stall;
    a.seq = seq;
    lm_head_stream_kernel<1><<<kLmStreamGroups, 64 * kLmStreamWaves, 0, stream>>>(a);
}

void launch_lm_head_pair(const uint16_t* lm_t, const float* final_norm, const DecodeScratch& s,
                         const PairScratch& pr, ArgmaxResult* host_out, uint32_t tag, hipStream_t stream,
                         unsigned seq) {
    LmStreamArgs a{};
    a.g.w = lm_t;
    a.g.in = pr.x;
    a.g.norm_w = final_norm;
    a.g.out = pr.logits;
    a.g.out_stride = kVocab;
    a.g.hidden = pr.hidden;
    a.words = s.lm_words;
    a.tag = tag;
    a.result = pr.result;
    a.host_out = host_out;
    a.stall = s.stall;
    a.seq = seq;
    lm_head_stream_kernel<2><<<kLmStreamGroups, 64 * kLmStreamWaves, 0, stream>>>(a);
}

void launch_norm_qkv(const uint16_t* qkv_t, const float* norm_w, const float* x, float* qkv, hipStream_t stream) {
    GemvArgs q{};
    q.w = qkv_t;
    q.in = x;
    q.norm_w = norm_w;
    q.out = qkv;
    launch_gemv<kHidden, kQKV>(q, kQKVRows, stream);
}

void launch_norm_gate_up(const uint16_t* gateup_t, const float* norm_w, const float* x, const float* parts,
                         float* act, float* raw, hipStream_t stream) {
    GemvArgs gu{};
    gu.raw = raw;
    gu.w = gateup_t;
    gu.in = x;
    gu.norm_w = norm_w;
    gu.parts = parts;
    gu.out = act;
    launch_gemv<kHidden, kGateUp>(gu, 2 * kFFN, stream);
}

namespace {
// x[q][j] = xm[q][j] + the 8 down slices of row j (fixed tree order): the
// residual after a layer whose FFN ran as the fused kernel.
__global__ __launch_bounds__(kHidden) void fold_residual_kernel(const float* __restrict__ xm,
                                                                const float* __restrict__ dparts, float* x) {
    const int q = blockIdx.x, j = threadIdx.x;
    float d[kFfnSlices];
#pragma unroll
    for (int g = 0; g < kFfnSlices; ++g) d[g] = dparts[(q * kFfnSlices + g) * kHidden + j];
    x[q * kHidden + j] = fold_slices(xm[q * kHidden + j], d);
}
}  // namespace

void launch_fold_residual(const float* xm, const float* dparts, float* x, int rows, hipStream_t stream) {
    require(rows == 1 || rows == 2, "fold: one or two rows");
    fold_residual_kernel<<<rows, kHidden, 0, stream>>>(xm, dparts, x);
}

void launch_fused_ffn(const uint16_t* gateup_t, const uint16_t* down_t, const float* norm_w, const float* x,
                      const float* parts, float* xm, float* dparts, uint64_t* exchange, int* stall, uint32_t tag,
                      hipStream_t stream) {
    launch_ffn_rows<1>(gateup_t, down_t, norm_w, x, parts, xm, dparts, exchange, stall, tag, stream);
}

void launch_norm_qkv_folded(const uint16_t* qkv_t, const float* norm_w, const float* xm, const float* dparts,
                            float* x, float* qkv, hipStream_t stream) {
    GemvArgs q{};
    q.w = qkv_t;
    q.in = xm;
    q.parts = dparts;
    q.norm_w = norm_w;
    q.out = qkv;
    q.x = x;
    launch_gemv<kHidden, kQKV>(q, kQKVRows, stream);
}

void launch_down_residual(const uint16_t* down_t, const float* act, const float* parts, float* x,
                          hipStream_t stream) {
    GemvArgs d{};
    d.w = down_t;
    d.in = act;
    d.parts = parts;
    d.x = x;
    launch_gemv<kFFN, kDown>(d, kHidden, stream);
}

}  // namespace qwen_hip

namespace qwen_hip {
namespace {
__global__ void copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
        dst[i] = src[i];
}
}  // namespace

void launch_copy(const void* src, void* dst, size_t bytes, hipStream_t stream) {
    require(bytes % 16 == 0, "copy: bytes must be a multiple of 16");
    const size_t n = bytes / 16;
    const unsigned blocks = unsigned(std::min<size_t>((n + 255) / 256, 8192));
    if (n) copy_kernel<<<blocks, 256, 0, stream>>>(static_cast<const uint4*>(src), static_cast<uint4*>(dst), n);
}
}  // namespace qwen_hip
