// Batched decode: one step for up to 8 independent sequences that share the
// weights (the prefix-reuse serving workload). The reference is
// single-stream; per sequence this computes what qwen_cpu::Model::step does
// (engine/core.cpp:353-646, 707-714), but every projection reads each weight
// matrix once for all rows: a skinny GEMM on the matrix cores instead of one
// GEMV per sequence.
//
// Skinny GEMM (bgemv_kernel): Y[b][o] = sum_k X[b][k] W[o][k], W natural
// row-major FP16, b < 8. Workgroup = 16 output rows per MFMA tile (one
// 16x16x32 tile, A = W rows, B = X^T with the 8 sequences in columns 0..7;
// the lm_head takes 4 tiles per workgroup) and one wave per 256 columns of K
// (4, 8 or 12 waves: a wave retires about one 1 KiB load per 100 ns, so the
// inputs and weights a workgroup streams are spread over that many waves);
// the waves' parts are summed in LDS in a fixed order. X enters the matrix cores
// as FP16 hi + lo (hi = fp16(x), lo = fp16(x - hi)), so the products are
// exact and the sums FP32, as in the prefill GEMMs. In each weight load the 4
// lanes of a tile row read 64 contiguous bytes (the summation order inside a
// 128-wide K block is a fixed permutation of k, applied to A and B alike).
// RMSNorm prologues (FP32 squares, FP64 sums per row) and the residual /
// SwiGLU / argmax epilogues are fused as in the batch-1 kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>

#include "batch.hpp"
#include "decode_dev.hpp"
#include "half_split.hpp"

namespace qwen_hip {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;  // waves of the K = 1024 kernels (norm prologues, lm_head)
using dev::xor_lanes;

__device__ __forceinline__ float h2f(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

enum BatchMode { kBPlain, kBQKV, kBO, kBGateUp, kBDown, kBLmHead };

struct BatchGemvArgs {
    const uint16_t* w;                 // natural [rows x K]; gate/up: 3072 gate rows then 3072 up rows
    const float* norm_w;               // RMSNorm weights (QKV, gate/up, lm_head)
    const float* in[kMaxBatch];        // input rows: x (norm modes), attention output (O), activation (down)
    const uint16_t* embed[kMaxBatch];  // QKV of the first layer: embedding rows instead of x
    float* out[kMaxBatch];             // output rows (plain, QKV, gate/up: activation, lm_head: logits)
    float* x[kMaxBatch];               // residual rows (O and down add; first layer stores E[token])
    float* hidden[kMaxBatch];          // lm_head: final normalized rows
    float* lm_value;                   // lm_head argmax partials [groups][kMaxBatch]
    int* lm_index;
    int* lm_bad;
    float* slices[kMaxBatch];          // down with K slices: [3][1024] partial sums per sequence (output)
    const float* pending[kMaxBatch];   // QKV, O: the previous layer's down slices still to add, or null
    int batch;
};

// RT = 16-row MFMA tiles per workgroup (gate/up: the gate tile and the
// matching up tile). The prologue loads every input row as float4 (thread t
// holds elements 4 t .. 4 t + 3), sums the squares of all rows in one
// pass (one barrier for the 8 norms) and stages FP16 hi / lo with 8-byte LDS
// stores; the weights are issued right after the inputs, so their HBM round
// trip overlaps the prologue.
// SPLITK > 1 (down): workgroup (tile, blockIdx.y) multiplies one slice of
// K / SPLITK = 1024 columns and stores its partial sums in the sequence's
// slice buffer; the next layer's QKV prologue adds them to the residual it
// normalizes, and its O epilogue adds them into the residual stream (both in
// slice order), so no workgroup waits for another.
template <int K, int MODE, int RT = 1, int SPLITK = 1>
__global__ __launch_bounds__(K / SPLITK / 4) void bgemv_kernel(const BatchGemvArgs a) {
    constexpr bool kNorm = MODE == kBQKV || MODE == kBGateUp || MODE == kBLmHead;
    constexpr int kTiles = MODE == kBGateUp ? 2 : RT;
    static_assert(MODE == kBGateUp ? RT == 1 : RT >= 1, "gate/up pairs one gate tile with one up tile");
    static_assert(SPLITK == 1 || (MODE == kBDown && SPLITK == kBatchSplitMax && RT == 1),
                  "K slices for the down projection");
    constexpr int KS = K / SPLITK;  // this workgroup's columns
    constexpr int WAVES = KS / 256, THREADS = 64 * WAVES, KW = 256, kBlocks = KW / 128, F4 = 1;
    static_assert(KS % 1024 == 0 && (!kNorm || WAVES == kWaves), "one wave per 256 columns; norms with 4 waves");
    const int k0 = KS * int(blockIdx.y);
    __shared__ __align__(16) _Float16 xh[kMaxBatch][KS + 8];
    __shared__ __align__(16) _Float16 xl[kMaxBatch][KS + 8];
    __shared__ double red[kWaves][kMaxBatch];
    __shared__ float part[WAVES][kTiles][64][4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, quad = lane >> 4;
    const int B = a.batch, o0 = blockIdx.x * (kBatchRows * RT);
    // Epilogue elements of this thread: row o0 + 16 t + 4 (l / 16) + r,
    // sequence l % 16 of each 16x16 accumulator (r = wave, l = lane).
    const int eb = lane & 15, erow = 4 * (lane >> 4) + (wave & 3);  // waves 0..3 run the epilogue

    // Loads complete in issue order per wave: inputs first (rows past the
    // batch repeat row B - 1 and are never stored), then norm weights and
    // residual entries, then the weights.
    float4 v[kMaxBatch][F4];
#pragma unroll
    for (int b = 0; b < kMaxBatch; ++b) {
        const int bb = min(b, B - 1);
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const int j4 = tid + THREADS * i;
            if constexpr (MODE == kBQKV) {
                if (a.embed[bb]) {
                    const uint2 e = reinterpret_cast<const uint2*>(a.embed[bb])[j4];
                    v[b][i] = make_float4(h2f(e.x & 0xffffu), h2f(e.x >> 16), h2f(e.y & 0xffffu), h2f(e.y >> 16));
                    continue;
                }
            }
            v[b][i] = reinterpret_cast<const float4*>(a.in[bb] + k0)[j4];
        }
    }
    if constexpr (MODE == kBQKV) {
        // The residual the norm sees: x plus the previous layer's down slices
        // (((s0 + s1) + s2), added as the O epilogue will add them).
        float4 sl[kMaxBatch][kBatchSplitMax];
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b) {
            const int bb = min(b, B - 1);
            if (a.pending[bb]) {
#pragma unroll
                for (int z = 0; z < kBatchSplitMax; ++z)
                    sl[b][z] = reinterpret_cast<const float4*>(a.pending[bb] + z * kHidden)[tid];
            }
        }
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b) {
            const int bb = min(b, B - 1);
            if (a.pending[bb]) {
                const float4 s01 = make_float4(sl[b][0].x + sl[b][1].x, sl[b][0].y + sl[b][1].y,
                                               sl[b][0].z + sl[b][1].z, sl[b][0].w + sl[b][1].w);
                v[b][0] = make_float4(v[b][0].x + (s01.x + sl[b][2].x), v[b][0].y + (s01.y + sl[b][2].y),
                                      v[b][0].z + (s01.z + sl[b][2].z), v[b][0].w + (s01.w + sl[b][2].w));
            }
        }
    }
    float4 wn[F4];
    if constexpr (kNorm) {
#pragma unroll
        for (int i = 0; i < F4; ++i) wn[i] = reinterpret_cast<const float4*>(a.norm_w)[tid + THREADS * i];
    }
    float xres = 0.f, pend[kBatchSplitMax] = {};
    if constexpr (MODE == kBO || (MODE == kBDown && SPLITK == 1)) xres = a.x[min(eb, B - 1)][o0 + erow];
    if constexpr (MODE == kBO) {
        const float* pb = a.pending[min(eb, B - 1)];
        if (pb) {
#pragma unroll
            for (int z = 0; z < kBatchSplitMax; ++z) pend[z] = pb[z * kHidden + o0 + erow];
        }
    }
    u32x4 wa[kTiles][kBlocks][4];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        const int row = MODE == kBGateUp ? o0 + col + (t ? kFFN : 0) : o0 + kBatchRows * t + col;
        const u32x4* wp = reinterpret_cast<const u32x4*>(a.w + size_t(row) * K + k0 + wave * KW) + quad;
#pragma unroll
        for (int blk = 0; blk < kBlocks; ++blk)
#pragma unroll
            for (int s = 0; s < 4; ++s) wa[t][blk][s] = __builtin_nontemporal_load(wp + 16 * blk + 4 * s);
    }
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (kNorm) {
        // RMSNorm per row (engine/core.cpp:207-215): FP32 squares summed in
        // FP64. A reduce-scatter inside each wave halves the rows a lane
        // carries at each of the exchanges over lane bits 5, 4 and 3, then
        // sums over bits 2..0, so lane l ends with the wave's total of row
        // (l >> 3) & 7; the 4 wave totals of a row are added by one thread,
        // which also forms the row's scale once.
        double sq[kMaxBatch];
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b) {
            double s = 0.0;
#pragma unroll
            for (int i = 0; i < F4; ++i) {
                const float e[4] = {v[b][i].x, v[b][i].y, v[b][i].z, v[b][i].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float square = e[k] * e[k];
                    s += static_cast<double>(square);
                }
            }
            sq[b] = s;
        }
        const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
        double r4[4], r2[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // keep rows 4 b5 + i, send the others
            const double keep = b5 ? sq[4 + i] : sq[i], send = b5 ? sq[i] : sq[4 + i];
            r4[i] = keep + xor_lanes<32>(send);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {  // rows 4 b5 + 2 b4 + i
            const double keep = b4 ? r4[2 + i] : r4[i], send = b4 ? r4[i] : r4[2 + i];
            r2[i] = keep + xor_lanes<16>(send);
        }
        double r1 = (b3 ? r2[1] : r2[0]) + xor_lanes<8>(b3 ? r2[0] : r2[1]);  // row (lane >> 3) & 7
        r1 += xor_lanes<4>(r1);
        r1 += xor_lanes<2>(r1);
        r1 += xor_lanes<1>(r1);
        if ((lane & 7) == 0) red[wave][lane >> 3] = r1;
        __syncthreads();
        __shared__ float inv_row[kMaxBatch];
        if (tid < kMaxBatch) {
            const double total = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
            inv_row[tid] = 1.0f / __builtin_sqrtf(static_cast<float>(total) / static_cast<float>(K) + 1e-6f);
        }
        if constexpr (MODE == kBQKV) {
            if (blockIdx.x == 0) {  // first layer: keep fp32(E[token]) as the residual stream
#pragma unroll
                for (int b = 0; b < kMaxBatch; ++b)
                    if (b < B && a.embed[b]) {
#pragma unroll
                        for (int i = 0; i < F4; ++i) reinterpret_cast<float4*>(a.x[b])[tid + THREADS * i] = v[b][i];
                    }
            }
        }
        __syncthreads();
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b) {
            const float inv = inv_row[b];
#pragma unroll
            for (int i = 0; i < F4; ++i) {
                v[b][i].x = (v[b][i].x * inv) * wn[i].x;
                v[b][i].y = (v[b][i].y * inv) * wn[i].y;
                v[b][i].z = (v[b][i].z * inv) * wn[i].z;
                v[b][i].w = (v[b][i].w * inv) * wn[i].w;
            }
        }
        if constexpr (MODE == kBLmHead) {
            if (blockIdx.x == 0) {
#pragma unroll
                for (int b = 0; b < kMaxBatch; ++b)
                    if (b < B) {
#pragma unroll
                        for (int i = 0; i < F4; ++i) reinterpret_cast<float4*>(a.hidden[b])[tid + THREADS * i] = v[b][i];
                    }
            }
        }
    }
#pragma unroll
    for (int b = 0; b < kMaxBatch; ++b)
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const float e[4] = {v[b][i].x, v[b][i].y, v[b][i].z, v[b][i].w};
            half4 hi, lo;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                _Float16 h, l;
                split_half(e[k], h, l);
                hi[k] = h;
                lo[k] = l;
            }
            const int j = 4 * (tid + THREADS * i);
            *reinterpret_cast<half4*>(&xh[b][j]) = hi;
            *reinterpret_cast<half4*>(&xl[b][j]) = lo;
        }
    __syncthreads();

    floatx4 acc[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    const half8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int blk = 0; blk < kBlocks; ++blk)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            // k slot (quad, i) of step s holds k = 128 blk + 32 s + 8 quad + i of this wave's range
            // (each weight load reads 64 contiguous bytes of every tile row).
            const int k = wave * KW + 128 * blk + 32 * s + 8 * quad;
            const half8 bh = col < kMaxBatch ? *reinterpret_cast<const half8*>(&xh[col & 7][k]) : zero;
            const half8 bl = col < kMaxBatch ? *reinterpret_cast<const half8*>(&xl[col & 7][k]) : zero;
#pragma unroll
            for (int t = 0; t < kTiles; ++t) {
                const half8 w8 = __builtin_bit_cast(half8, wa[t][blk][s]);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w8, bh, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w8, bl, acc[t], 0, 0, 0);
            }
        }
#pragma unroll
    for (int t = 0; t < kTiles; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) part[wave][t][lane][r] = acc[t][r];
    __syncthreads();

    // The waves' K parts of each output, summed in a fixed order (pairs,
    // then pairs of pairs; a third group of four comes last).
    if (wave >= 4) return;
    float y[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        auto quad_sum = [&](int w0) {
            return (part[w0][t][lane][wave] + part[w0 + 1][t][lane][wave]) +
                   (part[w0 + 2][t][lane][wave] + part[w0 + 3][t][lane][wave]);
        };
        y[t] = quad_sum(0);
        if constexpr (WAVES >= 8) y[t] = y[t] + quad_sum(4);
        if constexpr (WAVES >= 12) y[t] = y[t] + quad_sum(8);
        static_assert(WAVES == 4 || WAVES == 8 || WAVES == 12, "4, 8 or 12 waves");
    }
    const bool live = eb < B;
    const int eo = o0 + erow;
    if constexpr (MODE == kBPlain || MODE == kBQKV) {
        if (live) a.out[eb][eo] = y[0];
    } else if constexpr (MODE == kBO) {
        if (live) {
            const float base = a.pending[eb] ? xres + ((pend[0] + pend[1]) + pend[2]) : xres;
            a.x[eb][eo] = base + y[0];
        }
    } else if constexpr (MODE == kBDown) {
        if (live) {
            if constexpr (SPLITK == 1) a.x[eb][eo] = xres + y[0];
            else a.slices[eb][blockIdx.y * kHidden + eo] = y[0];
        }
    } else if constexpr (MODE == kBGateUp) {
        if (live) {  // SwiGLU (engine/core.cpp:636-639)
            const float gate = y[0], up = y[1];
            const float half_gate = gate * 0.5f;
            const float th = tanhf(half_gate);
            a.out[eb][eo] = gate * (0.5f + 0.5f * th) * up;
        }
    } else if constexpr (MODE == kBLmHead) {
        // Per-sequence argmax over this workgroup's rows: lowest id among
        // maxima, nonfinite values flagged (engine/main.cpp:51-59).
        float bv = -INFINITY;
        int bi = INT_MAX, bad = 0;
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            const int row = eo + kBatchRows * t;
            if (live) {
                a.out[eb][row] = y[t];
                bad |= !__builtin_isfinite(y[t]);
                if (better(y[t], row, bv, bi)) { bv = y[t]; bi = row; }
            }
        }
#pragma unroll
        for (int off = 16; off < 64; off <<= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            bad |= __shfl_xor(bad, off);
            if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        __shared__ float mv[kWaves][16];
        __shared__ int mi[kWaves][16], mb[kWaves][16];
        if (lane < 16) { mv[wave][lane] = bv; mi[wave][lane] = bi; mb[wave][lane] = bad; }
        __syncthreads();
        if (tid < B) {
            float v0 = mv[0][tid];
            int i0 = mi[0][tid], b0 = mb[0][tid];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) {
                b0 |= mb[w][tid];
                if (better(mv[w][tid], mi[w][tid], v0, i0)) { v0 = mv[w][tid]; i0 = mi[w][tid]; }
            }
            const size_t slot = size_t(blockIdx.x) * kMaxBatch + tid;
            a.lm_value[slot] = v0;
            a.lm_index[slot] = i0;
            a.lm_bad[slot] = b0;
        }
    }
}

// Second pass of the per-sequence greedy selection.
struct BatchResults {
    ArgmaxResult* device[kMaxBatch];
    ArgmaxResult* host[kMaxBatch];
    int* stall[kMaxBatch];  // the sequence's stall flag: copied to its result, then cleared
};

__global__ __launch_bounds__(1024) void batch_argmax_kernel(const float* __restrict__ value,
                                                            const int* __restrict__ index,
                                                            const int* __restrict__ bad_in, BatchResults out) {
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = -INFINITY;
    int bi = INT_MAX, bad = 0;
    for (int k = tid; k < kBatchLmGroups; k += 1024) {
        const size_t slot = size_t(k) * kMaxBatch + b;
        bad |= bad_in[slot];
        if (better(value[slot], index[slot], bv, bi)) { bv = value[slot]; bi = index[slot]; }
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        bad |= __shfl_xor(bad, off);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    __shared__ float wv[16];
    __shared__ int wi[16], wb[16];
    if (lane == 0) { wv[wave] = bv; wi[wave] = bi; wb[wave] = bad; }
    __syncthreads();
    if (tid == 0) {
        for (int k = 1; k < 16; ++k) {
            bad |= wb[k];
            if (better(wv[k], wi[k], bv, bi)) { bv = wv[k]; bi = wi[k]; }
        }
        const int stalled = *out.stall[b];
        *out.stall[b] = 0;
        out.device[b]->token = bi;
        out.device[b]->nonfinite = bad;
        out.device[b]->stalled = stalled;
        out.host[b]->token = bi;
        out.host[b]->nonfinite = bad;
        out.host[b]->stalled = stalled;
    }
}

template <int K, int MODE, int RT = 1, int SPLITK = 1>
void bgemv(const BatchGemvArgs& a, int rows, hipStream_t stream) {
    require(a.batch >= 1 && a.batch <= kMaxBatch, "batched GEMV: 1..8 rows");
    require(rows % (kBatchRows * RT) == 0 && rows > 0, "batched GEMV: rows must be a positive multiple of the tile rows");
    require(SPLITK == 1 || rows == kHidden, "batched GEMV: K slices for the down projection only");
    bgemv_kernel<K, MODE, RT, SPLITK><<<dim3(rows / (kBatchRows * RT), SPLITK), K / SPLITK / 4, 0, stream>>>(a);
}

}  // namespace

void launch_bgemv_plain(const uint16_t* w, const float* x, float* y, int batch, int rows, int cols,
                        hipStream_t stream) {
    BatchGemvArgs a{};
    a.w = w;
    a.batch = batch;
    for (int b = 0; b < batch; ++b) {
        a.in[b] = x + size_t(b) * cols;
        a.out[b] = y + size_t(b) * rows;
    }
    switch (cols) {
        case 1024: bgemv<1024, kBPlain>(a, rows, stream); break;
        case 2048: bgemv<2048, kBPlain>(a, rows, stream); break;
        case 3072: bgemv<3072, kBPlain>(a, rows, stream); break;
        default: throw std::runtime_error("batched GEMV: cols must be 1024, 2048 or 3072");
    }
}

void launch_decode_batch(const BatchSeq* seqs, int count, const uint16_t* embed, const float* final_norm,
                         const float* cosines, const float* sines, hipStream_t stream) {
    require(count >= 1 && count <= kMaxBatch, "batched decode: 1..8 sequences");
    for (int l = 0; l < kLayers; ++l) {
        const LayerDevice& W = seqs[0].layers[l];  // weights are shared; K/V are per sequence
        BatchGemvArgs q{};
        q.w = W.qkv_n;
        q.norm_w = W.in_norm;
        q.batch = count;
        for (int b = 0; b < count; ++b) {
            const DecodeScratch& s = seqs[b].s;
            q.in[b] = s.x;
            q.embed[b] = l == 0 ? embed + size_t(seqs[b].token) * kHidden : nullptr;
            q.out[b] = s.qkv;
            q.x[b] = s.x;
            q.pending[b] = l > 0 ? s.o_part : nullptr;  // the previous layer's down slices
        }
        bgemv<kHidden, kBQKV>(q, kQKVRows, stream);

        AttnSeq as[kMaxBatch];
        for (int b = 0; b < count; ++b) {
            const DecodeScratch& s = seqs[b].s;
            as[b] = AttnSeq{s.qkv,   seqs[b].layers[l].keys, seqs[b].layers[l].values, s.xpart,
                            s.attended, s.stall, seqs[b].pos, seqs[b].context, seqs[b].tags[l]};
        }
        launch_attention_batch(as, count, W.q_norm, W.k_norm, cosines, sines, stream);

        BatchGemvArgs o{};
        o.w = W.o_n;
        o.batch = count;
        for (int b = 0; b < count; ++b) {
            o.in[b] = seqs[b].s.attended;
            o.x[b] = seqs[b].s.x;
            o.pending[b] = l > 0 ? seqs[b].s.o_part : nullptr;
        }
        bgemv<kQDim, kBO>(o, kHidden, stream);

        BatchGemvArgs gu{};
        gu.w = W.gateup_n;
        gu.norm_w = W.post_norm;
        gu.batch = count;
        for (int b = 0; b < count; ++b) {
            gu.in[b] = seqs[b].s.x;
            gu.out[b] = seqs[b].s.act;
        }
        bgemv<kHidden, kBGateUp>(gu, kFFN, stream);

        BatchGemvArgs d{};
        d.w = W.down_n;
        d.batch = count;
        for (int b = 0; b < count; ++b) {
            d.in[b] = seqs[b].s.act;
            d.x[b] = seqs[b].s.x;
            d.slices[b] = seqs[b].s.o_part;  // [3][1024] of the sequence's partial buffer
        }
        // K slices leave their partial sums for the next layer; the last
        // layer's down adds into the residual itself (the lm_head reads it).
        if (l + 1 < kLayers)
            bgemv<kFFN, kBDown, 1, kBatchSplitMax>(d, kHidden, stream);
        else
            bgemv<kFFN, kBDown>(d, kHidden, stream);
    }
    BatchGemvArgs lm{};
    lm.w = embed;  // tied head (engine/core.cpp:643-645)
    lm.norm_w = final_norm;
    lm.batch = count;
    const DecodeScratch& s0 = seqs[0].s;
    lm.lm_value = s0.lm_value;
    lm.lm_index = s0.lm_index;
    lm.lm_bad = s0.lm_bad;
    BatchResults res{};
    for (int b = 0; b < count; ++b) {
        lm.in[b] = seqs[b].s.x;
        lm.out[b] = seqs[b].s.logits;
        lm.hidden[b] = seqs[b].s.hidden;
        res.device[b] = seqs[b].s.result;
        res.host[b] = seqs[b].host_out;
        res.stall[b] = seqs[b].s.stall;
    }
    bgemv<kHidden, kBLmHead, kBatchLmTiles>(lm, kVocab, stream);
    batch_argmax_kernel<<<count, 1024, 0, stream>>>(s0.lm_value, s0.lm_index, s0.lm_bad, res);
}

}  // namespace qwen_hip
