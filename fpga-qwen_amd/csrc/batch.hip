// Batched decode: one step for up to 8 independent sequences that share the
// weights (the prefix-reuse serving workload). The reference is
// single-stream; per sequence this computes what qwen_cpu::Model::step does
// (engine/core.cpp:353-646, 707-714), but every projection reads each weight
// matrix once for all sequences, on the matrix cores.
//
// A step is 28 pairs of launches of 256 workgroups (one per CU), then the
// head:
//  * attention (decode.hip, attn_batch_kernel): RMSNorm + QKV + QK-norm /
//    RoPE + attention over 64-position blocks + merge of the position pieces
//    + O + residual;
//  * FFN (ffn_batch_kernel, below): RMSNorm + gate/up + SwiGLU + down +
//    residual;
//  * lm_head_batch_kernel (final norm + tied head + per-workgroup best) and
//    batch_argmax_kernel (per-sequence greedy selection).
// Workgroup w runs on XCD w % 8; values move between workgroups as tagged
// words inside an XCD (its L2) or, for the residual shares, between XCDs.
// Every matrix product is v_mfma_f32_16x16x32_f16 with A = 16 weight rows
// (the 4 lanes of a row reading 64 contiguous bytes per load) and B = the 8
// sequences' inputs as FP16 hi + lo (hi = fp16(x), lo = fp16(x - hi)) in
// columns 0..7, so the products are exact and the sums FP32; a kernel's
// waves split K and their parts are added in a fixed order.
//
// bgemv_kernel is the plain skinny GEMM (Y[b] = W X[b], b < 8) behind the
// batched-GEMV parity entry.
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
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

using dev::exchange_gather;
using dev::exchange_gather_pipe;
using dev::masked_b;
using dev::exchange_put;
using dev::exchange_put_through;
using dev::xor_lanes;

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

struct BatchGemvArgs {
    const uint16_t* w;                 // natural [rows x K]
    const float* in[kMaxBatch];        // input rows
    float* out[kMaxBatch];             // output rows
    int batch;
};

// Y[b] = W X[b] on the matrix cores: one 16-row tile per workgroup, one
// wave per 256 columns. Every input row is loaded as float4 (thread t holds
// elements 4 t .. 4 t + 3) and staged in LDS as FP16 hi / lo; the weights
// are issued right after the inputs, so their HBM round trip overlaps the
// staging, and the waves' K parts are summed in a fixed order.
template <int K>
__global__ __launch_bounds__(K / 4) void bgemv_kernel(const BatchGemvArgs a) {
    constexpr int WAVES = K / 256, KW = 256, kBlocks = KW / 128;
    static_assert(WAVES == 4 || WAVES == 8 || WAVES == 12, "4, 8 or 12 waves");
    __shared__ __align__(16) _Float16 xh[kMaxBatch][K + 8];
    __shared__ __align__(16) _Float16 xl[kMaxBatch][K + 8];
    __shared__ float part[WAVES][64][4];
    __shared__ dev::SplitGuard guard;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, quad = lane >> 4;
    const int B = a.batch, o0 = blockIdx.x * kBatchRows;
    guard.init(tid);

    // Loads complete in issue order per wave: inputs first (rows past the
    // batch repeat row B - 1 and are never stored), then the weights.
    float4 v[kMaxBatch];
#pragma unroll
    for (int b = 0; b < kMaxBatch; ++b) v[b] = reinterpret_cast<const float4*>(a.in[min(b, B - 1)])[tid];
    u32x4 wa[kBlocks][4];
    __builtin_amdgcn_sched_barrier(0);
    {
        const u32x4* wp = reinterpret_cast<const u32x4*>(a.w + size_t(o0 + col) * K + wave * KW) + quad;
#pragma unroll
        for (int blk = 0; blk < kBlocks; ++blk)
#pragma unroll
            for (int s = 0; s < 4; ++s) wa[blk][s] = __builtin_nontemporal_load(wp + 16 * blk + 4 * s);
    }
    __builtin_amdgcn_sched_barrier(0);
    auto split_rows = [&](bool scaled) {
        float big = 0.f;
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b) {
            const float down = scaled ? pow2(-guard.seq_e[b]) : 1.f;
            const float e[4] = {v[b].x, v[b].y, v[b].z, v[b].w};
            half4 hi, lo;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                big = fmaxf(big, fabsf(e[k]));
                _Float16 h, l;
                split_half(e[k] * down, h, l);
                hi[k] = h;
                lo[k] = l;
            }
            *reinterpret_cast<half4*>(&xh[b][4 * tid]) = hi;
            *reinterpret_cast<half4*>(&xl[b][4 * tid]) = lo;
        }
        return big;
    };
    guard.post(split_rows(false), lane, wave);
    __syncthreads();
    if (guard.needed(WAVES)) {
#pragma unroll
        for (int b = 0; b < kMaxBatch; ++b)
            guard.offer(b, fmaxf(fmaxf(fabsf(v[b].x), fabsf(v[b].y)), fmaxf(fabsf(v[b].z), fabsf(v[b].w))));
        __syncthreads();
        if (tid < kMaxBatch) guard.seq_e[tid] = guard.exponent(tid);
        __syncthreads();
        split_rows(true);
        __syncthreads();
    }

    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int blk = 0; blk < kBlocks; ++blk)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            // k slot (quad, i) of step s holds k = 128 blk + 32 s + 8 quad + i of this wave's range
            // (each weight load reads 64 contiguous bytes of every tile row).
            const int k = wave * KW + 128 * blk + 32 * s + 8 * quad;
            const half8 bh = masked_b<half8>(&xh[col & 7][k], col < kMaxBatch);
            const half8 bl = masked_b<half8>(&xl[col & 7][k], col < kMaxBatch);
            const half8 w8 = __builtin_bit_cast(half8, wa[blk][s]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w8, bh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w8, bl, acc, 0, 0, 0);
        }
#pragma unroll
    for (int r = 0; r < 4; ++r) part[wave][lane][r] = acc[r];
    __syncthreads();

    // Element (row o0 + 4 (lane / 16) + wave, sequence lane % 16) for
    // waves 0..3: the waves' K parts in fixed order (pairs, then pairs of
    // pairs; further groups of four after).
    if (wave >= 4) return;
    auto quad_sum = [&](int w0) {
        return (part[w0][lane][wave] + part[w0 + 1][lane][wave]) + (part[w0 + 2][lane][wave] + part[w0 + 3][lane][wave]);
    };
    float y = quad_sum(0);
    if constexpr (WAVES >= 8) y = y + quad_sum(4);
    if constexpr (WAVES >= 12) y = y + quad_sum(8);
    const int eb = lane & 15;
    if (eb < B) a.out[eb][o0 + 4 * (lane >> 4) + wave] = y * guard.up(eb & 7);
}

// Norm + gate/up + SwiGLU + down + residual of one layer for the batched
// step in one launch (engine/core.cpp:627-641). 256 workgroups of 512
// threads, one per CU; XCD x owns activation columns 384 x .. 384 x + 383:
//  1. every workgroup forms RMSNorm(x) of all sequences (FP32 squares summed
//     in FP64) as FP16 hi + lo in LDS;
//  2. workgroup r of XCD x computes the 12 gate and 12 up rows of columns
//     384 x + 12 r .. + 11 on the matrix cores (two 16-row tiles, 4 rows of
//     each unused; the 8 waves split K, summed in a fixed tree), applies
//     SwiGLU (636-639) and posts the activations as tagged words in the
//     XCD's L2;
//  3. it gathers the XCD's 384 x 8 activations and multiplies them by down
//     rows 32 r .. 32 r + 31, columns 384 x .. + 383 (this XCD's share of K);
//  4. the 8 shares of a row, one per XCD, travel through memory (stores that
//     write through the L2, loads that bypass it; each XCD's shares of a
//     workgroup's rows fill whole lines), and workgroup (r, x) adds rows
//     32 r .. 32 r + 31 of sequence x in fixed order ((s0 + s1) + (s2 + s3))
//     + ((s4 + s5) + (s6 + s7)) to the residual (whole lines again).
// Every workgroup reads all of the input residual, so the output goes to a
// second buffer (the layers alternate between the two).
struct BatchFfnArgs {
    const uint16_t* gateup;            // gate / up tiles in matrix-core order (launch_gateup_order)
    const uint16_t* down;              // [1024 x 3072] in matrix-core order, 96-column blocks
    const float* norm_w;               // post-attention RMSNorm weights
    const float* x[kMaxBatch];         // residual in
    float* x_out[kMaxBatch];           // residual out
    uint64_t* act_words;               // [8 XCDs][kMaxBatch][384] tagged activations
    uint64_t* share_words;             // [32 row blocks][8 XCDs][kMaxBatch][32 rows] tagged down shares
    int* stall;
    int batch;
    uint32_t tag;
};

constexpr int kFfnOctant = kFFN / 8;  // 384 activation columns per XCD
static_assert(kBatchActWords == 8 * kMaxBatch * kFfnOctant, "activation words per XCD octant");

// The normalized rows (x * inv) * w of every sequence (elements 2 tid and
// 2 tid + 1) as FP16 hi / lo in LDS under the range guard; with `hidden`,
// also the unscaled FP32 rows of the first `batch` sequences. Ends with a
// barrier.
__device__ __forceinline__ void split_normalized(const float2 (&xv)[kMaxBatch], float2 wn,
                                                 const float (&inv_row)[kMaxBatch],
                                                 _Float16 (&xh)[kMaxBatch][kHidden + 8],
                                                 _Float16 (&xl)[kMaxBatch][kHidden + 8], dev::SplitGuard& guard,
                                                 int tid, float* const* hidden, int batch = 0) {
    const int lane = tid & 63, wave = tid >> 6;
    auto split_rows = [&](bool scaled) {
        float big = 0.f;
#pragma unroll
        for (int bb = 0; bb < kMaxBatch; ++bb) {
            const float inv = inv_row[bb];
            float n0 = (xv[bb].x * inv) * wn.x, n1 = (xv[bb].y * inv) * wn.y;
            if (!scaled && hidden != nullptr && bb < batch)
                reinterpret_cast<float2*>(hidden[bb])[tid] = make_float2(n0, n1);
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

__global__ __launch_bounds__(512) void ffn_batch_kernel(const BatchFfnArgs a) {
    const int xo = blockIdx.x & 7, r = blockIdx.x >> 3;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, quad = lane >> 4;
    const int B = a.batch;

    // Loads complete in issue order per wave: residual elements 2 tid,
    // 2 tid + 1 of every sequence (rows past the batch repeat row B - 1),
    // norm weights, gate/up weights, down weights.
    float2 xv[kMaxBatch];
#pragma unroll
    for (int bb = 0; bb < kMaxBatch; ++bb) xv[bb] = reinterpret_cast<const float2*>(a.x[min(bb, B - 1)])[tid];
    const float2 wn = reinterpret_cast<const float2*>(a.norm_w)[tid];
    // Gate/up tiles 32 xo + r (rows 384 xo + 12 r + col of the gate and up
    // halves, col < 12; lanes col >= 12 read row 11 again and are masked
    // at use); wave w takes columns 128 w .. 128 w + 127. 768 bytes
    // contiguous per load.
    const int tile = 32 * xo + r;
    u32x4 wg[4], wu[4];
    __builtin_amdgcn_sched_barrier(0);
    {
        const int l48 = 12 * quad + min(col, 11);
        const u32x4* gp = reinterpret_cast<const u32x4*>(a.gateup) + (size_t(2 * tile) * 8 + wave) * 4 * 48 + l48;
        const u32x4* up = reinterpret_cast<const u32x4*>(a.gateup) + (size_t(2 * tile + 1) * 8 + wave) * 4 * 48 + l48;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            wg[st] = __builtin_nontemporal_load(gp + 48 * st);
            wu[st] = __builtin_nontemporal_load(up + 48 * st);
        }
    }
    // Down tile tt = wave & 1 (rows 32 r + 16 tt + col), K range
    // 384 xo + 96 (wave >> 1) .. + 95 in 3 steps (96-column block
    // 4 xo + (wave >> 1)).
    const int tt = wave & 1, kq = wave >> 1;
    u32x4 wd[3];
    {
        const u32x4* dp = reinterpret_cast<const u32x4*>(a.down) + ((size_t(2 * r + tt) * 32 + 4 * xo + kq) * 3) * 64 + lane;
#pragma unroll
        for (int st = 0; st < 3; ++st) wd[st] = __builtin_nontemporal_load(dp + 64 * st);
    }
    __builtin_amdgcn_sched_barrier(0);

    __shared__ __align__(16) _Float16 xh[kMaxBatch][kHidden + 8];
    __shared__ __align__(16) _Float16 xl[kMaxBatch][kHidden + 8];
    __shared__ double nred[8][kMaxBatch];
    __shared__ float inv_row[kMaxBatch];
    __shared__ float part[8][2][64][4];
    __shared__ __align__(16) _Float16 ah[kMaxBatch][kFfnOctant + 8];
    __shared__ __align__(16) _Float16 al[kMaxBatch][kFfnOctant + 8];
    // Range guards (decode_dev.hpp): the normalized rows, then the XCD's
    // activations of each sequence.
    __shared__ dev::SplitGuard guard, act_guard;
    guard.init(tid);
    act_guard.init(tid);

    // 1. RMSNorm of every row (reduce-scatter inside each wave: lane l ends
    // with its wave's total of row (l >> 3) & 7; then the 8 waves in order).
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
        split_normalized(xv, wn, inv_row, xh, xl, guard, tid, nullptr);
    }

    // 2. Gate/up and SwiGLU.
    {
        floatx4 accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            // k slot (quad, e) of step st holds column 128 wave + 32 st + 8 quad + e.
            const int k = 128 * wave + 32 * st + 8 * quad;
            const half8 bh = masked_b<half8>(&xh[col & 7][k], col < kMaxBatch);
            const half8 bl = masked_b<half8>(&xl[col & 7][k], col < kMaxBatch);
            const u32x4 zero4 = {0u, 0u, 0u, 0u};
            const half8 g8 = __builtin_bit_cast(half8, col < 12 ? wg[st] : zero4);
            const half8 u8 = __builtin_bit_cast(half8, col < 12 ? wu[st] : zero4);
            accg = __builtin_amdgcn_mfma_f32_16x16x32_f16(g8, bh, accg, 0, 0, 0);
            accg = __builtin_amdgcn_mfma_f32_16x16x32_f16(g8, bl, accg, 0, 0, 0);
            accu = __builtin_amdgcn_mfma_f32_16x16x32_f16(u8, bh, accu, 0, 0, 0);
            accu = __builtin_amdgcn_mfma_f32_16x16x32_f16(u8, bl, accu, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            part[wave][0][lane][e] = accg[e];
            part[wave][1][lane][e] = accu[e];
        }
        __syncthreads();
        if (wave < 4) {  // element (row 4 (lane / 16) + wave, sequence lane % 16)
            auto tree = [&](int t) {
                return ((part[0][t][lane][wave] + part[1][t][lane][wave]) +
                        (part[2][t][lane][wave] + part[3][t][lane][wave])) +
                       ((part[4][t][lane][wave] + part[5][t][lane][wave]) +
                        (part[6][t][lane][wave] + part[7][t][lane][wave]));
            };
            const int row = 4 * (lane >> 4) + wave, seq = lane & 15;
            const float gate = tree(0) * guard.up(seq & 7), up = tree(1) * guard.up(seq & 7);
            if (row < 12 && seq < B) {
                const float half_gate = gate * 0.5f;
                const float th = tanhf(half_gate);
                const float act = gate * (0.5f + 0.5f * th) * up;
                exchange_put(a.act_words + (size_t(xo) * kMaxBatch + seq) * kFfnOctant + 12 * r + row, act, a.tag);
            }
        }
    }

    // 3. The XCD's activations (6 words per thread), staged as hi / lo.
    bool ok;
    {
        const uint64_t* words[6];
        float got[6];
        unsigned want = 0;
#pragma unroll
        for (int k = 0; k < 6; ++k) {
            const int idx = tid + 512 * k, seq = idx / kFfnOctant;
            words[k] = a.act_words + size_t(xo) * kMaxBatch * kFfnOctant + idx;
            got[k] = 0.f;
            if (seq < B) want |= 1u << k;
        }
        ok = exchange_gather_pipe<6, 2>(words, a.tag, got, want);
        auto split_acts = [&](bool scaled) {
            float big = 0.f;
#pragma unroll
            for (int k = 0; k < 6; ++k) {
                const int idx = tid + 512 * k, seq = idx / kFfnOctant, c = idx % kFfnOctant;
                big = fmaxf(big, fabsf(got[k]));
                _Float16 h, l;
                split_half(scaled ? got[k] * pow2(-act_guard.seq_e[seq]) : got[k], h, l);
                ah[seq][c] = h;
                al[seq][c] = l;
            }
            return big;
        };
        act_guard.post(split_acts(false), lane, wave);
        __syncthreads();
        if (act_guard.needed(8)) {
#pragma unroll
            for (int k = 0; k < 6; ++k) act_guard.offer((tid + 512 * k) / kFfnOctant, fabsf(got[k]));
            __syncthreads();
            if (tid < kMaxBatch) act_guard.seq_e[tid] = act_guard.exponent(tid);
            __syncthreads();
            split_acts(true);
            __syncthreads();
        }
    }
    // Down share of rows 32 r .. 32 r + 31 over this XCD's columns.
    {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < 3; ++st) {
            const int k = 96 * kq + 32 * st + 8 * quad;
            const half8 bh = masked_b<half8>(&ah[col & 7][k], col < kMaxBatch);
            const half8 bl = masked_b<half8>(&al[col & 7][k], col < kMaxBatch);
            const half8 d8 = __builtin_bit_cast(half8, wd[st]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(d8, bh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(d8, bl, acc, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) part[wave][0][lane][e] = acc[e];
        __syncthreads();
        // Thread (wave w < 4, lane): sequence 2 w + lane / 32, row
        // 32 r + rl (rl = lane % 32: tile rl / 16, element rl % 16 held by
        // MFMA lane 16 (rl / 4 % 4) + sequence, register rl % 4); the 4 K
        // ranges of the tile (waves tt, tt + 2, tt + 4, tt + 6) in fixed
        // order. A wave posts 64 consecutive words: the XCD's shares fill
        // whole lines (write-through stores of parts of a line cost far more).
        if (wave < 4) {
            const int seq = 2 * wave + (lane >> 5), rl = lane & 31;
            const int tt2 = rl >> 4, e4 = rl & 3, el = 16 * ((rl >> 2) & 3) + seq;
            const float y = ((part[tt2][0][el][e4] + part[tt2 + 2][0][el][e4]) +
                             (part[tt2 + 4][0][el][e4] + part[tt2 + 6][0][el][e4])) *
                            act_guard.up(seq);
            if (seq < B)
                exchange_put_through(a.share_words + ((size_t(r) * 8 + xo) * kMaxBatch + seq) * 32 + rl, y, a.tag);
        }
    }

    // 4. Rows 32 r .. 32 r + 31 of sequence xo (threads 0..31, one row
    // each: a whole line of the residual): x + the 8 XCD shares.
    if (tid < 32) {
        const int row = 32 * r + tid, seq = xo;
        const bool live = seq < B;
        const uint64_t* words[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) words[k] = a.share_words + ((size_t(r) * 8 + k) * kMaxBatch + seq) * 32 + tid;
        float s8[8] = {};
        if (ok) ok = exchange_gather_pipe<8, 6>(words, a.tag, s8, live ? 0xffu : 0u);
        if (live) {
            const float down = ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
            a.x_out[seq][row] = a.x[seq][row] + down;
        }
    }
    if (!ok) *a.stall = 1;
}

// Final norm + tied lm_head + first pass of the per-sequence greedy
// selection for the batched step (engine/core.cpp:642-645, main.cpp:51-59)
// as one workgroup per CU: every workgroup forms RMSNorm(x) of all
// sequences as FP16 hi + lo in LDS, then streams the 16-row tiles
// w, w + 256, ... of the embedding matrix with kLmInFlight tiles in flight
// (the 8 waves split K, summed in a fixed tree per tile), writes the logits
// and keeps each sequence's best (largest value, lowest id among equals,
// nonfinite flagged) for the second pass.
constexpr int kLmInFlight = 4;
constexpr int kLmTiles = kVocab / kBatchRows;  // 9496
constexpr int kLmTilesPerGroup = (kLmTiles + kBatchLmGroups - 1) / kBatchLmGroups;
static_assert(kVocab % kBatchRows == 0, "whole 16-row tiles");

struct BatchLmArgs {
    const uint16_t* w;         // embedding matrix (tied head) in matrix-core order (launch_mfma_order)
    const float* norm_w;       // final RMSNorm weights
    const float* x[kMaxBatch];
    float* hidden[kMaxBatch];  // final normalized rows
    float* logits[kMaxBatch];
    float* lm_value;           // [kBatchLmGroups][kMaxBatch] per-group best
    int* lm_index;
    int* lm_bad;
    int batch;
};

__global__ __launch_bounds__(512) void lm_head_batch_kernel(const BatchLmArgs a) {
    const int w = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, quad = lane >> 4;
    const int B = a.batch;
    float2 xv[kMaxBatch];
#pragma unroll
    for (int bb = 0; bb < kMaxBatch; ++bb) xv[bb] = reinterpret_cast<const float2*>(a.x[min(bb, B - 1)])[tid];
    const float2 wn = reinterpret_cast<const float2*>(a.norm_w)[tid];
    // Tile k of this workgroup: rows 16 (w + 256 k) ..; loads past the last
    // tile repeat it and are not used.
    const int ntiles = (kLmTiles - w + kBatchLmGroups - 1) / kBatchLmGroups;
    auto load_tile = [&](u32x4 (&wt)[4], int k) {
        const int t = min(w + kBatchLmGroups * k, kLmTiles - 1);
        // Piece (t, wave, st) of the matrix-core copy: 64 lanes x 16 bytes
        // in a row, so that every load reads 1 KiB contiguous.
        const u32x4* wp = reinterpret_cast<const u32x4*>(a.w) + (size_t(t) * 8 + wave) * 256 + lane;
#pragma unroll
        for (int st = 0; st < 4; ++st) wt[st] = __builtin_nontemporal_load(wp + 64 * st);
    };
    // Epilogue element of threads 0..255: row 4 (lane / 16) + wave of the
    // tile, sequence lane % 16; its running best over the tiles.
    const int eb = lane & 15, erow = 4 * (lane >> 4) + (wave & 3);
    // Loaded before the stream and waited for (by the empty asm that uses
    // it) right after the first tiles are issued: a pointer still pending
    // inside the loop would wait behind the tiles in flight.
    float* out = a.logits[min(eb, B - 1)];
    // The first tiles do not depend on the norm: issued behind the residual
    // rows (which return first), they stream while the norm is formed.
    u32x4 ring[kLmInFlight][4];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kLmInFlight; ++u) load_tile(ring[u], u);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" : "+v"(out));

    __shared__ __align__(16) _Float16 xh[kMaxBatch][kHidden + 8];
    __shared__ __align__(16) _Float16 xl[kMaxBatch][kHidden + 8];
    __shared__ double nred[8][kMaxBatch];
    __shared__ float inv_row[kMaxBatch];
    __shared__ float part[2][8][64][4];
    __shared__ dev::SplitGuard guard;
    guard.init(tid);
    // RMSNorm of every row (as in ffn_batch_kernel).
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
        split_normalized(xv, wn, inv_row, xh, xl, guard, tid, w == 0 ? a.hidden : nullptr, B);
    }

    float bv = -INFINITY, lg[kLmTilesPerGroup];
    int bi = INT_MAX, bad = 0;
    // Fully unrolled (compile-time ring slots and tile counts, so every wait
    // covers exactly the oldest tile).
#pragma unroll
    for (int k0 = 0; k0 < kLmTilesPerGroup; k0 += kLmInFlight) {
#pragma unroll
        for (int u = 0; u < kLmInFlight; ++u) {
            const int k = k0 + u;
            if (k >= kLmTilesPerGroup) break;
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const int kk = 128 * wave + 32 * st + 8 * quad;
                const half8 bh = masked_b<half8>(&xh[col & 7][kk], col < kMaxBatch);
                const half8 bl = masked_b<half8>(&xl[col & 7][kk], col < kMaxBatch);
                const half8 w8 = __builtin_bit_cast(half8, ring[u][st]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w8, bh, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(w8, bl, acc, 0, 0, 0);
            }
            if (k + kLmInFlight < kLmTilesPerGroup) load_tile(ring[u], k + kLmInFlight);
#pragma unroll
            for (int e = 0; e < 4; ++e) part[k & 1][wave][lane][e] = acc[e];
            __syncthreads();
            if (wave < 4) {
                const auto f = [&](int v8) { return part[k & 1][v8][lane][wave]; };
                const float y = (((f(0) + f(1)) + (f(2) + f(3))) + ((f(4) + f(5)) + (f(6) + f(7)))) *
                                guard.up(eb & 7);
                const int row = kBatchRows * (w + kBatchLmGroups * k) + erow;
                lg[k] = y;
                const bool use = k < ntiles && eb < B;
                bad |= use && !__builtin_isfinite(y);
                if (use && better(y, row, bv, bi)) { bv = y; bi = row; }
            }
        }
    }
    // The logits are stored after the stream: on this GPU a store counts
    // among the outstanding loads, and conditional stores inside the loop
    // would make every wait cover all the tiles in flight.
    if (wave < 4 && eb < B) {
#pragma unroll
        for (int k = 0; k < kLmTilesPerGroup; ++k)
            if (k < ntiles) out[kBatchRows * (w + kBatchLmGroups * k) + erow] = lg[k];
    }
    // Best per sequence over the 16 rows' threads (lanes l, l ^ 16, l ^ 32,
    // l ^ 48 of waves 0-3), then this group's entry.
    __shared__ float mv[4][16];
    __shared__ int mi[4][16], mb[4][16];
    if (wave < 4) {
#pragma unroll
        for (int off = 16; off < 64; off <<= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            bad |= __shfl_xor(bad, off);
            if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        if (lane < 16) { mv[wave][lane] = bv; mi[wave][lane] = bi; mb[wave][lane] = bad; }
    }
    __syncthreads();
    if (tid < B) {
        float v0 = mv[0][tid];
        int i0 = mi[0][tid], b0 = mb[0][tid];
#pragma unroll
        for (int q = 1; q < 4; ++q) {
            b0 |= mb[q][tid];
            if (better(mv[q][tid], mi[q][tid], v0, i0)) { v0 = mv[q][tid]; i0 = mi[q][tid]; }
        }
        const size_t slot = size_t(w) * kMaxBatch + tid;
        a.lm_value[slot] = v0;
        a.lm_index[slot] = i0;
        a.lm_bad[slot] = b0;
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

template <int K>
void bgemv(const BatchGemvArgs& a, int rows, hipStream_t stream) {
    require(a.batch >= 1 && a.batch <= kMaxBatch, "batched GEMV: 1..8 rows");
    require(rows % kBatchRows == 0 && rows > 0, "batched GEMV: rows must be a positive multiple of 16");
    bgemv_kernel<K><<<rows / kBatchRows, K / 4, 0, stream>>>(a);
}

// dst in matrix-core order of W (natural [rows x K], rows % 16 == 0,
// K % BW == 0, BW % 32 == 0): 16-byte piece
// u = ((t (K / BW) + b) (BW / 32) + st) 64 + l holds
// W[16 t + l % 16][BW b + 32 st + 8 (l / 16) .. + 7], the A operand of lane
// l in step st of the wave that takes columns BW b .. + BW - 1 of tile t.
__global__ void mfma_order_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, int rows, int K,
                                  int BW) {
    const size_t u = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int blocks = K / BW, steps = BW / 32;
    if (u >= size_t(rows) / 16 * blocks * steps * 64) return;
    const int l = int(u & 63);
    const size_t q = u >> 6;
    const int st = int(q % steps), b = int((q / steps) % blocks);
    const size_t t = q / steps / blocks;
    const u32x4* s4 = reinterpret_cast<const u32x4*>(src + (16 * t + (l & 15)) * size_t(K) + BW * b + 32 * st + 8 * (l >> 4));
    reinterpret_cast<u32x4*>(dst)[u] = *s4;
}

// Gate / up rows of the batched FFN in matrix-core order: tile T holds gate
// (h = 0) or up (h = 1) rows 12 T .. 12 T + 11; piece
// u = (((2 T + h) 8 + w) 4 + st) 48 + 12 q + c (c < 12) holds
// W[h 3072 + 12 T + c][128 w + 32 st + 8 q .. + 7], the A operand of lane
// 16 q + c in step st of wave w (lanes with l % 16 >= 12 read piece c = 11
// again and are masked).
__global__ void gateup_order_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst) {
    const size_t u = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (u >= kGateupOrderHalves / 8) return;
    const int l48 = int(u % 48), q = l48 / 12, c = l48 % 12;
    const size_t rest = u / 48;
    const int st = int(rest & 3), w = int((rest >> 2) & 7), h = int((rest >> 5) & 1);
    const int T = int(rest >> 6);
    const int row = h * kFFN + 12 * T + c;
    const u32x4* s4 = reinterpret_cast<const u32x4*>(src + size_t(row) * kHidden + 128 * w + 32 * st + 8 * q);
    reinterpret_cast<u32x4*>(dst)[u] = *s4;
}

}  // namespace

void launch_mfma_order(const uint16_t* src, uint16_t* dst, int rows, int K, int BW, hipStream_t stream) {
    require(rows > 0 && rows % 16 == 0 && BW > 0 && BW % 32 == 0 && K > 0 && K % BW == 0,
            "mfma order: rows % 16 == 0, K % BW == 0, BW % 32 == 0");
    const size_t pieces = size_t(rows) / 16 * (K / BW) * (BW / 32) * 64;
    mfma_order_kernel<<<unsigned((pieces + 255) / 256), 256, 0, stream>>>(src, dst, rows, K, BW);
}

void launch_gateup_order(const uint16_t* gateup, uint16_t* dst, hipStream_t stream) {
    const size_t pieces = kGateupOrderHalves / 8;
    gateup_order_kernel<<<unsigned((pieces + 255) / 256), 256, 0, stream>>>(gateup, dst);
}

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
        case 1024: bgemv<1024>(a, rows, stream); break;
        case 2048: bgemv<2048>(a, rows, stream); break;
        case 3072: bgemv<3072>(a, rows, stream); break;
        default: throw std::runtime_error("batched GEMV: cols must be 1024, 2048 or 3072");
    }
}

void launch_decode_batch(const BatchSeq* seqs, int count, const uint16_t* embed, const uint16_t* embed_mfma,
                         const float* final_norm, const float* cosines, const float* sines, const uint32_t* tags,
                         hipStream_t stream) {
    require(count >= 1 && count <= kMaxBatch, "batched decode: 1..8 sequences");
    for (int l = 0; l < kBatchTagsPerLayer * kLayers; ++l) require(tags[l] != 0, "batched decode: exchange tags are nonzero");
    uint64_t* const words = seqs[0].s.bexchange;
    for (int b = 0; b < count; ++b) {
        const BatchSeq& q = seqs[b];
        require(q.shared_seq >= 0 && q.shared_seq < count && q.shared >= 0 && q.shared % 64 == 0 &&
                    q.shared <= q.pos && q.shared <= seqs[q.shared_seq].pos,
                "batched decode: shared rows outside both caches");
    }
    for (int l = 0; l < kLayers; ++l) {
        const LayerDevice& W = seqs[0].layers[l];  // weights are shared; K/V are per sequence
        // The residual is in x at each layer's start; attention + O leave it
        // in xm, the FFN brings it back to x.
        AttnSeq as[kMaxBatch];
        for (int b = 0; b < count; ++b) {
            const DecodeScratch& s = seqs[b].s;
            as[b] = AttnSeq{s.x,
                            l == 0 ? embed + size_t(seqs[b].token) * kHidden : nullptr,
                            s.xm,
                            seqs[b].layers[l].keys,
                            seqs[b].layers[l].values,
                            seqs[b].pos,
                            seqs[b].context,
                            seqs[seqs[b].shared_seq].layers[l].keys,
                            seqs[seqs[b].shared_seq].layers[l].values,
                            seqs[seqs[b].shared_seq].context,
                            seqs[b].shared};
        }
        launch_attention_o_batch(as, count, W.qkv_m, W.o_m, W.in_norm, W.q_norm, W.k_norm, cosines, sines, words,
                                 seqs[0].s.stall, tags[kBatchTagsPerLayer * l], stream);

        BatchFfnArgs f{};
        f.gateup = W.gateup_m;
        f.down = W.down_m;
        f.norm_w = W.post_norm;
        f.act_words = words + kBatchActOffset;
        f.share_words = words + kBatchShareOffset;
        f.stall = seqs[0].s.stall;
        f.batch = count;
        f.tag = tags[kBatchTagsPerLayer * l + 1];
        for (int b = 0; b < count; ++b) {
            f.x[b] = seqs[b].s.xm;
            f.x_out[b] = seqs[b].s.x;
        }
        ffn_batch_kernel<<<256, 512, 0, stream>>>(f);
    }
    BatchLmArgs lm{};
    lm.w = embed_mfma;  // tied head (engine/core.cpp:643-645)
    lm.norm_w = final_norm;
    lm.batch = count;
    const DecodeScratch& s0 = seqs[0].s;
    lm.lm_value = s0.lm_value;
    lm.lm_index = s0.lm_index;
    lm.lm_bad = s0.lm_bad;
    BatchResults res{};
    for (int b = 0; b < count; ++b) {
        lm.x[b] = seqs[b].s.x;
        lm.logits[b] = seqs[b].s.logits;
        lm.hidden[b] = seqs[b].s.hidden;
        res.device[b] = seqs[b].s.result;
        res.host[b] = seqs[b].host_out;
        res.stall[b] = seqs[b].s.stall;
    }
    lm_head_batch_kernel<<<kBatchLmGroups, 512, 0, stream>>>(lm);
    batch_argmax_kernel<<<count, 1024, 0, stream>>>(s0.lm_value, s0.lm_index, s0.lm_bad, res);
}

}  // namespace qwen_hip
