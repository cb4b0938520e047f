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
// Attention: flash-decoding over position splits. Each workgroup owns one KV
// head (both GQA query heads 2g, 2g+1 share every K/V row it loads) and a
// contiguous range of positions; the last split to finish combines the
// (max, sum, output) partials in fixed split order, so results do not depend
// on scheduling. The workgroup holding the current position also applies
// QK-norm + RoPE to k and writes K/V (FP16, round-to-nearest-even) into the
// cache (engine/core.cpp:395-406) and uses them from LDS.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <climits>

#include "kernels.hpp"

namespace qwen_hip {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

// Eight chain steps from one 16-byte block: halves i = 0..7 with activations xa/xb.
__device__ __forceinline__ float chain8(float acc, u32x4 w, float4 xa, float4 xb) {
    acc = __builtin_fmaf(xa.x, h2f(w.x & 0xffffu), acc);
    acc = __builtin_fmaf(xa.y, h2f(w.x >> 16), acc);
    acc = __builtin_fmaf(xa.z, h2f(w.y & 0xffffu), acc);
    acc = __builtin_fmaf(xa.w, h2f(w.y >> 16), acc);
    acc = __builtin_fmaf(xb.x, h2f(w.z & 0xffffu), acc);
    acc = __builtin_fmaf(xb.y, h2f(w.z >> 16), acc);
    acc = __builtin_fmaf(xb.z, h2f(w.w & 0xffffu), acc);
    acc = __builtin_fmaf(xb.w, h2f(w.w >> 16), acc);
    return acc;
}

// Lane c of each 8-lane group holds chain c; returns
// ((c0+c4)+(c1+c5)) + ((c2+c6)+(c3+c7)) in every lane of the group.
__device__ __forceinline__ float combine_chains(float acc) {
    const float t1 = acc + __shfl_xor(acc, 4);
    const float t2 = t1 + __shfl_xor(t1, 1);
    return t2 + __shfl_xor(t2, 2);
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// Position of activation j in the permuted LDS vector: j = 64b + 8i + c is
// stored at 64b + 8c + i, so chain c reads its 8 values contiguously.
__device__ __forceinline__ int xperm(int j) { return (j & ~63) | ((j & 7) << 3) | ((j >> 3) & 7); }

// RMSNorm of x[0..N) into permuted LDS (and optionally to `copy`).
template <int N, int THREADS>
__device__ __forceinline__ void norm_to_lds(const float* __restrict__ x, const float* __restrict__ w, float* xs,
                                            double* red, float* copy) {
    constexpr int PER = N / THREADS;
    const int tid = threadIdx.x;
    float v[PER];
    double part = 0.0;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        v[k] = x[tid + k * THREADS];
        const float square = v[k] * v[k];
        part += static_cast<double>(square);
    }
    part = wave_sum(part);
    if ((tid & 63) == 0) red[tid >> 6] = part;
    __syncthreads();
    double total = 0.0;
#pragma unroll
    for (int i = 0; i < THREADS / 64; ++i) total += red[i];
    const float sum = static_cast<float>(total);
    const float inv = 1.0f / __builtin_sqrtf(sum / static_cast<float>(N) + 1e-6f);
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int j = tid + k * THREADS;
        const float o = (v[k] * inv) * w[j];
        xs[xperm(j)] = o;
        if (copy) copy[j] = o;
    }
}

template <int N, int THREADS>
__device__ __forceinline__ void copy_to_lds(const float* __restrict__ x, float* xs) {
#pragma unroll
    for (int k = 0; k < N / THREADS; ++k) {
        const int j = threadIdx.x + k * THREADS;
        xs[xperm(j)] = x[j];
    }
}

// Chain dot of one 8-row tile against the permuted LDS vector.
template <int N>
__device__ __forceinline__ float tile_dot(const uint16_t* __restrict__ w_t, const float* xs, size_t tile, int lane) {
    constexpr int NB = N / 64;
    constexpr int U = NB < 16 ? NB : 16;
    const u32x4* wp = reinterpret_cast<const u32x4*>(w_t) + tile * (NB * 64) + lane;
    const float4* xs4 = reinterpret_cast<const float4*>(xs);
    const int c = lane & 7;
    float acc = 0.f;
#pragma unroll
    for (int b0 = 0; b0 < NB; b0 += U) {
        u32x4 wv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) wv[u] = __builtin_nontemporal_load(wp + (b0 + u) * 64);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int b = b0 + u;
            acc = chain8(acc, wv[u], xs4[16 * b + 2 * c], xs4[16 * b + 2 * c + 1]);
        }
    }
    return combine_chains(acc);
}

enum GemvMode { kPlain, kQKV, kO, kGateUp, kDown, kLmHead };

struct GemvArgs {
    const uint16_t* w;        // chain-tiled weights
    const float* in;          // input vector (plain/O/down), residual x (norm modes)
    const float* norm_w;      // RMSNorm weights (QKV, gate/up, lm_head)
    const uint16_t* embed;    // natural embedding, first layer only (QKV)
    const StepParams* params; // token for the embedding gather
    float* out;               // plain/QKV: y; gate/up: activation; lm_head: logits
    float* x;                 // residual stream (O/down add, first-layer QKV store)
    float* hidden;            // lm_head: final normalized hidden
    float* lm_value;
    int* lm_index;
    int* lm_bad;
    unsigned* lm_count;
    ArgmaxResult* result;
};

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

template <int N, int WAVES, int MODE>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(const GemvArgs a) {
    constexpr int THREADS = WAVES * 64;
    __shared__ float4 xs4[N / 4];
    __shared__ double red[WAVES];
    float* xs = reinterpret_cast<float*>(xs4);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    if constexpr (MODE == kQKV) {
        const float* src = a.in;
        if (a.embed) {
            // First layer: x = fp32(E[token]) (engine/core.cpp:382-383), kept as the residual.
            __shared__ float xe[N];
            const uint16_t* row = a.embed + size_t(a.params->token) * N;
            for (int j = tid; j < N; j += THREADS) {
                const float v = h2f(row[j]);
                xe[j] = v;
                if (blockIdx.x == 0) a.x[j] = v;
            }
            __syncthreads();
            src = xe;
        }
        norm_to_lds<N, THREADS>(src, a.norm_w, xs, red, nullptr);
    } else if constexpr (MODE == kGateUp) {
        norm_to_lds<N, THREADS>(a.in, a.norm_w, xs, red, nullptr);
    } else if constexpr (MODE == kLmHead) {
        norm_to_lds<N, THREADS>(a.in, a.norm_w, xs, red, blockIdx.x == 0 ? a.hidden : nullptr);
    } else {
        copy_to_lds<N, THREADS>(a.in, xs);
    }
    __syncthreads();

    const size_t tile = size_t(blockIdx.x) * WAVES + wave;
    const float y = tile_dot<N>(a.w, xs, tile, lane);
    const int c = lane & 7, r = lane >> 3;
    const int row = int(tile) * 8 + r;

    if constexpr (MODE == kPlain || MODE == kQKV) {
        if (c == 0) a.out[row] = y;
    } else if constexpr (MODE == kO || MODE == kDown) {
        if (c == 0) a.x[row] = a.x[row] + y;
    } else if constexpr (MODE == kGateUp) {
        // Tile rows 0-3 are gate rows 4T..4T+3, rows 4-7 the matching up rows.
        const float up = __shfl(y, (lane + 32) & 63);
        if (lane < 32 && c == 0) {
            const float gate = y;
            const float half_gate = gate * 0.5f;
            const float t = tanhf(half_gate);
            a.out[int(tile) * 4 + r] = gate * (0.5f + 0.5f * t) * up;
        }
    } else if constexpr (MODE == kLmHead) {
        if (c == 0) a.out[row] = y;
        // Workgroup argmax: lowest id among maxima; any nonfinite value flagged.
        float bv = -INFINITY;
        int bi = INT_MAX, bad = 0;
        if (c == 0) {
            bad = !__builtin_isfinite(y);
            if (better(y, row, bv, bi)) { bv = y; bi = row; }
        }
#pragma unroll
        for (int off = 8; off < 64; off <<= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            bad |= __shfl_xor(bad, off);
            if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        __shared__ float wv[WAVES];
        __shared__ int wi[WAVES], wb[WAVES];
        __shared__ int last;
        if (lane == 0) { wv[wave] = bv; wi[wave] = bi; wb[wave] = bad; }
        __syncthreads();
        if (tid == 0) {
            for (int k = 1; k < WAVES; ++k) {
                bad |= wb[k];
                if (better(wv[k], wi[k], bv, bi)) { bv = wv[k]; bi = wi[k]; }
            }
            __hip_atomic_store(a.lm_value + blockIdx.x, bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.lm_index + blockIdx.x, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.lm_bad + blockIdx.x, bad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __threadfence();
            const unsigned prev = __hip_atomic_fetch_add(a.lm_count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            last = prev == gridDim.x - 1;
        }
        __syncthreads();
        if (!last) return;
        __threadfence();
        bv = -INFINITY;
        bi = INT_MAX;
        bad = 0;
        for (int k = tid; k < int(gridDim.x); k += THREADS) {
            const float v = __hip_atomic_load(a.lm_value + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int i = __hip_atomic_load(a.lm_index + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            bad |= __hip_atomic_load(a.lm_bad + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (better(v, i, bv, bi)) { bv = v; bi = i; }
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            bad |= __shfl_xor(bad, off);
            if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        __syncthreads();
        if (lane == 0) { wv[wave] = bv; wi[wave] = bi; wb[wave] = bad; }
        __syncthreads();
        if (tid == 0) {
            for (int k = 1; k < WAVES; ++k) {
                bad |= wb[k];
                if (better(wv[k], wi[k], bv, bi)) { bv = wv[k]; bi = wi[k]; }
            }
            a.result->token = bi;
            a.result->nonfinite = bad;
            __hip_atomic_store(a.lm_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
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
    const StepParams* params;
    float* partial;        // [8][kAttnSplits][kAttnPartial]
    unsigned* counters;    // [8]
    float* attended;       // [2048]
    int context;
    float scale;           // 1.0f / sqrt(128.0f)
};

__device__ __forceinline__ int kperm(int j) { return ((j & 7) << 4) | (j >> 3); }

// RMSNorm over 128 values held one per thread by two consecutive waves
// (engine/core.cpp:397-398), then rotate-half RoPE (216-218).
__device__ __forceinline__ float head_norm_rope(float raw, const float* w, const float* cs, const float* sn,
                                                double* red2, float* buf, int j) {
    const int lane = threadIdx.x & 63;
    const float square = raw * raw;
    const double part = wave_sum(static_cast<double>(square));
    if (lane == 0) red2[(j >> 6)] = part;
    __syncthreads();
    const float sum = static_cast<float>(red2[0] + red2[1]);
    const float inv = 1.0f / __builtin_sqrtf(sum / 128.0f + 1e-6f);
    const float normed = (raw * inv) * w[j];
    buf[j] = normed;
    __syncthreads();
    float out;
    if (j < 64) {
        const float x0 = buf[j], x1 = buf[j + 64];
        out = x0 * cs[j] - x1 * sn[j];
    } else {
        const int jj = j - 64;
        const float x0 = buf[jj], x1 = buf[j];
        out = x1 * cs[jj] + x0 * sn[jj];
    }
    return out;
}

__global__ __launch_bounds__(256) void attn_decode_kernel(const AttnArgs a) {
    const int s = blockIdx.x, g = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos = a.params->pos, n = pos + 1;
    int chunk = (n + kAttnSplits - 1) / kAttnSplits;
    chunk = max(64, (chunk + 63) & ~63);
    const int ns = (n + chunk - 1) / chunk;
    if (s >= ns) return;
    const int t0 = s * chunk, m = min(n, t0 + chunk) - t0;  // 1 <= m <= 128
    const bool owner = t0 + m == n;

    __shared__ float qp[2][128];
    __shared__ float buf[2][128];
    __shared__ float sc[2][128];
    __shared__ float opart[2][2][128];
    __shared__ uint16_t kcur[128], vcur[128];
    __shared__ double red[2][2];
    __shared__ float redm[4], reds[4];
    __shared__ int last;

    const float* cs = a.cosines + size_t(pos) * 64;
    const float* sn = a.sines + size_t(pos) * 64;
    const size_t head_base = size_t(g) * a.context;

    {  // q heads 2g, 2g+1: one head per pair of waves
        const int h = tid >> 7, j = tid & 127;
        const float raw = a.qkv[(2 * g + h) * 128 + j];
        const float q = head_norm_rope(raw, a.q_norm, cs, sn, red[h], buf[h], j);
        qp[h][kperm(j)] = q;
    }
    if (owner) {  // current k and v into the cache and LDS (owner is block-uniform)
        __syncthreads();
        // Both wave pairs normalize the same k head into separate buffers so
        // every wave meets the same barriers; pair 0 stores k, pair 1 stores v.
        const int h = tid >> 7, j = tid & 127;
        const float raw = a.qkv[2048 + g * 128 + j];
        const float k = head_norm_rope(raw, a.k_norm, cs, sn, red[h], buf[h], j);
        if (h == 0) {
            const uint16_t bits = f2h(k);
            kcur[kperm(j)] = bits;
            a.keys[(head_base + pos) * 128 + kperm(j)] = bits;
        } else {
            const uint16_t bits = f2h(a.qkv[3072 + g * 128 + j]);
            vcur[j] = bits;
            a.values[(head_base + pos) * 128 + j] = bits;
        }
    }
    __syncthreads();

    // Scores: 8 threads per position, thread c runs chain c over the 16
    // steps of the 128-long dot for both query heads (engine/core.cpp:612).
    {
        const int c = tid & 7;
        for (int base = 0; base < m; base += 32) {
            const int tl = base + (tid >> 3);
            float acc0 = 0.f, acc1 = 0.f;
            if (tl < m) {
                const int t = t0 + tl;
                uint32_t kw[8];
                if (t == pos) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) kw[i] = uint32_t(kcur[c * 16 + 2 * i]) | (uint32_t(kcur[c * 16 + 2 * i + 1]) << 16);
                } else {
                    const u32x4* kp = reinterpret_cast<const u32x4*>(a.keys + (head_base + t) * 128 + c * 16);
                    const u32x4 lo = kp[0], hi = kp[1];
                    kw[0] = lo.x; kw[1] = lo.y; kw[2] = lo.z; kw[3] = lo.w;
                    kw[4] = hi.x; kw[5] = hi.y; kw[6] = hi.z; kw[7] = hi.w;
                }
                const float* q0 = &qp[0][c * 16];
                const float* q1 = &qp[1][c * 16];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float k0 = h2f(kw[i] & 0xffffu), k1 = h2f(kw[i] >> 16);
                    acc0 = __builtin_fmaf(q0[2 * i], k0, acc0);
                    acc1 = __builtin_fmaf(q1[2 * i], k0, acc1);
                    acc0 = __builtin_fmaf(q0[2 * i + 1], k1, acc0);
                    acc1 = __builtin_fmaf(q1[2 * i + 1], k1, acc1);
                }
            }
            const float d0 = combine_chains(acc0), d1 = combine_chains(acc1);
            if (c == 0 && tl < m) {
                sc[0][tl] = d0 * a.scale;
                sc[1][tl] = d1 * a.scale;
            }
        }
    }
    __syncthreads();

    // Split-local softmax statistics per head.
    float head_max, head_sum;
    {
        const int h = tid >> 7, i = tid & 127;
        const float v = i < m ? sc[h][i] : -INFINITY;
        const float mx = wave_max(v);
        if (lane == 0) redm[wave] = mx;
        __syncthreads();
        head_max = fmaxf(redm[2 * h], redm[2 * h + 1]);
        const float p = i < m ? expf(v - head_max) : 0.f;
        if (i < m) sc[h][i] = p;
        const float sm = wave_sum(p);
        if (lane == 0) reds[wave] = sm;
        __syncthreads();
        head_sum = reds[2 * h] + reds[2 * h + 1];
    }

    // P.V: wave pair per head; lane = channel group (8 channels) + position lane.
    {
        const int h = wave >> 1, cg = lane & 15, pl = ((wave & 1) << 2) | (lane >> 4);
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.f;
        for (int tl = pl; tl < m; tl += 8) {
            const int t = t0 + tl;
            const float p = sc[h][tl];
            uint32_t vw[4];
            if (t == pos) {
#pragma unroll
                for (int i = 0; i < 4; ++i) vw[i] = uint32_t(vcur[cg * 8 + 2 * i]) | (uint32_t(vcur[cg * 8 + 2 * i + 1]) << 16);
            } else {
                const u32x4 v = *reinterpret_cast<const u32x4*>(a.values + (head_base + t) * 128 + cg * 8);
                vw[0] = v.x; vw[1] = v.y; vw[2] = v.z; vw[3] = v.w;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc[2 * i] = __builtin_fmaf(h2f(vw[i] & 0xffffu), p, acc[2 * i]);
                acc[2 * i + 1] = __builtin_fmaf(h2f(vw[i] >> 16), p, acc[2 * i + 1]);
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            acc[i] += __shfl_xor(acc[i], 16);
            acc[i] += __shfl_xor(acc[i], 32);
        }
        if (lane < 16) {
#pragma unroll
            for (int i = 0; i < 8; ++i) opart[wave & 1][h][cg * 8 + i] = acc[i];
        }
    }
    __syncthreads();

    float* part = a.partial + (size_t(g) * kAttnSplits + s) * kAttnPartial;
    {
        const int h = tid >> 7, j = tid & 127;
        const float o = opart[0][h][j] + opart[1][h][j];
        __hip_atomic_store(part + h * 132 + j, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (j == 0) {
            __hip_atomic_store(part + h * 132 + 128, head_max, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(part + h * 132 + 129, head_sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(a.counters + g, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last = prev == unsigned(ns - 1);
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    {  // combine splits in fixed order
        const int h = tid >> 7, j = tid & 127;
        const float* base = a.partial + size_t(g) * kAttnSplits * kAttnPartial + h * 132;
        float mx = -INFINITY;
        for (int k = 0; k < ns; ++k)
            mx = fmaxf(mx, __hip_atomic_load(base + k * kAttnPartial + 128, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        float o = 0.f, l = 0.f;
        for (int k = 0; k < ns; ++k) {
            const float* p = base + k * kAttnPartial;
            const float w = expf(__hip_atomic_load(p + 128, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - mx);
            o += w * __hip_atomic_load(p + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            l += w * __hip_atomic_load(p + 129, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        a.attended[(2 * g + h) * 128 + j] = o / l;
    }
    if (tid == 0) __hip_atomic_store(a.counters + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

constexpr int kLayerWaves = 2;

template <int N, int MODE>
void launch_gemv(const GemvArgs& a, int rows, hipStream_t stream) {
    gemv_kernel<N, kLayerWaves, MODE><<<rows / (8 * kLayerWaves), 64 * kLayerWaves, 0, stream>>>(a);
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

void launch_layer_kernel(int which, const LayerDevice& L, const uint16_t* embed, const StepParams* params,
                         const float* cosines, const float* sines, int context, const DecodeScratch& s,
                         hipStream_t stream) {
    switch (which) {
        case 0: {
            GemvArgs q{};
            q.w = L.qkv_t;
            q.in = s.x;
            q.norm_w = L.in_norm;
            q.embed = embed;
            q.params = params;
            q.out = s.qkv;
            q.x = s.x;
            launch_gemv<kHidden, kQKV>(q, kQKVRows, stream);
            break;
        }
        case 1: {
            AttnArgs at{};
            at.qkv = s.qkv;
            at.q_norm = L.q_norm;
            at.k_norm = L.k_norm;
            at.cosines = cosines;
            at.sines = sines;
            at.keys = L.keys;
            at.values = L.values;
            at.params = params;
            at.partial = s.attn_partial;
            at.counters = s.attn_count;
            at.attended = s.attended;
            at.context = context;
            at.scale = 1.0f / std::sqrt(128.0f);
            attn_decode_kernel<<<dim3(kAttnSplits, kKVHeads), 256, 0, stream>>>(at);
            break;
        }
        case 2: {
            GemvArgs o{};
            o.w = L.o_t;
            o.in = s.attended;
            o.x = s.x;
            launch_gemv<kQDim, kO>(o, kHidden, stream);
            break;
        }
        case 3: {
            GemvArgs gu{};
            gu.w = L.gateup_t;
            gu.in = s.x;
            gu.norm_w = L.post_norm;
            gu.out = s.act;
            launch_gemv<kHidden, kGateUp>(gu, 2 * kFFN, stream);
            break;
        }
        case 4: {
            GemvArgs d{};
            d.w = L.down_t;
            d.in = s.act;
            d.x = s.x;
            launch_gemv<kFFN, kDown>(d, kHidden, stream);
            break;
        }
        default: throw std::runtime_error("unknown decode kernel");
    }
}

void launch_decode_layer(const LayerDevice& L, const uint16_t* embed, const StepParams* params, const float* cosines,
                         const float* sines, int context, const DecodeScratch& s, hipStream_t stream) {
    for (int which = 0; which < 5; ++which)
        launch_layer_kernel(which, L, which == 0 ? embed : nullptr, params, cosines, sines, context, s, stream);
}

void launch_lm_head(const uint16_t* lm_t, const float* final_norm, const DecodeScratch& s, hipStream_t stream) {
    GemvArgs a{};
    a.w = lm_t;
    a.in = s.x;
    a.norm_w = final_norm;
    a.out = s.logits;
    a.hidden = s.hidden;
    a.lm_value = s.lm_value;
    a.lm_index = s.lm_index;
    a.lm_bad = s.lm_bad;
    a.lm_count = s.lm_count;
    a.result = s.result;
    gemv_kernel<kHidden, kLmWaves, kLmHead><<<kLmGroups, 64 * kLmWaves, 0, stream>>>(a);
}

}  // namespace qwen_hip
