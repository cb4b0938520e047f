// Batched prefill kernels for gfx950: a chunk of up to 512 prompt rows runs
// through each layer as GEMMs on the matrix cores plus row kernels
// (engine/core.cpp:353-646 with batch > 1).
//
// GEMM: C[M x N] = A[M x K] . W[N x K]^T with natural FP16 weights on
// v_mfma_f32_32x32x16_f16. The FP32 activations are split exactly into
// hi = fp16(a) and lo = fp16(a - hi) (a - hi is exact in FP32), and both
// halves are multiplied: about 22 significant bits of each activation enter
// the FP32 accumulation, close to the reference's FP32 SGEMM
// (engine/core.cpp:293-294) at twice the MFMA work of a plain FP16 GEMM.
// Each output element's K order is fixed by its column, so a row's result
// does not depend on how many rows the chunk holds.
#include <hip/hip_runtime.h>

#include <cfloat>

#include "kernels.hpp"
#include "prefill.hpp"

namespace qwen_hip {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

constexpr int kTileM = 64, kTileN = 64, kTileK = 64;
constexpr int kLdsRow = kTileK + 8;  // halves per LDS row (padding against bank conflicts)

// Epilogue: 0 store, 1 add into C (residual).
template <int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const float* __restrict__ A, const uint16_t* __restrict__ W,
                                                   float* __restrict__ C, int M, int N, int K) {
    __shared__ _Float16 a_hi[kTileM][kLdsRow];
    __shared__ _Float16 a_lo[kTileM][kLdsRow];
    __shared__ _Float16 b_s[kTileN][kLdsRow];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * kTileM, n0 = blockIdx.x * kTileN;
    const int wm = wave & 1, wn = wave >> 1;
    // Tile loads: thread -> (row, 16 consecutive k).
    const int lr = tid >> 2, lk = (tid & 3) * 16;
    const bool a_ok = m0 + lr < M;
    const float* a_row = A + size_t(m0 + lr) * K + lk;
    const uint16_t* b_row = W + size_t(n0 + lr) * K + lk;
    floatx16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;

    for (int k0 = 0; k0 < K; k0 += kTileK) {
        float4 av[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            av[i] = a_ok ? reinterpret_cast<const float4*>(a_row + k0)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        const u32x4 bv0 = reinterpret_cast<const u32x4*>(b_row + k0)[0];
        const u32x4 bv1 = reinterpret_cast<const u32x4*>(b_row + k0)[1];
        __syncthreads();  // previous tile fully consumed
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v[4] = {av[i].x, av[i].y, av[i].z, av[i].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const _Float16 hi = static_cast<_Float16>(v[e]);
                const _Float16 lo = static_cast<_Float16>(v[e] - static_cast<float>(hi));
                a_hi[lr][lk + 4 * i + e] = hi;
                a_lo[lr][lk + 4 * i + e] = lo;
            }
        }
        *reinterpret_cast<u32x4*>(&b_s[lr][lk]) = bv0;
        *reinterpret_cast<u32x4*>(&b_s[lr][lk + 8]) = bv1;
        __syncthreads();
        const int fr = lane & 31, fk = (lane >> 5) * 8;
#pragma unroll
        for (int ks = 0; ks < kTileK; ks += 16) {
            const half8 ah = *reinterpret_cast<const half8*>(&a_hi[wm * 32 + fr][ks + fk]);
            const half8 al = *reinterpret_cast<const half8*>(&a_lo[wm * 32 + fr][ks + fk]);
            const half8 bb = *reinterpret_cast<const half8*>(&b_s[wn * 32 + fr][ks + fk]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bb, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bb, acc, 0, 0, 0);
        }
    }
    // D layout: lane -> column (lane & 31); register r -> row 8(r/4) + 4(lane/32) + r%4.
    const int n = n0 + wn * 32 + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < M) {
            float* c = C + size_t(m) * N + n;
            if constexpr (EPI == 1)
                *c = *c + acc[r];
            else
                *c = acc[r];
        }
    }
}

// x[b] = fp32(E[ids[b]]) (engine/core.cpp:382-383).
__global__ __launch_bounds__(256) void embed_rows_kernel(const int* __restrict__ ids, const uint16_t* __restrict__ E,
                                                         float* __restrict__ X) {
    const int b = blockIdx.x;
    const uint16_t* row = E + size_t(ids[b]) * kHidden;
    for (int j = threadIdx.x; j < kHidden; j += 256) X[size_t(b) * kHidden + j] = h2f(row[j]);
}

// out[b] = RMSNorm(x[b]) (engine/core.cpp:207-215): FP32 squares, FP64 sum.
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* __restrict__ X, const float* __restrict__ w,
                                                           float* __restrict__ out) {
    const int b = blockIdx.x, tid = threadIdx.x;
    const float* x = X + size_t(b) * kHidden;
    float v[4];
    double part = 0.0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        v[k] = x[tid + 256 * k];
        const float square = v[k] * v[k];
        part += static_cast<double>(square);
    }
    part = wave_sum(part);
    __shared__ double red[4];
    if ((tid & 63) == 0) red[tid >> 6] = part;
    __syncthreads();
    const float sum = static_cast<float>((red[0] + red[1]) + (red[2] + red[3]));
    const float inv = 1.0f / __builtin_sqrtf(sum / 1024.0f + 1e-6f);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int j = tid + 256 * k;
        out[size_t(b) * kHidden + j] = (v[k] * inv) * w[j];
    }
}

// Per (row, head): QK-norm + RoPE for the 16 q heads (written back in the
// key's chain-permuted order) and the 8 k heads (FP16 into the cache), V to
// the cache (engine/core.cpp:395-406). Grid (rows, 24), 128 threads.
__global__ __launch_bounds__(128) void qk_rope_kv_kernel(float* __restrict__ QKV, const float* __restrict__ q_norm,
                                                         const float* __restrict__ k_norm,
                                                         const float* __restrict__ cosines,
                                                         const float* __restrict__ sines, uint16_t* __restrict__ keys,
                                                         uint16_t* __restrict__ values, int pos0, int context) {
    const int b = blockIdx.x, head = blockIdx.y, j = threadIdx.x, lane = j & 63;
    const int pos = pos0 + b;
    float* row = QKV + size_t(b) * kQKVRows;
    const bool is_q = head < kQHeads;
    const int kh = head - kQHeads;
    float* src = is_q ? row + head * kHeadDim : row + kQDim + kh * kHeadDim;
    const float raw = src[j];
    const float square = raw * raw;
    const double part = wave_sum(static_cast<double>(square));
    __shared__ double red[2];
    __shared__ float buf[128];
    if (lane == 0) red[j >> 6] = part;
    __syncthreads();
    const float sum = static_cast<float>(red[0] + red[1]);
    const float inv = 1.0f / __builtin_sqrtf(sum / 128.0f + 1e-6f);
    buf[j] = (raw * inv) * (is_q ? q_norm : k_norm)[j];
    __syncthreads();
    const float* cs = cosines + size_t(pos) * 64;
    const float* sn = sines + size_t(pos) * 64;
    float out;
    if (j < 64) {
        out = buf[j] * cs[j] - buf[j + 64] * sn[j];
    } else {
        const int jj = j - 64;
        out = buf[j] * cs[jj] + buf[jj] * sn[jj];
    }
    if (is_q) {
        __syncthreads();  // all raw values read before the in-place write
        src[kperm(j)] = out;
    } else {
        const size_t slot = (size_t(kh) * context + pos) * kHeadDim;
        keys[slot + kperm(j)] = f2h(out);
        values[slot + j] = f2h(row[kQDim + kKVDim + kh * kHeadDim + j]);
    }
}

// Causal attention for a chunk (engine/core.cpp:407-605): workgroup = 16
// query rows x the two query heads of KV head g; keys in tiles of 64 from
// the FP16 cache, online softmax per query. q rows hold the chain-permuted
// order of the cached keys, so plain index order gives the same dot.
constexpr int kQRows = 16, kKeyTile = 64;
__global__ __launch_bounds__(256) void attn_prefill_kernel(const float* __restrict__ QKV,
                                                           const uint16_t* __restrict__ keys,
                                                           const uint16_t* __restrict__ values,
                                                           float* __restrict__ attended, int rows, int pos0,
                                                           int context, float scale) {
    __shared__ float qs[2 * kQRows][kHeadDim];
    __shared__ uint16_t ks[kKeyTile][kHeadDim + 8];
    __shared__ uint16_t vs[kKeyTile][kHeadDim];
    __shared__ float ps[2 * kQRows][kKeyTile];
    const int b0 = blockIdx.x * kQRows, g = blockIdx.y, tid = threadIdx.x;
    const int nrows = min(kQRows, rows - b0);
    // query vector qi = 2 * row + head
    for (int i = tid; i < 2 * kQRows * kHeadDim; i += 256) {
        const int qi = i / kHeadDim, d = i % kHeadDim, r = qi >> 1;
        qs[qi][d] = r < nrows ? QKV[size_t(b0 + r) * kQKVRows + (2 * g + (qi & 1)) * kHeadDim + d] : 0.f;
    }
    const int qi = tid >> 3, sub = tid & 7, row = qi >> 1;
    const int qpos = pos0 + b0 + row;  // causal limit for this query
    const int last = pos0 + b0 + nrows - 1;
    const size_t head_base = size_t(g) * context;
    float m_run = -INFINITY, l_run = 0.f;
    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;

    for (int t0 = 0; t0 <= last; t0 += kKeyTile) {
        __syncthreads();
        for (int i = tid; i < kKeyTile * 16; i += 256) {  // 16-byte pieces
            const int key = i >> 4, piece = i & 15, t = t0 + key;
            u32x4 kv = {0, 0, 0, 0}, vv = {0, 0, 0, 0};
            if (t <= last) {
                kv = reinterpret_cast<const u32x4*>(keys + (head_base + t) * kHeadDim)[piece];
                vv = reinterpret_cast<const u32x4*>(values + (head_base + t) * kHeadDim)[piece];
            }
            *reinterpret_cast<u32x4*>(&ks[key][piece * 8]) = kv;
            *reinterpret_cast<u32x4*>(&vs[key][piece * 8]) = vv;
        }
        __syncthreads();
        float s[8];
        float tile_max = -INFINITY;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const int key = sub + 8 * jj, t = t0 + key;
            float dotv = 0.f;
#pragma unroll 8
            for (int d = 0; d < kHeadDim; ++d) dotv = __builtin_fmaf(qs[qi][d], h2f(ks[key][d]), dotv);
            s[jj] = (t <= qpos && row < nrows) ? dotv * scale : -INFINITY;
            tile_max = fmaxf(tile_max, s[jj]);
        }
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) tile_max = fmaxf(tile_max, __shfl_xor(tile_max, off));
        const float m_new = fmaxf(m_run, tile_max);
        const float rescale = m_new == -INFINITY ? 1.f : (m_run == -INFINITY ? 0.f : expf(m_run - m_new));
        float psum = 0.f;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const float p = s[jj] == -INFINITY ? 0.f : expf(s[jj] - m_new);
            ps[qi][sub + 8 * jj] = p;
            psum += p;
        }
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) psum += __shfl_xor(psum, off);
        l_run = l_run * rescale + psum;
        m_run = m_new;
        // ps[qi] is written and read by the same 8 lanes of one wave.
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] *= rescale;
        for (int key = 0; key < kKeyTile; ++key) {
            const float p = ps[qi][key];
            const u32x4 v0 = *reinterpret_cast<const u32x4*>(&vs[key][sub * 16]);
            const u32x4 v1 = *reinterpret_cast<const u32x4*>(&vs[key][sub * 16 + 8]);
            const uint32_t w[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                acc[2 * i] = __builtin_fmaf(h2f(uint16_t(w[i] & 0xffffu)), p, acc[2 * i]);
                acc[2 * i + 1] = __builtin_fmaf(h2f(uint16_t(w[i] >> 16)), p, acc[2 * i + 1]);
            }
        }
    }
    if (row < nrows) {
        float* out = attended + size_t(b0 + row) * kQDim + (2 * g + (qi & 1)) * kHeadDim + sub * 16;
#pragma unroll
        for (int i = 0; i < 16; ++i) out[i] = acc[i] / l_run;
    }
}

// act[b][i] = g * (0.5 + 0.5 * tanh(0.5 g)) * u with g = GU[b][i], u = GU[b][3072 + i]
// (engine/core.cpp:636-639).
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const float* __restrict__ GU, float* __restrict__ act,
                                                          int total) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const int b = idx / kFFN, i = idx % kFFN;
    const float gate = GU[size_t(b) * 2 * kFFN + i], up = GU[size_t(b) * 2 * kFFN + kFFN + i];
    const float half_gate = gate * 0.5f;
    const float t = tanhf(half_gate);
    act[idx] = gate * (0.5f + 0.5f * t) * up;
}

template <int EPI>
void gemm(const float* A, const uint16_t* W, float* C, int M, int N, int K, hipStream_t stream) {
    require(N % kTileN == 0 && K % kTileK == 0 && M > 0, "gemm: unsupported shape");
    gemm_kernel<EPI><<<dim3(N / kTileN, (M + kTileM - 1) / kTileM), 256, 0, stream>>>(A, W, C, M, N, K);
}

}  // namespace

void launch_gemm(const float* A, const uint16_t* W, float* C, int M, int N, int K, bool accumulate,
                 hipStream_t stream) {
    if (accumulate)
        gemm<1>(A, W, C, M, N, K, stream);
    else
        gemm<0>(A, W, C, M, N, K, stream);
}

void launch_prefill_chunk(const PrefillLayer* layers, const uint16_t* embed, const int* ids_dev, int rows, int pos0,
                          const float* cosines, const float* sines, int context, const PrefillScratch& s,
                          hipStream_t stream) {
    require(rows >= 1 && rows <= kChunk, "prefill chunk: bad row count");
    embed_rows_kernel<<<rows, 256, 0, stream>>>(ids_dev, embed, s.x);
    const float scale = 1.0f / std::sqrt(128.0f);
    for (int l = 0; l < kLayers; ++l) {
        const PrefillLayer& L = layers[l];
        rmsnorm_rows_kernel<<<rows, 256, 0, stream>>>(s.x, L.in_norm, s.h);
        gemm<0>(s.h, L.qkv_n, s.qkv, rows, kQKVRows, kHidden, stream);
        qk_rope_kv_kernel<<<dim3(rows, kQHeads + kKVHeads), 128, 0, stream>>>(s.qkv, L.q_norm, L.k_norm, cosines, sines,
                                                                             L.keys, L.values, pos0, context);
        attn_prefill_kernel<<<dim3((rows + kQRows - 1) / kQRows, kKVHeads), 256, 0, stream>>>(
            s.qkv, L.keys, L.values, s.attended, rows, pos0, context, scale);
        gemm<1>(s.attended, L.o_n, s.x, rows, kHidden, kQDim, stream);
        rmsnorm_rows_kernel<<<rows, 256, 0, stream>>>(s.x, L.post_norm, s.h);
        gemm<0>(s.h, L.gateup_n, s.gu, rows, 2 * kFFN, kHidden, stream);
        swiglu_rows_kernel<<<(rows * kFFN + 255) / 256, 256, 0, stream>>>(s.gu, s.act, rows * kFFN);
        gemm<1>(s.act, L.down_n, s.x, rows, kHidden, kFFN, stream);
    }
}

}  // namespace qwen_hip
