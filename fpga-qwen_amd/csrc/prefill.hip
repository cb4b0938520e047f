// Batched prefill kernels for gfx950: up to 4096 prompt rows run through
// each layer as GEMMs on the matrix cores plus row kernels
// (engine/core.cpp:353-646 with batch > 1). QK-norm, RoPE and the K/V cache
// writes run in the QKV GEMM's epilogue, SwiGLU in the gate/up GEMM's, and
// the residual adds of the K-split O and down GEMMs in the next RMSNorm.
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

// C[M x N] (+)= A[M x K] . W[N x K]^T on the matrix cores. Workgroup tile TM
// x 128 (TM = 64 or 32), K in steps of 64; 4 waves, each owning 32 rows x
// (64 or 32) columns of C as 32x32 MFMA tiles. A (FP32) enters LDS as
// FP16 hi = fp16(a) and lo = fp16(a - hi), W as its FP16 values; every
// product runs twice (hi, lo), so products are exact and sums FP32. The next
// K step's global loads are issued before the current step's MFMAs. Each
// output element accumulates its K terms in the same order whatever TM and
// its row position, so results do not depend on M or on how rows are grouped.
constexpr int kTileN = 128, kTileK = 64;
constexpr int kLdsRow = kTileK + 8;  // halves per LDS row (padding against bank conflicts)

// Per-head work fused into the QKV GEMM (EPI 4): QK-norm, RoPE and the K/V
// cache writes of engine/core.cpp:395-406.
struct QkvEpilogue {
    const float* q_norm;
    const float* k_norm;
    const float* cosines;
    const float* sines;
    uint16_t* keys;
    uint16_t* values;
    int pos0;
    int context;
};

// Epilogue: 0 store, 1 add into C (residual), 2 store the partial product
// of K range blockIdx.z (K / gridDim.z columns) at C + blockIdx.z M N,
// 3 SwiGLU (W = gate rows then up rows, N = 2F: tile t multiplies gate rows
// 64t.. and up rows F + 64t.. and stores act[m][64t + i], C has F columns),
// 4 QKV rows (tile t = head t): q heads QK-normed, rotated and stored in the
// key's chain-permuted order, k heads QK-normed, rotated and written to the
// cache as FP16, v heads written to the cache. Epilogues 3 and 4 stage the
// finished tile in LDS.
template <int TM, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const float* __restrict__ A, const uint16_t* __restrict__ W,
                                                   float* __restrict__ C, int M, int N, int K, QkvEpilogue ep) {
    static_assert(TM == 64 || TM == 32, "tile height");
    constexpr int kWaveRows = TM / 32, kWaveCols = 4 / kWaveRows;  // wave grid
    constexpr int kColTiles = kTileN / kWaveCols / 32;              // 32-column MFMA tiles per wave
    constexpr int kAThreadsPerRow = 256 / TM;   // threads loading one A row of the K step
    constexpr int kAF4 = kTileK / 4 / kAThreadsPerRow;  // float4 loads per thread
    constexpr int kCPitch = kTileN + 4;                     // floats per row of the staged C tile
    constexpr int kABytes = TM * kLdsRow * 2, kBBytes = kTileN * kLdsRow * 2;
    constexpr int kSmem = 2 * kABytes + kBBytes > TM * kCPitch * 4 ? 2 * kABytes + kBBytes : TM * kCPitch * 4;
    __shared__ __align__(16) unsigned char smem[kSmem];
    _Float16(*a_hi)[kLdsRow] = reinterpret_cast<_Float16(*)[kLdsRow]>(smem);
    _Float16(*a_lo)[kLdsRow] = reinterpret_cast<_Float16(*)[kLdsRow]>(smem + kABytes);
    _Float16(*b_s)[kLdsRow] = reinterpret_cast<_Float16(*)[kLdsRow]>(smem + 2 * kABytes);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * TM, n0 = blockIdx.x * kTileN;
    const int wm = wave % kWaveRows, wn = wave / kWaveRows;
    // Global loads: A row ar (rows past M repeat row M - 1 and are not
    // stored), 4 * kAF4 consecutive k; W row br, 32 consecutive k.
    const int ar = tid / kAThreadsPerRow, ak = (tid % kAThreadsPerRow) * 4 * kAF4;
    const int br = tid >> 1, bk = (tid & 1) * 32;
    const int ks = K / gridDim.z, kz = blockIdx.z * ks;  // this workgroup's K range
    const float* a_row = A + size_t(min(m0 + ar, M - 1)) * K + kz + ak;
    const int wr = EPI == 3 ? (br < 64 ? n0 / 2 + br : N / 2 + n0 / 2 + br - 64) : n0 + br;  // W row of tile row br
    const uint16_t* b_row = W + size_t(wr) * K + kz + bk;
    float4 av[kAF4];
    u32x4 bv[4];
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < kAF4; ++i) av[i] = reinterpret_cast<const float4*>(a_row + k0)[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) bv[i] = reinterpret_cast<const u32x4*>(b_row + k0)[i];
    };
    floatx16 acc[kColTiles];
#pragma unroll
    for (int jt = 0; jt < kColTiles; ++jt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[jt][r] = 0.f;

    load(0);
    const int fr = lane & 31, fk = (lane >> 5) * 8;
    for (int k0 = 0; k0 < ks; k0 += kTileK) {
        __syncthreads();  // the previous step's fragments are consumed
#pragma unroll
        for (int i = 0; i < kAF4; i += 2) {  // 8 values -> one 16-byte store per plane
            const float v[8] = {av[i].x, av[i].y, av[i].z, av[i].w, av[i + 1].x, av[i + 1].y, av[i + 1].z, av[i + 1].w};
            half8 hi8, lo8;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const _Float16 hi = static_cast<_Float16>(v[e]);
                hi8[e] = hi;
                lo8[e] = static_cast<_Float16>(v[e] - static_cast<float>(hi));
            }
            *reinterpret_cast<half8*>(&a_hi[ar][ak + 4 * i]) = hi8;
            *reinterpret_cast<half8*>(&a_lo[ar][ak + 4 * i]) = lo8;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(&b_s[br][bk + 8 * i]) = bv[i];
        __syncthreads();
        if (k0 + kTileK < ks) load(k0 + kTileK);
#pragma unroll
        for (int ks = 0; ks < kTileK; ks += 16) {
            const half8 ah = *reinterpret_cast<const half8*>(&a_hi[wm * 32 + fr][ks + fk]);
            const half8 al = *reinterpret_cast<const half8*>(&a_lo[wm * 32 + fr][ks + fk]);
            half8 bb[kColTiles];
#pragma unroll
            for (int jt = 0; jt < kColTiles; ++jt)
                bb[jt] = *reinterpret_cast<const half8*>(&b_s[wn * 32 * kColTiles + 32 * jt + fr][ks + fk]);
#pragma unroll
            for (int jt = 0; jt < kColTiles; ++jt) {
                acc[jt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bb[jt], acc[jt], 0, 0, 0);
                acc[jt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bb[jt], acc[jt], 0, 0, 0);
            }
        }
    }
    // D layout: lane -> column (lane & 31); register r -> row 8(r/4) + 4(lane/32) + r%4.
    if constexpr (EPI <= 2) {
#pragma unroll
        for (int jt = 0; jt < kColTiles; ++jt) {
            const int n = n0 + wn * 32 * kColTiles + 32 * jt + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < M) {
                    float* c = C + (size_t(blockIdx.z) * M + m) * N + n;
                    if constexpr (EPI == 1)
                        *c = *c + acc[jt][r];
                    else
                        *c = acc[jt][r];
                }
            }
        }
        return;
    }
    float(*ct)[kCPitch] = reinterpret_cast<float(*)[kCPitch]>(smem);
    __syncthreads();  // every wave is done with the operand tiles
#pragma unroll
    for (int jt = 0; jt < kColTiles; ++jt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            ct[wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)][wn * 32 * kColTiles + 32 * jt + (lane & 31)] =
                acc[jt][r];
    __syncthreads();
    if constexpr (EPI == 3) {
        // SwiGLU (engine/core.cpp:636-639): thread -> row tid / 4, outputs 16 (tid % 4) .. +15.
        const int row = tid >> 2, c0 = (tid & 3) * 16, m = m0 + row;
        if (row < TM && m < M) {
            float* out = C + size_t(m) * (N / 2) + n0 / 2 + c0;
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float gate = ct[row][c0 + i + e], up = ct[row][64 + c0 + i + e];
                    const float half_gate = gate * 0.5f;
                    const float t = tanhf(half_gate);
                    o[e] = gate * (0.5f + 0.5f * t) * up;
                }
                *reinterpret_cast<float4*>(out + i) = make_float4(o[0], o[1], o[2], o[3]);
            }
        }
    } else {
        // Thread -> row tid / 4, channels j in [16 s, 16 s + 16) and j + 64 (s = tid % 4).
        const int row = tid >> 2, s4 = tid & 3, m = m0 + row, head = blockIdx.x;
        if (row < TM && m < M) {
            const int pos = ep.pos0 + m;
            if (head >= kQHeads + kKVHeads) {  // v: FP16 into the cache
                uint16_t* vrow = ep.values + (size_t(head - kQHeads - kKVHeads) * ep.context + pos) * kHeadDim;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    vrow[16 * s4 + i] = f2h(ct[row][16 * s4 + i]);
                    vrow[64 + 16 * s4 + i] = f2h(ct[row][64 + 16 * s4 + i]);
                }
            } else {
                const bool is_q = head < kQHeads;
                const float* w = is_q ? ep.q_norm : ep.k_norm;
                float x0[16], x1[16];
                double part = 0.0;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    x0[i] = ct[row][16 * s4 + i];
                    x1[i] = ct[row][64 + 16 * s4 + i];
                    const float s0 = x0[i] * x0[i], s1 = x1[i] * x1[i];
                    part += static_cast<double>(s0);
                    part += static_cast<double>(s1);
                }
                part += __shfl_xor(part, 1);
                part += __shfl_xor(part, 2);
                const float inv = 1.0f / __builtin_sqrtf(static_cast<float>(part) / 128.0f + 1e-6f);
                const float* cs = ep.cosines + size_t(pos) * 64;
                const float* sn = ep.sines + size_t(pos) * 64;
                float* qrow = C + size_t(m) * N + head * kHeadDim;
                uint16_t* krow = ep.keys + (size_t(head - kQHeads) * ep.context + pos) * kHeadDim;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int j = 16 * s4 + i;
                    const float n0v = (x0[i] * inv) * w[j], n1v = (x1[i] * inv) * w[j + 64];
                    const float o0 = n0v * cs[j] - n1v * sn[j];
                    const float o1 = n1v * cs[j] + n0v * sn[j];
                    if (is_q) {
                        qrow[kperm(j)] = o0;
                        qrow[kperm(j + 64)] = o1;
                    } else {
                        krow[kperm(j)] = f2h(o0);
                        krow[kperm(j + 64)] = f2h(o1);
                    }
                }
            }
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

// x + the SPLITS partial products of a K-split GEMM in a fixed order.
template <int SPLITS>
__device__ __forceinline__ float fold_splits(float x, const float* p, size_t stride) {
    if constexpr (SPLITS == 0) return x;
    else if constexpr (SPLITS == 2) return x + (p[0] + p[stride]);
    else return x + ((p[0] + p[stride]) + p[2 * stride]);
}

// out[b] = RMSNorm(x[b]) (engine/core.cpp:207-215): FP32 squares, FP64 sum.
// With SPLITS > 0 the residual first absorbs the pending partial products of
// a K-split GEMM (parts[z][b], z < SPLITS) and is written back.
template <int SPLITS = 0>
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(float* __restrict__ X, const float* __restrict__ w,
                                                           float* __restrict__ out, const float* __restrict__ parts,
                                                           int rows) {
    const int b = blockIdx.x, tid = threadIdx.x;
    float* x = X + size_t(b) * kHidden;
    float v[4];
    double part = 0.0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int j = tid + 256 * k;
        v[k] = x[j];
        if constexpr (SPLITS > 0) {
            v[k] = fold_splits<SPLITS>(v[k], parts + size_t(b) * kHidden + j, size_t(rows) * kHidden);
            x[j] = v[k];
        }
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

// Causal attention for a prefill chunk on the matrix cores (engine/core.cpp:
// 407-605, same math as the decode path): workgroup = 32 consecutive query
// rows x one query head; its 4 waves take every 4th tile of 32 keys, each
// with its own online softmax, and merge (max, sum, output) at the end.
//   S^T = K Q^T  (A = 32 keys x 16 dims straight from the cache, B = Q^T as
//                 FP16 hi + lo of the FP32 q, so products are exact)
//   O^T += V^T P^T (A = V^T through a per-wave LDS transpose, B = P^T as
//                 FP16 hi + lo of the FP32 probabilities)
// With S^T in the 32x32 accumulator layout each lane holds 16 keys of one
// query (lane % 32), so the softmax statistics stay in the lane: one
// exchange with lane ^ 32 per tile. q and the cached keys share the
// chain-permuted channel order, which leaves q . k unchanged.
constexpr int kFaRows = 32, kFaKeys = 32, kFaWaves = 4, kVtPitch = 36, kFaccPitch = 132;
typedef _Float16 half4 __attribute__((ext_vector_type(4)));

// Two waves per SIMD (at most 256 registers per lane, two workgroups per
// CU): one wave's softmax and V^T work overlaps the other's matrix ops.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_prefill_mfma_kernel(const float* __restrict__ QKV,
                                                                const uint16_t* __restrict__ keys,
                                                                const uint16_t* __restrict__ values,
                                                                float* __restrict__ attended, int rows, int pos0,
                                                                int context, float scale) {
    // LDS: per-wave V^T tiles during the key loop, then the 4 waves' outputs.
    __shared__ __align__(16) unsigned char lds[kFaWaves * kFaRows * kFaccPitch * 4];
    __shared__ float fm[kFaWaves][kFaRows], fl[kFaWaves][kFaRows];
    const int qb = blockIdx.x, head = blockIdx.y, g = head >> 1;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, hf = lane >> 5;
    const int b0 = qb * kFaRows, nrows = min(kFaRows, rows - b0);
    const int last = pos0 + b0 + nrows - 1;  // last key any query of the block attends to
    const int ntiles = last / kFaKeys + 1;
    const size_t head_base = size_t(g) * context;
    const int qpos = pos0 + b0 + col;        // causal limit of this lane's query
    // Softmax in base 2: scores scaled by log2(e) / sqrt(128), weights 2^(s - m)
    // = e^(scaled score - max) from the hardware exp2.
    const float scale2 = scale * 1.4426950408889634f;
    uint16_t(*vt)[kVtPitch] = reinterpret_cast<uint16_t(*)[kVtPitch]>(lds + wave * 128 * kVtPitch * 2);

    // Q^T operand: query b0 + col (rows past the chunk repeat its last row
    // and are never written), channels 16s + 8hf .. +7.
    half8 qh[8], ql[8];
    {
        const float* qrow = QKV + size_t(b0 + min(col, nrows - 1)) * kQKVRows + head * kHeadDim + 8 * hf;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const float4 x0 = reinterpret_cast<const float4*>(qrow + 16 * s)[0];
            const float4 x1 = reinterpret_cast<const float4*>(qrow + 16 * s)[1];
            const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const _Float16 h = static_cast<_Float16>(v[i]);
                qh[s][i] = h;
                ql[s][i] = static_cast<_Float16>(v[i] - static_cast<float>(h));
            }
        }
    }
    float m = -INFINITY, l = 0.f;
    floatx16 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;

    const int vp = lane & 15, vg = lane >> 4;  // V^T fill: key pair vp, channel group vg
    for (int kt = wave; kt < ntiles; kt += kFaWaves) {
        const int t0 = kt * kFaKeys;
        // Keys past `last` load row `last` and are masked below.
        const u32x4* krow = reinterpret_cast<const u32x4*>(keys + (head_base + min(t0 + col, last)) * kHeadDim);
        half8 ka[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) ka[s] = __builtin_bit_cast(half8, krow[2 * s + hf]);
        const u32x4* va_row = reinterpret_cast<const u32x4*>(values + (head_base + min(t0 + 2 * vp, last)) * kHeadDim);
        const u32x4* vb_row =
            reinterpret_cast<const u32x4*>(values + (head_base + min(t0 + 2 * vp + 1, last)) * kHeadDim);
        u32x4 va[4], vb[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            va[r] = va_row[vg + 4 * r];
            vb[r] = vb_row[vg + 4 * r];
        }
        floatx16 st;
#pragma unroll
        for (int r = 0; r < 16; ++r) st[r] = 0.f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            st = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[s], qh[s], st, 0, 0, 0);
            st = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[s], ql[s], st, 0, 0, 0);
        }
        // V^T: channel 32r + 8vg + e, keys 2vp (low half) and 2vp + 1 (high half).
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t aw[4] = {va[r].x, va[r].y, va[r].z, va[r].w};
            const uint32_t bw[4] = {vb[r].x, vb[r].y, vb[r].z, vb[r].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ch = 32 * r + 8 * vg + 2 * i;
                *reinterpret_cast<uint32_t*>(&vt[ch][2 * vp]) = (aw[i] & 0xffffu) | (bw[i] << 16);
                *reinterpret_cast<uint32_t*>(&vt[ch + 1][2 * vp]) = (aw[i] >> 16) | (bw[i] & 0xffff0000u);
            }
        }
        // Online softmax; register r holds key t0 + 8(r/4) + 4hf + r%4.
        float sv[16];
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + 8 * (r >> 2) + 4 * hf + (r & 3);
            sv[r] = t <= qpos ? st[r] * scale2 : -INFINITY;
            tmax = fmaxf(tmax, sv[r]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float mnew = fmaxf(m, tmax);
        const float factor = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mnew);
        half8 ph[2], pl[2];
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = sv[r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sv[r] - mnew);
            psum += p;
            const _Float16 h = static_cast<_Float16>(p);
            ph[r >> 3][r & 7] = h;
            pl[r >> 3][r & 7] = static_cast<_Float16>(p - static_cast<float>(h));
        }
        psum += __shfl_xor(psum, 32);
        l = l * factor + psum;
        // Rescaling by 1 changes nothing; skip it when no lane's maximum moved.
        if (__builtin_amdgcn_ballot_w64(mnew != m) != 0) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[dt][r] *= factor;
        }
        m = mnew;
        // vt is written and read by this wave only.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const uint16_t* vrow = vt[32 * dt + col];
                const half4 lo4 = *reinterpret_cast<const half4*>(vrow + 16 * j + 4 * hf);
                const half4 hi4 = *reinterpret_cast<const half4*>(vrow + 16 * j + 8 + 4 * hf);
                const half8 a = __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
                acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, ph[j], acc[dt], 0, 0, 0);
                acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pl[j], acc[dt], 0, 0, 0);
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // Merge the 4 waves: O^T register r of tile dt is channel 32dt + 8(r/4) + 4hf + r%4 of query col.
    __syncthreads();  // every wave is done with its V^T tile
    float(*facc)[kFaccPitch] = reinterpret_cast<float(*)[kFaccPitch]>(lds + wave * kFaRows * kFaccPitch * 4);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) facc[col][32 * dt + 8 * (r >> 2) + 4 * hf + (r & 3)] = acc[dt][r];
    if (hf == 0) {
        fm[wave][col] = m;
        fl[wave][col] = l;
    }
    __syncthreads();
    const int q = tid >> 3, c0 = (tid & 7) * 16;
    if (q < nrows) {
        float mx = fm[0][q];
#pragma unroll
        for (int w = 1; w < kFaWaves; ++w) mx = fmaxf(mx, fm[w][q]);
        float e[kFaWaves], lsum = 0.f;
#pragma unroll
        for (int w = 0; w < kFaWaves; ++w) {
            e[w] = fm[w][q] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(fm[w][q] - mx);
            lsum = __builtin_fmaf(e[w], fl[w][q], lsum);
        }
        float* out = attended + size_t(b0 + q) * kQDim + head * kHeadDim + c0;
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) {
            float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int w = 0; w < kFaWaves; ++w) {
                const float4 v = *reinterpret_cast<const float4*>(
                    reinterpret_cast<const float*>(lds + w * kFaRows * kFaccPitch * 4) + q * kFaccPitch + c0 + 4 * k4);
                o[0] = __builtin_fmaf(e[w], v.x, o[0]);
                o[1] = __builtin_fmaf(e[w], v.y, o[1]);
                o[2] = __builtin_fmaf(e[w], v.z, o[2]);
                o[3] = __builtin_fmaf(e[w], v.w, o[3]);
            }
            reinterpret_cast<float4*>(out)[k4] = make_float4(o[0] / lsum, o[1] / lsum, o[2] / lsum, o[3] / lsum);
        }
    }
}

// X[b] += the SPLITS partial products of a K-split GEMM (rows x 1024).
template <int SPLITS>
__global__ __launch_bounds__(256) void fold_rows_kernel(float* __restrict__ X, const float* __restrict__ parts,
                                                        int rows) {
    const size_t idx = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (idx < size_t(rows) * kHidden) X[idx] = fold_splits<SPLITS>(X[idx], parts + idx, size_t(rows) * kHidden);
}

// 64-row tiles when they give every CU a workgroup, else 32-row tiles.
// `splits` K ranges (EPI 2) count towards the workgroups.
template <int EPI>
void gemm(const float* A, const uint16_t* W, float* C, int M, int N, int K, hipStream_t stream, int splits = 1,
          const QkvEpilogue& ep = {}) {
    require(N % kTileN == 0 && K % (kTileK * splits) == 0 && M > 0 && (splits == 1 || EPI == 2),
            "gemm: unsupported shape");
    if ((M + 63) / 64 * (N / kTileN) * splits >= 256)
        gemm_kernel<64, EPI><<<dim3(N / kTileN, (M + 63) / 64, splits), 256, 0, stream>>>(A, W, C, M, N, K, ep);
    else
        gemm_kernel<32, EPI><<<dim3(N / kTileN, (M + 31) / 32, splits), 256, 0, stream>>>(A, W, C, M, N, K, ep);
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
    require(rows >= 1 && rows <= kPrefillRows, "prefill chunk: bad row count");
    embed_rows_kernel<<<rows, 256, 0, stream>>>(ids_dev, embed, s.x);
    const float scale = 1.0f / std::sqrt(128.0f);
    // The O and down GEMMs (1024 output columns, K = 2048 / 3072) split K
    // into 1024-wide ranges for parallelism at any row count; the row kernel
    // after each adds the partials to the residual in a fixed order, so a
    // row's result still does not depend on the rows around it.
    constexpr int kOSplits = kQDim / 1024, kDownSplits = kFFN / 1024;
    for (int l = 0; l < kLayers; ++l) {
        const PrefillLayer& L = layers[l];
        if (l == 0)
            rmsnorm_rows_kernel<<<rows, 256, 0, stream>>>(s.x, L.in_norm, s.h, nullptr, rows);
        else
            rmsnorm_rows_kernel<kDownSplits><<<rows, 256, 0, stream>>>(s.x, L.in_norm, s.h, s.part, rows);
        const QkvEpilogue ep{L.q_norm, L.k_norm, cosines, sines, L.keys, L.values, pos0, context};
        gemm<4>(s.h, L.qkv_n, s.qkv, rows, kQKVRows, kHidden, stream, 1, ep);
        attn_prefill_mfma_kernel<<<dim3((rows + kFaRows - 1) / kFaRows, kQHeads), 256, 0, stream>>>(
            s.qkv, L.keys, L.values, s.attended, rows, pos0, context, scale);
        gemm<2>(s.attended, L.o_n, s.part, rows, kHidden, kQDim, stream, kOSplits);
        rmsnorm_rows_kernel<kOSplits><<<rows, 256, 0, stream>>>(s.x, L.post_norm, s.h, s.part, rows);
        gemm<3>(s.h, L.gateup_n, s.act, rows, 2 * kFFN, kHidden, stream);
        gemm<2>(s.act, L.down_n, s.part, rows, kHidden, kFFN, stream, kDownSplits);
    }
    fold_rows_kernel<kDownSplits><<<(rows * kHidden + 255) / 256, 256, 0, stream>>>(s.x, s.part, rows);
}

}  // namespace qwen_hip
