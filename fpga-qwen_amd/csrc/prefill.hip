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
#include <mutex>
#include <type_traits>

#include "half_split.hpp"
#include "kernels.hpp"
#include "prefill.hpp"

namespace qwen_hip {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return to_half_bits(f); }

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// C[M x N] (+)= A[M x K] . W[N x K]^T on the matrix cores
// (v_mfma_f32_32x32x16_f16). A arrives as two FP16 planes written by the
// kernel that produced it, hi = fp16(a) and lo = fp16(a - hi) (a - hi is
// exact in FP32), W as its FP16 values; every product runs twice (hi, lo), so
// products are exact and sums FP32. Workgroup tile BM x 128 (BM = 128, 64 or
// 32), K in steps of 64 through a ring of LDS stages filled by direct global
// -> LDS loads (global_load_lds_dwordx4) one or two steps ahead of the matrix
// cores, one barrier per step. A wave retires roughly one 1 KiB load
// instruction per 240 cycles on this chip, so the loads are spread over 16
// (BM = 128) or 8 waves per workgroup; 4 (BM = 64: 8) of them also run the
// MFMAs, each on 64x64 (BM = 128) or 32x32 tiles of C. Epilogues stage C in LDS and write 16 bytes per
// lane. Each output element accumulates its K terms in the same order
// whatever BM and its row position, so results do not depend on M or on how
// rows are grouped.
constexpr int kTileN = 128, kTileK = 64;

// BN = 192 or 256 (only with BM = 128): 1.5x or 2x the columns per
// workgroup, so every A byte streamed feeds more MFMA work; 8 MFMA waves, two
// per SIMD, on 32x96 (BN = 192) or 64x64 tiles (6 waves of 64x64 put two
// SIMDs' worth of MFMAs on two of the four), and 2 stages of 56 or 64 KiB
// (the LDS holds no third). At
// BN = 192 a stage is 56 loads of 1 KiB, so half of the 16 waves issue 4 and
// half 3 (with two stages every wait is for all of a wave's loads).
template <int BM, int BN = kTileN>
struct GemmShape {
    static_assert(BN == kTileN || ((BN == 192 || BN == 256) && BM == 128), "wide tiles with 128 rows only");
    static constexpr int kWaves = BM == 128 ? 16 : 8;            // waves per workgroup (all load)
    static constexpr int kMma = BM == 64 || BN == 192 || BN == 256 ? 8 : 4;  // waves running the MFMAs
    static constexpr int TI = BM == 128 && BN != 192 ? 2 : 1;    // 32-row tiles per MFMA wave
    static constexpr int WR = BM / 32 / TI, WC = kMma / WR;      // MFMA wave grid
    static constexpr int TJ = BN / WC / 32;                      // 32-column tiles per MFMA wave
    static constexpr int kASlots = BM * 8, kBSlots = BN * 8;     // 16-byte slots per stage
    static constexpr int kStageBytes = (2 * kASlots + kBSlots) * 16;
    static constexpr int kStageLoads = (2 * kASlots + kBSlots) / 64;         // 1 KiB loads per stage
    static constexpr int kLoads = (kStageLoads + kWaves - 1) / kWaves;       // per thread per stage (at most)
    static constexpr int kStages = BN == kTileN ? (BM == 128 ? 3 : 4) : 2;
    static_assert(kStageLoads * 64 == 2 * kASlots + kBSlots && WR * WC == kMma && TJ * WC * 32 == BN,
                  "tile shape");
    static_assert(kLoads * kWaves == kStageLoads || kStages == 2, "uneven loads need whole-stage waits");
};

// LDS operand tiles hold rows of 64 halves (eight 16-byte pieces): piece p of
// row r sits in 16-byte slot 8 r + (p ^ swz(r)), so the 8 (or 16) lanes
// served in one LDS cycle read distinct banks.
__device__ __forceinline__ int swz(int r) { return ((r >> 1) ^ ((r & 1) << 2)) & 7; }

// Work fused into the epilogue. QKV (EPI 4): QK-norm, RoPE and the K/V cache
// writes of engine/core.cpp:395-406. Gate/up (EPI 3): SwiGLU, written as the
// FP16 hi / lo planes the down GEMM reads.
//
// Range guard of the FP16 split (split_exponent): A row m that its producer
// split as a * 2^-row_exp[m] has its products scaled back by 2^row_exp[m]
// (EPI 0, 1, 3, 4; row_exp null: no row was scaled). The SwiGLU epilogue
// splits each group of 8 activations with its own exponent, stored in
// act_exp [M][N / 16], and raises act_flag [M][4] (one word per K range of
// the down GEMM, cleared by the kernel before the gate/up GEMM) to the
// largest exponent in the range. The down GEMM (EPI 2 with act_flag) runs
// its plain K loop, and a workgroup whose rows saw a nonzero flag runs the
// loop again with every group rescaled in LDS to its row's flag exponent
// and the products scaled back: a row that fits keeps its bits.
struct GemmEpilogue {
    const float* q_norm;
    const float* k_norm;
    const float* cosines;
    const float* sines;
    uint16_t* keys;
    uint16_t* values;
    int pos0;
    int context;
    uint16_t* act_hi;
    uint16_t* act_lo;
    const int* row_exp;
    int* act_flag;
    uint8_t* act_exp;
};

// Exponent of row m in row_exp (0 without one).
__device__ __forceinline__ float row_scale(const int* row_exp, int m) {
    return row_exp ? pow2(row_exp[m]) : 1.f;
}

// FP32 value -> the FP16 hi / lo pair the GEMMs read (hi = fp16(v), lo = fp16(v - hi)).
__device__ __forceinline__ void split_store(float v, uint16_t* hi, uint16_t* lo, size_t i) {
    _Float16 h, l;
    split_half(v, h, l);
    hi[i] = __builtin_bit_cast(uint16_t, h);
    lo[i] = __builtin_bit_cast(uint16_t, l);
}

// 16 bytes per lane from global memory straight into LDS at
// lds + 16 lane (lds wave-uniform); counted by vmcnt like any load.
__device__ __forceinline__ void load_lds16(const void* src, unsigned char* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
#endif
}

// vmcnt <= n (expcnt and lgkmcnt unconstrained).
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

// lgkmcnt == 0 (this wave's LDS accesses have completed).
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }

// Workgroup barrier without a memory fence: the waits before it already
// cover the direct-to-LDS loads (a fenced barrier would wait for every load
// in flight, including the later stages). The empty asm statements keep the
// compiler from moving LDS accesses across it.
__device__ __forceinline__ void stage_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Epilogue: 0 store, 1 add into C (residual), 2 store the partial product
// of K range blockIdx.z (K / gridDim.z columns) at C + blockIdx.z M N,
// 3 SwiGLU (W = gate rows then up rows, N = 2F: tile t multiplies gate rows
// 64t.. and up rows F + 64t.. and stores act[m][64t + i] as FP16 hi / lo),
// 4 QKV rows (tile t = head t): q heads QK-normed, rotated and stored in the
// key's chain-permuted order, k heads QK-normed, rotated and written to the
// cache as FP16, v heads written to the cache.
template <int BM, int EPI, int BN = kTileN>
__global__ __launch_bounds__((GemmShape<BM, BN>::kWaves * 64)) void gemm_kernel(
    const uint16_t* __restrict__ Ah, const uint16_t* __restrict__ Al, const uint16_t* __restrict__ W,
    float* __restrict__ C, int M, int N, int K, GemmEpilogue ep) {
    using S = GemmShape<BM, BN>;
    static_assert(EPI != 4 || BN == kTileN, "the QKV epilogue takes one head per tile");
    constexpr int kStages = S::kStages, kLoads = S::kLoads, kStageBytes = S::kStageBytes;
    constexpr int kASlots = S::kASlots, WR = S::WR, TI = S::TI, TJ = S::TJ;
    // Overlapped operand reads (below) for 2 x 2 MFMA tiles per wave; the
    // K-split 192-column instance keeps the plain order (8 more registers
    // would spill there).
    constexpr bool kPipelined = TI == 2 && TJ == 2 && !(EPI == 2 && BN == 192);
    constexpr int kThreads = S::kWaves * 64;
    constexpr int kCPitch = BN + 4;  // floats per row of the staged C tile
    constexpr int kEpiBytes = BM * kCPitch * 4 + (EPI == 4 ? BM * kHeadDim * 2 : 0);
    constexpr int kSmem = kStages * kStageBytes > kEpiBytes ? kStages * kStageBytes : kEpiBytes;
    __shared__ __align__(16) unsigned char smem[kSmem];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Tile of this workgroup: workgroup w runs on XCD w % 8 (round-robin
    // dispatch). With 4 or more row tiles per XCD, XCD x takes row tiles
    // x, x + 8, ... and walks the column tiles (its 32 CUs hold 4 row tiles
    // x 8 column tiles at a time). With fewer (prompts up to 3 x 8 x BM
    // rows), f = 4 or 2 XCDs pool their row tiles and split the column tiles
    // by residue mod f, so that the tiles an XCD runs at once still share
    // A and W rows in its L2: at 1024 rows 4 x 8 tiles per XCD instead of
    // 1 x 32 (each W tile fetched by 2 XCDs instead of 8). The grid is
    // rounded up to whole XCD rows; the extra workgroups have no tile.
    const int mtiles = (M + BM - 1) / BM, per = (mtiles + 7) / 8, ntiles = N / BN;
    const int f = per >= 4 ? 1 : per == 1 && ntiles % 4 == 0 ? 4 : ntiles % 2 == 0 ? 2 : 1;
    const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8, rows = f * per;
    const int rr = slot % rows, cc = slot / rows;
    const int mt = (xcd / f) * f + rr % f + 8 * (rr / f), nt = xcd % f + f * cc;
    if (mt >= mtiles) return;
    const int m0 = mt * BM, n0 = nt * BN;
    const bool mma = wave < S::kMma;
    const int wm = wave % WR, wn = wave / WR;
    const int ks = K / gridDim.z, kz = blockIdx.z * ks, nk = ks / kTileK;  // this workgroup's K range

    // Load j of this thread fills slot 64 (wave + kWaves j) + lane of a
    // stage: a wave-uniform operand plane (A hi, A lo, W) and one 16-byte
    // piece of a row. A rows past M repeat row M - 1 and are never stored.
    const uint16_t* src[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int q = 64 * (wave + S::kWaves * j) + lane;
        if (q < 2 * kASlots) {
            const int qa = q < kASlots ? q : q - kASlots, r = qa >> 3, p = (qa & 7) ^ swz(r);
            src[j] = (q < kASlots ? Ah : Al) + size_t(min(m0 + r, M - 1)) * K + kz + 8 * p;
        } else {
            const int qb = q - 2 * kASlots, r = qb >> 3, p = (qb & 7) ^ swz(r);
            const int wr = EPI == 3 ? (r < BN / 2 ? n0 / 2 + r : N / 2 + n0 / 2 + r - BN / 2) : n0 + r;
            src[j] = W + size_t(wr) * K + kz + 8 * p;
        }
    }
    auto issue = [&](int kt) {
        unsigned char* stage = smem + (kt % kStages) * kStageBytes;
#pragma unroll
        for (int j = 0; j < kLoads; ++j)
            if (kLoads * S::kWaves == S::kStageLoads || wave + S::kWaves * j < S::kStageLoads)
                load_lds16(src[j] + kt * kTileK, stage + 1024 * (wave + S::kWaves * j));
    };

    // Range guard of the down GEMM (EPI 2 with act_flag): the flags of this
    // workgroup's rows in its K range (lane l: rows m0 + l and m0 + 64 + l),
    // loaded before the stream so that they have arrived when the loop ends.
    int flag0 = 0, flag1 = 0;
    if constexpr (EPI == 2) {
        if (ep.act_flag != nullptr && lane < BM) {
            flag0 = ep.act_flag[size_t(min(m0 + lane, M - 1)) * 4 + blockIdx.z];
            if (BM > 64) flag1 = ep.act_flag[size_t(min(m0 + 64 + lane, M - 1)) * 4 + blockIdx.z];
        }
    }

    floatx16 acc[TI][TJ];
    const int fr = lane & 31;
    // Rescales the A groups of stage kt in LDS to their row's flag
    // exponent (the second pass of a guarded down GEMM): exact, being
    // multiplications of FP16 values by powers of two no greater than 1.
    auto rescale_stage = [&](int kt) {
        unsigned char* stage = smem + (kt % kStages) * kStageBytes;
        for (int q = tid; q < kASlots; q += kThreads) {
            const int r = q >> 3, p = (q & 7) ^ swz(r), m = min(m0 + r, M - 1);
            const int er = ep.act_flag[size_t(m) * 4 + blockIdx.z];
            if (er != 0) {
                const int e8 = ep.act_exp[size_t(m) * (K / 8) + (kz + kt * kTileK) / 8 + p];
                const float sc = pow2(e8 - er);
                half8* h = reinterpret_cast<half8*>(stage + 16 * q);
                half8* l = reinterpret_cast<half8*>(stage + 16 * (kASlots + q));
                half8 hv = *h, lv = *l;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    hv[e] = static_cast<_Float16>(static_cast<float>(hv[e]) * sc);
                    lv[e] = static_cast<_Float16>(static_cast<float>(lv[e]) * sc);
                }
                *h = hv;
                *l = lv;
            }
        }
    };
    auto k_loop = [&](auto rescale_tag) {
        constexpr bool kRescale = decltype(rescale_tag)::value;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int jt = 0; jt < TJ; ++jt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][jt][r] = 0.f;
#pragma unroll
        for (int s = 0; s < kStages - 1; ++s)
            if (s < nk) issue(s);
        for (int kt = 0; kt < nk; ++kt) {
            // Step kt has landed once no more than the later steps' loads are
            // pending; the barrier then also tells every wave that all waves are
            // done reading the stage the next issue overwrites.
            if (kt + kStages - 2 < nk)
                wait_vmcnt<(kStages - 2) * kLoads>();
            else
                wait_vmcnt<0>();
            stage_barrier();
            if (kt + kStages - 1 < nk) issue(kt + kStages - 1);
            if constexpr (kRescale) {
                rescale_stage(kt);
                wait_lgkm0();
                stage_barrier();
            }
            if (mma) {
                if constexpr (kPipelined) {
                    // Operand reads of sub-step sub + 1 overlap the MFMAs of sub:
                    // the B pair and row tile 0 of sub + 1 are read while row tile
                    // 1 of sub multiplies, row tile 1 of sub + 1 while row tile 0
                    // of sub + 1 does. Each accumulator still takes hi then lo of
                    // sub 0, 1, 2, 3 in turn.
                    const unsigned char* stage = smem + (kt % kStages) * kStageBytes;
                    auto read_a = [&](int sub, int i, half8& h, half8& l) {
                        const int p = 2 * sub + (lane >> 5);
                        const int ra = (wm * TI + i) * 32 + fr, sa = 8 * ra + (p ^ swz(ra));
                        h = *reinterpret_cast<const half8*>(stage + 16 * sa);
                        l = *reinterpret_cast<const half8*>(stage + 16 * (kASlots + sa));
                    };
                    auto read_b = [&](int sub, half8 (&b)[TJ]) {
                        const int p = 2 * sub + (lane >> 5);
#pragma unroll
                        for (int jt = 0; jt < TJ; ++jt) {
                            const int rb = wn * (BN / S::WC) + 32 * jt + fr;
                            b[jt] = *reinterpret_cast<const half8*>(stage + 16 * (2 * kASlots + 8 * rb + (p ^ swz(rb))));
                        }
                    };
                    half8 a0h, a0l, a1h, a1l, bb[2][TJ];
                    read_a(0, 0, a0h, a0l);
                    read_b(0, bb[0]);
                    read_a(0, 1, a1h, a1l);
#pragma unroll
                    for (int sub = 0; sub < 4; ++sub) {
                        half8(&cur)[TJ] = bb[sub & 1];
#pragma unroll
                        for (int jt = 0; jt < TJ; ++jt)
                            acc[0][jt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0h, cur[jt], acc[0][jt], 0, 0, 0);
#pragma unroll
                        for (int jt = 0; jt < TJ; ++jt)
                            acc[0][jt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0l, cur[jt], acc[0][jt], 0, 0, 0);
                        __builtin_amdgcn_sched_barrier(0);
                        if (sub < 3) {
                            read_b(sub + 1, bb[(sub + 1) & 1]);
                            read_a(sub + 1, 0, a0h, a0l);
                        }
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int jt = 0; jt < TJ; ++jt)
                            acc[1][jt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1h, cur[jt], acc[1][jt], 0, 0, 0);
#pragma unroll
                        for (int jt = 0; jt < TJ; ++jt)
                            acc[1][jt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1l, cur[jt], acc[1][jt], 0, 0, 0);
                        __builtin_amdgcn_sched_barrier(0);
                        if (sub < 3) read_a(sub + 1, 1, a1h, a1l);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                } else {
                    const unsigned char* stage = smem + (kt % kStages) * kStageBytes;
#pragma unroll
                    for (int sub = 0; sub < 4; ++sub) {
                        const int p = 2 * sub + (lane >> 5);  // k = 16 sub + 8 (lane / 32) .. + 7 of the step
                        half8 ah[TI], al[TI], bb[TJ];
#pragma unroll
                        for (int i = 0; i < TI; ++i) {
                            const int ra = (wm * TI + i) * 32 + fr, sa = 8 * ra + (p ^ swz(ra));
                            ah[i] = *reinterpret_cast<const half8*>(stage + 16 * sa);
                            al[i] = *reinterpret_cast<const half8*>(stage + 16 * (kASlots + sa));
                        }
#pragma unroll
                        for (int jt = 0; jt < TJ; ++jt) {
                            const int rb = wn * (BN / S::WC) + 32 * jt + fr;
                            bb[jt] = *reinterpret_cast<const half8*>(stage + 16 * (2 * kASlots + 8 * rb + (p ^ swz(rb))));
                        }
#pragma unroll
                        for (int i = 0; i < TI; ++i)
#pragma unroll
                            for (int jt = 0; jt < TJ; ++jt) {
                                acc[i][jt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bb[jt], acc[i][jt], 0, 0, 0);
                                acc[i][jt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bb[jt], acc[i][jt], 0, 0, 0);
                            }
                    }
                }
            }
        }
    };
    k_loop(std::false_type{});
    // Every wave read the same flags, so every wave takes the same branch.
    bool rescaled = false;
    if constexpr (EPI == 2) {
        if (ep.act_flag != nullptr && __builtin_amdgcn_ballot_w64(flag0 != 0 || flag1 != 0) != 0) {
            rescaled = true;
            stage_barrier();  // every wave is done with the stages (all loads were waited for)
            k_loop(std::true_type{});
        }
    }

    // Stage C in LDS. D layout: lane -> column (lane & 31); register r ->
    // row 8(r/4) + 4(lane/32) + r%4 of the wave's 32-row tile.
    float(*ct)[kCPitch] = reinterpret_cast<float(*)[kCPitch]>(smem);
    stage_barrier();  // every wave is done with the operand stages (all loads were waited for)
    if (mma) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int jt = 0; jt < TJ; ++jt)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    ct[(wm * TI + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)]
                      [wn * (BN / S::WC) + 32 * jt + fr] = acc[i][jt][r];
    }
    __syncthreads();
    if constexpr (EPI <= 2) {
        // 16-byte pieces: row q / (BN / 4), columns 4 (q % (BN / 4)) .. + 3.
#pragma unroll
        for (int q = tid; q < BM * (BN / 4); q += kThreads) {
            const int row = q / (BN / 4), c4 = q % (BN / 4), m = m0 + row;
            if (m < M) {
                float4* c = reinterpret_cast<float4*>(C + (size_t(blockIdx.z) * M + m) * N + n0) + c4;
                float4 v = *reinterpret_cast<const float4*>(&ct[row][4 * c4]);
                float sc = 1.f;
                if constexpr (EPI == 2) {
                    if (rescaled) sc = pow2(ep.act_flag[size_t(m) * 4 + blockIdx.z]);
                } else {
                    sc = row_scale(ep.row_exp, m);
                }
                v = make_float4(v.x * sc, v.y * sc, v.z * sc, v.w * sc);
                if constexpr (EPI == 1) {
                    const float4 o = *c;
                    *c = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
                } else {
                    *c = v;
                }
            }
        }
    } else if constexpr (EPI == 3) {
        // SwiGLU (engine/core.cpp:636-639): task q = row q / (BN / 16), act
        // columns n0 / 2 + 8 (q % (BN / 16)) .. + 7, stored as one 16-byte
        // piece per plane (gate in tile columns 0 .. BN / 2 - 1, up after).
#pragma unroll
        for (int q = tid; q < BM * (BN / 16); q += kThreads) {
            const int row = q / (BN / 16), c8 = 8 * (q % (BN / 16)), m = m0 + row;
            if (m < M) {
                const float sc = row_scale(ep.row_exp, m);
                float o[8], big = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float gate = ct[row][c8 + e] * sc, up = ct[row][BN / 2 + c8 + e] * sc;
                    const float half_gate = gate * 0.5f;
                    const float t = tanhf(half_gate);
                    o[e] = gate * (0.5f + 0.5f * t) * up;
                    big = fmaxf(big, fabsf(o[e]));
                }
                // This group's exponent; the K range's flag holds the largest.
                const int e8 = split_exponent(big), col = n0 / 2 + c8;
                const float down = pow2(-e8);
                half8 hi, lo;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    _Float16 h, l;
                    split_half(o[e] * down, h, l);
                    hi[e] = h;
                    lo[e] = l;
                }
                const size_t at = size_t(m) * (N / 2) + col;
                *reinterpret_cast<half8*>(ep.act_hi + at) = hi;
                *reinterpret_cast<half8*>(ep.act_lo + at) = lo;
                ep.act_exp[size_t(m) * (N / 16) + col / 8] = static_cast<uint8_t>(e8);
                if (e8 != 0) atomicMax(ep.act_flag + size_t(m) * 4 + col / (N / 8), e8);
            }
        }
    } else {
        // Per row (one wave per row, rows wave, wave + kWaves, ...; lane l on
        // channels l and l + 64): QK-norm and RoPE in place, the row left in
        // LDS in its stored order (q: FP32 chain-permuted; k: FP16
        // chain-permuted; v: FP16), then written out 16 bytes per lane.
        uint16_t(*ht)[kHeadDim] = reinterpret_cast<uint16_t(*)[kHeadDim]>(smem + BM * kCPitch * 4);
        const int head = nt, j = lane;
        const bool is_q = head < kQHeads, is_v = head >= kQHeads + kKVHeads;
        constexpr int kRows = BM / S::kWaves;
        if (is_v) {
#pragma unroll
            for (int k = 0; k < kRows; ++k) {
                const int rr = wave + S::kWaves * k;
                const float sc = row_scale(ep.row_exp, min(m0 + rr, M - 1));
                ht[rr][j] = f2h(ct[rr][j] * sc);
                ht[rr][j + 64] = f2h(ct[rr][j + 64] * sc);
            }
        } else {
            const float* w = is_q ? ep.q_norm : ep.k_norm;
            const float w0 = w[j], w1 = w[j + 64];
            float rc[kRows], rs[kRows];
#pragma unroll
            for (int k = 0; k < kRows; ++k) {
                const int pos = ep.pos0 + min(m0 + wave + S::kWaves * k, M - 1);
                rc[k] = ep.cosines[size_t(pos) * 64 + j];
                rs[k] = ep.sines[size_t(pos) * 64 + j];
            }
#pragma unroll
            for (int k = 0; k < kRows; ++k) {
                const int rr = wave + S::kWaves * k;
                const float sc = row_scale(ep.row_exp, min(m0 + rr, M - 1));
                const float x0 = ct[rr][j] * sc, x1 = ct[rr][j + 64] * sc;
                const float s0 = x0 * x0, s1 = x1 * x1;
                double part = static_cast<double>(s0) + static_cast<double>(s1);
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
                const float inv = 1.0f / __builtin_sqrtf(static_cast<float>(part) / 128.0f + 1e-6f);
                const float n0v = (x0 * inv) * w0, n1v = (x1 * inv) * w1;
                const float o0 = n0v * rc[k] - n1v * rs[k];
                const float o1 = n1v * rc[k] + n0v * rs[k];
                if (is_q) {
                    ct[rr][kperm(j)] = o0;  // the row's reads above came first
                    ct[rr][kperm(j + 64)] = o1;
                } else {
                    ht[rr][kperm(j)] = f2h(o0);
                    ht[rr][kperm(j + 64)] = f2h(o1);
                }
            }
        }
        __syncthreads();
        if (is_q) {
#pragma unroll
            for (int q = tid; q < BM * 32; q += kThreads) {
                const int row = q >> 5, c4 = q & 31, m = m0 + row;
                if (m < M)
                    reinterpret_cast<float4*>(C + size_t(m) * N + head * kHeadDim)[c4] =
                        *reinterpret_cast<const float4*>(&ct[row][4 * c4]);
            }
        } else {
            uint16_t* cache = (is_v ? ep.values + size_t(head - kQHeads - kKVHeads) * ep.context * kHeadDim
                                    : ep.keys + size_t(head - kQHeads) * ep.context * kHeadDim);
#pragma unroll
            for (int q = tid; q < BM * 16; q += kThreads) {
                const int row = q >> 4, c8 = q & 15, m = m0 + row;
                if (m < M)
                    reinterpret_cast<u32x4*>(cache + size_t(ep.pos0 + m) * kHeadDim)[c8] =
                        *reinterpret_cast<const u32x4*>(&ht[row][8 * c8]);
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
    static_assert(SPLITS == 0 || SPLITS == 4, "K-split GEMMs use 4 ranges");
    if constexpr (SPLITS == 0) return x;
    else return x + ((p[0] + p[stride]) + (p[2 * stride] + p[3 * stride]));
}


// out[b] = RMSNorm(x[b]) (engine/core.cpp:207-215): FP32 squares, FP64 sum,
// written as the FP16 hi / lo planes of the next GEMM's A operand, split as
// out * 2^-row_exp[b] (split_exponent of the row's largest magnitude; 0
// wherever the row fits FP16). With SPLITS > 0 the residual first absorbs the
// pending partial products of a K-split GEMM (parts[z][b], z < SPLITS) and is
// written back. clear_flags (optional) zeroes the row's 4 SwiGLU range flags
// ahead of the gate/up GEMM.
template <int SPLITS = 0>
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(float* __restrict__ X, const float* __restrict__ w,
                                                           uint16_t* __restrict__ out_hi,
                                                           uint16_t* __restrict__ out_lo,
                                                           const float* __restrict__ parts, int rows,
                                                           int* __restrict__ row_exp, int* __restrict__ clear_flags) {
    const int b = blockIdx.x, tid = threadIdx.x;
    // Thread t holds columns 4t .. 4t + 3 (16-byte accesses).
    float4* xr = reinterpret_cast<float4*>(X + size_t(b) * kHidden) + tid;
    float4 v4 = *xr;
    if constexpr (SPLITS > 0) {
        const size_t stride = size_t(rows) * kHidden / 4;
        const float4* pr = reinterpret_cast<const float4*>(parts + size_t(b) * kHidden) + tid;
        const float4 p0 = pr[0], p1 = pr[stride], p2 = pr[2 * stride], p3 = pr[3 * stride];
        v4.x = v4.x + ((p0.x + p1.x) + (p2.x + p3.x));
        v4.y = v4.y + ((p0.y + p1.y) + (p2.y + p3.y));
        v4.z = v4.z + ((p0.z + p1.z) + (p2.z + p3.z));
        v4.w = v4.w + ((p0.w + p1.w) + (p2.w + p3.w));
        *xr = v4;
    }
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    double part = 0.0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float square = v[k] * v[k];
        part += static_cast<double>(square);
    }
    part = wave_sum(part);
    __shared__ double red[4];
    if ((tid & 63) == 0) red[tid >> 6] = part;
    __syncthreads();
    const float sum = static_cast<float>((red[0] + red[1]) + (red[2] + red[3]));
    const float inv = 1.0f / __builtin_sqrtf(sum / 1024.0f + 1e-6f);
    const float4 w4 = reinterpret_cast<const float4*>(w)[tid];
    const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
    float n[4], big = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        n[k] = (v[k] * inv) * wv[k];
        big = fmaxf(big, fabsf(n[k]));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) big = fmaxf(big, __shfl_xor(big, off));
    __shared__ float bred[4];
    if ((tid & 63) == 0) bred[tid >> 6] = big;
    __syncthreads();
    const int e = split_exponent(fmaxf(fmaxf(bred[0], bred[1]), fmaxf(bred[2], bred[3])));
    const float down = pow2(-e);
    if (tid == 0) row_exp[b] = e;
    if (clear_flags != nullptr && tid < 4) clear_flags[size_t(b) * 4 + tid] = 0;
    uint16_t hi[4], lo[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        _Float16 h, l;
        split_half(n[k] * down, h, l);
        hi[k] = __builtin_bit_cast(uint16_t, h);
        lo[k] = __builtin_bit_cast(uint16_t, l);
    }
    const size_t at = size_t(b) * kHidden + 4 * tid;
    *reinterpret_cast<uint2*>(out_hi + at) = make_uint2(hi[0] | (unsigned(hi[1]) << 16), hi[2] | (unsigned(hi[3]) << 16));
    *reinterpret_cast<uint2*>(out_lo + at) = make_uint2(lo[0] | (unsigned(lo[1]) << 16), lo[2] | (unsigned(lo[3]) << 16));
}

// Causal attention for a prefill chunk on the matrix cores (engine/core.cpp:
// 407-605, same math as the decode path):
//   S^T = K Q^T  (A = 32 keys x 16 dims, B = Q^T as FP16 hi + lo of the FP32
//                 q, so products are exact)
//   O^T += V^T P^T (A = V^T, B = P^T as FP16 hi + lo of the FP32
//                 probabilities)
// With S^T in the 32x32 accumulator layout each lane holds 16 keys of one
// query (lane % 32), so the softmax statistics stay in the lane: one
// exchange with lane ^ 32 per tile. q and the cached keys share the
// chain-permuted channel order, which leaves q . k unchanged.
constexpr int kFaRows = 32, kFaKeys = 32, kFaccPitch = 132;
// A query keeps the reference maximum of its online softmax until a score
// exceeds it by more than this (log2 units), so probabilities stay <= 2^8 and
// most tiles need no rescaling of the output accumulators.
constexpr float kFaLazyMax = 8.f;

// Workgroup = 32 consecutive query rows x one KV head g, 8 waves: wave
// (h, s) = (wave & 1, wave >> 1) runs query head 2g + h over the key tiles
// kt = s (mod 4) with its own online softmax, and the 4 key splits of each
// head are merged at the end. The two waves of a split use the same tiles:
// they load each K/V tile together (direct global -> LDS loads, 8 KiB each)
// into a double-buffered LDS ring, one tile ahead of the matrix cores, so a
// wave streams half a tile per step instead of a whole one (a wave retires
// only about 10 GB/s of loads). K is read from LDS as the S^T operand and V^T
// with the LDS transpose load (ds_read_b64_tr_b16), so V needs no transpose
// pass through registers.
constexpr int kFbTileBytes = kFaKeys * kHeadDim * 2;        // one K or V tile (8 KiB)
constexpr int kFbSplitBytes = 2 * kFbTileBytes;             // K then V of one split
constexpr int kFbStageBytes = 4 * kFbSplitBytes;            // the 4 splits' tiles of one step
constexpr int kFbMergeBytes = 8 * kFaRows * kFaccPitch * 4; // 8 waves' outputs
constexpr int kFbLds = 2 * kFbStageBytes > kFbMergeBytes ? 2 * kFbStageBytes : kFbMergeBytes;
typedef short short4_t __attribute__((ext_vector_type(4)));

// K and V tiles in LDS: rows of 128 halves (sixteen 16-byte pieces), piece p
// of key row r in 16-byte slot 16 r + (p ^ fb_swz(r)). fb_swz is a bijection
// of r % 16, so 16 consecutive rows at one piece (the K operand reads) fill
// 16 distinct slots of a 256-byte bank cycle, and 4 consecutive rows (r % 4
// in bits 2-3) at 4 aligned pieces (bits 0-1) -- what 32 lanes of the V^T
// transpose load touch -- also fill 16 distinct slots.
__device__ __forceinline__ int fb_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
__device__ __forceinline__ int fb_slot(int r, int p) { return 16 * r + (p ^ fb_swz(r)); }

// ds_read_b64_tr_b16 (gfx950): within each 16-lane group, lane 4a + b
// receives element b of the 8-byte chunks addressed by lanes a, a + 4,
// a + 8 and a + 12, in that order.
__device__ __forceinline__ short4_t lds_read_tr16(const unsigned char* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) short4_t*)(const_cast<unsigned char*>(p)));
#else
    (void)p;
    return short4_t{0, 0, 0, 0};
#endif
}

__global__ __launch_bounds__(512) void attn_prefill_mfma_kernel(const float* __restrict__ QKV,
                                                                  const uint16_t* __restrict__ keys,
                                                                  const uint16_t* __restrict__ values,
                                                                  uint16_t* __restrict__ att_hi,
                                                                  uint16_t* __restrict__ att_lo, int rows, int pos0,
                                                                  int context, float scale) {
    __shared__ __align__(16) unsigned char lds[kFbLds];
    __shared__ float fm[8][kFaRows], fl[8][kFaRows];
    // Workgroup w runs on XCD w % 8 (round-robin dispatch): KV head g = w % 8
    // keeps every workgroup reading one head's K/V rows on one XCD, so they
    // stay in its L2; the query blocks run heaviest (latest) first.
    const int nqb = gridDim.x / kKVHeads;
    const int g = blockIdx.x % kKVHeads, qb = nqb - 1 - blockIdx.x / kKVHeads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = wave & 1, sp = wave >> 1, head = 2 * g + h;
    const int col = lane & 31, hf = lane >> 5;
    const int b0 = qb * kFaRows, nrows = min(kFaRows, rows - b0);
    const int last = pos0 + b0 + nrows - 1;  // last key any query of the block attends to
    const int ntiles = last / kFaKeys + 1;
    const int nsteps = (ntiles + 3) / 4;     // steps of 4 tiles (one per split)
    const size_t head_base = size_t(g) * context;
    const int qpos = pos0 + b0 + col;        // causal limit of this lane's query
    const float scale2 = scale * 1.4426950408889634f;

    // Direct loads of step i: split sp's tile kt = 4 i + sp; load j of this
    // wave fills 16-byte slot 64 (2 j + h) + lane of the split's K tile
    // (j < 4) or V tile; rows past `last` repeat row `last` (masked).
    int ld_row[8], ld_col[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q = (64 * (2 * j + h) + lane) & 511, r = q >> 4;
        ld_row[j] = r;
        ld_col[j] = 8 * ((q & 15) ^ fb_swz(r));
    }
    auto issue = [&](int step) {
        const int kt = 4 * step + sp;
        unsigned char* dst = lds + (step & 1) * kFbStageBytes + sp * kFbSplitBytes;
        if (kt < ntiles) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int key = min(kt * kFaKeys + ld_row[j], last);
                const uint16_t* src = (j < 4 ? keys : values) + (head_base + key) * kHeadDim + ld_col[j];
                load_lds16(src, dst + 1024 * (2 * j + h));
            }
        }
    };
    issue(0);

    // Q^T operand: query b0 + col (rows past the chunk repeat its last row
    // and are never written), channels 16s + 8hf .. +7, scaled by
    // scale * log2(e) so that the scores come out in the exp2 domain.
    // A query row whose largest magnitude reaches 65504 is split as
    // q * 2^-eq (split_exponent) and its scores scaled back by 2^eq.
    half8 qh[8], ql[8];
    int eq;
    {
        const float* qrow = QKV + size_t(b0 + min(col, nrows - 1)) * kQKVRows + head * kHeadDim + 8 * hf;
        float v[8][8], big = 0.f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const float4 x0 = reinterpret_cast<const float4*>(qrow + 16 * s)[0];
            const float4 x1 = reinterpret_cast<const float4*>(qrow + 16 * s)[1];
            const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[s][i] = x[i] * scale2;
                big = fmaxf(big, fabsf(v[s][i]));
            }
        }
        eq = split_exponent(fmaxf(big, __shfl_xor(big, 32)));
        const float down = pow2(-eq);
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                _Float16 hh, ll;
                split_half(v[s][i] * down, hh, ll);
                qh[s][i] = hh;
                ql[s][i] = ll;
            }
    }
    const bool q_scaled = __builtin_amdgcn_ballot_w64(eq != 0) != 0;
    const float q_up = pow2(eq);
    float m = -INFINITY, l = 0.f;
    floatx16 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;

    // Transpose-load addresses in a V tile: lane j of 16-lane group G hands
    // over key row 8 hh + 4 (G / 2) + jj / 4 (+ 16 per key step), channels
    // 32 dt + 16 (G % 2) + 4 (jj % 4) (jj = j % 16).
    const int grp = lane >> 4, jj = lane & 15;
    const int tr_row = 4 * (grp >> 1) + (jj >> 2), tr_ch = 16 * (grp & 1) + 4 * (jj & 3);
    for (int step = 0; step < nsteps; ++step) {
        wait_vmcnt<0>();       // this wave's loads of the step have landed
        stage_barrier();       // everyone's have; the other buffer is free again
        if (step + 1 < nsteps) issue(step + 1);
        const int kt = 4 * step + sp, t0 = kt * kFaKeys;
        if (kt >= ntiles) continue;  // wave-uniform: this split has no tile in the last step
        const unsigned char* k_lds = lds + (step & 1) * kFbStageBytes + sp * kFbSplitBytes;
        const unsigned char* v_lds = k_lds + kFbTileBytes;
        floatx16 st;
#pragma unroll
        for (int r = 0; r < 16; ++r) st[r] = 0.f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const half8 ka = *reinterpret_cast<const half8*>(k_lds + 16 * fb_slot(col, 2 * s + hf));
            st = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qh[s], st, 0, 0, 0);
            st = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, ql[s], st, 0, 0, 0);
        }
        if (q_scaled) {
#pragma unroll
            for (int r = 0; r < 16; ++r) st[r] *= q_up;
        }
        // Online softmax; register r holds key t0 + 8(r/4) + 4hf + r%4. A
        // tile entirely at or before the block's first query needs no causal
        // mask (and its maximum is finite), which saves the per-key compares
        // and selects on all but the diagonal tiles.
        float sv[16], mnew, factor, psum = 0.f;
        bool grow;
        half8 ph[2], pl[2];
        auto softmax = [&](auto masked) {
            constexpr bool kMask = decltype(masked)::value;
            float tmax = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = t0 + 8 * (r >> 2) + 4 * hf + (r & 3);
                sv[r] = !kMask || t <= qpos ? st[r] : -INFINITY;
                tmax = fmaxf(tmax, sv[r]);
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            grow = tmax > m + kFaLazyMax;  // per query (both halves agree)
            mnew = grow ? tmax : m;
            factor = !grow ? 1.f : m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mnew);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = kMask && sv[r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sv[r] - mnew);
                psum += p;
                _Float16 hh, ll;
                split_half(p, hh, ll);
                ph[r >> 3][r & 7] = hh;
                pl[r >> 3][r & 7] = ll;
            }
        };
        if (t0 + kFaKeys - 1 <= pos0 + b0)
            softmax(std::false_type{});
        else
            softmax(std::true_type{});
        psum += __shfl_xor(psum, 32);
        l = l * factor + psum;
        // Rescaling by 1 changes nothing; skip it when no lane's reference moved.
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[dt][r] *= factor;
        }
        m = mnew;
        // P^T k slot 8 hf + i of key step j is key 16 j + 8 (i / 4) + 4 hf + i % 4;
        // transpose load hh covers keys 16 j + 8 hh + 4 hf + 0..3 of channel
        // 32 dt + lane % 32, the same order.
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const int c = 32 * dt + tr_ch;
                const int r0 = 16 * j + tr_row, r1 = r0 + 8;
                const short4_t lo4 = lds_read_tr16(v_lds + 16 * fb_slot(r0, c >> 3) + 2 * (c & 7));
                const short4_t hi4 = lds_read_tr16(v_lds + 16 * fb_slot(r1, c >> 3) + 2 * (c & 7));
                const half8 a = __builtin_bit_cast(half8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, ph[j], acc[dt], 0, 0, 0);
                acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pl[j], acc[dt], 0, 0, 0);
            }
    }

    // Merge the 4 splits of each head: O^T register r of tile dt is channel
    // 32dt + 8(r/4) + 4hf + r%4 of query col.
    stage_barrier();  // every wave is done with the K/V stages (all loads were waited for)
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
    // Thread -> head hm = tid / 256, query q, channels c0 .. c0 + 15.
    const int hm = tid >> 8, q = (tid >> 3) & 31, c0 = (tid & 7) * 16;
    if (q < nrows) {
        float mx = fm[hm][q];
#pragma unroll
        for (int s = 1; s < 4; ++s) mx = fmaxf(mx, fm[2 * s + hm][q]);
        float e[4], lsum = 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int w = 2 * s + hm;
            e[s] = fm[w][q] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(fm[w][q] - mx);
            lsum = __builtin_fmaf(e[s], fl[w][q], lsum);
        }
        const size_t out = size_t(b0 + q) * kQDim + (2 * g + hm) * kHeadDim + c0;
        half8 hi[2], lo[2];
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) {
            float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const float4 v = *reinterpret_cast<const float4*>(
                    reinterpret_cast<const float*>(lds + (2 * s + hm) * kFaRows * kFaccPitch * 4) + q * kFaccPitch +
                    c0 + 4 * k4);
                o[0] = __builtin_fmaf(e[s], v.x, o[0]);
                o[1] = __builtin_fmaf(e[s], v.y, o[1]);
                o[2] = __builtin_fmaf(e[s], v.z, o[2]);
                o[3] = __builtin_fmaf(e[s], v.w, o[3]);
            }
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {  // the O GEMM's A operand as FP16 hi / lo
                const float v = o[e4] / lsum;
                _Float16 hh, ll;
                split_half(v, hh, ll);
                hi[k4 >> 1][4 * (k4 & 1) + e4] = hh;
                lo[k4 >> 1][4 * (k4 & 1) + e4] = ll;
            }
        }
        *reinterpret_cast<half8*>(att_hi + out) = hi[0];
        *reinterpret_cast<half8*>(att_hi + out + 8) = hi[1];
        *reinterpret_cast<half8*>(att_lo + out) = lo[0];
        *reinterpret_cast<half8*>(att_lo + out + 8) = lo[1];
    }
}

// X[b] += the SPLITS partial products of a K-split GEMM (rows x 1024).
template <int SPLITS>
__global__ __launch_bounds__(256) void fold_rows_kernel(float* __restrict__ X, const float* __restrict__ parts,
                                                        int rows) {
    const size_t idx = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (idx < size_t(rows) * kHidden) X[idx] = fold_splits<SPLITS>(X[idx], parts + idx, size_t(rows) * kHidden);
}

// The tallest tile (128, 64 or 32 rows) that still gives every CU a
// workgroup; `splits` K ranges (EPI 2) count towards the workgroups.
template <int EPI>
void gemm(const uint16_t* Ah, const uint16_t* Al, const uint16_t* W, float* C, int M, int N, int K,
          hipStream_t stream, int splits = 1, const GemmEpilogue& ep = {}) {
    require(N % kTileN == 0 && K % (kTileK * splits) == 0 && M > 0 && (splits == 1 || EPI == 2),
            "gemm: unsupported shape");
    const int tiles = N / kTileN * splits;
    auto launch = [&](auto bm, auto bn) {
        constexpr int BM = decltype(bm)::value, BN = decltype(bn)::value;
        const int per = ((M + BM - 1) / BM + 7) / 8;  // row tiles per XCD
        gemm_kernel<BM, EPI, BN><<<dim3(8 * per * (N / BN), 1, splits), GemmShape<BM, BN>::kWaves * 64, 0, stream>>>(
            Ah, Al, W, C, M, N, K, ep);
    };
    using I128 = std::integral_constant<int, 128>;
        // 128-row tiles of 128, 192 or 256 columns (the QKV epilogue takes one
    // head per tile): the fewest rounds of 256 workgroups, each round priced
    // at the measured time of one workgroup of that width relative to 128.
    if constexpr (EPI != 4) {
        const int mtiles = (M + 127) / 128;
        auto cost = [&](int bn, double per_round) {
            const long groups = long(mtiles) * (N / bn) * splits;
            return (groups + 255) / 256 * per_round;
        };
        if (mtiles * tiles >= 256) {
            const double c128 = cost(128, 1.0);
            const double c192 = N % 192 == 0 ? cost(192, 1.45) : 1e30;
            const double c256 = N % 256 == 0 ? cost(256, 1.91) : 1e30;
            if (c256 <= c192 && c256 <= c128) {
                launch(I128{}, std::integral_constant<int, 256>{});
                return;
            }
            if (c192 <= c128) {
                launch(I128{}, std::integral_constant<int, 192>{});
                return;
            }
        }
    }
    if ((M + 127) / 128 * tiles >= 256)
        launch(I128{}, I128{});
    else if ((M + 63) / 64 * tiles >= 256)
        launch(std::integral_constant<int, 64>{}, I128{});
    else
        launch(std::integral_constant<int, 32>{}, I128{});
}

// FP32 rows [M x K] -> FP16 hi / lo planes (GEMM operands handed over as
// FP32), one workgroup per row: the row is split as a * 2^-row_exp[m]
// (split_exponent of its largest magnitude).
__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ A, uint16_t* __restrict__ hi,
                                                         uint16_t* __restrict__ lo, int* __restrict__ row_exp, int K) {
    const size_t base = size_t(blockIdx.x) * K;
    const int tid = threadIdx.x;
    float big = 0.f;
    for (int i = tid; i < K; i += 256) big = fmaxf(big, fabsf(A[base + i]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) big = fmaxf(big, __shfl_xor(big, off));
    __shared__ float bred[4];
    if ((tid & 63) == 0) bred[tid >> 6] = big;
    __syncthreads();
    const int e = split_exponent(fmaxf(fmaxf(bred[0], bred[1]), fmaxf(bred[2], bred[3])));
    const float down = pow2(-e);
    if (tid == 0) row_exp[blockIdx.x] = e;
    for (int i = tid; i < K; i += 256) split_store(A[base + i] * down, hi, lo, base + i);
}

}  // namespace

// Runs fn(hi, lo, row_exp) on FP16 hi / lo planes of the FP32 rows
// A[M x K] and their row exponents, held in device memory allocated for this
// call (an operator entry point for tests and benchmarks, not on the
// inference path), then waits for the stream.
template <class F>
static void with_planes(const float* A, int M, int K, hipStream_t stream, F&& fn) {
    require(M > 0 && K > 0, "gemm: unsupported shape");
    const size_t n = size_t(M) * K;
    auto check = [](hipError_t e, const char* what) {
        require(e == hipSuccess, std::string("HIP error: ") + hipGetErrorString(e) + " (" + what + ")");
    };
    uint16_t* planes = nullptr;
    check(hipMalloc(&planes, 2 * n * sizeof(uint16_t) + size_t(M) * sizeof(int)), "hipMalloc");
    int* row_exp = reinterpret_cast<int*>(planes + 2 * n);
    split_rows_kernel<<<M, 256, 0, stream>>>(A, planes, planes + n, row_exp, K);
    fn(planes, planes + n, row_exp);
    const hipError_t launched = hipGetLastError();
    const hipError_t done = hipStreamSynchronize(stream);
    check(hipFree(planes), "hipFree");
    check(launched, "gemm launch");
    check(done, "hipStreamSynchronize");
}

void launch_gemm(const float* A, const uint16_t* W, float* C, int M, int N, int K, bool accumulate,
                 hipStream_t stream) {
    with_planes(A, M, K, stream, [&](const uint16_t* hi, const uint16_t* lo, const int* row_exp) {
        GemmEpilogue ep{};
        ep.row_exp = row_exp;
        if (accumulate)
            gemm<1>(hi, lo, W, C, M, N, K, stream, 1, ep);
        else
            gemm<0>(hi, lo, W, C, M, N, K, stream, 1, ep);
    });
}

void launch_gemm_swiglu(const float* A, const uint16_t* W, uint16_t* act_hi, uint16_t* act_lo, uint8_t* act_exp,
                        int M, int N, int K, hipStream_t stream) {
    require(N % 256 == 0, "gemm swiglu: N must be a multiple of 256");
    int* flags = nullptr;
    require(hipMalloc(&flags, size_t(M) * 4 * sizeof(int)) == hipSuccess, "gemm swiglu: hipMalloc failed");
    const hipError_t cleared = hipMemsetAsync(flags, 0, size_t(M) * 4 * sizeof(int), stream);
    GemmEpilogue ep{};
    ep.act_hi = act_hi;
    ep.act_lo = act_lo;
    ep.act_exp = act_exp;
    ep.act_flag = flags;
    try {
        require(cleared == hipSuccess, "gemm swiglu: hipMemsetAsync failed");
        with_planes(A, M, K, stream, [&](const uint16_t* hi, const uint16_t* lo, const int* row_exp) {
            ep.row_exp = row_exp;
            gemm<3>(hi, lo, W, nullptr, M, N, K, stream, 1, ep);
        });
    } catch (...) {
        (void)hipFree(flags);
        throw;
    }
    require(hipFree(flags) == hipSuccess, "gemm swiglu: hipFree failed");
}

// Operand planes and row exponents of launch_gemm_static: a file-scope
// device array, so the call allocates nothing. Each device holds its own copy
// at its own address (from hipGetSymbolAddress, taken once per device); host
// code uses only that address, never the array's name.
inline constexpr size_t kStaticGemmRows = kStaticGemmElements / kTileK;  // K >= 64
static __device__ __align__(256) uint16_t scratch[2 * kStaticGemmElements + 2 * kStaticGemmRows];

static uint16_t* static_planes() {
    constexpr int kMaxDevices = 64;
    static std::mutex lock;
    static uint16_t* by_device[kMaxDevices] = {};
    int device = -1;
    hipError_t e = hipGetDevice(&device);
    require(e == hipSuccess && device >= 0 && device < kMaxDevices,
            std::string("gemm static: no usable current device (") + hipGetErrorString(e) + ")");
    std::lock_guard<std::mutex> guard(lock);
    if (!by_device[device]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        require(e == hipSuccess && ptr != nullptr,
                std::string("gemm static: hipGetSymbolAddress failed (") + hipGetErrorString(e) + ")");
        by_device[device] = static_cast<uint16_t*>(ptr);
    }
    return by_device[device];
}

void launch_gemm_static(const float* A, const uint16_t* W, float* C, int M, int N, int K, bool accumulate,
                        hipStream_t stream) {
    require(M > 0 && K > 0 && N > 0 && N % kTileN == 0 && K % kTileK == 0, "gemm: unsupported shape");
    require(size_t(M) * size_t(K) <= kStaticGemmElements,
            "gemm static: M x K exceeds the 1048576 operand elements of the static planes");
    uint16_t* hi = static_planes();
    uint16_t* lo = hi + kStaticGemmElements;
    int* row_exp = reinterpret_cast<int*>(hi + 2 * kStaticGemmElements);
    split_rows_kernel<<<M, 256, 0, stream>>>(A, hi, lo, row_exp, K);
    GemmEpilogue ep{};
    ep.row_exp = row_exp;
    if (accumulate)
        gemm<1>(hi, lo, W, C, M, N, K, stream, 1, ep);
    else
        gemm<0>(hi, lo, W, C, M, N, K, stream, 1, ep);
}

void launch_attention_prefill(const float* qkv, const uint16_t* keys, const uint16_t* values, uint16_t* att_hi,
                              uint16_t* att_lo, int rows, int pos0, int context, hipStream_t stream) {
    require(rows >= 1 && rows <= kPrefillRows && pos0 >= 0 && context > 0 && pos0 + rows <= context,
            "attention: bad rows / position / context");
    attn_prefill_mfma_kernel<<<(rows + kFaRows - 1) / kFaRows * kKVHeads, 512, 0, stream>>>(
        qkv, keys, values, att_hi, att_lo, rows, pos0, context, 1.0f / std::sqrt(128.0f));
}

void launch_prefill_chunk(const PrefillLayer* layers, const uint16_t* embed, const int* ids_dev, int rows, int pos0,
                          const float* cosines, const float* sines, int context, const PrefillScratch& s,
                          hipStream_t stream) {
    require(rows >= 1 && rows <= kPrefillRows, "prefill chunk: bad row count");
    embed_rows_kernel<<<rows, 256, 0, stream>>>(ids_dev, embed, s.x);
    // The O and down GEMMs (1024 output columns, K = 2048 / 3072) split K
    // into 4 ranges for parallelism at any row count; the row kernel after
    // each adds the partials to the residual in a fixed order, so a row's
    // result still does not depend on the rows around it.
    constexpr int kSplits = 4;
    for (int l = 0; l < kLayers; ++l) {
        const PrefillLayer& L = layers[l];
        if (l == 0)
            rmsnorm_rows_kernel<<<rows, 256, 0, stream>>>(s.x, L.in_norm, s.h_hi, s.h_lo, nullptr, rows, s.row_exp,
                                                          nullptr);
        else
            rmsnorm_rows_kernel<kSplits><<<rows, 256, 0, stream>>>(s.x, L.in_norm, s.h_hi, s.h_lo, s.part, rows,
                                                                   s.row_exp, nullptr);
        GemmEpilogue ep{L.q_norm, L.k_norm, cosines, sines, L.keys, L.values, pos0, context, s.act_hi, s.act_lo,
                        s.row_exp, s.act_flag, s.act_exp};
        gemm<4>(s.h_hi, s.h_lo, L.qkv_n, s.qkv, rows, kQKVRows, kHidden, stream, 1, ep);
        launch_attention_prefill(s.qkv, L.keys, L.values, s.att_hi, s.att_lo, rows, pos0, context, stream);
        // The attention output is a convex combination of FP16 values: it fits FP16 unscaled.
        gemm<2>(s.att_hi, s.att_lo, L.o_n, s.part, rows, kHidden, kQDim, stream, kSplits);
        rmsnorm_rows_kernel<kSplits><<<rows, 256, 0, stream>>>(s.x, L.post_norm, s.h_hi, s.h_lo, s.part, rows,
                                                               s.row_exp, s.act_flag);
        gemm<3>(s.h_hi, s.h_lo, L.gateup_n, nullptr, rows, 2 * kFFN, kHidden, stream, 1, ep);
        GemmEpilogue down{};
        down.act_flag = s.act_flag;
        down.act_exp = s.act_exp;
        gemm<2>(s.act_hi, s.act_lo, L.down_n, s.part, rows, kHidden, kFFN, stream, kSplits, down);
    }
    fold_rows_kernel<kSplits><<<(rows * kHidden + 255) / 256, 256, 0, stream>>>(s.x, s.part, rows);
}

}  // namespace qwen_hip
