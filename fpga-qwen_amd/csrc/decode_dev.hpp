// Device arithmetic of the batch-1 decode kernels (decode.hip): the
// reference dot's chain steps and combine (engine/core.cpp:119-147), RMSNorm
// (207-215), QK-norm and rotate-half RoPE (216-218, 395-402), and the
// chain-permuted key reads.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "half_split.hpp"
#include "kernels.hpp"

namespace qwen_hip {
namespace dev {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}
__device__ __forceinline__ uint16_t f2h(float f) { return to_half_bits(f); }

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

// The value of lane (this lane ^ OFF), at register speed instead of the
// cross-lane permute through the LDS unit (a round trip of 100+ clocks on
// the dependent chains of the reductions): inside a 16-lane row DPP row
// moves (quad_perm for 1 and 2; row_shl / row_shr plus a lane select for 4
// and 8), across rows the gfx950 row swaps (v_permlane16_swap,
// v_permlane32_swap; token kernel 324.5 -> 322.6 us at 109 positions, 353.5
// -> 348.3 at 201). Every lane receives the same value as from __shfl_xor,
// so reductions keep their exact order. The lane select reads threadIdx.x,
// so callers run one-dimensional workgroups (threadIdx.x % 64 is the lane),
// as every decode kernel does.
template <int OFF>
__device__ __forceinline__ int xor_lanes_bits(int v) {
    static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "power-of-two lane offset");
    if constexpr (OFF == 1) {
        return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (OFF == 2) {
        return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (OFF == 4 || OFF == 8) {
        const int up = __builtin_amdgcn_update_dpp(v, v, 0x100 + OFF, 0xF, 0xF, false);  // row_shl: lane + OFF
        const int down = __builtin_amdgcn_update_dpp(v, v, 0x110 + OFF, 0xF, 0xF, false);  // row_shr: lane - OFF
        return (threadIdx.x & OFF) ? down : up;
    } else if constexpr (OFF == 16) {
        // Odd 16-lane rows of the first operand trade places with even rows
        // of the second: with v in both, the first holds lane - 16 in the
        // odd rows and the second lane + 16 in the even rows.
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return int((threadIdx.x & 16) ? r[0] : r[1]);
    } else {
        // The upper half of the first operand trades places with the lower
        // half of the second.
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return int((threadIdx.x & 32) ? r[0] : r[1]);
    }
}
template <int OFF>
__device__ __forceinline__ int xor_lanes(int v) { return xor_lanes_bits<OFF>(v); }
template <int OFF>
__device__ __forceinline__ float xor_lanes(float v) { return __int_as_float(xor_lanes_bits<OFF>(__float_as_int(v))); }
template <int OFF>
__device__ __forceinline__ double xor_lanes(double v) {
    const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(v));
    const unsigned lo = static_cast<unsigned>(xor_lanes_bits<OFF>(static_cast<int>(b & 0xffffffffu)));
    const unsigned hi = static_cast<unsigned>(xor_lanes_bits<OFF>(static_cast<int>(b >> 32)));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// Lane c of each 8-lane group holds chain c; returns
// ((c0+c4)+(c1+c5)) + ((c2+c6)+(c3+c7)) in every lane of the group.
__device__ __forceinline__ float combine_chains(float acc) {
    const float t1 = acc + xor_lanes<4>(acc);
    const float t2 = t1 + xor_lanes<1>(t1);
    return t2 + xor_lanes<2>(t2);
}

__device__ __forceinline__ double wave_sum(double v) {
    v += xor_lanes<32>(v);
    v += xor_lanes<16>(v);
    v += xor_lanes<8>(v);
    v += xor_lanes<4>(v);
    v += xor_lanes<2>(v);
    v += xor_lanes<1>(v);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, xor_lanes<32>(v));
    v = fmaxf(v, xor_lanes<16>(v));
    v = fmaxf(v, xor_lanes<8>(v));
    v = fmaxf(v, xor_lanes<4>(v));
    v = fmaxf(v, xor_lanes<2>(v));
    return fmaxf(v, xor_lanes<1>(v));
}

// Range guard of the batched matrix-core inputs (split_exponent): a launch
// first splits every sequence's values unscaled and each wave records the
// largest magnitude it split (wave_big). Only if one of them reaches the FP16
// limit (rare: every wave sees the same LDS, so all take the same branch)
// does the workgroup find each sequence's exact maximum and split again as
// v * 2^-e; the products of sequence s are scaled back by 2^e[s]
// (SplitGuard::up, 1 while no sequence was scaled).
struct SplitGuard {
    float wave_big[16];
    unsigned seq_big[kMaxBatch];
    int seq_e[kMaxBatch];

    // Before the first barrier of the launch.
    __device__ void init(int tid) {
        if (tid < kMaxBatch) {
            seq_big[tid] = 0u;
            seq_e[tid] = 0;
        }
    }
    // Every wave after its unscaled splits, before the barrier that ends them.
    __device__ void post(float big, int lane, int wave) {
        big = wave_max(big);
        if (lane == 0) wave_big[wave] = big;
    }
    // After that barrier.
    __device__ bool needed(int waves) const {
        float big = 0.f;
        for (int w = 0; w < waves; ++w) big = fmaxf(big, wave_big[w]);
        return big >= kSplitLimit;
    }
    // Slow path: every thread offers the maximum of its values of sequence
    // s; after a barrier, exponent(s) is that sequence's exponent.
    __device__ void offer(int s, float big) { atomicMax(&seq_big[s], __float_as_uint(big)); }
    __device__ int exponent(int s) const { return split_exponent(__uint_as_float(seq_big[s])); }
    __device__ float up(int s) const { return pow2(seq_e[s]); }
};

// Position of activation j in the permuted LDS vector: j = 64b + 8i + c is
// stored at 64b + 8c + i, so chain c reads its 8 values contiguously.
__device__ __forceinline__ int xperm(int j) { return (j & ~63) | ((j & 7) << 3) | ((j >> 3) & 7); }

// RMSNorm (engine/core.cpp:207-215) of N values held PER = N / THREADS per
// thread (element j = tid + k THREADS, or j = PER tid + k when CONTIG), with
// their norm weights, into permuted LDS (and optionally to `copy`).
template <int N, int THREADS, bool CONTIG = false>
__device__ __forceinline__ void norm_to_lds(const float (&v)[N / THREADS], const float (&w)[N / THREADS], float* xs,
                                            double* red, float* copy) {
    constexpr int PER = N / THREADS;
    const int tid = threadIdx.x;
    double part = 0.0;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
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
        const int j = CONTIG ? PER * tid + k : tid + k * THREADS;
        const float o = (v[k] * inv) * w[k];
        xs[xperm(j)] = o;
        if (copy) copy[j] = o;
    }
}

// 8 FP16 values of an MFMA B operand from LDS, zeroed for lanes whose column
// is not a live sequence. Read unconditionally and masked (no branch): a
// branch around the read makes the next wait cover every load in flight.
template <class H8>
__device__ __forceinline__ H8 masked_b(const _Float16* p, bool live) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
    const unsigned m = live ? 0xffffffffu : 0u;
    return __builtin_bit_cast(H8, u32x4{v.x & m, v.y & m, v.z & m, v.w & m});
}

// Two 16-byte pieces of a chain-permuted key row as the 8 chain steps each
// of lane c: pieces c and c + 8 (see kperm).
__device__ __forceinline__ void key_pieces(const uint16_t* row, int c, u32x4& lo, u32x4& hi) {
    const u32x4* kp = reinterpret_cast<const u32x4*>(row);
    lo = kp[c];
    hi = kp[c + 8];
}

// The same 16 halves of the current key row, from LDS.
__device__ __forceinline__ void key_pieces_lds(const uint16_t* kcur, int c, uint32_t (&kw)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int base = (i < 4 ? 8 * c : 64 + 8 * c) + 2 * (i & 3);
        kw[i] = uint32_t(kcur[base]) | (uint32_t(kcur[base + 1]) << 16);
    }
}

// Chain c of q . k for one key: steps s = 0..15 in order; q in kperm order.
__device__ __forceinline__ float key_chain(const float* qperm, int c, const uint32_t (&kw)[8], float acc) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int base = (i < 4 ? 8 * c : 64 + 8 * c) + 2 * (i & 3);
        acc = __builtin_fmaf(qperm[base], h2f(kw[i] & 0xffffu), acc);
        acc = __builtin_fmaf(qperm[base + 1], h2f(kw[i] >> 16), acc);
    }
    return acc;
}

// RMSNorm over 128 values held one per thread by two consecutive waves
// (engine/core.cpp:397-398), then rotate-half RoPE (216-218). w, cs, sn are
// this thread's norm weight and the cosine / sine of its rotation pair
// (index j % 64), loaded by the caller ahead of its other loads.
__device__ __forceinline__ float head_norm_rope(float raw, float w, float cs, float sn, double* red2, float* buf,
                                                int j) {
    const int lane = threadIdx.x & 63;
    const float square = raw * raw;
    const double part = wave_sum(static_cast<double>(square));
    if (lane == 0) red2[(j >> 6)] = part;
    __syncthreads();
    const float sum = static_cast<float>(red2[0] + red2[1]);
    const float inv = 1.0f / __builtin_sqrtf(sum / 128.0f + 1e-6f);
    const float normed = (raw * inv) * w;
    buf[j] = normed;
    __syncthreads();
    float out;
    if (j < 64) {
        const float x0 = buf[j], x1 = buf[j + 64];
        out = x0 * cs - x1 * sn;
    } else {
        const int jj = j - 64;
        const float x0 = buf[jj], x1 = buf[j];
        out = x1 * cs + x0 * sn;
    }
    return out;
}

// Exchange between the workgroups of one XCD. A launch's workgroups are
// dispatched round-robin over the 8 XCDs (workgroup w on XCD w % 8, measured
// on this chip also right after launches of odd sizes), whose CUs share the
// XCD's L2. A plain store reaches that L2 (the vector L1 is write-through),
// and an agent-scope load skips the reader's L1 and finds the line there.
// (Invalidating L1 with buffer_inv sc0 does not work here: outside
// thread-group-split mode it leaves the stale line in place.) Each value
// travels with its launch's tag in one 8-byte store, so a word left by an
// earlier launch is never taken for a fresh one: placement decides only
// whether a value arrives, never which value is read. Polls are bounded; a
// consumer that gives up raises the stall flag, which the step's argmax
// copies to the host. Measured: 0.40 us per exchange inside an XCD, against
// 2.37 us per dependent kernel launch.
constexpr unsigned kExchangeSpins = 1u << 18;  // ~0.1 s of polling; an exchange takes about a microsecond

__device__ __forceinline__ void exchange_put(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, (uint64_t(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// For a reader on another XCD: an agent-scope store writes through the L2
// (such a reader's agent-scope load then finds it in memory).
__device__ __forceinline__ void exchange_put_through(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, (uint64_t(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Two consecutive tagged words; false if they did not both carry `tag`
// within kExchangeSpins polls. The loop runs while any lane of the wave still
// waits (a wave-uniform exit), and each lane's result comes from its own
// flag: lanes leaving a loop at different iterations would otherwise hand the
// compiler a divergent loop exit for the result.
__device__ __forceinline__ bool exchange_get2(const uint64_t* p, uint32_t tag, float& a, float& b,
                                              unsigned limit = kExchangeSpins) {
    unsigned missing = 1;
    for (unsigned spin = 0; spin < limit && __any(missing); ++spin) {
        if (missing) {
            const uint64_t u = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint64_t w = __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (uint32_t(u >> 32) == tag && uint32_t(w >> 32) == tag) {
                a = __uint_as_float(uint32_t(u));
                b = __uint_as_float(uint32_t(w));
                missing = 0;
            }
        }
    }
    return missing == 0;
}

// N tagged words at once: every round issues the loads of all words still
// missing (bit k of `want`), then checks them, so a round costs one L2 round
// trip however many words there are. False if some word did not carry `tag`
// within kExchangeSpins rounds.
template <int N>
__device__ __forceinline__ bool exchange_gather(const uint64_t* const (&p)[N], uint32_t tag, float (&out)[N],
                                                unsigned want, unsigned limit = kExchangeSpins) {
    // Wave-uniform loop exit, per-lane result from `want` (see exchange_get2).
    for (unsigned spin = 0; spin < limit && __any(want != 0); ++spin) {
        uint64_t u[N];
#pragma unroll
        for (int k = 0; k < N; ++k)
            u[k] = (want >> k) & 1 ? __hip_atomic_load(p[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
#pragma unroll
        for (int k = 0; k < N; ++k)
            if (((want >> k) & 1) && uint32_t(u[k] >> 32) == tag) {
                out[k] = __uint_as_float(uint32_t(u[k]));
                want &= ~(1u << k);
            }
    }
    return want == 0;
}

// exchange_gather with two rounds in flight: every round loads all N words
// (the caller's addresses must be valid for every lane, wanted or not), the
// second round issued D x 64 clocks after the first, so memory is sampled
// about twice per round trip and the compiler's waits count one round.
template <int N, int D>
__device__ __forceinline__ bool exchange_gather_pipe(const uint64_t* const (&p)[N], uint32_t tag, float (&out)[N],
                                                     unsigned want, unsigned limit = kExchangeSpins) {
    uint64_t a[N], b[N];
    auto issue = [&](uint64_t(&u)[N]) {
#pragma unroll
        for (int k = 0; k < N; ++k) u[k] = __hip_atomic_load(p[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto take = [&](const uint64_t(&u)[N]) {
#pragma unroll
        for (int k = 0; k < N; ++k)
            if (((want >> k) & 1) && uint32_t(u[k] >> 32) == tag) {
                out[k] = __uint_as_float(uint32_t(u[k]));
                want &= ~(1u << k);
            }
    };
    issue(a);
    __builtin_amdgcn_s_sleep(D);
    for (unsigned spin = 0;;) {
        issue(b);
        take(a);
        if (!__any(want != 0) || ++spin >= limit) break;
        issue(a);
        take(b);
        if (!__any(want != 0) || ++spin >= limit) break;
    }
    return want == 0;
}

}  // namespace dev
}  // namespace qwen_hip
