// One launch per decode token for gfx950 (CDNA4, wave64): the 28 layers of
// a batch-1 step (engine/core.cpp:353-646 for one row) in one persistent
// kernel.
//
// Why one launch: between two dependent kernels the GPU spends ~1.2 us of
// launch gap and ~2.5 us until the next kernel's first data arrives (its
// inputs were just written on other XCDs, and every workgroup starts by
// loading them together with its weights), 57 times per token. Inside one
// launch the two residual hand-overs of a layer are exchanges through memory
// (~1.1-1.5 us each), and each phase's weights are already in LDS when it
// starts.
//
// Workgroup w = g + 8 s (XCD g, slot s), 12 waves:
// * waves 0-7 (compute) run the phases of the fused QKV + attention + O
//   kernel and of the fused FFN kernel (decode.hip) with the same thread
//   layouts and arithmetic, so every row is bit-identical to that path, and
//   do every exchange poll;
// * waves 8-11 (load) copy the layer's weight tiles into LDS with direct
//   global -> LDS loads, one region per phase (QKV tiles with the input and
//   QK norm weights, O rows, gate/up tiles with the post-attention norm
//   weights, down tiles). A region is refilled with the next layer's tiles
//   as soon as its phase is done, so the weights stream a layer ahead of the
//   arithmetic. Load waves never poll: a wave's loads complete in issue
//   order, so a poll issued behind weight loads would wait for them.
// All 12 waves pass the same barriers (s_barrier without a memory fence).
// Compute waves wait for their own LDS accesses before each barrier; load
// waves wait for the region the next phase reads with an exact vmcnt (the
// loads they issued after it may stay in flight).
//
// Residual hand-overs across XCDs (the O projection's 16 head partials, the
// FFN's 8 down slices): producers post their rows with write-through stores;
// the 8 workgroups of slot s (one per XCD) each gather rows 32 s .. 32 s +
// 31, fold them in the fixed tree order of the two-kernel path, and post
// the 32 sums inside their XCD, where every workgroup gathers all 1024.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <type_traits>

#include "decode_dev.hpp"
#include "token.hpp"

#ifndef QWEN_TOK_STAGGER_XCD
#define QWEN_TOK_STAGGER_XCD 2
#endif
#ifndef QWEN_TOK_STAGGER_CROSS
#define QWEN_TOK_STAGGER_CROSS 6
#endif

namespace qwen_hip {
namespace {

using namespace dev;

constexpr int kComputeWaves = 8, kLoadWaves = 4;
constexpr int kTokenThreads = 64 * (kComputeWaves + kLoadWaves);

// LDS regions (bytes) and the direct loads (1 KiB each) each load wave issues for them.
constexpr int kRegQkv = 2 * 16384;   // QKV tiles li = 2s, 2s + 1 of the head group
constexpr int kRegO = 64 * 256;       // O rows 64 (s / 2) .. + 63 over head h's 128 columns
constexpr int kRegGu = 3 * 16384;     // gate/up tiles 96 g + 3 s .. + 2
constexpr int kRegDown = 4 * 6144;    // down tiles 4 s .. 4 s + 3 over slice g's 6 column blocks
constexpr int kLoadsQkv = 10;         // 8 tile blocks, a quarter of the input norm, the QK norms
constexpr int kLoadsO = 4;
constexpr int kLoadsGu = 13;          // 12 tile blocks, a quarter of the post-attention norm
constexpr int kLoadsDown = 6;
constexpr int kLoadsPrefetch = 2;     // next layer's K/V lines into L2
static_assert(kRegQkv / 1024 == 8 * kLoadWaves && kRegO / 1024 == kLoadsO * kLoadWaves &&
                  kRegGu / 1024 == 12 * kLoadWaves && kRegDown / 1024 == kLoadsDown * kLoadWaves,
              "every load wave issues the same loads");
// When each region's loads are issued. A CU returns loads in issue order, so
// an exchange poll issued behind weight loads waits for them, and a load
// wave that issues a long burst holds up the next barrier (the issue rate is
// bound by HBM when every CU streams). So each region's loads are spread
// over several barrier intervals, a few per interval, in intervals without
// polls where possible. Interval k runs from barrier Bk to Bk+1 (B0: the
// previous layer's last barrier). Per layer l, per load wave:
//   k = 0: gate/up(l) loads 0-4        k = 5: QKV(l + 1) 3-4
//   k = 1: gate/up(l) 5-8              k = 6: QKV(l + 1) 5-6
//   k = 3: gate/up(l) 9-12, prefetch 0 k = 8: O(l + 1) 0-2
//   k = 4: down(l) 0-5, prefetch 1,    k = 9: O(l + 1) 3, QKV(l + 1) 7-9
//          QKV(l + 1) 0-2
// At the start: QKV(0) and O(0) in the order of intervals 4-9. A region's
// wait comes after its interval's loads; it allows the loads issued after
// the region (the same count for every layer but the last, which waits for
// all):
//   QKV(l) in interval 0: gate/up(l) 0-4                          = 5
//   O(l) in interval 4: QKV(l) 7-9, gate/up(l), prefetch, down(l),
//     QKV(l + 1) 0-2                                               = 27
//   gate/up(l) in interval 8: prefetch 0-1, down, QKV(l + 1) 0-6,
//     O(l + 1) 0-2 (less prefetch 0, issued with gate/up 9-12)     = 18
//   down(l) in interval 10: prefetch 1, QKV(l + 1), O(l + 1)       = 15
// In the split form the partial merge (interval 5) stores and polls behind
// whatever the CU still has in flight, and beyond ~1000 positions the
// prefetch makes intervals 3-4 ask for more than HBM delivers in them: so
// there prefetch 1 goes out in interval 8 (before O(l + 1) 0-2) and
// QKV(l + 1) 3-4 after B6b, and the O(l) wait allows one load fewer (the
// other counts stay: prefetch 1 is still issued after down(l) and before
// the gate/up wait). With two passes (beyond 2048 positions) only load
// waves 2-3 move their prefetch 1; waves 0-1 keep it in interval 4, so the
// two windows share it (each wave's waits count its own loads).
constexpr int kAfterQkv = 5;
constexpr int kAfterO = 3 + kLoadsGu + kLoadsPrefetch + kLoadsDown + 3;
constexpr int kAfterOSplit = kAfterO - 1;
constexpr int kAfterGu = 1 + kLoadsDown + 1 + 7 + 3;
constexpr int kAfterDown = 1 + kLoadsQkv + kLoadsO;
static_assert(kAfterO == 27 && kAfterGu == 18 && kAfterDown == 15, "wait counts of the load plan");

constexpr int kXPart = kHeadDim + 2;  // attention partial: 128 outputs, max, sum

// 16 bytes per lane from global memory into LDS at lds + 16 lane (lds
// wave-uniform), counted by vmcnt.
__device__ __forceinline__ void dma16(const void* src, void* lds) {
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

// Barrier of all 12 waves without a memory fence (a fenced barrier would
// make the load waves wait for every load in flight). Each wave first waits
// for its own LDS accesses, so what it wrote is visible after the barrier;
// the empty asm statements keep the compiler from moving memory accesses
// across it.
__device__ __forceinline__ void barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Exchange polls that also give up as soon as another workgroup raised the
// step's stall word (so one missing post costs one poll limit, not one per
// waiting workgroup and phase).
//
// Two rounds are in flight at once, the second issued about half a round
// trip after the first (s_sleep D, D x 64 clocks), so memory is sampled twice
// per round trip: a word that lands is seen about a quarter round trip
// sooner on average than with one round at a time. Every round loads all N
// words (every caller's addresses are valid for every lane), so each round is
// the same N instructions and the compiler's waits count exactly one round.
template <int N, int D>
__device__ __forceinline__ bool tok_gather(const uint64_t* const (&p)[N], uint32_t tag, float (&out)[N], unsigned want,
                                           const int* stall, unsigned limit) {
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
        // Every polling wave of the launch reads the one stall word: read it
        // every 16th pair of rounds only.
        if ((spin & 31) == 30 && __any(__hip_atomic_load(stall, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0))
            break;
    }
    // A give-up raises the stall word at once: the other workgroups stop
    // polling and the step's argmax reports it.
    if (want != 0) __hip_atomic_store(const_cast<int*>(stall), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return want == 0;
}

// Stagger of the second round in flight (s_sleep units of 64 clocks): about
// half the round trip of a poll inside an XCD (L2) and across XCDs (memory).
constexpr int kStaggerXcd = QWEN_TOK_STAGGER_XCD, kStaggerCross = QWEN_TOK_STAGGER_CROSS;

__device__ __forceinline__ bool tok_get2(const uint64_t* p, uint32_t tag, float& a, float& b, const int* stall,
                                         unsigned limit) {
    const uint64_t* const words[2] = {p, p + 1};
    float got[2] = {0.f, 0.f};
    const bool ok = tok_gather<2, kStaggerXcd>(words, tag, got, 3u, stall, limit);
    a = got[0];
    b = got[1];
    return ok;
}

// Global-memory views of the K/V cache pointers (which the kernel reads from
// its arguments, so the compiler cannot infer their address space and would
// use flat accesses, which also count in lgkmcnt).
typedef __attribute__((address_space(1))) const u32x4 global_u32x4;
typedef __attribute__((address_space(1))) uint16_t global_u16;
__device__ __forceinline__ const global_u32x4* global_rows(const uint16_t* p) {
    return (const global_u32x4*)(p);
}
__device__ __forceinline__ global_u16* global_halves(uint16_t* p) { return (global_u16*)(p); }

__device__ __forceinline__ float fold_slices(float xm, const float (&d)[kFfnSlices]) {
    return xm + (((d[0] + d[1]) + (d[2] + d[3])) + ((d[4] + d[5]) + (d[6] + d[7])));
}

// QKV tile of local index li (0..63) of head group g: q tiles 32 g + li,
// k tiles 256 + 16 g + li - 32, v tiles 384 + 16 g + li - 48.
__device__ __forceinline__ int qkv_tile(int g, int li) {
    return li < 32 ? 32 * g + li : li < 48 ? 256 + 16 * g + (li - 32) : 384 + 16 * g + (li - 48);
}

// LDS of a workgroup. Weight regions (bytes): one row: QKV, O, gate/up,
// down; two rows (verification): O shares the down region (O rows are used
// before the down tiles are loaded, and the next layer's O rows are loaded
// after them), which leaves room for the second row's state.
template <int ROWS>
struct Lds {
    static constexpr int kQkvAt = 0;
    static constexpr int kGuAt = kQkvAt + kRegQkv;
    static constexpr int kDownAt = kGuAt + kRegGu;
    static constexpr int kOAt = ROWS == 1 ? kDownAt + kRegDown : kDownAt;
    static constexpr int kWeights = ROWS == 1 ? kOAt + kRegO : kDownAt + kRegDown;
    static_assert(kRegO <= kRegDown, "O rows fit the down region");
    unsigned char w[kWeights];
    float nin[kHidden];       // input RMSNorm weights
    float npost[kHidden];     // post-attention RMSNorm weights
    float nqk[2 * kHeadDim];  // q norm, k norm
    unsigned char junk[1024];  // target of the K/V prefetch loads
    float rope[ROWS][2][64];  // cos, sin of each row's position
    // Per row. Buffers whose lifetimes do not overlap share storage: the
    // attention partials (between the scores and the O rows) with the
    // normalized input and the post-attention residual, the probabilities
    // with the activations.
    struct Row {
        float x[kHidden];  // residual the layer starts from
        union {
            struct {
                float4 xs4[kHidden / 4];  // normalized input, chain-permuted
                float xm[kHidden];        // residual after the attention block
            } n;
            float opart[8][2][128];
        } u;
        union {
            float4 as4[kFfnSlice / 4];  // this XCD's activations, chain-permuted
            float prob[2][128];
        } v;
        double red[4];
        float qp[2][128];
        uint16_t kcur[128], vcur[128];
        float wmax[8][2], wsum[8][2];
        float gm[4], gl[4], go[4][128];
        float att[128];
    } r[ROWS];
    __device__ unsigned char* wq() { return w + kQkvAt; }
    __device__ unsigned char* wo() { return w + kOAt; }
    __device__ unsigned char* wgu() { return w + kGuAt; }
    __device__ unsigned char* wdn() { return w + kDownAt; }
};
static_assert(sizeof(Lds<1>) <= 163840 && sizeof(Lds<2>) <= 163840, "LDS of one workgroup per CU");

// Load waves: one load of a region for layer `layer` (lw = load wave 0..3).
template <int ROWS>
struct Loader {
    const TokenLaunch& a;  // the kernel arguments (layer pointers read with scalar loads)
    Lds<ROWS>& m;
    int g, s, lw, lane, context, pos;

    // Load i (0-9) of the QKV region: 8 tile blocks, a quarter of the input
    // norm weights, the QK norm weights.
    __device__ void qkv(int layer, int i) const {
        const TokenLayer& L = a.layers[layer];
        if (i < 8) {
            const int k = 8 * lw + i, t = k >> 4, b = k & 15;
            const int tile = qkv_tile(g, 2 * s + t);
            dma16(L.qkv_t + (size_t(tile) * 16 + b) * 512 + 8 * lane, m.wq() + 1024 * k);
        } else if (i == 8) {
            dma16(L.in_norm + 256 * lw + 4 * lane, reinterpret_cast<unsigned char*>(m.nin) + 1024 * lw);
        } else {
            dma16(L.qk_norm + 4 * lane, m.nqk);
        }
    }
    __device__ void o(int layer, int i) const {
        const TokenLayer& L = a.layers[layer];
        const int h = 2 * g + (s & 1), rb = s >> 1;
        const int k = kLoadsO * lw + i, r = 4 * k + (lane >> 4), piece = lane & 15;
        dma16(L.o_n + size_t(64 * rb + r) * kQDim + 128 * h + 8 * piece, m.wo() + 1024 * k);
    }
    // Load i (0-12) of the gate/up region: 12 tile blocks, a quarter of the
    // post-attention norm weights.
    __device__ void gu(int layer, int i) const {
        const TokenLayer& L = a.layers[layer];
        if (i < 12) {
            const int k = 12 * lw + i;
            dma16(L.gateup_t + (size_t(96 * g + 3 * s) * 16 + k) * 512 + 8 * lane, m.wgu() + 1024 * k);
        } else {
            dma16(L.post_norm + 256 * lw + 4 * lane, reinterpret_cast<unsigned char*>(m.npost) + 1024 * lw);
        }
    }
    __device__ void down(int layer, int b) const {
        const TokenLayer& L = a.layers[layer];
        const int tile = 4 * s + lw;
        dma16(L.down_t + (size_t(tile) * (kFFN / 64) + 6 * g + b) * 512 + 8 * lane,
              m.wdn() + 1024 * (6 * lw + b));
    }
    // Lines of the K/V rows [0, pos) of head g in layer `layer`, a 1/32
    // share per workgroup of the XCD (128-byte lines, one lane each; lanes
    // past the rows read line 0), into L2 ahead of the compute waves' loads.
    // With `on` false the same load re-reads the QK norm weights into the
    // junk area (the waits count loads).
    __device__ void prefetch(int layer, int i, bool on) const {
        const TokenLayer& L = a.layers[layer];
        if (!on) {
            dma16(L.qk_norm + 4 * lane, m.junk);
            return;
        }
        const size_t base = size_t(g) * context * 128;     // halves
        const size_t kv = size_t(kKVHeads) * context * 128;  // values after the keys
        const int lines = 2 * pos;                         // per matrix
        const int q = 512 * s + 64 * (kLoadsPrefetch * lw + i) + lane;
        // Key lines, then the value lines (kv halves further on).
        const size_t at = q < lines ? base + 64 * size_t(q) : q < 2 * lines ? kv + base + 64 * size_t(q - lines) : base;
        dma16(L.keys + at, m.junk);
    }
    __device__ void qkv_range(int layer, int first, int count) const {
        for (int i = first; i < first + count; ++i) qkv(layer, i);
    }
    __device__ void o_range(int layer, int first, int count) const {
        for (int i = first; i < first + count; ++i) o(layer, i);
    }
    __device__ void gu_range(int layer, int first, int count) const {
        for (int i = first; i < first + count; ++i) gu(layer, i);
    }
    __device__ void down_range(int layer, int first, int count) const {
        for (int b = first; b < first + count; ++b) down(layer, b);
    }
};

// The load plan of two rows, where O shares the down region: down(l) is
// loaded after O(l) is used (B7), O(l + 1) after down(l) is used (B12). Per
// layer l, per load wave:
//   k = 0: gate/up(l) 0-4           k = 6: QKV(l + 1) 5-6
//   k = 1: gate/up(l) 5-8           k = 7: down(l) 0-2
//   k = 3: gate/up(l) 9-12,         k = 8: down(l) 3-5
//          prefetch 0               k = 9: QKV(l + 1) 7-9
//   k = 4: prefetch 1, QKV(l + 1)   k = 12: O(l + 1) 0-3
//          0-2
//   k = 5: QKV(l + 1) 3-4
// At the start: QKV(0), then O(0). Waits (loads issued after the region):
//   QKV(l) in interval 0: O(l), gate/up(l) 0-4                     = 9
//   O(l) in interval 4: gate/up(l), prefetch, QKV(l + 1) 0-2       = 18
//   gate/up(l) in interval 8: prefetch, QKV(l + 1) 0-6, down(l)    = 15
//   down(l) in interval 10: QKV(l + 1) 7-9                         = 3
constexpr int kPairAfterQkv = kLoadsO + 5;
constexpr int kPairAfterO = kLoadsGu + kLoadsPrefetch + 3;
constexpr int kPairAfterGu = kLoadsPrefetch + 7 + kLoadsDown;
constexpr int kPairAfterDown = 3;
static_assert(kPairAfterQkv == 9 && kPairAfterO == 18 && kPairAfterGu == 15, "wait counts of the two-row plan");

// The chain dot of NB 16-byte LDS blocks (block b at w[64 b]) against the
// permuted LDS vector of each row (block b's 8 values at x4[16 b],
// x4[16 b + 1]) in the reference's FMA order; the rows share every weight
// read. The next two blocks are read while the chain steps of the current
// two run, which bounds the registers the dot holds (about 50 per row
// instead of the ~190 of all 16 blocks read up front).
template <int NB, int ROWS>
__device__ __forceinline__ void lds_chain(const u32x4* w, const float4* const (&x4)[ROWS], float (&acc)[ROWS]) {
    static_assert(NB % 2 == 0, "pairs of blocks");
    u32x4 w0 = w[0], w1 = w[64];
    float4 a0[ROWS], b0[ROWS], a1[ROWS], b1[ROWS];
#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        a0[q] = x4[q][0];
        b0[q] = x4[q][1];
        a1[q] = x4[q][16];
        b1[q] = x4[q][17];
        acc[q] = 0.f;
    }
#pragma unroll
    for (int b = 0; b < NB; b += 2) {
        u32x4 nw0 = w0, nw1 = w1;
        float4 na0[ROWS], nb0[ROWS], na1[ROWS], nb1[ROWS];
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            na0[q] = a0[q];
            nb0[q] = b0[q];
            na1[q] = a1[q];
            nb1[q] = b1[q];
        }
        if (b + 2 < NB) {
            nw0 = w[64 * (b + 2)];
            nw1 = w[64 * (b + 3)];
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                na0[q] = x4[q][16 * (b + 2)];
                nb0[q] = x4[q][16 * (b + 2) + 1];
                na1[q] = x4[q][16 * (b + 3)];
                nb1[q] = x4[q][16 * (b + 3) + 1];
            }
        }
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            acc[q] = chain8(acc[q], w0, a0[q], b0[q]);
            acc[q] = chain8(acc[q], w1, a1[q], b1[q]);
        }
        w0 = nw0;
        w1 = nw1;
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            a0[q] = na0[q];
            b0[q] = nb0[q];
            a1[q] = na1[q];
            b1[q] = nb1[q];
            // Orders the chain steps before the next reads (a scheduling
            // barrier alone leaves the arithmetic free to sink below every read).
            asm volatile("" : "+v"(acc[q]));
        }
    }
}

// RMSNorm sums of one row (engine/core.cpp:207-215: FP32 squares summed in
// FP64): thread tid < 256 holds entries 4 tid .. 4 tid + 3 in v; wave w's
// sum goes to red[w].
__device__ __forceinline__ void norm_sums(const float (&v)[4], double* red, int wave, int lane) {
    double part = 0.0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float square = v[k] * v[k];
        part += static_cast<double>(square);
    }
    part = wave_sum(part);
    if (lane == 0) red[wave] = part;
}

// FULL (PASSES <= 4 passes of 64 positions, n <= 256): every workgroup
// attends its query head over all positions; else the split form (passes s
// and s + 32 of both heads, partials merged inside the XCD). ROWS = 2: the
// two rows of a verification at positions pos and pos + 1 (row 1 attends to
// row 0's new K/V from LDS), every weight read once for both, each row with
// the arithmetic of a single step; the attention form and pass count are
// row 1's (extra passes add nothing to row 0: its positions past pos + 1
// score -inf and weigh 0).
//
// The load waves and the compute waves run separate loops that pass the
// same barriers, numbered B0 .. B13 below (the split form adds B6b).
template <int PASSES, bool FULL, int ROWS>
__global__ __launch_bounds__(kTokenThreads) void token_kernel(const TokenLaunch a) {
    static_assert(ROWS == 1 || ROWS == 2, "one or two rows");
    __shared__ Lds<ROWS> m;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = int(blockIdx.x & 7), s = int(blockIdx.x >> 3);
    const int L = a.layer_count;

    if (wave >= kComputeWaves) {
        // lw in a scalar register: every load below must be one instruction
        // executed by the whole wave (the waits count them), never a load
        // under a divergent branch.
        const int lw = __builtin_amdgcn_readfirstlane(wave - kComputeWaves);
        const Loader<ROWS> ld{a, m, g, s, lw, lane, a.context, a.pos};
        const bool pf = a.prefetch != 0;
        constexpr bool kSplitPlan = ROWS == 1 && !FULL;  // the split form's moved loads (above)
        const bool late_pf = kSplitPlan && (PASSES == 1 || lw >= 2);  // prefetch 1 after fold 1
        if constexpr (ROWS == 1) {
            // QKV(0) and O(0) in the order of intervals 4-9 of a layer.
            ld.qkv_range(0, 0, 3);
            ld.qkv_range(0, 3, 2);
            ld.qkv_range(0, 5, 2);
            ld.o_range(0, 0, 3);
            ld.o_range(0, 3, 1);
            ld.qkv_range(0, 7, 3);
        } else {
            ld.qkv_range(0, 0, kLoadsQkv);
            ld.o_range(0, 0, kLoadsO);
        }
        barrier();  // B0
        for (int l = 0; l < L; ++l) {
            const bool last = l + 1 == L;
            ld.gu_range(l, 0, 5);
            wait_vmcnt<ROWS == 1 ? kAfterQkv : kPairAfterQkv>();  // QKV(l) and the input / QK norm weights
            barrier();  // B1
            ld.gu_range(l, 5, 4);
            barrier();  // B2
            barrier();  // B3
            ld.gu_range(l, 9, 4);
            if (!last) ld.prefetch(l + 1, 0, pf);
            barrier();  // B4
            if constexpr (ROWS == 1) ld.down_range(l, 0, kLoadsDown);
            if (!last) {
                if (!late_pf) ld.prefetch(l + 1, 1, pf);
                ld.qkv_range(l + 1, 0, 3);
            }
            if (last) wait_vmcnt<0>();
            else if (late_pf) wait_vmcnt<kAfterOSplit>();
            else wait_vmcnt<ROWS == 2 ? kPairAfterO : kAfterO>();  // O(l)
            barrier();  // B5
            if (!kSplitPlan && !last) ld.qkv_range(l + 1, 3, 2);
            barrier();  // B6
            if (!FULL) barrier();  // B6b
            if (kSplitPlan && !last) ld.qkv_range(l + 1, 3, 2);
            if (!last) ld.qkv_range(l + 1, 5, 2);
            barrier();  // B7: O(l) is used
            if constexpr (ROWS == 2) ld.down_range(l, 0, 3);
            barrier();  // B8
            if constexpr (ROWS == 1) {
                if (!last) {
                    if (late_pf) ld.prefetch(l + 1, 1, pf);
                    ld.o_range(l + 1, 0, 3);
                }
            } else {
                ld.down_range(l, 3, 3);
            }
            if (last) wait_vmcnt<0>();
            else wait_vmcnt<ROWS == 1 ? kAfterGu : kPairAfterGu>();  // gate/up(l), post-attention norm weights
            barrier();  // B9
            if (!last) {
                if constexpr (ROWS == 1) ld.o_range(l + 1, 3, 1);
                ld.qkv_range(l + 1, 7, 3);
            }
            barrier();  // B10
            if (last) wait_vmcnt<0>();
            else wait_vmcnt<ROWS == 1 ? kAfterDown : kPairAfterDown>();  // down(l)
            barrier();  // B11
            barrier();  // B12: down(l) is used
            if constexpr (ROWS == 2) {
                if (!last) ld.o_range(l + 1, 0, kLoadsO);
            }
            barrier();  // B13
        }
        return;
    }

    // Compute waves.
    const int pos = a.pos;
    int n[ROWS], active[ROWS];
#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        n[q] = pos + 1 + q;
        active[q] = min((n[q] + 63) >> 6, 32);
    }
    const bool mine = FULL || s < active[ROWS - 1];
    const size_t head_base = size_t(g) * a.context;
    const int hq = s & 1, h = 2 * g + hq, rb = s >> 1;
    const unsigned spins = a.spins;
    bool ok = true;
    auto pass_base = [&](int p) { return FULL ? 64 * p : 64 * (s + 32 * p); };

    // Layer 0 starts from the embedding rows (engine/core.cpp:354-356).
#pragma unroll
    for (int q = 0; q < ROWS; ++q) {
        if (tid < 256) {
            const uint2 e = *reinterpret_cast<const uint2*>(a.embed + size_t(a.token[q]) * kHidden + 4 * tid);
            *reinterpret_cast<float4*>(&m.r[q].x[4 * tid]) =
                make_float4(h2f(e.x & 0xffffu), h2f(e.x >> 16), h2f(e.y & 0xffffu), h2f(e.y >> 16));
        }
        if (wave == 0) {
            m.rope[q][0][lane] = a.cosines[size_t(pos + q) * 64 + lane];
            m.rope[q][1][lane] = a.sines[size_t(pos + q) * 64 + lane];
        }
    }
    // K/V rows of this workgroup's passes in layer `layer` from the cache
    // (the rows at pos and pos + 1 come from LDS; positions past them, and
    // all of an inactive workgroup's, read row 0).
    auto load_kv = [&](int layer, int t_id, u32x4 (&kreg)[PASSES][2], u32x4 (&vreg)[PASSES][2]) {
        const TokenLayer& KL = a.layers[layer];
        const uint16_t* kv_values = KL.keys + size_t(kKVHeads) * a.context * 128;
        const int kl = t_id & 63, kw = t_id >> 6, kc = t_id & 7, kg = t_id >> 3;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int t = pass_base(p) + kg;
            const int tl = mine && t < pos ? t : 0;
            const global_u32x4* kp = global_rows(KL.keys + (head_base + tl) * 128);
            kreg[p][0] = kp[kc];
            kreg[p][1] = kp[kc + 8];
        }
#pragma unroll
        for (int p = 0; p < PASSES; ++p)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const int t = pass_base(p) + 8 * kw + 4 * hf + (kl >> 4);
                const int tl = mine && t < pos ? t : 0;
                vreg[p][hf] = global_rows(kv_values + (head_base + tl) * 128)[kl & 15];
            }
    };
    // One row with up to 3 passes: each layer's K/V loads are issued in the
    // last interval of the layer before (the first layer's here): by the
    // waves that do not fold as it starts, by the folding waves after their
    // fold, so that they land while the fold is gathered and under the norm
    // instead of holding up the norm waves at the layer start (token kernel
    // 329 -> 325 us at 109 positions, 477 -> 457 at 4034, the same bits);
    // more passes, or two rows, would spill, and load at the layer start.
    constexpr bool kEarlyKv = ROWS == 1 && PASSES <= 3;
    u32x4 knext[PASSES][2], vnext[PASSES][2];
    if constexpr (kEarlyKv) load_kv(0, int(threadIdx.x), knext, vnext);
    barrier();  // B0

    for (int l = 0; l < L; ++l) {
        const TokenLayer& TL = a.layers[l];
        uint16_t* const values = TL.keys + size_t(kKVHeads) * a.context * 128;
        const uint32_t tag = a.tag + uint32_t(l);
        // The thread index, opaque to the compiler in each iteration:
        // otherwise it hoists every per-thread address out of the layer loop
        // and spills them.
        int tid = threadIdx.x;
        asm volatile("" : "+v"(tid));
        uint64_t* W[ROWS];
#pragma unroll
        for (int q = 0; q < ROWS; ++q) W[q] = a.words + size_t(q) * kTokWords;
        const int lane = tid & 63, wave = tid >> 6;
        const int j = tid & 127, c = tid & 7, grp = tid >> 3;
        const int vsub = lane >> 4, vcg = lane & 15;
        const int orow_local = tid >> 3, opart_id = tid & 7;
        const int orow = 64 * rb + orow_local;
        const int gu_tile = 96 * g + 3 * s + min(wave, 2);
        const int down_tile = 4 * s + wave;

        // ---- attention block (engine/core.cpp:384-406, 606-626) ----
        u32x4 kreg[PASSES][2], vreg[PASSES][2];
        if constexpr (kEarlyKv) {
#pragma unroll
            for (int p = 0; p < PASSES; ++p)
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    kreg[p][e] = knext[p][e];
                    vreg[p][e] = vnext[p][e];
                }
        } else {
#pragma unroll
            for (int p = 0; p < PASSES; ++p) {
                const int t = pass_base(p) + grp;
                const int tl = mine && t < pos ? t : 0;
                const global_u32x4* kp = global_rows(TL.keys + (head_base + tl) * 128);
                kreg[p][0] = kp[c];
                kreg[p][1] = kp[c + 8];
            }
#pragma unroll
            for (int p = 0; p < PASSES; ++p)
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const int t = pass_base(p) + 8 * wave + 4 * hf + vsub;
                    const int tl = mine && t < pos ? t : 0;
                    vreg[p][hf] = global_rows(values + (head_base + tl) * 128)[vcg];
                }
        }
        // RMSNorm of the residual: waves 0-3 hold entries 4 tid .. 4 tid + 3.
        float v[ROWS][4];
        if (tid < 256) {
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                const float4 f = *reinterpret_cast<const float4*>(&m.r[q].x[4 * tid]);
                v[q][0] = f.x; v[q][1] = f.y; v[q][2] = f.z; v[q][3] = f.w;
                norm_sums(v[q], m.r[q].red, wave, lane);
            }
        }
        barrier();  // B1
        if (tid < 256) {
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                const double* red = m.r[q].red;
                const float sum = static_cast<float>(((red[0] + red[1]) + red[2]) + red[3]);
                const float inv = 1.0f / __builtin_sqrtf(sum / static_cast<float>(kHidden) + 1e-6f);
                float* xs = reinterpret_cast<float*>(m.r[q].u.n.xs4);
#pragma unroll
                for (int k = 0; k < 4; ++k) xs[xperm(4 * tid + k)] = (v[q][k] * inv) * m.nin[4 * tid + k];
            }
        }
        barrier();  // B2

        // QKV rows (the reference's chain-ordered dot): wave t < 2 runs tile
        // li = 2 s + t over all 16 column blocks and posts its 8 rows.
        if (wave < 2) {
            const float4* x4[ROWS];
#pragma unroll
            for (int q = 0; q < ROWS; ++q) x4[q] = m.r[q].u.n.xs4 + 2 * c;
            float acc[ROWS];
            lds_chain<16, ROWS>(reinterpret_cast<const u32x4*>(m.wq() + 16384 * wave) + lane, x4, acc);
            const int li = 2 * s + wave;
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                const float y = combine_chains(acc[q]);
                if (c == 0 && !(q == 0 && l == 0 && int(blockIdx.x) == a.withhold))
                    exchange_put(W[q] + kTokQkvOffset + g * 512 + 8 * li + (lane >> 3), y, tag);
            }
        }
        // Wave w < 4 takes head-group rows 128 w + lane and 128 w + 64 + lane
        // (q0, q1, k, v) of each row: QK-norm (engine/core.cpp:397-398) and
        // rotate-half RoPE (216-218) inside the wave; the workgroup holding
        // the pass of a row's position writes its new K/V row (403-406).
        if (tid < 256) {
            const uint64_t* words[2 * ROWS];
            float got[2 * ROWS];
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                words[2 * q] = W[q] + kTokQkvOffset + g * 512 + 128 * wave + lane;
                words[2 * q + 1] = W[q] + kTokQkvOffset + g * 512 + 128 * wave + 64 + lane;
                got[2 * q] = got[2 * q + 1] = 0.f;
            }
            if (ok) ok = tok_gather<2 * ROWS, kStaggerXcd>(words, tag, got, (1u << (2 * ROWS)) - 1, a.stall, spins);
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                const int at = pos + q;
                const float x0 = got[2 * q], x1 = got[2 * q + 1];
                const bool owner = ((at >> 6) & 31) == s;
                auto& R = m.r[q];
                if (wave < 3) {
                    const float* hw = m.nqk + (wave == 2 ? kHeadDim : 0);
                    const float sq0 = x0 * x0, sq1 = x1 * x1;
                    const double lo = wave_sum(static_cast<double>(sq0)), hi = wave_sum(static_cast<double>(sq1));
                    const float sum = static_cast<float>(lo + hi);
                    const float inv = 1.0f / __builtin_sqrtf(sum / 128.0f + 1e-6f);
                    const float n0 = (x0 * inv) * hw[lane], n1 = (x1 * inv) * hw[lane + 64];
                    const float rc = m.rope[q][0][lane], rs = m.rope[q][1][lane];
                    const float r0 = n0 * rc - n1 * rs, r1 = n1 * rc + n0 * rs;
                    if (wave < 2) {
                        R.qp[wave][kperm(lane)] = r0;
                        R.qp[wave][kperm(lane + 64)] = r1;
                    } else {
                        const uint16_t b0 = f2h(r0), b1 = f2h(r1);
                        R.kcur[kperm(lane)] = b0;
                        R.kcur[kperm(lane + 64)] = b1;
                        if (owner) {
                            global_halves(TL.keys)[(head_base + at) * 128 + kperm(lane)] = b0;
                            global_halves(TL.keys)[(head_base + at) * 128 + kperm(lane + 64)] = b1;
                        }
                    }
                } else {
                    const uint16_t b0 = f2h(x0), b1 = f2h(x1);
                    R.vcur[lane] = b0;
                    R.vcur[lane + 64] = b1;
                    if (owner) {
                        global_halves(values)[(head_base + at) * 128 + lane] = b0;
                        global_halves(values)[(head_base + at) * 128 + lane + 64] = b1;
                    }
                }
            }
        }
        barrier();  // B3

        // Scores (engine/core.cpp:606-612): the 8 lanes of a position run its
        // chains; each head's maximum over this workgroup's positions.
        float s0[ROWS][PASSES], s1[ROWS][PASSES];
        float m0[ROWS], m1[ROWS];
#pragma unroll
        for (int q = 0; q < ROWS; ++q) m0[q] = m1[q] = -INFINITY;
        if (mine) {
#pragma unroll
            for (int p = 0; p < PASSES; ++p) {
                const int t = pass_base(p) + grp;
                uint32_t kw[8];
                if (t == pos) {
                    key_pieces_lds(m.r[0].kcur, c, kw);
                } else if (ROWS == 2 && t == pos + 1) {
                    key_pieces_lds(m.r[ROWS - 1].kcur, c, kw);
                } else {
                    kw[0] = kreg[p][0].x; kw[1] = kreg[p][0].y; kw[2] = kreg[p][0].z; kw[3] = kreg[p][0].w;
                    kw[4] = kreg[p][1].x; kw[5] = kreg[p][1].y; kw[6] = kreg[p][1].z; kw[7] = kreg[p][1].w;
                }
#pragma unroll
                for (int q = 0; q < ROWS; ++q) {
                    if constexpr (FULL) {
                        const float d0 = combine_chains(key_chain(m.r[q].qp[hq], c, kw, 0.f)) * a.scale;
                        s0[q][p] = t < n[q] ? d0 : -INFINITY;
                        m0[q] = fmaxf(m0[q], s0[q][p]);
                    } else {
                        const float d0 = combine_chains(key_chain(m.r[q].qp[0], c, kw, 0.f)) * a.scale;
                        const float d1 = combine_chains(key_chain(m.r[q].qp[1], c, kw, 0.f)) * a.scale;
                        s0[q][p] = t < n[q] ? d0 : -INFINITY;
                        s1[q][p] = t < n[q] ? d1 : -INFINITY;
                        m0[q] = fmaxf(m0[q], s0[q][p]);
                        m1[q] = fmaxf(m1[q], s1[q][p]);
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                m0[q] = fmaxf(m0[q], xor_lanes<8>(m0[q]));
                m0[q] = fmaxf(m0[q], xor_lanes<16>(m0[q]));
                m0[q] = fmaxf(m0[q], xor_lanes<32>(m0[q]));
                if constexpr (!FULL) {
                    m1[q] = fmaxf(m1[q], xor_lanes<8>(m1[q]));
                    m1[q] = fmaxf(m1[q], xor_lanes<16>(m1[q]));
                    m1[q] = fmaxf(m1[q], xor_lanes<32>(m1[q]));
                }
                if (lane == 0) {
                    m.r[q].wmax[wave][0] = m0[q];
                    m.r[q].wmax[wave][1] = m1[q];
                }
            }
        }
        barrier();  // B4

        // Probabilities and P.V (engine/core.cpp:613-624): one maximum per
        // head over the workgroup (so the waves' sums add without
        // rescaling), each wave's sums over its positions.
        if (mine) {
            float l0[ROWS], l1[ROWS];
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                auto& R = m.r[q];
                m0[q] = R.wmax[0][0];
                m1[q] = R.wmax[0][1];
#pragma unroll
                for (int w = 1; w < 8; ++w) {
                    m0[q] = fmaxf(m0[q], R.wmax[w][0]);
                    m1[q] = fmaxf(m1[q], R.wmax[w][1]);
                }
                l0[q] = l1[q] = 0.f;
#pragma unroll
                for (int p = 0; p < PASSES; ++p) {
                    const int t = pass_base(p) + grp;
                    const float p0 = t < n[q] ? expf(s0[q][p] - m0[q]) : 0.f;
                    l0[q] += p0;
                    if constexpr (FULL) {
                        if (c == 0) R.v.prob[t >> 7][t & 127] = p0;
                    } else {
                        const float p1 = t < n[q] ? expf(s1[q][p] - m1[q]) : 0.f;
                        l1[q] += p1;
                        if (c == 0) {
                            R.v.prob[0][p * 64 + grp] = p0;
                            R.v.prob[1][p * 64 + grp] = p1;
                        }
                    }
                }
                l0[q] += xor_lanes<8>(l0[q]);
                l0[q] += xor_lanes<16>(l0[q]);
                l0[q] += xor_lanes<32>(l0[q]);
                if constexpr (!FULL) {
                    l1[q] += xor_lanes<8>(l1[q]);
                    l1[q] += xor_lanes<16>(l1[q]);
                    l1[q] += xor_lanes<32>(l1[q]);
                }
            }
            // prob of this wave's positions is written and read by this wave only.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            constexpr int kHeads = FULL ? 1 : 2;
            float acc[ROWS][kHeads][8];
#pragma unroll
            for (int q = 0; q < ROWS; ++q)
#pragma unroll
                for (int hh = 0; hh < kHeads; ++hh)
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[q][hh][i] = 0.f;
#pragma unroll
            for (int p = 0; p < PASSES; ++p)
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const int t = pass_base(p) + 8 * wave + 4 * hf + vsub;
                    if (t < n[ROWS - 1]) {
                        uint32_t vw[4];
                        if (t == pos) {
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                vw[i] = uint32_t(m.r[0].vcur[vcg * 8 + 2 * i]) |
                                        (uint32_t(m.r[0].vcur[vcg * 8 + 2 * i + 1]) << 16);
                        } else if (ROWS == 2 && t == pos + 1) {
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                vw[i] = uint32_t(m.r[ROWS - 1].vcur[vcg * 8 + 2 * i]) |
                                        (uint32_t(m.r[ROWS - 1].vcur[vcg * 8 + 2 * i + 1]) << 16);
                        } else {
                            vw[0] = vreg[p][hf].x; vw[1] = vreg[p][hf].y; vw[2] = vreg[p][hf].z; vw[3] = vreg[p][hf].w;
                        }
#pragma unroll
                        for (int q = 0; q < ROWS; ++q) {
                            if (t < n[q]) {
                                if constexpr (FULL) {
                                    const float p0 = m.r[q].v.prob[t >> 7][t & 127];
#pragma unroll
                                    for (int i = 0; i < 4; ++i) {
                                        acc[q][0][2 * i] = __builtin_fmaf(h2f(vw[i] & 0xffffu), p0, acc[q][0][2 * i]);
                                        acc[q][0][2 * i + 1] = __builtin_fmaf(h2f(vw[i] >> 16), p0, acc[q][0][2 * i + 1]);
                                    }
                                } else {
                                    const int tl = p * 64 + 8 * wave + 4 * hf + vsub;
                                    const float p0 = m.r[q].v.prob[0][tl], p1 = m.r[q].v.prob[1][tl];
#pragma unroll
                                    for (int i = 0; i < 4; ++i) {
                                        const float v0 = h2f(vw[i] & 0xffffu), v1 = h2f(vw[i] >> 16);
                                        acc[q][0][2 * i] = __builtin_fmaf(v0, p0, acc[q][0][2 * i]);
                                        acc[q][0][2 * i + 1] = __builtin_fmaf(v1, p0, acc[q][0][2 * i + 1]);
                                        acc[q][kHeads - 1][2 * i] = __builtin_fmaf(v0, p1, acc[q][kHeads - 1][2 * i]);
                                        acc[q][kHeads - 1][2 * i + 1] =
                                            __builtin_fmaf(v1, p1, acc[q][kHeads - 1][2 * i + 1]);
                                    }
                                }
                            }
                        }
                    }
                }
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
#pragma unroll
                for (int hh = 0; hh < kHeads; ++hh)
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        acc[q][hh][i] += xor_lanes<16>(acc[q][hh][i]);
                        acc[q][hh][i] += xor_lanes<32>(acc[q][hh][i]);
                    }
                if (vsub == 0) {
#pragma unroll
                    for (int hh = 0; hh < kHeads; ++hh)
#pragma unroll
                        for (int i = 0; i < 8; i += 4)
                            *reinterpret_cast<float4*>(&m.r[q].u.opart[wave][hh][vcg * 8 + i]) =
                                make_float4(acc[q][hh][i], acc[q][hh][i + 1], acc[q][hh][i + 2], acc[q][hh][i + 3]);
                }
                if (lane == 0) {
                    m.r[q].wsum[wave][0] = l0[q];
                    m.r[q].wsum[wave][1] = l1[q];
                }
            }
        }
        barrier();  // B5

        if constexpr (FULL) {
            if (tid < 128 * ROWS) {  // the 8 waves' sums in a fixed tree
                auto& R = m.r[tid >> 7];
                const float o = ((R.u.opart[0][0][j] + R.u.opart[1][0][j]) + (R.u.opart[2][0][j] + R.u.opart[3][0][j])) +
                                ((R.u.opart[4][0][j] + R.u.opart[5][0][j]) + (R.u.opart[6][0][j] + R.u.opart[7][0][j]));
                const float lsum = ((R.wsum[0][0] + R.wsum[1][0]) + (R.wsum[2][0] + R.wsum[3][0])) +
                                   ((R.wsum[4][0] + R.wsum[5][0]) + (R.wsum[6][0] + R.wsum[7][0]));
                R.att[j] = o / lsum;
            }
            barrier();  // B6
        } else {
            // Each workgroup with positions writes (output, max, sum) of both
            // heads as plain floats and, once a wave's stores are in the
            // XCD's L2, posts that wave's flag; workgroup (g, s) polls the
            // flags of the active partials, reads them in one pass and merges
            // head h (4 groups of 8 against their own maximum, then
            // combined). Polling the 32 x 130 tagged words themselves cost
            // 2-3 us per layer of rounds that re-read all of them.
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                if (s < active[q] && tid < 256) {
                    auto& R = m.r[q];
                    const int hh = tid >> 7;
                    const float o = ((R.u.opart[0][hh][j] + R.u.opart[1][hh][j]) +
                                     (R.u.opart[2][hh][j] + R.u.opart[3][hh][j])) +
                                    ((R.u.opart[4][hh][j] + R.u.opart[5][hh][j]) +
                                     (R.u.opart[6][hh][j] + R.u.opart[7][hh][j]));
                    const float lsum = ((R.wsum[0][hh] + R.wsum[1][hh]) + (R.wsum[2][hh] + R.wsum[3][hh])) +
                                       ((R.wsum[4][hh] + R.wsum[5][hh]) + (R.wsum[6][hh] + R.wsum[7][hh]));
                    float* pay = reinterpret_cast<float*>(W[q] + kTokPartOffset) + ((size_t(g) * 32 + s) * 2 + hh) * kXPart;
                    pay[j] = o;
                    if (j == 0) {
                        pay[128] = hh ? m1[q] : m0[q];
                        pay[129] = lsum;
                    }
                }
            }
            // The floats of this wave are in the XCD's L2 once its stores
            // have completed; then its flag tells the readers.
            if (tid < 256) {
                __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0)
#pragma unroll
                for (int q = 0; q < ROWS; ++q)
                    if (s < active[q] && lane == 0)
                        exchange_put(W[q] + kTokPartFlagOffset + (size_t(g) * 32 + s) * 4 + wave, 0.f, tag);
            }
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                const int gq = tid >> 7;
                float mv[8], lv[8], ovl[8];
                {
                    // Lanes 0-15 of each wave poll the flags of the group's
                    // 8 partials (the two posting waves of head hq); then
                    // every lane reads its output entry of the 8 partials,
                    // lane k < 8 the maximum of partial k and lane 8 + k its
                    // sum, which every lane then reads from those lanes.
                    const int kf = lane & 7;
                    const uint64_t* const flag[1] = {W[q] + kTokPartFlagOffset + (size_t(g) * 32 + 8 * gq + kf) * 4 +
                                                     2 * hq + ((lane >> 3) & 1)};
                    float unused[1] = {0.f};
                    const unsigned want = lane < 16 && 8 * gq + kf < active[q] ? 1u : 0u;
                    if (ok) ok = tok_gather<1, kStaggerXcd>(flag, tag, unused, want, a.stall, spins);
                    const uint32_t* pay = reinterpret_cast<const uint32_t*>(W[q] + kTokPartOffset) +
                                          (size_t(g) * 32 + 8 * gq) * 2 * kXPart + hq * kXPart;
                    uint32_t raw[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k)
                        raw[k] = __hip_atomic_load(pay + k * 2 * kXPart + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    const uint32_t ml = __hip_atomic_load(pay + kf * 2 * kXPart + (lane < 8 ? 128 : 129),
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        ovl[k] = 8 * gq + k < active[q] ? __uint_as_float(raw[k]) : 0.f;
                        mv[k] = 8 * gq + k < active[q] ? __uint_as_float(__shfl(ml, k)) : -INFINITY;
                        lv[k] = __uint_as_float(__shfl(ml, 8 + k));
                    }
                }
                float mx = -INFINITY;
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    if (8 * gq + k < active[q]) mx = fmaxf(mx, mv[k]);
                float lsum = 0.f, o = 0.f;
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    if (8 * gq + k < active[q]) {
                        const float w = expf(mv[k] - mx);
                        lsum += w * lv[k];
                        o += w * ovl[k];
                    }
                auto& R = m.r[q];
                if (j == 0) {
                    R.gm[gq] = mx;
                    R.gl[gq] = lsum;
                }
                R.go[gq][j] = o;
            }
            barrier();  // B6
            if (tid < 128 * ROWS) {
                auto& R = m.r[tid >> 7];
                float m2 = R.gm[0];
#pragma unroll
                for (int gq = 1; gq < 4; ++gq) m2 = fmaxf(m2, R.gm[gq]);
                float lt = 0.f, ot = 0.f;
#pragma unroll
                for (int gq = 0; gq < 4; ++gq)
                    if (R.gm[gq] != -INFINITY) {  // a group without partials adds nothing
                        const float w = expf(R.gm[gq] - m2);
                        lt += w * R.gl[gq];
                        ot += w * R.go[gq][j];
                    }
                R.att[j] = ot / lt;
            }
            barrier();  // B6b
        }

        // O rows 64 rb .. + 63 against head h's attention output of each row;
        // each row's partial goes to the fold across XCDs.
        {
            const u32x4* wrow = reinterpret_cast<const u32x4*>(m.wo() + 256 * orow_local) + opart_id;
            const u32x4 w0 = wrow[0], w1 = wrow[8];
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                const float4* at4 = reinterpret_cast<const float4*>(m.r[q].att) + 2 * opart_id;
                float y = chain8(0.f, w0, at4[0], at4[1]);
                y = chain8(y, w1, at4[16], at4[17]);
                y += xor_lanes<1>(y);
                y += xor_lanes<2>(y);
                y += xor_lanes<4>(y);
                if (opart_id == 0) exchange_put_through(W[q] + kTokOCrossOffset + size_t(h) * kHidden + orow, y, tag);
            }
        }
        barrier();  // B7

        // Fold 1 (engine/core.cpp:626): wave q forms rows 32 s .. + 31 of row
        // q's x + the 16 head partials (lane = row, half: heads 8 half .. + 7;
        // the tree of the two-kernel path) and posts them inside the XCD;
        // every thread then gathers two of the XCD's 1024 sums of each row.
        if (wave < ROWS) {
            const int row = 32 * s + (lane >> 1), half = lane & 1;
            const uint64_t* base = W[wave] + kTokOCrossOffset + size_t(8 * half) * kHidden + row;
            const uint64_t* const words[8] = {base, base + kHidden, base + 2 * kHidden, base + 3 * kHidden,
                                              base + 4 * kHidden, base + 5 * kHidden, base + 6 * kHidden,
                                              base + 7 * kHidden};
            float p8[8] = {};
            if (ok) ok = tok_gather<8, kStaggerCross>(words, tag, p8, 0xffu, a.stall, spins);
            const float part = ((p8[0] + p8[1]) + (p8[2] + p8[3])) + ((p8[4] + p8[5]) + (p8[6] + p8[7]));
            const float other = xor_lanes<1>(part);
            const float lo = half ? other : part, hi = half ? part : other;
            const float xm = m.r[wave].x[row] + (lo + hi);
            if (half == 0) exchange_put(W[wave] + kTokXmOffset + g * kHidden + row, xm, tag);
        }
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            float x0 = 0.f, x1 = 0.f;
            if (ok) ok = tok_get2(W[q] + kTokXmOffset + g * kHidden + 2 * tid, tag, x0, x1, a.stall, spins);
            m.r[q].u.n.xm[2 * tid] = x0;
            m.r[q].u.n.xm[2 * tid + 1] = x1;
        }
        barrier();  // B8

        // ---- FFN block (engine/core.cpp:627-641) ----
        if (tid < 256) {
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                const float4 f = *reinterpret_cast<const float4*>(&m.r[q].u.n.xm[4 * tid]);
                v[q][0] = f.x; v[q][1] = f.y; v[q][2] = f.z; v[q][3] = f.w;
                norm_sums(v[q], m.r[q].red, wave, lane);
            }
        }
        barrier();  // B9
        if (tid < 256) {
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                double total = 0.0;
#pragma unroll
                for (int i = 0; i < 4; ++i) total += m.r[q].red[i];
                const float sum = static_cast<float>(total);
                const float inv = 1.0f / __builtin_sqrtf(sum / static_cast<float>(kHidden) + 1e-6f);
                float* xs = reinterpret_cast<float*>(m.r[q].u.n.xs4);
#pragma unroll
                for (int k = 0; k < 4; ++k) xs[xperm(4 * tid + k)] = (v[q][k] * inv) * m.npost[4 * tid + k];
            }
        }
        barrier();  // B10

        // Gate/up tile 96 g + 3 s + w (waves 0-2; rows 0-3 gate, 4-7 up),
        // SwiGLU (engine/core.cpp:636-639), the XCD's 384 activations
        // exchanged.
        if (wave < 3) {
            const float4* x4[ROWS];
#pragma unroll
            for (int q = 0; q < ROWS; ++q) x4[q] = m.r[q].u.n.xs4 + 2 * c;
            float acc[ROWS];
            lds_chain<16, ROWS>(reinterpret_cast<const u32x4*>(m.wgu() + 16384 * wave) + lane, x4, acc);
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                const float y = combine_chains(acc[q]);
                const float up = __shfl(y, (lane + 32) & 63);
                if (lane < 32 && c == 0) {
                    const float gate = y;
                    const float half_gate = gate * 0.5f;
                    const float t = tanhf(half_gate);
                    exchange_put(W[q] + kTokActOffset + 4 * gu_tile + (lane >> 3), gate * (0.5f + 0.5f * t) * up, tag);
                }
            }
        }
        if (tid < kFfnSlice / 2) {
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                float a0 = 0.f, a1 = 0.f;
                if (ok) ok = tok_get2(W[q] + kTokActOffset + kFfnSlice * g + 2 * tid, tag, a0, a1, a.stall, spins);
                float* as = reinterpret_cast<float*>(m.r[q].v.as4);
                as[xperm(2 * tid)] = a0;
                as[xperm(2 * tid + 1)] = a1;
            }
        }
        barrier();  // B11

        // Down tile 4 s + w (waves 0-3) over the slice's 384 columns; the
        // rows go to the fold across XCDs.
        if (wave < 4) {
            const float4* x4[ROWS];
#pragma unroll
            for (int q = 0; q < ROWS; ++q) x4[q] = m.r[q].v.as4 + 2 * c;
            float acc[ROWS];
            lds_chain<6, ROWS>(reinterpret_cast<const u32x4*>(m.wdn() + 6144 * wave) + lane, x4, acc);
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                const float y = combine_chains(acc[q]);
                if (c == 0)
                    exchange_put_through(W[q] + kTokDCrossOffset + size_t(g) * kHidden + 8 * down_tile + (lane >> 3), y,
                                         tag);
            }
        }
        barrier();  // B12

        // Fold 2: wave q forms rows 32 s .. + 31 of row q's xm + the 8 down
        // slices (the tree of the two-kernel path), posted inside the XCD;
        // every thread gathers two entries of each row's next residual.
        // The waves that do not fold issue the next layer's K/V loads first
        // (their polls cannot succeed before the folds are posted anyway);
        // the folding waves after their fold.
        if constexpr (kEarlyKv) {
            if (l + 1 < L && wave >= ROWS) load_kv(l + 1, tid, knext, vnext);
        }
        if (wave < ROWS && lane < 32) {
            const int row = 32 * s + lane;
            const uint64_t* base = W[wave] + kTokDCrossOffset + row;
            const uint64_t* const words[8] = {base, base + kHidden, base + 2 * kHidden, base + 3 * kHidden,
                                              base + 4 * kHidden, base + 5 * kHidden, base + 6 * kHidden,
                                              base + 7 * kHidden};
            float d8[8] = {};
            if (ok) ok = tok_gather<8, kStaggerCross>(words, tag, d8, 0xffu, a.stall, spins);
            exchange_put(W[wave] + kTokXOffset + g * kHidden + row, fold_slices(m.r[wave].u.n.xm[row], d8), tag);
        }
        if constexpr (kEarlyKv) {
            if (l + 1 < L && wave < ROWS) load_kv(l + 1, tid, knext, vnext);
        }
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            float x0 = 0.f, x1 = 0.f;
            if (ok) ok = tok_get2(W[q] + kTokXOffset + g * kHidden + 2 * tid, tag, x0, x1, a.stall, spins);
            m.r[q].x[2 * tid] = x0;
            m.r[q].x[2 * tid + 1] = x1;
        }
        barrier();  // B13
    }

    if (blockIdx.x == 0) {
        int t = threadIdx.x;  // opaque: keeps the address from being formed (and held) before the loop
        asm volatile("" : "+v"(t));
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            a.x_out[q * kHidden + 2 * t] = m.r[q].x[2 * t];
            a.x_out[q * kHidden + 2 * t + 1] = m.r[q].x[2 * t + 1];
        }
    }
}

}  // namespace

bool token_pair_supported(int pos) {
    const int n0 = pos + 1, n1 = pos + 2;
    return (n0 <= 256) == (n1 <= 256);  // the same attention form for both rows
}

void launch_token_layers(const TokenLaunch& t, hipStream_t stream) {
    require(t.layer_count >= 1 && t.layer_count <= kLayers, "token kernel: bad layer table");
    require(t.rows == 1 || t.rows == 2, "token kernel: one or two rows");
    require(t.pos >= 0 && t.pos + t.rows <= t.context && t.context <= kMaxContext,
            "token kernel: position outside the cache");
    for (int q = 0; q < t.rows; ++q) require(t.token[q] >= 0 && t.token[q] < kVocab, "token kernel: token out of range");
    require(t.rows == 1 || token_pair_supported(t.pos), "token kernel: the two rows take different attention forms");
    require(t.tag != 0 && uint64_t(t.tag) + uint64_t(t.layer_count) - 1 <= 0xFFFFFFFFull,
            "token kernel: tags must be nonzero and not wrap");
    require(t.spins >= 1, "token kernel: poll limit must be positive");
    const int passes = (t.pos + t.rows + 63) / 64;  // of the last row
    auto go = [&](auto rows_tag) {
        constexpr int R = decltype(rows_tag)::value;
        auto launch = [&](auto kernel) { kernel<<<256, kTokenThreads, 0, stream>>>(t); };
        switch (passes <= 4 ? passes : 0) {
            case 1: launch(token_kernel<1, true, R>); break;
            case 2: launch(token_kernel<2, true, R>); break;
            case 3: launch(token_kernel<3, true, R>); break;
            case 4: launch(token_kernel<4, true, R>); break;
            default:
                if (passes > 32) launch(token_kernel<2, false, R>);
                else launch(token_kernel<1, false, R>);
        }
    };
    if (t.rows == 1) go(std::integral_constant<int, 1>{});
    else go(std::integral_constant<int, 2>{});
}

}  // namespace qwen_hip
