// Batched prefill (up to kPrefillRows rows per pass; engine/core.cpp:353-646, 712).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "qwen_common.hpp"

namespace qwen_hip {

// Natural row-major FP16 weights of one layer for the matrix-core GEMMs.
struct PrefillLayer {
    const uint16_t* qkv_n;     // [4096 x 1024]: q rows, k rows, v rows
    const uint16_t* o_n;       // [1024 x 2048]
    const uint16_t* gateup_n;  // [6144 x 1024]: 3072 gate rows then 3072 up rows
    const uint16_t* down_n;    // [1024 x 3072]
    const float* in_norm;
    const float* post_norm;
    const float* q_norm;
    const float* k_norm;
    uint16_t* keys;            // [8][context][128], chain-permuted rows
    uint16_t* values;          // [8][context][128]
};

// Activations of one batched pass (up to kPrefillRows rows each). GEMM
// inputs are kept as FP16 hi / lo planes (hi = fp16(v), lo = fp16(v - hi)).
struct PrefillScratch {
    float* x;           // [rows x 1024] residual stream (FP32)
    uint16_t* h_hi;     // [rows x 1024] normalized
    uint16_t* h_lo;
    float* qkv;         // [rows x 4096] (FP32; q heads normed and rotated)
    uint16_t* att_hi;   // [rows x 2048] attention output
    uint16_t* att_lo;
    uint16_t* act_hi;   // [rows x 3072] SwiGLU output
    uint16_t* act_lo;
    float* part;        // [4 x rows x 1024] K-split partial products of the O and down GEMMs
    // Range guard of the FP16 split (values from 65504 up do not fit FP16):
    int* row_exp;       // [rows] the normalized row was split as h * 2^-row_exp
    int* act_flag;      // [rows x 4] largest SwiGLU group exponent per K range of the down GEMM
    uint8_t* act_exp;   // [rows x 384] exponent of each group of 8 activations
};

// C[M x N] (+)= A[M x K] . W[N x K]^T; A FP32 split into FP16 hi + lo on the
// matrix cores; N a multiple of 128, K of 32.
void launch_gemm(const float* A, const uint16_t* W, float* C, int M, int N, int K, bool accumulate,
                 hipStream_t stream);

// launch_gemm without allocating: the FP16 operand planes live in a static
// device array of 2 x kStaticGemmElements halves (4 MiB per device, held until
// the process ends) shared by every call on a device, so calls that overlap
// on one device race. Enqueues on `stream` and returns (no synchronization).
inline constexpr size_t kStaticGemmElements = size_t(1) << 20;  // M x K limit
void launch_gemm_static(const float* A, const uint16_t* W, float* C, int M, int N, int K, bool accumulate,
                        hipStream_t stream);

// Gate/up projection with the SwiGLU epilogue of the prefill path: W holds
// N / 2 gate rows then N / 2 up rows (natural [N x K]); act[m][i] =
// SwiGLU(gate_i, up_i) of row m, written as FP16 hi / lo planes [M x N / 2]
// of act * 2^-act_exp[m][i / 8] (act_exp [M x N / 16]: 0 wherever the group
// of 8 fits FP16). N a multiple of 256, K of 64.
void launch_gemm_swiglu(const float* A, const uint16_t* W, uint16_t* act_hi, uint16_t* act_lo, uint8_t* act_exp,
                        int M, int N, int K, hipStream_t stream);

// Causal GQA attention of a prefill chunk (the layer step between the QKV
// and O GEMMs): queries from qkv [rows x 4096] (columns 0..2047, 16 heads),
// keys / values of positions 0 .. pos0 + rows - 1 from the [8][context][128]
// caches; output [rows x 2048] as FP16 hi + lo planes. rows in 1..4096 and
// pos0 + rows <= context.
void launch_attention_prefill(const float* qkv, const uint16_t* keys, const uint16_t* values, uint16_t* att_hi,
                              uint16_t* att_lo, int rows, int pos0, int context, hipStream_t stream);

// All 28 layers for `rows` prompt ids (device) at positions pos0..pos0+rows-1:
// K/V land in the cache, the final residual rows in s.x.
void launch_prefill_chunk(const PrefillLayer* layers, const uint16_t* embed, const int* ids_dev, int rows, int pos0,
                          const float* cosines, const float* sines, int context, const PrefillScratch& s,
                          hipStream_t stream);

}  // namespace qwen_hip
