// FP32 -> FP16 conversions of the device code, and the exact two-plane split
// hi = fp16(v), lo = fp16(v - hi) that carries FP32 activations into the FP16
// matrix-core products (v - hi is exact in FP32, so hi + lo holds v to 2^-22).
//
// Each converted value first passes an empty asm statement. Without it the
// compiler may fuse the multiply that produced the value into the conversion
// (v_fma_mixlo_f16: the exact product rounded once to FP16 instead of the FP32
// product rounded), and may do so for one use of a value and not for another:
// in a split the stored hi then differs from the hi that lo was computed
// against, and hi + lo is off by one FP16 ulp of hi.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace qwen_hip {

// v as an FP32 value the compiler cannot see through.
__device__ __forceinline__ float fp32_fixed(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ _Float16 to_half(float v) { return static_cast<_Float16>(fp32_fixed(v)); }

__device__ __forceinline__ uint16_t to_half_bits(float v) { return __builtin_bit_cast(uint16_t, to_half(v)); }

__device__ __forceinline__ void split_half(float v, _Float16& hi, _Float16& lo) {
    v = fp32_fixed(v);
    hi = static_cast<_Float16>(v);
    lo = to_half(v - static_cast<float>(hi));
}

// Range guard of the split. FP32 values from 65520 up round to an infinite
// FP16 hi (and a NaN lo), where the FP32 reference carries on. A group of
// values that feeds one dot product (a row of a GEMM operand, or a slice of
// one) is therefore split as v * 2^-e with e the smallest exponent that
// brings its largest magnitude below 65504, and the FP32 product is scaled
// back by 2^e: both scalings are exact, so the result is the unscaled
// product's, and e = 0 (no scaling at all) wherever the group fits, which
// leaves those bits unchanged. Non-finite maxima keep e = 0: they propagate
// as the reference's FP32 arithmetic would.
inline constexpr float kSplitLimit = 65504.f;

__device__ __forceinline__ int split_exponent(float max_abs) {
    if (!(max_abs >= kSplitLimit) || max_abs == __builtin_huge_valf()) return 0;
    // max_abs in [2^k, 2^(k+1)), k >= 15: v * 2^-(k - 14) lies below 2^15.
    return ((__builtin_bit_cast(int, max_abs) >> 23) - 127) - 14;
}

// 2^e as an FP32 value, e in [-126, 127].
__device__ __forceinline__ float pow2(int e) { return __builtin_bit_cast(float, (127 + e) << 23); }

}  // namespace qwen_hip
