// MFMA fragment helpers shared by the GEMM and attention kernels (gfx950).
//
// Fragment convention for the 16x16 MFMAs used here: lane l supplies row/column l % 16 and the
// k values of lane group g = l / 16:
//   FP32  v_mfma_f32_16x16x4_f32  : a 16-wide k chunk; group g holds k = 4g..4g+3 (one per MFMA)
//   BF16  v_mfma_f32_16x16x32_bf16: a 32-wide k chunk; group g holds 8 k values
// Both operands of a product use the same assignment, so every MFMA sums the right products.
// A 16x16 accumulator block holds, at lane l, column l % 16 and rows 4*(l/16) + r, r = 0..3.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace it {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// FP32 -> BF16 round-to-nearest-even on the hardware converter (v_cvt_pk_bf16_f32, two values per
// instruction); NaN stays a quiet NaN. Same results as the reference's round-half-even formula
// (src/precision.rs:24-29) for every non-NaN input, denormals included.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Logistic sigmoid 1 / (1 + e^-x) from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32; a
// few ulps): e^-x = 2^(-x log2 e). Large negative x gives 2^+inf = inf and a sigmoid of 0; NaN
// stays NaN.
__device__ __forceinline__ float sigmoid_fast(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// acc += a . b over one fragment chunk.
template <typename T>
__device__ __forceinline__ void mma16(f32x4 &acc, const u32x4 &a, const u32x4 &b) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[s]), __uint_as_float(b[s]),
                                                       acc, 0, 0, 0);
    } else {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
    }
}

}  // namespace it
