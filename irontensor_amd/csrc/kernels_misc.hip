// Row and elementwise kernels around the contractions: zero-fill, BF16 conversion, the attention
// softmax (forward and backward) with causal awareness.
//
// Semantics follow src/shaders/softmax.metal:14-45 (max-subtracted exp, sum, divide),
// src/shaders/backward/softmax.metal:22-45 (y * (g - dot(g, y))), the causal -inf mask of
// src/shaders/attention.metal:186-207 and the conversions of src/shaders/bf16_ops.metal:339-357.
#include <cmath>

#include "internal.hpp"
#include "mfma.hpp"

namespace it {
namespace {

__global__ void zero_bytes(char *dst, size_t n16, size_t bytes) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t v = i; v < n16; v += stride) ((u32x4 *)dst)[v] = u32x4{0u, 0u, 0u, 0u};
    for (size_t b = n16 * 16 + i; b < bytes; b += stride) dst[b] = 0;
}

// Conversions move 8 elements per thread and iteration (two 16-byte FP32 accesses, one 16-byte
// BF16 access) when both buffers are 16-byte aligned; the tail and unaligned buffers go element
// by element.
__global__ void f32_to_bf16_kernel(const float *src, uint16_t *dst, int64_t n, int64_t n8) {
    const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t v = i0; v < n8; v += stride) {
        const f32x4 a = ((const f32x4 *)src)[2 * v], b = ((const f32x4 *)src)[2 * v + 1];
        ((u32x4 *)dst)[v] = u32x4{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]),
                                  pack_bf16x2(b[2], b[3])};
    }
    for (int64_t i = n8 * 8 + i0; i < n; i += stride) dst[i] = f32_to_bf16_rne(src[i]);
}

__global__ void bf16_to_f32_kernel(const uint16_t *src, float *dst, int64_t n, int64_t n8) {
    const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t v = i0; v < n8; v += stride) {
        const u32x4 h = ((const u32x4 *)src)[v];
        f32x4 a, b;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            a[2 * e] = __uint_as_float(h[e] << 16);
            a[2 * e + 1] = __uint_as_float(h[e] & 0xffff0000u);
            b[2 * e] = __uint_as_float(h[2 + e] << 16);
            b[2 * e + 1] = __uint_as_float(h[2 + e] & 0xffff0000u);
        }
        ((f32x4 *)dst)[2 * v] = a;
        ((f32x4 *)dst)[2 * v + 1] = b;
    }
    for (int64_t i = n8 * 8 + i0; i < n; i += stride) dst[i] = bf16_to_f32(src[i]);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// One wave64 per row, 4 rows per 256-thread block.
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float *S, void *P, int p_bf16,
                                                           int64_t total_rows, int64_t rows,
                                                           int64_t cols, int causal,
                                                           int64_t causal_offset) {
    const int lane = threadIdx.x & 63;
    const int64_t grow = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (grow >= total_rows) return;
    const int64_t r = grow % rows;
    const float *s = S + grow * cols;
    int64_t valid = cols;
    if (causal) valid = max((int64_t)0, min(cols, r + causal_offset + 1));

    float mx = -INFINITY;
    for (int64_t c = lane; c < valid; c += 64) mx = fmaxf(mx, s[c]);
    mx = wave_max(mx);
    float sum = 0.f;
    for (int64_t c = lane; c < valid; c += 64) sum += expf(s[c] - mx);
    sum = wave_sum(sum);

    if (p_bf16) {
        uint16_t *p = (uint16_t *)P + grow * cols;
        for (int64_t c = lane; c < cols; c += 64)
            p[c] = c < valid ? f32_to_bf16_rne(expf(s[c] - mx) / sum) : (uint16_t)0;
    } else {
        float *p = (float *)P + grow * cols;
        for (int64_t c = lane; c < cols; c += 64) p[c] = c < valid ? expf(s[c] - mx) / sum : 0.f;
    }
}

__global__ __launch_bounds__(256) void softmax_backward_kernel(const float *dY, const void *Y,
                                                               int y_bf16, void *dX, int dx_bf16,
                                                               int64_t total_rows, int64_t rows,
                                                               int64_t cols, int causal) {
    const int lane = threadIdx.x & 63;
    const int64_t grow = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (grow >= total_rows) return;
    const int64_t r = grow % rows;
    const int64_t valid = causal ? min(cols, r + 1) : cols;
    const float *gy = dY + grow * cols;
    auto yv = [&](int64_t c) -> float {
        return y_bf16 ? bf16_to_f32(((const uint16_t *)Y)[grow * cols + c])
                      : ((const float *)Y)[grow * cols + c];
    };
    float dot = 0.f;
    for (int64_t c = lane; c < valid; c += 64) dot += gy[c] * yv(c);
    dot = wave_sum(dot);
    for (int64_t c = lane; c < cols; c += 64) {
        const float v = c < valid ? yv(c) * (gy[c] - dot) : 0.f;
        if (dx_bf16)
            ((uint16_t *)dX)[grow * cols + c] = f32_to_bf16_rne(v);
        else
            ((float *)dX)[grow * cols + c] = v;
    }
}

unsigned grid_for(int64_t n, int per_block) {
    int64_t b = (n + per_block - 1) / per_block;
    if (b < 1) b = 1;
    if (b > 65536) b = 65536;
    return (unsigned)b;
}

}  // namespace

it_status launch_zero(hipStream_t s, void *dst, size_t bytes) {
    const size_t n16 = ((uintptr_t)dst % 16 == 0) ? bytes / 16 : 0;
    hipLaunchKernelGGL(zero_bytes, dim3(grid_for((int64_t)(n16 ? n16 : bytes), 256)), dim3(256), 0, s,
                       (char *)dst, n16, bytes);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

static int64_t vec8_count(const void *a, const void *b, int64_t n) {
    return ((uintptr_t)a % 16 == 0 && (uintptr_t)b % 16 == 0) ? n / 8 : 0;
}

it_status launch_f32_to_bf16(hipStream_t s, const float *src, uint16_t *dst, int64_t n) {
    const int64_t n8 = vec8_count(src, dst, n);
    hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(grid_for(n8 ? n8 : n, 256)), dim3(256), 0, s, src, dst, n, n8);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_bf16_to_f32(hipStream_t s, const uint16_t *src, float *dst, int64_t n) {
    const int64_t n8 = vec8_count(src, dst, n);
    hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(grid_for(n8 ? n8 : n, 256)), dim3(256), 0, s, src, dst, n, n8);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_softmax_rows(hipStream_t s, const float *S, void *P, int p_bf16, int64_t batch,
                              int64_t rows, int64_t cols, int causal, int64_t causal_offset,
                              int64_t, int64_t) {
    const int64_t total = batch * rows;
    const int64_t blocks = (total + 3) / 4;
    if (blocks > 0x7fffffff) return fail(IT_ERR_DIMS, "softmax: too many rows");
    hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, s, S, P, p_bf16,
                       total, rows, cols, causal, causal_offset);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_softmax_backward(hipStream_t s, const float *dY, const void *Y, int y_bf16,
                                  void *dX, int dx_bf16, int64_t batch, int64_t rows,
                                  int64_t cols, int causal) {
    const int64_t total = batch * rows;
    const int64_t blocks = (total + 3) / 4;
    if (blocks > 0x7fffffff) return fail(IT_ERR_DIMS, "softmax_backward: too many rows");
    hipLaunchKernelGGL(softmax_backward_kernel, dim3((unsigned)blocks), dim3(256), 0, s, dY, Y,
                       y_bf16, dX, dx_bf16, total, rows, cols, causal);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

}  // namespace it
