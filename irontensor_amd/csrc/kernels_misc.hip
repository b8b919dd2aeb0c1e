// Row and elementwise kernels around the contractions: zero-fill, BF16 conversion, the attention
// softmax (forward and backward) with causal awareness, the batched transpose and causal mask of
// the reference's attention helpers, and the seeded normal fill used for synthetic inputs.
//
// Semantics follow src/shaders/softmax.metal:14-45 (max-subtracted exp, sum, divide),
// src/shaders/backward/softmax.metal:22-45 (y * (g - dot(g, y))), the causal -inf mask of
// src/shaders/attention.metal:186-207, transpose_3d_f32 (attention.metal:163-182) and the
// conversions of src/shaders/bf16_ops.metal:339-357.
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

// [batch, m, n] -> [batch, n, m] through a 64 x 64 LDS tile (pitch 65 floats: the column reads of
// the store phase hit 64 distinct banks). Each wave reads and writes 256 contiguous bytes per
// instruction; tiles are numbered (batch, tile row, tile column) over a 1-D grid.
__global__ __launch_bounds__(256) void transpose_3d_kernel(const float *in, float *out, int64_t m, int64_t n,
                                                          int64_t tiles_m, int64_t tiles_n) {
    __shared__ float tile[64][65];
    const int64_t t = blockIdx.x;
    const int64_t per_batch = tiles_m * tiles_n;
    const int64_t b = t / per_batch;
    const int64_t r = t - b * per_batch;
    const int64_t i0 = (r / tiles_n) * 64, j0 = (r % tiles_n) * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const float *src = in + b * m * n;
    float *dst = out + b * m * n;
    const bool full = i0 + 64 <= m && j0 + 64 <= n;
    if (full) {
#pragma unroll
        for (int k = 0; k < 16; ++k) tile[ty + 4 * k][tx] = src[(i0 + ty + 4 * k) * n + j0 + tx];
    } else {
        for (int k = 0; k < 16; ++k) {
            const int64_t i = i0 + ty + 4 * k, j = j0 + tx;
            if (i < m && j < n) tile[ty + 4 * k][tx] = src[i * n + j];
        }
    }
    __syncthreads();
    if (full) {
#pragma unroll
        for (int k = 0; k < 16; ++k) dst[(j0 + ty + 4 * k) * m + i0 + tx] = tile[tx][ty + 4 * k];
    } else {
        for (int k = 0; k < 16; ++k) {
            const int64_t j = j0 + ty + 4 * k, i = i0 + tx;
            if (i < m && j < n) dst[j * m + i] = tile[tx][ty + 4 * k];
        }
    }
}

// out[b, r, c] = c > r ? -inf : in[b, r, c] over [batch, seq, seq]; one wave per row, masked
// columns written without being read. VEC: 16-byte accesses (seq % 4 == 0, aligned buffers).
template <bool VEC>
__global__ __launch_bounds__(256) void causal_mask_3d_kernel(const float *in, float *out, int64_t rows,
                                                            int64_t seq) {
    const int lane = threadIdx.x & 63;
    const int64_t grow = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (grow >= rows) return;
    const int64_t r = grow % seq;
    const float *s = in + grow * seq;
    float *d = out + grow * seq;
    if (VEC) {
        for (int64_t c = 4 * lane; c < seq; c += 256) {
            f32x4 v;
            if (c + 3 <= r) {
                v = *(const f32x4 *)(s + c);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = c + e <= r ? s[c + e] : -INFINITY;
            }
            *(f32x4 *)(d + c) = v;
        }
    } else {
        for (int64_t c = lane; c < seq; c += 64) d[c] = c <= r ? s[c] : -INFINITY;
    }
}

// Seeded N(0, std^2) values, element e of the stream being normal number (offset + e) of `seed`:
// SplitMix64 output i of the seed is mix(seed + (i + 1) * 0x9E3779B97F4A7C15) (Steele, Lea and
// Flood 2014); uniforms take the top 53 bits, u = (bits + 0.5) / 2^53; normals pair consecutive
// uniforms by Box-Muller (element 2p = r cos(2 pi u2), 2p + 1 = r sin(2 pi u2) with
// r = sqrt(-2 ln u1)), in float64, then scaled by std (a separate multiply and add, no FMA) and
// rounded to float32 (and to BF16, round-to-nearest-even, for IT_BF16). One thread per pair.
__device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ double uniform_at(uint64_t seed, uint64_t i) {
    return __dmul_rn(__dadd_rn((double)(splitmix64_at(seed, i) >> 11), 0.5), 1.0 / 9007199254740992.0);
}

template <bool BF16>
__global__ __launch_bounds__(256) void fill_normal_kernel(void *dst, uint64_t seed, int64_t offset, int64_t n,
                                                         double std_dev, int64_t pair0, int64_t pairs) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < pairs; q += stride) {
        const int64_t p = pair0 + q;
        const double u1 = uniform_at(seed, (uint64_t)(2 * p));
        const double u2 = uniform_at(seed, (uint64_t)(2 * p + 1));
        const double rad = sqrt(__dmul_rn(-2.0, log(u1)));
        const double ang = __dmul_rn(2.0 * M_PI, u2);
        const double z[2] = {__dmul_rn(rad, cos(ang)), __dmul_rn(rad, sin(ang))};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t e = 2 * p + h - offset;
            if (e < 0 || e >= n) continue;
            const float v = (float)__dadd_rn(__dmul_rn(z[h], std_dev), 0.0);
            if (BF16) {
                // RNE from the FP32 bits (the values are finite): written on the bits so that the
                // compiler cannot fold the two roundings into one float64 -> BF16 conversion.
                const uint32_t b = __float_as_uint(v);
                ((uint16_t *)dst)[e] = (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
            } else {
                ((float *)dst)[e] = v;
            }
        }
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

it_status launch_transpose_3d(hipStream_t s, const float *in, float *out, int64_t batch, int64_t m, int64_t n) {
    const int64_t tm = (m + 63) / 64, tn = (n + 63) / 64;
    const int64_t blocks = batch * tm * tn;
    if (blocks > 0x7fffffff) return fail(IT_ERR_DIMS, "transpose_3d_gpu: too many tiles");
    hipLaunchKernelGGL(transpose_3d_kernel, dim3((unsigned)blocks), dim3(256), 0, s, in, out, m, n, tm, tn);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_causal_mask_3d(hipStream_t s, const float *in, float *out, int64_t batch, int64_t seq) {
    const int64_t rows = batch * seq;
    const int64_t blocks = (rows + 3) / 4;
    if (blocks > 0x7fffffff) return fail(IT_ERR_DIMS, "causal_mask_3d_gpu: too many rows");
    const bool vec = seq % 4 == 0 && (uintptr_t)in % 16 == 0 && (uintptr_t)out % 16 == 0;
    if (vec)
        hipLaunchKernelGGL(causal_mask_3d_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, in, out, rows, seq);
    else
        hipLaunchKernelGGL(causal_mask_3d_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, in, out, rows, seq);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_fill_normal(hipStream_t s, bool bf16, void *dst, uint64_t seed, int64_t offset, int64_t n,
                             double std_dev) {
    const int64_t pair0 = offset / 2;
    const int64_t pairs = (offset + n + 1) / 2 - pair0;
    const unsigned grid = grid_for(pairs, 256);
    if (bf16)
        hipLaunchKernelGGL(fill_normal_kernel<true>, dim3(grid), dim3(256), 0, s, dst, seed, offset, n, std_dev,
                           pair0, pairs);
    else
        hipLaunchKernelGGL(fill_normal_kernel<false>, dim3(grid), dim3(256), 0, s, dst, seed, offset, n, std_dev,
                           pair0, pairs);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

}  // namespace it
