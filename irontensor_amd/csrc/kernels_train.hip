// The training step's row and elementwise work around the contractions: RMSNorm forward (with the
// residual add fused in front) and backward (with the residual-gradient add fused behind and a
// deterministic dgamma), RoPE, embedding gather and its deterministic scatter-add, fused cross
// entropy with the mean loss, SwiGLU backward, the global gradient norm with the clip factor, and
// the Lion update.
//
// Semantics follow the reference kernels: src/shaders/norm.metal:16-44 and
// src/shaders/backward/norm.metal:22-69 (RMSNorm), src/shaders/rope.metal:22-62 and
// src/shaders/backward/rope.metal:25-62 (RoPE), src/shaders/embedding.metal and
// src/ops/backward/embedding.rs:21-61 (embedding), src/shaders/loss.metal:91-131 with the
// 1/rows gradient scale of src/ops/backward/loss.rs:248-330 (cross entropy),
// src/shaders/backward/elementwise.metal:101-126 (SwiGLU backward), src/ops/reduction.rs:94-158 with
// the clip rule of src/train/trainer/train_step.rs:405-414 (gradient norm), src/shaders/lion.metal
// (lion_step_f32) and src/optim/lion/optimizer.rs:54-106 (Lion).
//
// Every reduction here runs in a fixed order (no floating-point atomics), so a step is bit-for-bit
// repeatable; all are memory-bound and sized for one wave (rows) or 16-byte accesses (elementwise).
#include <cmath>

#include "internal.hpp"
#include "mfma.hpp"

namespace it {
namespace {

template <typename T>
__device__ __forceinline__ float ldv(const T *p, int64_t i);
template <>
__device__ __forceinline__ float ldv<float>(const float *p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ldv<uint16_t>(const uint16_t *p, int64_t i) { return bf16_to_f32(p[i]); }

template <typename T>
__device__ __forceinline__ void stv(T *p, int64_t i, float v);
template <>
__device__ __forceinline__ void stv<float>(float *p, int64_t i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void stv<uint16_t>(uint16_t *p, int64_t i, float v) { p[i] = f32_to_bf16_rne(v); }

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ double wsum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wmax(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

unsigned blocks_for(int64_t n, int64_t per_block, int64_t cap = 0x7fffffff) {
    int64_t b = (n + per_block - 1) / per_block;
    if (b < 1) b = 1;
    if (b > cap) b = cap;
    return (unsigned)b;
}

// ------------------------------------------------------------------ RMSNorm forward

// One wave per row, lane-strided columns (lane + 64 k): s = x (+ res); sum_out = s;
// y = s * (1 / sqrt(sum(s^2) / dim + eps)) * gamma. Columns are read twice; the second pass hits
// the cache (rows are at most a few KB).
template <typename TY>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const float *x, const float *res, float *sum_out,
                                                          const float *gamma, TY *y, int64_t rows,
                                                          int64_t dim, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * dim;
    const float *rr = res ? res + row * dim : nullptr;
    float ss = 0.f;
    for (int64_t c = lane; c < dim; c += 64) {
        const float s = rr ? xr[c] + rr[c] : xr[c];
        if (sum_out) sum_out[row * dim + c] = s;
        ss += s * s;
    }
    ss = wsum(ss);
    const float rms = sqrtf(ss / (float)dim + eps);
    const float inv = 1.0f / rms;
    for (int64_t c = lane; c < dim; c += 64) {
        const float s = rr ? xr[c] + rr[c] : xr[c];
        stv<TY>(y, row * dim + c, s * inv * gamma[c]);
    }
}

// ------------------------------------------------------------------ RMSNorm backward

// Rows are split over blocks of RB_ROWS; each wave takes every fourth row of its block. Per row:
// s = 1/rms, dot = sum(dy * gamma * x), dx = gres + dy * gamma * s - (1/dim) s^3 x dot. Each lane
// keeps its columns' dgamma partial sum (dy * x * s) in registers over the block's rows; the four
// waves combine in a fixed order into part[block][dim], which rmsnorm_dgamma_reduce sums over
// blocks in order.
constexpr int RB_ROWS = 16;

template <int MAXK>  // columns per lane: dim <= 64 * MAXK
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const float *dy, const float *x, const float *gamma,
                                                          const float *gres, float *dx, float *part,
                                                          int64_t rows, int64_t dim, float eps) {
    extern __shared__ float red[];  // [4][dim]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * RB_ROWS;
    const float n = (float)dim;
    float acc[MAXK];
#pragma unroll
    for (int k = 0; k < MAXK; ++k) acc[k] = 0.f;
    for (int64_t row = r0 + wave; row < min(rows, r0 + RB_ROWS); row += 4) {
        const float *xr = x + row * dim, *gr = dy + row * dim;
        float xv[MAXK], gv[MAXK];
        float ss = 0.f, dot = 0.f;
#pragma unroll
        for (int k = 0; k < MAXK; ++k) {
            const int64_t c = lane + 64 * k;
            xv[k] = c < dim ? xr[c] : 0.f;
            gv[k] = c < dim ? gr[c] : 0.f;
            ss += xv[k] * xv[k];
            dot += gv[k] * (c < dim ? gamma[c] : 0.f) * xv[k];
        }
        ss = wsum(ss);
        dot = wsum(dot);
        const float rms = sqrtf(ss / n + eps);
        const float s = 1.0f / rms, s3 = s * s * s;
#pragma unroll
        for (int k = 0; k < MAXK; ++k) {
            const int64_t c = lane + 64 * k;
            if (c < dim) {
                float v = gv[k] * gamma[c] * s - (1.0f / n) * s3 * xv[k] * dot;
                if (gres) v = gres[row * dim + c] + v;
                dx[row * dim + c] = v;
                acc[k] += gv[k] * xv[k] * s;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
        const int64_t c = lane + 64 * k;
        if (c < dim) red[wave * dim + c] = acc[k];
    }
    __syncthreads();
    for (int64_t c = threadIdx.x; c < dim; c += 256)
        part[(int64_t)blockIdx.x * dim + c] = ((red[c] + red[dim + c]) + red[2 * dim + c]) + red[3 * dim + c];
}

// dgamma[c] = sum over blocks of part[b][c]: 64 columns per block (lane = column), the four waves
// take every fourth partial row and combine in a fixed order.
__global__ __launch_bounds__(256) void rmsnorm_dgamma_reduce(const float *part, float *dgamma, int64_t blocks,
                                                             int64_t dim) {
    __shared__ float red[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t c = (int64_t)blockIdx.x * 64 + lane;
    float s = 0.f;
    if (c < dim) {
        int64_t b = wave;
        for (; b + 12 < blocks; b += 16) {
            const float v0 = part[b * dim + c], v1 = part[(b + 4) * dim + c];
            const float v2 = part[(b + 8) * dim + c], v3 = part[(b + 12) * dim + c];
            s += v0;
            s += v1;
            s += v2;
            s += v3;
        }
        for (; b < blocks; b += 4) s += part[b * dim + c];
    }
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && c < dim) dgamma[c] = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
}

// ------------------------------------------------------------------ RoPE

// One block per row (b, s) of src, at (b * seq + s) * src_rs; its threads take the rotated pairs:
// heads * head_dim columns rotated pairwise ((2i, 2i+1) of each head, theta_i = 1 / base^(2i /
// head_dim), angle = (s + offset) * theta_i); the backward applies the transposed rotation. When
// src and dst differ, copy_cols further columns are copied after the rotated ones (the V block of a
// fused QKV gradient changing precision).
// theta_i = 1 / base^(2i / head_dim) with the power evaluated in double and rounded once: the
// correctly rounded powf. The angle (s + offset) * theta_i multiplies a position of up to a few
// thousand by it, so one unit in the last place of theta_i would show in every rotated value; the
// correctly rounded power is what an accurate host powf returns for these arguments.
__device__ __forceinline__ float rope_theta(float base, int i, int64_t head_dim) {
    const float e = (float)(i * 2) / (float)head_dim;
    return 1.0f / (float)pow((double)base, (double)e);
}

constexpr int ROPE_TABLE = 256;  // pairs per head whose theta is tabulated per block

template <typename TS, typename TD>
__global__ __launch_bounds__(256) void rope_kernel(const TS *src, TD *dst, int64_t seq, int64_t heads,
                                                   int64_t head_dim, int64_t src_rs, int64_t dst_rs,
                                                   int64_t copy_cols, float base, int64_t offset, int backward) {
    const int64_t row = blockIdx.x;
    const int64_t s = row % seq;
    const int half = (int)(head_dim / 2);
    const TS *sp = src + row * src_rs;
    TD *dp = dst + row * dst_rs;
    __shared__ float theta_s[ROPE_TABLE];
    if (threadIdx.x < min(half, ROPE_TABLE)) theta_s[threadIdx.x] = rope_theta(base, threadIdx.x, head_dim);
    __syncthreads();
    const int64_t pairs = heads * half;
    for (int64_t j = threadIdx.x; j < pairs; j += 256) {
        const int i = (int)(j % half);
        const int64_t c = (j / half) * head_dim + 2 * i;
        const float theta = i < ROPE_TABLE ? theta_s[i] : rope_theta(base, i, head_dim);
        const float angle = (float)(s + offset) * theta;
        float sn, cs;
        sincosf(angle, &sn, &cs);
        const float x0 = ldv<TS>(sp, c), x1 = ldv<TS>(sp, c + 1);
        if (!backward) {
            stv<TD>(dp, c, x0 * cs - x1 * sn);
            stv<TD>(dp, c + 1, x0 * sn + x1 * cs);
        } else {
            stv<TD>(dp, c, x0 * cs + x1 * sn);
            stv<TD>(dp, c + 1, -x0 * sn + x1 * cs);
        }
    }
    const int64_t c0 = heads * head_dim;
    for (int64_t c = c0 + threadIdx.x; c < c0 + copy_cols; c += 256) stv<TD>(dp, c, ldv<TS>(sp, c));
}

// ------------------------------------------------------------------ embedding

// One wave per token: out[i] = table[ids[i]]. An id outside the vocabulary yields a zero row (the
// host mirrors reject such ids before upload; the guard only keeps the read in bounds).
template <typename TW, typename TO>
__global__ __launch_bounds__(256) void embedding_fwd_kernel(const TW *table, const uint32_t *ids, TO *out,
                                                            int64_t n, int64_t dim, int64_t vocab) {
    const int lane = threadIdx.x & 63;
    const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= n) return;
    const uint32_t id = ids[i];
    const bool ok = (int64_t)id < vocab;
    const TW *src = table + (ok ? (int64_t)id * dim : 0);
    for (int64_t c = lane; c < dim; c += 64) stv<TO>(out, i * dim + c, ok ? ldv<TW>(src, c) : 0.f);
}

// Scatter-add without atomics: block b owns vocabulary rows [EB_ROWS b, EB_ROWS (b+1)). It scans the
// ids in windows of EB_WIN tokens, compacts the tokens that hit its rows into an index-ordered list
// in LDS, and each thread adds dy[token][c] into its own columns c of the owned rows, in token
// order. Every element is therefore summed in index order, as a sequential loop would, and rows no
// token hits are written as zeros.
constexpr int EB_ROWS = 16;
constexpr int EB_WIN = 2048;

__global__ __launch_bounds__(256) void embedding_bwd_kernel(const float *dy, const uint32_t *ids, float *dw,
                                                            int64_t n, int64_t dim, int64_t vocab) {
    __shared__ int tok[EB_WIN];
    __shared__ uint8_t hit_row[EB_WIN];
    __shared__ int wave_cnt[4];
    __shared__ int row_cnt[EB_ROWS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t v0 = (int64_t)blockIdx.x * EB_ROWS;
    const int nrows = (int)min((int64_t)EB_ROWS, vocab - v0);
    for (int64_t w0 = 0; w0 < n || w0 == 0; w0 += EB_WIN) {
        const int64_t wend = min(n, w0 + EB_WIN);
        if (tid < EB_ROWS) row_cnt[tid] = 0;
        int count = 0;
        __syncthreads();
        for (int64_t c0 = w0; c0 < wend; c0 += 256) {
            const int64_t i = c0 + tid;
            const uint32_t id = i < wend ? ids[i] : 0xffffffffu;
            const int64_t r = (int64_t)id - v0;
            const bool hit = i < wend && r >= 0 && r < nrows;
            const uint64_t mask = __ballot(hit);
            const int before = __popcll(mask & ((1ull << lane) - 1ull));
            if (lane == 0) wave_cnt[wave] = __popcll(mask);
            __syncthreads();
            int base = count;
            for (int w = 0; w < wave; ++w) base += wave_cnt[w];
            if (hit) {
                tok[base + before] = (int)(i - w0);
                hit_row[base + before] = (uint8_t)r;
                atomicAdd(&row_cnt[r], 1);  // integer count: order-free
            }
            count += wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
            __syncthreads();
        }
        for (int r = 0; r < nrows; ++r) {
            const int cnt_r = row_cnt[r];
            if (w0 > 0 && cnt_r == 0) continue;  // earlier windows already wrote this row
            float *out = dw + (v0 + r) * dim;
            for (int64_t c = tid; c < dim; c += 256) {
                float acc = w0 == 0 ? 0.f : out[c];
                if (cnt_r)
                    for (int m = 0; m < count; ++m)
                        if (hit_row[m] == r) acc += dy[(w0 + tok[m]) * dim + c];
                out[c] = acc;
            }
        }
        __syncthreads();
        if (n == 0) break;
    }
}

// ------------------------------------------------------------------ cross entropy

// One 256-thread block per row. With NPT > 0 the row (vocab <= 256 * NPT, logits and gradient 16-byte
// aligned, vocab % 4 == 0) is held in registers: one HBM read, one write. NPT == 0 reads the row
// three times (max; exp-sum; gradient), the later passes mostly from cache.
// loss = -x[t] + (max + log(sum exp(x - max))); grad = (exp(x - max) / sum - onehot) * grad_scale.
template <int NPT, typename TG>
__global__ __launch_bounds__(256) void ce_kernel(const float *logits, const uint32_t *targets, float *losses,
                                                 TG *grad, int64_t rows, int64_t vocab, float grad_scale) {
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = blockIdx.x;
    const float *x = logits + row * vocab;
    TG *g = grad + row * vocab;
    const uint32_t t = targets[row];

    auto block_max = [&](float v) {
        v = wmax(v);
        if (lane == 0) red[wave] = v;
        __syncthreads();
        v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();
        return v;
    };
    auto block_sum = [&](float v) {
        v = wsum(v);
        if (lane == 0) red[wave] = v;
        __syncthreads();
        v = ((red[0] + red[1]) + red[2]) + red[3];
        __syncthreads();
        return v;
    };

    float mx = -INFINITY, sum = 0.f;
    if constexpr (NPT > 0) {
        constexpr int NV = NPT / 4;
        f32x4 v[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int64_t e = 4 * ((int64_t)tid + 256 * k);
            v[k] = e < vocab ? *(const f32x4 *)(x + e) : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
            for (int q = 0; q < 4; ++q) mx = fmaxf(mx, v[k][q]);
        }
        mx = block_max(mx);
#pragma unroll
        for (int k = 0; k < NV; ++k)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v[k][q] = expf(v[k][q] - mx);  // exp(-inf) = 0 for the padding
                sum += v[k][q];
            }
        sum = block_sum(sum);
        const float inv = 1.0f / sum;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int64_t e = 4 * ((int64_t)tid + 256 * k);
            if (e < vocab) {
                f32x4 o;
#pragma unroll
                for (int q = 0; q < 4; ++q) o[q] = (v[k][q] * inv - ((uint64_t)(e + q) == t ? 1.0f : 0.0f)) * grad_scale;
                if constexpr (sizeof(TG) == 4)
                    *(f32x4 *)(g + e) = o;
                else
                    *(u32x2 *)(g + e) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
            }
        }
    } else {
        for (int64_t e = tid; e < vocab; e += 256) mx = fmaxf(mx, x[e]);
        mx = block_max(mx);
        for (int64_t e = tid; e < vocab; e += 256) sum += expf(x[e] - mx);
        sum = block_sum(sum);
        const float inv = 1.0f / sum;
        for (int64_t e = tid; e < vocab; e += 256)
            stv<TG>(g, e, (expf(x[e] - mx) * inv - ((uint64_t)e == t ? 1.0f : 0.0f)) * grad_scale);
    }
    if (tid == 0) losses[row] = (int64_t)t < vocab ? -x[t] + (mx + logf(sum)) : NAN;
}

// Mean of `n` values in a fixed order (one block): per-thread strided sums, then a tree.
__global__ __launch_bounds__(256) void mean_kernel(const float *v, int64_t n, float *out) {
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float s = 0.f;
    for (int64_t i = tid; i < n; i += 256) s += v[i];
    s = wsum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (tid == 0) out[0] = (((red[0] + red[1]) + red[2]) + red[3]) / (float)n;
}

// ------------------------------------------------------------------ SwiGLU backward

// grad_up = dh * silu(g); grad_gate = dh * u * sig(g) (1 + g (1 - sig(g))), sig(g) = 1 / (1 + exp(-g)).
// One block per row.
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const float *dh, int64_t ld_dh, const TI *gate,
                                                         const TI *up, int64_t ld_gu, TO *dgate, TO *dup,
                                                         int64_t ld_out, int64_t cols) {
    const int64_t r = blockIdx.x;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
        const float g = ldv<TI>(gate, r * ld_gu + c), u = ldv<TI>(up, r * ld_gu + c);
        const float go = dh[r * ld_dh + c];
        const float sig = 1.0f / (1.0f + expf(-g));
        const float silu = g * sig;
        stv<TO>(dup, r * ld_out + c, go * silu);
        const float d_silu = sig * (1.0f + g * (1.0f - sig));
        stv<TO>(dgate, r * ld_out + c, go * u * d_silu);
    }
}

// ------------------------------------------------------------------ gradient norm and Lion

constexpr int MT_MAX = 24;  // tensors per launch (the table travels in the kernel arguments)

struct TensorTable {
    int count;
    float *w[MT_MAX];
    float *m[MT_MAX];
    const float *g[MT_MAX];
    int64_t n[MT_MAX];
    int64_t first_block[MT_MAX + 1];  // block ranges per tensor
};

constexpr int MT_ELEMS = 4096;  // elements per block

__device__ __forceinline__ int table_find(const TensorTable &t, int64_t b) {
    int i = 0;
    while (i + 1 < t.count && b >= t.first_block[i + 1]) ++i;
    return i;
}

// Sum of squares in double: each block sums its MT_ELEMS-element chunk of one tensor into part[slot].
__global__ __launch_bounds__(256) void sumsq_kernel(const TensorTable t, double *part) {
    __shared__ double red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t b = blockIdx.x;
    const int i = table_find(t, b);
    const int64_t e0 = (b - t.first_block[i]) * MT_ELEMS;
    const int64_t e1 = min(t.n[i], e0 + MT_ELEMS);
    const float *g = t.g[i];
    double s = 0.0;
    for (int64_t e = e0 + tid; e < e1; e += 256) {
        const double v = (double)g[e];
        s += v * v;
    }
    s = wsum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (tid == 0) part[b] = ((red[0] + red[1]) + red[2]) + red[3];
}

// out[0] = sqrt(sum of parts) (float), out[1] = max_norm / norm when norm > max_norm, else 1.
__global__ __launch_bounds__(256) void norm_finish_kernel(const double *part, int64_t n, float max_norm,
                                                          float *out) {
    __shared__ double red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    double s = 0.0;
    for (int64_t i = tid; i < n; i += 256) s += part[i];
    s = wsum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (tid == 0) {
        const float norm = (float)sqrt(((red[0] + red[1]) + red[2]) + red[3]);
        out[0] = norm;
        out[1] = norm > max_norm ? max_norm / norm : 1.0f;
    }
}

// Lion, per element: g' = g * scale; u = beta2 m + (1 - beta2) g'; m = beta1 m + (1 - beta1) g';
// w = w - lr sign(u) - lr wd w. scale and lr come from device memory when given (a clip factor
// computed on the GPU, a schedule value updated between graph replays).
__global__ __launch_bounds__(256) void lion_kernel(const TensorTable t, float lr, float beta1, float beta2,
                                                   float wd, const float *scale_dev, const float *lr_dev) {
#pragma clang fp contract(off)  // separate roundings, as the reference's expression is written
    const int64_t b = blockIdx.x;
    const int i = table_find(t, b);
    const int64_t e0 = (b - t.first_block[i]) * MT_ELEMS;
    const int64_t e1 = min(t.n[i], e0 + MT_ELEMS);
    const float scale = scale_dev ? scale_dev[0] : 1.0f;
    const float rate = lr_dev ? lr_dev[0] : lr;
    float *w = t.w[i], *m = t.m[i];
    const float *g = t.g[i];
    for (int64_t e = e0 + threadIdx.x; e < e1; e += 256) {
        const float gi = g[e] * scale;
        const float mi = m[e], wi = w[e];
        const float u = beta2 * mi + (1.0f - beta2) * gi;
        const float dir = u > 0.f ? 1.f : (u < 0.f ? -1.f : 0.f);
        m[e] = beta1 * mi + (1.0f - beta1) * gi;
        w[e] = wi - rate * dir - rate * wd * wi;
    }
}

}  // namespace

// ------------------------------------------------------------------ launchers

it_status launch_rmsnorm_forward(hipStream_t s, bool y_bf16, int64_t rows, int64_t dim, float eps, const float *x,
                                 const float *res, const float *gamma, float *sum_out, void *y) {
    const unsigned grid = blocks_for(rows, 4);
    if (y_bf16)
        hipLaunchKernelGGL(rmsnorm_fwd_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, x, res, sum_out, gamma,
                           (uint16_t *)y, rows, dim, eps);
    else
        hipLaunchKernelGGL(rmsnorm_fwd_kernel<float>, dim3(grid), dim3(256), 0, s, x, res, sum_out, gamma,
                           (float *)y, rows, dim, eps);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

int64_t rmsnorm_backward_scratch_bytes(int64_t rows, int64_t dim) {
    return ((rows + RB_ROWS - 1) / RB_ROWS) * dim * (int64_t)sizeof(float);
}

it_status launch_rmsnorm_backward(hipStream_t s, int64_t rows, int64_t dim, float eps, const float *dy,
                                  const float *x, const float *gamma, const float *gres, float *dx,
                                  float *dgamma, float *part) {
    const int64_t blocks = (rows + RB_ROWS - 1) / RB_ROWS;
    const size_t lds = 4 * (size_t)dim * sizeof(float);
    if (dim <= 256)
        hipLaunchKernelGGL(rmsnorm_bwd_kernel<4>, dim3((unsigned)blocks), dim3(256), lds, s, dy, x, gamma, gres, dx,
                           part, rows, dim, eps);
    else if (dim <= 1024)
        hipLaunchKernelGGL(rmsnorm_bwd_kernel<16>, dim3((unsigned)blocks), dim3(256), lds, s, dy, x, gamma, gres,
                           dx, part, rows, dim, eps);
    else
        hipLaunchKernelGGL(rmsnorm_bwd_kernel<32>, dim3((unsigned)blocks), dim3(256), lds, s, dy, x, gamma, gres,
                           dx, part, rows, dim, eps);
    IT_HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(rmsnorm_dgamma_reduce, dim3(blocks_for(dim, 64)), dim3(256), 0, s, part, dgamma, blocks,
                       dim);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_rope(hipStream_t s, bool src_bf16, bool dst_bf16, int64_t batch, int64_t seq, int64_t heads,
                      int64_t head_dim, float base, int64_t offset, int backward, const void *src, int64_t src_rs,
                      void *dst, int64_t dst_rs, int64_t copy_cols) {
    const dim3 grid((unsigned)(batch * seq));
#define IT_ROPE(TS, TD)                                                                                        \
    hipLaunchKernelGGL((rope_kernel<TS, TD>), grid, dim3(256), 0, s, (const TS *)src, (TD *)dst, seq, heads,   \
                       head_dim, src_rs, dst_rs, copy_cols, base, offset, backward)
    if (!src_bf16 && !dst_bf16)
        IT_ROPE(float, float);
    else if (!src_bf16 && dst_bf16)
        IT_ROPE(float, uint16_t);
    else if (src_bf16 && dst_bf16)
        IT_ROPE(uint16_t, uint16_t);
    else
        IT_ROPE(uint16_t, float);
#undef IT_ROPE
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_embedding_forward(hipStream_t s, bool table_bf16, bool out_bf16, int64_t n, int64_t dim,
                                   int64_t vocab, const void *table, const uint32_t *ids, void *out) {
    const unsigned grid = blocks_for(n, 4);
#define IT_EMB(TW, TO)                                                                                         \
    hipLaunchKernelGGL((embedding_fwd_kernel<TW, TO>), dim3(grid), dim3(256), 0, s, (const TW *)table, ids,      \
                       (TO *)out, n, dim, vocab)
    if (!table_bf16 && !out_bf16)
        IT_EMB(float, float);
    else if (!table_bf16 && out_bf16)
        IT_EMB(float, uint16_t);
    else if (table_bf16 && out_bf16)
        IT_EMB(uint16_t, uint16_t);
    else
        IT_EMB(uint16_t, float);
#undef IT_EMB
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_embedding_backward(hipStream_t s, int64_t n, int64_t dim, int64_t vocab, const float *dy,
                                    const uint32_t *ids, float *dw) {
    const int64_t blocks = (vocab + EB_ROWS - 1) / EB_ROWS;
    hipLaunchKernelGGL(embedding_bwd_kernel, dim3((unsigned)blocks), dim3(256), 0, s, dy, ids, dw, n, dim, vocab);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_cross_entropy(hipStream_t s, bool grad_bf16, int64_t rows, int64_t vocab, const float *logits,
                               const uint32_t *targets, float *losses, void *grad, float *loss_mean,
                               bool vec_ok) {
    const float gs = 1.0f / (float)rows;
    const dim3 grid((unsigned)rows), block(256);
#define IT_CE(NPT, TG)                                                                                         \
    hipLaunchKernelGGL((ce_kernel<NPT, TG>), grid, block, 0, s, logits, targets, losses, (TG *)grad, rows, vocab, gs)
#define IT_CE_T(NPT)            \
    if (grad_bf16)              \
        IT_CE(NPT, uint16_t);   \
    else                        \
        IT_CE(NPT, float);
    if (vec_ok && vocab <= 256 * 16) {
        IT_CE_T(16)
    } else if (vec_ok && vocab <= 256 * 64) {
        IT_CE_T(64)
    } else if (vec_ok && vocab <= 256 * 128) {
        IT_CE_T(128)
    } else {
        IT_CE_T(0)
    }
#undef IT_CE_T
#undef IT_CE
    IT_HIP_TRY(hipGetLastError());
    if (loss_mean) {
        hipLaunchKernelGGL(mean_kernel, dim3(1), dim3(256), 0, s, losses, rows, loss_mean);
        IT_HIP_TRY(hipGetLastError());
    }
    return IT_OK;
}

it_status launch_swiglu_backward(hipStream_t s, bool in_bf16, bool out_bf16, int64_t rows, int64_t cols,
                                 const float *dh, int64_t ld_dh, const void *gate, const void *up, int64_t ld_gu,
                                 void *dgate, void *dup, int64_t ld_out) {
    const dim3 grid((unsigned)rows);
#define IT_SWB(TI, TO)                                                                                          \
    hipLaunchKernelGGL((swiglu_bwd_kernel<TI, TO>), grid, dim3(256), 0, s, dh, ld_dh, (const TI *)gate,         \
                       (const TI *)up, ld_gu, (TO *)dgate, (TO *)dup, ld_out, cols)
    if (!in_bf16 && !out_bf16)
        IT_SWB(float, float);
    else if (!in_bf16 && out_bf16)
        IT_SWB(float, uint16_t);
    else if (in_bf16 && out_bf16)
        IT_SWB(uint16_t, uint16_t);
    else
        IT_SWB(uint16_t, float);
#undef IT_SWB
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

// Builds launch tables of at most MT_MAX tensors; `fn(table, blocks)` launches one.
template <typename F>
static it_status for_tables(int count, float *const *w, float *const *m, const float *const *g, const int64_t *n,
                            F fn) {
    for (int i0 = 0; i0 < count; i0 += MT_MAX) {
        TensorTable t{};
        t.count = 0;
        int64_t blocks = 0;
        for (int i = i0; i < count && i < i0 + MT_MAX; ++i) {
            if (n[i] == 0) continue;
            const int k = t.count++;
            t.w[k] = w ? w[i] : nullptr;
            t.m[k] = m ? m[i] : nullptr;
            t.g[k] = g[i];
            t.n[k] = n[i];
            t.first_block[k] = blocks;
            blocks += (n[i] + MT_ELEMS - 1) / MT_ELEMS;
        }
        t.first_block[t.count] = blocks;
        if (t.count == 0) continue;
        if (const it_status st = fn(t, blocks); st != IT_OK) return st;
    }
    return IT_OK;
}

int64_t grad_norm_partials(int count, const int64_t *n) {
    int64_t blocks = 0;
    for (int i = 0; i < count; ++i) blocks += (n[i] + MT_ELEMS - 1) / MT_ELEMS;
    return blocks;
}

it_status launch_grad_norm(hipStream_t s, int count, const float *const *g, const int64_t *n, float max_norm,
                           float *out, double *part) {
    int64_t slot = 0;
    const it_status st = for_tables(count, nullptr, nullptr, g, n, [&](const TensorTable &t, int64_t blocks) {
        if (blocks > 0x7fffffff) return fail(IT_ERR_DIMS, "grad_norm: tensor too large");
        hipLaunchKernelGGL(sumsq_kernel, dim3((unsigned)blocks), dim3(256), 0, s, t, part + slot);
        IT_HIP_TRY(hipGetLastError());
        slot += blocks;
        return IT_OK;
    });
    if (st != IT_OK) return st;
    hipLaunchKernelGGL(norm_finish_kernel, dim3(1), dim3(256), 0, s, part, slot, max_norm, out);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_lion(hipStream_t s, int count, float *const *w, float *const *m, const float *const *g,
                      const int64_t *n, float lr, float beta1, float beta2, float wd, const float *scale_dev,
                      const float *lr_dev) {
    return for_tables(count, w, m, g, n, [&](const TensorTable &t, int64_t blocks) {
        if (blocks > 0x7fffffff) return fail(IT_ERR_DIMS, "lion: tensor too large");
        hipLaunchKernelGGL(lion_kernel, dim3((unsigned)blocks), dim3(256), 0, s, t, lr, beta1, beta2, wd, scale_dev,
                           lr_dev);
        IT_HIP_TRY(hipGetLastError());
        return IT_OK;
    });
}

}  // namespace it
