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

// One wave per row, lane-strided columns (c = lane + 64 k): s = x (+ res); sum_out = s;
// y = s * (1 / sqrt(sum(s^2) / dim + eps)) * gamma. With MAXK > 0 (dim <= 64 MAXK) the row stays in
// registers (every load issued before the reduction: one pass over HBM); MAXK == 0 reads the row
// twice for any dim.
template <typename TY, int MAXK>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const float *x, const float *res, float *sum_out,
                                                          const float *gamma, TY *y, int64_t rows,
                                                          int64_t dim, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * dim;
    const float *rr = res ? res + row * dim : nullptr;
    float ss = 0.f;
    if constexpr (MAXK > 0) {
        float sv[MAXK];
#pragma unroll
        for (int k = 0; k < MAXK; ++k) {
            const int64_t c = lane + 64 * k;
            sv[k] = c < dim ? (rr ? xr[c] + rr[c] : xr[c]) : 0.f;
            ss += sv[k] * sv[k];
        }
        ss = wsum(ss);
        const float rms = sqrtf(ss / (float)dim + eps);
        const float inv = 1.0f / rms;
#pragma unroll
        for (int k = 0; k < MAXK; ++k) {
            const int64_t c = lane + 64 * k;
            if (c < dim) {
                if (sum_out) sum_out[row * dim + c] = sv[k];
                stv<TY>(y, row * dim + c, sv[k] * inv * gamma[c]);
            }
        }
    } else {
        for (int64_t c = lane; c < dim; c += 64) {
            const float v = rr ? xr[c] + rr[c] : xr[c];
            if (sum_out) sum_out[row * dim + c] = v;
            ss += v * v;
        }
        ss = wsum(ss);
        const float rms = sqrtf(ss / (float)dim + eps);
        const float inv = 1.0f / rms;
        for (int64_t c = lane; c < dim; c += 64) {
            const float v = rr ? xr[c] + rr[c] : xr[c];
            stv<TY>(y, row * dim + c, v * inv * gamma[c]);
        }
    }
}

// ------------------------------------------------------------------ RMSNorm backward

// Each wave takes RPW consecutive rows and loads all of them (x, dy and the residual gradient)
// before reducing (RPW rows of memory latency overlap); a block's four waves cover 4 RPW rows. Per row: s = 1/rms,
// dot = sum(dy * gamma * x), dx = gres + dy * gamma * s - (1/dim) s^3 x dot. Each lane keeps its
// columns' dgamma partial sum (dy * x * s, rows in order) in registers; the four waves combine in a
// fixed order into part[block][dim], summed over blocks in order by rmsnorm_dgamma_reduce.
template <int MAXK, int RPW>  // columns per lane (dim <= 64 MAXK), rows per wave
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const float *dy, const float *x, const float *gamma,
                                                          const float *gres, float *dx, float *part,
                                                          int64_t rows, int64_t dim, float eps) {
    extern __shared__ float red[];  // [4][dim]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r0 = ((int64_t)blockIdx.x * 4 + wave) * RPW;
    const float n = (float)dim;
    float gm[MAXK], acc[MAXK];
    float xv[RPW][MAXK], gv[RPW][MAXK], rv[RPW][MAXK];
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
        const int64_t c = lane + 64 * k;
        gm[k] = c < dim ? gamma[c] : 0.f;
        acc[k] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        const int64_t row = r0 + j;
#pragma unroll
        for (int k = 0; k < MAXK; ++k) {
            const int64_t c = lane + 64 * k;
            const bool ok = row < rows && c < dim;
            xv[j][k] = ok ? x[row * dim + c] : 0.f;
            gv[j][k] = ok ? dy[row * dim + c] : 0.f;
            rv[j][k] = ok && gres ? gres[row * dim + c] : 0.f;  // in flight with x and dy
        }
    }
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        const int64_t row = r0 + j;
        float ss = 0.f, dot = 0.f;
#pragma unroll
        for (int k = 0; k < MAXK; ++k) {
            ss += xv[j][k] * xv[j][k];
            dot += gv[j][k] * gm[k] * xv[j][k];
        }
        ss = wsum(ss);
        dot = wsum(dot);
        if (row >= rows) continue;
        const float rms = sqrtf(ss / n + eps);
        const float s = 1.0f / rms, s3 = s * s * s;
#pragma unroll
        for (int k = 0; k < MAXK; ++k) {
            const int64_t c = lane + 64 * k;
            if (c < dim) {
                float v = gv[j][k] * gm[k] * s - (1.0f / n) * s3 * xv[j][k] * dot;
                if (gres) v = rv[j][k] + v;
                dx[row * dim + c] = v;
                acc[k] += gv[j][k] * xv[j][k] * s;
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

// dgamma[c] = sum over blocks b of part[b][c]: one 1024-thread block per 64 columns (lane =
// column); wave w sums rows b = w (mod 16) with sixteen loads in flight, then the 16 waves combine
// in a fixed order.
__global__ __launch_bounds__(1024) void rmsnorm_dgamma_reduce(const float *part, float *dgamma, int64_t blocks,
                                                              int64_t dim) {
    __shared__ float red[16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t c = (int64_t)blockIdx.x * 64 + lane;
    float s = 0.f;
    if (c < dim) {
        int64_t b = wave;
        for (; b + 15 * 16 < blocks; b += 256) {
            float v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = part[(b + 16 * j) * dim + c];
#pragma unroll
            for (int j = 0; j < 16; ++j) s += v[j];
        }
        for (; b < blocks; b += 16) s += part[b * dim + c];
    }
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && c < dim) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < 16; ++w) t += red[w][lane];
        dgamma[c] = t;
    }
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

// table[s][i] = (cos, sin) of angle (s + offset) * theta_i, for s < seq and i < head_dim / 2.
__global__ __launch_bounds__(256) void rope_table_kernel(float2 *table, int64_t seq, int64_t head_dim, float base,
                                                         int64_t offset) {
    const int64_t half = head_dim / 2;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= seq * half) return;
    const int64_t s = t / half;
    const int i = (int)(t % half);
    const float angle = (float)(s + offset) * rope_theta(base, i, head_dim);
    float sn, cs;
    sincosf(angle, &sn, &cs);
    table[t] = make_float2(cs, sn);
}

// One thread per rotated pair (2i, 2i+1) of each head, over rows (b, s) of src at
// (b * seq + s) * src_rs, with (cos, sin) from the table; the backward applies the transposed
// rotation. When src and dst differ, copy_cols further columns are copied after the rotated ones
// (the V block of a fused QKV gradient changing precision).
template <typename TS, typename TD>
__global__ __launch_bounds__(256) void rope_kernel(const TS *src, TD *dst, const float2 *table, int64_t rows,
                                                   int64_t seq, int heads, int half, int64_t src_rs, int64_t dst_rs,
                                                   int copy_cols, int backward) {
    const int per_row = heads * half + (copy_cols + 1) / 2;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= rows * per_row) return;
    const int64_t row = t / per_row;
    const int j = (int)(t - row * per_row);
    const TS *sp = src + row * src_rs;
    TD *dp = dst + row * dst_rs;
    if (j < heads * half) {
        const int i = j % half;
        const int64_t c = 2 * (int64_t)j;  // (j / half) * head_dim + 2 i
        const float2 cs = table[(row % seq) * half + i];
        const float x0 = ldv<TS>(sp, c), x1 = ldv<TS>(sp, c + 1);
        if (!backward) {
            stv<TD>(dp, c, x0 * cs.x - x1 * cs.y);
            stv<TD>(dp, c + 1, x0 * cs.y + x1 * cs.x);
        } else {
            stv<TD>(dp, c, x0 * cs.x + x1 * cs.y);
            stv<TD>(dp, c + 1, -x0 * cs.y + x1 * cs.x);
        }
    } else {
        const int64_t c0 = 2 * (int64_t)j;
        const int64_t end = 2 * (int64_t)heads * half + copy_cols;
        for (int64_t c = c0; c < min(c0 + 2, end); ++c) stv<TD>(dp, c, ldv<TS>(sp, c));
    }
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
// ids in windows of EB_WIN tokens (each thread loads EB_PER consecutive ids), compacts the tokens
// that hit its rows into an index-ordered list in LDS with one block-wide prefix sum, and each thread
// adds dy[token][c] into its own columns c of the owned rows, in token order. Every element is
// therefore summed in index order, as a sequential loop would, and rows no token hits are written
// as zeros.
constexpr int EB_ROWS = 16;
constexpr int EB_PER = 16;
constexpr int EB_WIN = 256 * EB_PER;

__global__ __launch_bounds__(256) void embedding_bwd_kernel(const float *dy, const uint32_t *ids, float *dw,
                                                            int64_t n, int64_t dim, int64_t vocab) {
    __shared__ int tok[EB_WIN];
    __shared__ uint8_t hit_row[EB_WIN];
    __shared__ int wave_tot[4];
    __shared__ int row_cnt[EB_ROWS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t v0 = (int64_t)blockIdx.x * EB_ROWS;
    const int nrows = (int)min((int64_t)EB_ROWS, vocab - v0);
    for (int64_t w0 = 0; w0 < n || w0 == 0; w0 += EB_WIN) {
        if (tid < EB_ROWS) row_cnt[tid] = 0;
        // this thread's tokens: [w0 + EB_PER tid, w0 + EB_PER (tid + 1)), all loads issued first
        const int64_t t0 = w0 + (int64_t)EB_PER * tid;
        int r[EB_PER];
        int mine = 0;
#pragma unroll
        for (int e = 0; e < EB_PER; ++e) {
            const int64_t i = t0 + e;
            const int64_t d = i < n ? (int64_t)ids[i] - v0 : -1;
            r[e] = (d >= 0 && d < nrows) ? (int)d : -1;
            mine += r[e] >= 0;
        }
        // exclusive prefix of `mine` over the block, in thread order
        int incl = mine;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o, 64);
            if (lane >= o) incl += v;
        }
        if (lane == 63) wave_tot[wave] = incl;
        __syncthreads();
        int base = incl - mine;
        for (int w = 0; w < wave; ++w) base += wave_tot[w];
        const int count = wave_tot[0] + wave_tot[1] + wave_tot[2] + wave_tot[3];
#pragma unroll
        for (int e = 0; e < EB_PER; ++e)
            if (r[e] >= 0) {
                tok[base] = (int)(t0 + e - w0);
                hit_row[base] = (uint8_t)r[e];
                atomicAdd(&row_cnt[r[e]], 1);  // integer count: order-free
                ++base;
            }
        __syncthreads();
        for (int rr = 0; rr < nrows; ++rr) {
            const int cnt_r = row_cnt[rr];
            if (w0 > 0 && cnt_r == 0) continue;  // earlier windows already wrote this row
            float *out = dw + (v0 + rr) * dim;
            for (int64_t c = tid; c < dim; c += 256) {
                float acc = w0 == 0 ? 0.f : out[c];
                if (cnt_r)
                    for (int m = 0; m < count; ++m)
                        if (hit_row[m] == rr) acc += dy[(w0 + tok[m]) * dim + c];
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
                                                 TG *grad, float2 *stats, int64_t rows, int64_t vocab,
                                                 float grad_scale) {
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
            if (!stats && e < vocab) {
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
        for (int64_t e = tid; !stats && e < vocab; e += 256)
            stv<TG>(g, e, (expf(x[e] - mx) * inv - ((uint64_t)e == t ? 1.0f : 0.0f)) * grad_scale);
    }
    if (tid == 0) {
        losses[row] = (int64_t)t < vocab ? -x[t] + (mx + logf(sum)) : NAN;
        // Stats mode: the row's max and 1 / sum, from which a GEMM rebuilds the gradient.
        if (stats) stats[row] = float2{mx, 1.0f / sum};
    }
}

// Mean of `n` values in a fixed order (one block): per-thread sums of a strided slice (eight loads
// in flight), then a tree.
__global__ __launch_bounds__(256) void mean_kernel(const float *v, int64_t n, float *out) {
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float s = 0.f;
    int64_t i = tid;
    for (; i + 7 * 256 < n; i += 8 * 256) {
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = v[i + 256 * j];
#pragma unroll
        for (int j = 0; j < 8; ++j) s += t[j];
    }
    for (; i < n; i += 256) s += v[i];
    s = wsum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (tid == 0) out[0] = (((red[0] + red[1]) + red[2]) + red[3]) / (float)n;
}

// ------------------------------------------------------------------ fused linear + cross entropy

// The logits are produced one vocabulary chunk [rows, vc] at a time by the GEMM; these kernels
// reduce a chunk to per-row (max, sum exp(x - max)) and the target's logit, combine the chunks into
// the row log-sum-exp and loss, and turn a (recomputed) chunk into the unscaled gradient
// softmax - onehot in place. A target outside [0, vocab) marks an ignored row.
__device__ __forceinline__ bool target_ok(int32_t t, int64_t vocab) { return t >= 0 && (int64_t)t < vocab; }

__global__ __launch_bounds__(256) void flce_chunk_stats(const float *x, int64_t ld, int64_t vc, int64_t v0,
                                                        const int32_t *targets, int64_t vocab, float2 *stats,
                                                        int64_t nchunks, int64_t chunk, float *tlogit) {
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = blockIdx.x;
    const float *xr = x + row * ld;
    float mx = -INFINITY;
    for (int64_t c = tid; c < vc; c += 256) mx = fmaxf(mx, xr[c]);
    mx = wmax(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float sum = 0.f;
    for (int64_t c = tid; c < vc; c += 256) sum += expf(xr[c] - mx);
    sum = wsum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    if (tid == 0) {
        stats[row * nchunks + chunk] = make_float2(mx, ((red[0] + red[1]) + red[2]) + red[3]);
        const int32_t t = targets[row];
        if (target_ok(t, vocab) && (int64_t)t >= v0 && (int64_t)t < v0 + vc) tlogit[row] = xr[t - v0];
    }
}

// One block: per row lse = M + log(sum_c s_c exp(m_c - M)) and loss = lse - logit[target] (0 when
// ignored); then the valid count, the mean loss and 1 / count, in a fixed order.
__global__ __launch_bounds__(1024) void flce_combine(const float2 *stats, int64_t nchunks, const float *tlogit,
                                                     const int32_t *targets, int64_t vocab, int64_t rows,
                                                     float *lse, float *losses, float *mean_out, float *scale_out) {
    __shared__ float rs[16];
    __shared__ int rc[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float tot = 0.f;
    int cnt = 0;
    for (int64_t r = tid; r < rows; r += 1024) {
        const float2 *st = stats + r * nchunks;
        float m = -INFINITY;
        for (int64_t c = 0; c < nchunks; ++c) m = fmaxf(m, st[c].x);
        float s = 0.f;
        for (int64_t c = 0; c < nchunks; ++c) s += st[c].y * expf(st[c].x - m);
        const float l = m + logf(s);
        lse[r] = l;
        if (target_ok(targets[r], vocab)) {
            losses[r] = l - tlogit[r];
            tot += losses[r];
            ++cnt;
        } else {
            losses[r] = 0.f;
        }
    }
    tot = wsum(tot);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
    if (lane == 0) {
        rs[wave] = tot;
        rc[wave] = cnt;
    }
    __syncthreads();
    if (tid == 0) {
        float t = 0.f;
        int n = 0;
        for (int w = 0; w < 16; ++w) {
            t += rs[w];
            n += rc[w];
        }
        mean_out[0] = n > 0 ? t / (float)n : 0.f;
        scale_out[0] = n > 0 ? 1.0f / (float)n : 0.f;
    }
}

// In place over a chunk: x <- exp(x - lse[row]) - [v0 + c == target] for valid rows, 0 otherwise.
__global__ __launch_bounds__(256) void flce_chunk_grad(float *x, int64_t ld, int64_t vc, int64_t v0,
                                                       const int32_t *targets, int64_t vocab, const float *lse) {
    const int64_t row = blockIdx.x;
    float *xr = x + row * ld;
    const int32_t t = targets[row];
    const bool ok = target_ok(t, vocab);
    const float l = lse[row];
    for (int64_t c = threadIdx.x; c < vc; c += 256)
        xr[c] = ok ? expf(xr[c] - l) - ((int64_t)t == v0 + c ? 1.0f : 0.0f) : 0.f;
}

// x[i] *= s[0] (the 1 / valid-count scale of grad_hidden, known only on the device).
__global__ __launch_bounds__(256) void scale_by_device_kernel(float *x, int64_t n, const float *s) {
    const float f = s[0];
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) x[i] *= f;
}

// ------------------------------------------------------------------ SwiGLU backward

// grad_up = dh * silu(g); grad_gate = dh * u * sig(g) (1 + g (1 - sig(g))), sig(g) = 1 / (1 + exp(-g)).
// One block per row; VEC consecutive columns per thread (VEC = 4 when every row start is aligned
// for 16-byte f32 / 8-byte bf16 accesses and cols % 4 == 0).
__device__ __forceinline__ void swiglu_grad(float go, float g, float u, float &dg, float &du) {
    const float sig = sigmoid_fast(g);
    const float silu = g * sig;
    du = go * silu;
    const float d_silu = sig * (1.0f + g * (1.0f - sig));
    dg = go * u * d_silu;
}

template <typename T>
__device__ __forceinline__ f32x4 ld4(const T *p) {
    if constexpr (sizeof(T) == 4) {
        return *(const f32x4 *)p;
    } else {
        const u32x2 h = *(const u32x2 *)p;
        return f32x4{__uint_as_float(h[0] << 16), __uint_as_float(h[0] & 0xffff0000u), __uint_as_float(h[1] << 16),
                     __uint_as_float(h[1] & 0xffff0000u)};
    }
}

template <typename T>
__device__ __forceinline__ void st4(T *p, f32x4 v) {
    if constexpr (sizeof(T) == 4)
        *(f32x4 *)p = v;
    else
        *(u32x2 *)p = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
}

template <typename TI, typename TO, int VEC>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const float *dh, int64_t ld_dh, const TI *gate,
                                                         const TI *up, int64_t ld_gu, TO *dgate, TO *dup,
                                                         int64_t ld_out, int64_t cols) {
    const int64_t r = blockIdx.x;
    if constexpr (VEC == 4) {
        for (int64_t c = 4 * (int64_t)threadIdx.x; c < cols; c += 1024) {
            const f32x4 go = *(const f32x4 *)(dh + r * ld_dh + c);
            const f32x4 g = ld4<TI>(gate + r * ld_gu + c), u = ld4<TI>(up + r * ld_gu + c);
            f32x4 dg, du;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float a, b;
                swiglu_grad(go[q], g[q], u[q], a, b);
                dg[q] = a;
                du[q] = b;
            }
            st4<TO>(dgate + r * ld_out + c, dg);
            st4<TO>(dup + r * ld_out + c, du);
        }
    } else {
        for (int64_t c = threadIdx.x; c < cols; c += 256) {
            float dg, du;
            swiglu_grad(dh[r * ld_dh + c], ldv<TI>(gate, r * ld_gu + c), ldv<TI>(up, r * ld_gu + c), dg, du);
            stv<TO>(dup, r * ld_out + c, du);
            stv<TO>(dgate, r * ld_out + c, dg);
        }
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
// 16-byte loads (four in flight per thread) where the tensor is 16-byte aligned; elementwise otherwise.
__global__ __launch_bounds__(256) void sumsq_kernel(const TensorTable t, double *part) {
    __shared__ double red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t b = blockIdx.x;
    const int i = table_find(t, b);
    const int64_t e0 = (b - t.first_block[i]) * MT_ELEMS;
    const int64_t e1 = min(t.n[i], e0 + MT_ELEMS);
    const float *g = t.g[i];
    double s = 0.0;
    if ((uintptr_t)g % 16 == 0 && e1 - e0 == MT_ELEMS) {
        f32x4 v[MT_ELEMS / 1024];
#pragma unroll
        for (int k = 0; k < MT_ELEMS / 1024; ++k) v[k] = *(const f32x4 *)(g + e0 + 4 * (tid + 256 * k));
#pragma unroll
        for (int k = 0; k < MT_ELEMS / 1024; ++k)
#pragma unroll
            for (int q = 0; q < 4; ++q) s += (double)v[k][q] * (double)v[k][q];
    } else {
        for (int64_t e = e0 + tid; e < e1; e += 256) {
            const double v = (double)g[e];
            s += v * v;
        }
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
// computed on the GPU, a schedule value updated between graph replays). 16-byte accesses where all
// three buffers are 16-byte aligned and the chunk is whole.
__device__ __forceinline__ void lion_elem(float &w, float &m, float g, float rate, float beta1, float beta2,
                                          float wd, float scale) {
#pragma clang fp contract(off)  // separate roundings, as the reference's expression is written
    const float gi = g * scale;
    const float u = beta2 * m + (1.0f - beta2) * gi;
    const float dir = u > 0.f ? 1.f : (u < 0.f ? -1.f : 0.f);
    m = beta1 * m + (1.0f - beta1) * gi;
    w = w - rate * dir - rate * wd * w;
}

__global__ __launch_bounds__(256) void lion_kernel(const TensorTable t, float lr, float beta1, float beta2,
                                                   float wd, const float *scale_dev, const float *lr_dev) {
    const int64_t b = blockIdx.x;
    const int i = table_find(t, b);
    const int64_t e0 = (b - t.first_block[i]) * MT_ELEMS;
    const int64_t e1 = min(t.n[i], e0 + MT_ELEMS);
    const float scale = scale_dev ? scale_dev[0] : 1.0f;
    const float rate = lr_dev ? lr_dev[0] : lr;
    float *w = t.w[i], *m = t.m[i];
    const float *g = t.g[i];
    const bool vec = ((uintptr_t)w | (uintptr_t)m | (uintptr_t)g) % 16 == 0 && e1 - e0 == MT_ELEMS;
    if (vec) {
        constexpr int NV = MT_ELEMS / 1024;
        f32x4 wv[NV], mv[NV], gv[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int64_t e = e0 + 4 * (threadIdx.x + 256 * k);
            wv[k] = *(const f32x4 *)(w + e);
            mv[k] = *(const f32x4 *)(m + e);
            gv[k] = *(const f32x4 *)(g + e);
        }
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int64_t e = e0 + 4 * (threadIdx.x + 256 * k);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float wq = wv[k][q], mq = mv[k][q];
                lion_elem(wq, mq, gv[k][q], rate, beta1, beta2, wd, scale);
                wv[k][q] = wq;
                mv[k][q] = mq;
            }
            *(f32x4 *)(w + e) = wv[k];
            *(f32x4 *)(m + e) = mv[k];
        }
    } else {
        for (int64_t e = e0 + threadIdx.x; e < e1; e += 256) {
            float wi = w[e], mi = m[e];
            lion_elem(wi, mi, g[e], rate, beta1, beta2, wd, scale);
            m[e] = mi;
            w[e] = wi;
        }
    }
}

}  // namespace

// ------------------------------------------------------------------ launchers

it_status launch_rmsnorm_forward(hipStream_t s, bool y_bf16, int64_t rows, int64_t dim, float eps, const float *x,
                                 const float *res, const float *gamma, float *sum_out, void *y) {
    const unsigned grid = blocks_for(rows, 4);
#define IT_RMSF(TY, K)                                                                                         \
    hipLaunchKernelGGL((rmsnorm_fwd_kernel<TY, K>), dim3(grid), dim3(256), 0, s, x, res, sum_out, gamma, (TY *)y, \
                       rows, dim, eps)
#define IT_RMSF_K(TY)          \
    if (dim <= 256)            \
        IT_RMSF(TY, 4);        \
    else if (dim <= 1024)      \
        IT_RMSF(TY, 16);       \
    else if (dim <= 2048)      \
        IT_RMSF(TY, 32);       \
    else                       \
        IT_RMSF(TY, 0);
    if (y_bf16) {
        IT_RMSF_K(uint16_t)
    } else {
        IT_RMSF_K(float)
    }
#undef IT_RMSF_K
#undef IT_RMSF
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

// Rows per block of the backward kernel: 4 waves x rows per wave.
static int64_t rmsnorm_bwd_rows_per_block(int64_t dim) { return dim <= 256 ? 16 : 4; }

int64_t rmsnorm_backward_scratch_bytes(int64_t rows, int64_t dim) {
    const int64_t rpb = rmsnorm_bwd_rows_per_block(dim);
    return ((rows + rpb - 1) / rpb) * dim * (int64_t)sizeof(float);
}

it_status launch_rmsnorm_backward(hipStream_t s, int64_t rows, int64_t dim, float eps, const float *dy,
                                  const float *x, const float *gamma, const float *gres, float *dx,
                                  float *dgamma, float *part) {
    const int64_t rpb = rmsnorm_bwd_rows_per_block(dim);
    const int64_t blocks = (rows + rpb - 1) / rpb;
    if (blocks > 0x7fffffff) return fail(IT_ERR_DIMS, "rmsnorm_backward: too many rows");
    const size_t lds = 4 * (size_t)dim * sizeof(float);
    if (dim <= 256)
        hipLaunchKernelGGL((rmsnorm_bwd_kernel<4, 4>), dim3((unsigned)blocks), dim3(256), lds, s, dy, x, gamma, gres,
                           dx, part, rows, dim, eps);
    else if (dim <= 1024)
        hipLaunchKernelGGL((rmsnorm_bwd_kernel<16, 1>), dim3((unsigned)blocks), dim3(256), lds, s, dy, x, gamma,
                           gres, dx, part, rows, dim, eps);
    else
        hipLaunchKernelGGL((rmsnorm_bwd_kernel<32, 1>), dim3((unsigned)blocks), dim3(256), lds, s, dy, x, gamma,
                           gres, dx, part, rows, dim, eps);
    IT_HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(rmsnorm_dgamma_reduce, dim3(blocks_for(dim, 64)), dim3(1024), 0, s, part, dgamma, blocks, dim);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_rope_table(hipStream_t s, int64_t seq, int64_t head_dim, float base, int64_t offset, void *table) {
    const int64_t n = seq * (head_dim / 2);
    if (n == 0) return IT_OK;
    hipLaunchKernelGGL(rope_table_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, (float2 *)table, seq, head_dim,
                       base, offset);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_rope(hipStream_t s, bool src_bf16, bool dst_bf16, int64_t batch, int64_t seq, int64_t heads,
                      int64_t head_dim, const void *table, int backward, const void *src, int64_t src_rs,
                      void *dst, int64_t dst_rs, int64_t copy_cols) {
    const int64_t rows = batch * seq;
    const int half = (int)(head_dim / 2);
    if (heads * half > 0x3fffffff || copy_cols > 0x3fffffff) return fail(IT_ERR_DIMS, "rope: rows too wide");
    const int64_t per_row = heads * half + (copy_cols + 1) / 2;
    const int64_t blocks = (rows * per_row + 255) / 256;
    if (blocks > 0x7fffffff) return fail(IT_ERR_DIMS, "rope: too many elements");
    if (blocks == 0) return IT_OK;
#define IT_ROPE(TS, TD)                                                                                         \
    hipLaunchKernelGGL((rope_kernel<TS, TD>), dim3((unsigned)blocks), dim3(256), 0, s, (const TS *)src, (TD *)dst, \
                       (const float2 *)table, rows, seq, (int)heads, half, src_rs, dst_rs, (int)copy_cols, backward)
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
                               const uint32_t *targets, float *losses, void *grad, float *stats, float *loss_mean,
                               bool vec_ok) {
    const float gs = 1.0f / (float)rows;
    const dim3 grid((unsigned)rows), block(256);
#define IT_CE(NPT, TG)                                                                                    \
    hipLaunchKernelGGL((ce_kernel<NPT, TG>), grid, block, 0, s, logits, targets, losses, (TG *)grad,       \
                       (float2 *)stats, rows, vocab, gs)
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

it_status launch_flce_chunk_stats(hipStream_t s, const float *x, int64_t ld, int64_t rows, int64_t vc, int64_t v0,
                                  const int32_t *targets, int64_t vocab, void *stats, int64_t nchunks, int64_t chunk,
                                  float *tlogit) {
    hipLaunchKernelGGL(flce_chunk_stats, dim3((unsigned)rows), dim3(256), 0, s, x, ld, vc, v0, targets, vocab,
                       (float2 *)stats, nchunks, chunk, tlogit);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_flce_combine(hipStream_t s, const void *stats, int64_t nchunks, const float *tlogit,
                              const int32_t *targets, int64_t vocab, int64_t rows, float *lse, float *losses,
                              float *mean_out, float *scale_out) {
    hipLaunchKernelGGL(flce_combine, dim3(1), dim3(1024), 0, s, (const float2 *)stats, nchunks, tlogit, targets, vocab,
                       rows, lse, losses, mean_out, scale_out);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_flce_chunk_grad(hipStream_t s, float *x, int64_t ld, int64_t rows, int64_t vc, int64_t v0,
                                 const int32_t *targets, int64_t vocab, const float *lse) {
    hipLaunchKernelGGL(flce_chunk_grad, dim3((unsigned)rows), dim3(256), 0, s, x, ld, vc, v0, targets, vocab, lse);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_scale_by_device(hipStream_t s, float *x, int64_t n, const float *scale) {
    hipLaunchKernelGGL(scale_by_device_kernel, dim3(blocks_for(n, 256 * 4, 65536)), dim3(256), 0, s, x, n, scale);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_swiglu_backward(hipStream_t s, bool in_bf16, bool out_bf16, int64_t rows, int64_t cols,
                                 const float *dh, int64_t ld_dh, const void *gate, const void *up, int64_t ld_gu,
                                 void *dgate, void *dup, int64_t ld_out) {
    const dim3 grid((unsigned)rows);
    const uintptr_t ia = in_bf16 ? 8 : 16, oa = out_bf16 ? 8 : 16;
    const bool vec = cols % 4 == 0 && ld_dh % 4 == 0 && ld_gu % 4 == 0 && ld_out % 4 == 0 && (uintptr_t)dh % 16 == 0 &&
                     (uintptr_t)gate % ia == 0 && (uintptr_t)up % ia == 0 && (uintptr_t)dgate % oa == 0 &&
                     (uintptr_t)dup % oa == 0;
#define IT_SWB(TI, TO)                                                                                           \
    if (vec)                                                                                                     \
        hipLaunchKernelGGL((swiglu_bwd_kernel<TI, TO, 4>), grid, dim3(256), 0, s, dh, ld_dh, (const TI *)gate,   \
                           (const TI *)up, ld_gu, (TO *)dgate, (TO *)dup, ld_out, cols);                         \
    else                                                                                                         \
        hipLaunchKernelGGL((swiglu_bwd_kernel<TI, TO, 1>), grid, dim3(256), 0, s, dh, ld_dh, (const TI *)gate,   \
                           (const TI *)up, ld_gu, (TO *)dgate, (TO *)dup, ld_out, cols);
    if (!in_bf16 && !out_bf16) {
        IT_SWB(float, float)
    } else if (!in_bf16 && out_bf16) {
        IT_SWB(float, uint16_t)
    } else if (in_bf16 && out_bf16) {
        IT_SWB(uint16_t, uint16_t)
    } else {
        IT_SWB(uint16_t, float)
    }
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
