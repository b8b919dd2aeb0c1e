/*
 * IronTensor matmul-path CPU ORACLE -- test infrastructure only (see ref.h for the contract and
 * for what pins each function).  Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 */
#include "ref.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#if defined(__FAST_MATH__)
#error "the oracle must not be built with fast-math"
#endif

/* ------------------------------------------------------------------ threading helper */

typedef void (*row_fn)(void *ctx, int64_t row_begin, int64_t row_end);

typedef struct {
    row_fn fn;
    void *ctx;
    int64_t begin, end;
} row_task;

static void *row_task_main(void *p) {
    row_task *t = (row_task *)p;
    t->fn(t->ctx, t->begin, t->end);
    return NULL;
}

/* Split [0, rows) into contiguous chunks, one per thread.  Each output row is produced by exactly
 * one thread with the sequential loop, so the thread count never changes any result. */
static void parallel_rows(row_fn fn, void *ctx, int64_t rows, int nthreads) {
    if (nthreads <= 1 || rows < 2) {
        fn(ctx, 0, rows);
        return;
    }
    if (nthreads > rows) nthreads = (int)rows;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    row_task tasks[256];
    int64_t chunk = (rows + nthreads - 1) / nthreads;
    int launched = 0;
    for (int t = 0; t < nthreads; ++t) {
        int64_t b = (int64_t)t * chunk, e = b + chunk;
        if (b >= rows) break;
        if (e > rows) e = rows;
        tasks[t].fn = fn;
        tasks[t].ctx = ctx;
        tasks[t].begin = b;
        tasks[t].end = e;
        if (pthread_create(&th[t], NULL, row_task_main, &tasks[t]) != 0) {
            row_task_main(&tasks[t]); /* run inline if a thread cannot be created */
            th[t] = 0;
        }
        ++launched;
    }
    for (int t = 0; t < launched; ++t)
        if (th[t]) pthread_join(th[t], NULL);
}

int ref_default_threads(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

/* ------------------------------------------------------------------ bf16 (precision.rs) */

uint16_t ref_f32_to_bf16(float x) {
    /* src/precision.rs:24-29: bits + (0x7FFF + ((bits >> 16) & 1)), wrapping, then >> 16. */
    uint32_t bits;
    memcpy(&bits, &x, 4);
    uint32_t round = ((bits >> 16) & 1u) + 0x7FFFu;
    return (uint16_t)((bits + round) >> 16);
}

float ref_bf16_to_f32(uint16_t x) {
    /* src/precision.rs:33-35 */
    uint32_t bits = (uint32_t)x << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void ref_f32_to_bf16_n(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = ref_f32_to_bf16(src[i]);
}

void ref_bf16_to_f32_n(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = ref_bf16_to_f32(src[i]);
}

/* ------------------------------------------------------------------ GEMM loops */

typedef struct {
    int transA, transB;
    int64_t M, N, K;
    const void *A;
    int64_t lda, sA;
    const void *B;
    int64_t ldb, sB;
    void *C;
    int64_t ldc, sC;
    int kind; /* 0: f32 in/out; 1: f32 in, f64 acc/out; 2: bf16 in, f32 out; 3: bf16 in, bf16 out */
} gemm_ctx;

static inline int64_t a_index(const gemm_ctx *g, int64_t i, int64_t p) {
    return g->transA ? p * g->lda + i : i * g->lda + p;
}
static inline int64_t b_index(const gemm_ctx *g, int64_t p, int64_t j) {
    return g->transB ? j * g->ldb + p : p * g->ldb + j;
}

/* One "row" of work is one (batch, i) pair; the inner loops are the reference's triple loop. */
static void gemm_rows(void *vctx, int64_t r0, int64_t r1) {
    const gemm_ctx *g = (const gemm_ctx *)vctx;
    for (int64_t r = r0; r < r1; ++r) {
        int64_t b = r / g->M, i = r % g->M;
        switch (g->kind) {
        case 0: {
            const float *A = (const float *)g->A + b * g->sA;
            const float *B = (const float *)g->B + b * g->sB;
            float *C = (float *)g->C + b * g->sC + i * g->ldc;
            for (int64_t j = 0; j < g->N; ++j) {
                float acc = 0.0f;
                for (int64_t p = 0; p < g->K; ++p) {
                    float prod = A[a_index(g, i, p)] * B[b_index(g, p, j)];
                    acc = acc + prod;
                }
                C[j] = acc;
            }
            break;
        }
        case 1: {
            const float *A = (const float *)g->A + b * g->sA;
            const float *B = (const float *)g->B + b * g->sB;
            double *C = (double *)g->C + b * g->sC + i * g->ldc;
            for (int64_t j = 0; j < g->N; ++j) {
                double acc = 0.0;
                for (int64_t p = 0; p < g->K; ++p)
                    acc += (double)A[a_index(g, i, p)] * (double)B[b_index(g, p, j)];
                C[j] = acc;
            }
            break;
        }
        default: {
            const uint16_t *A = (const uint16_t *)g->A + b * g->sA;
            const uint16_t *B = (const uint16_t *)g->B + b * g->sB;
            for (int64_t j = 0; j < g->N; ++j) {
                float acc = 0.0f;
                for (int64_t p = 0; p < g->K; ++p) {
                    float prod = ref_bf16_to_f32(A[a_index(g, i, p)]) *
                                 ref_bf16_to_f32(B[b_index(g, p, j)]);
                    acc = acc + prod;
                }
                if (g->kind == 2)
                    ((float *)g->C)[b * g->sC + i * g->ldc + j] = acc;
                else
                    ((uint16_t *)g->C)[b * g->sC + i * g->ldc + j] = ref_f32_to_bf16(acc);
            }
            break;
        }
        }
    }
}

static void run_gemm(gemm_ctx *g, int64_t batch, int nthreads) {
    if (g->M <= 0 || g->N <= 0 || batch <= 0) return;
    parallel_rows(gemm_rows, g, batch * g->M, nthreads);
}

void ref_gemm_f32(int transA, int transB, int64_t M, int64_t N, int64_t K,
                  const float *A, int64_t lda, int64_t strideA,
                  const float *B, int64_t ldb, int64_t strideB,
                  float *C, int64_t ldc, int64_t strideC, int64_t batch, int nthreads) {
    gemm_ctx g = {transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB, C, ldc, strideC, 0};
    run_gemm(&g, batch, nthreads);
}

void ref_gemm_f64(int transA, int transB, int64_t M, int64_t N, int64_t K,
                  const float *A, int64_t lda, int64_t strideA,
                  const float *B, int64_t ldb, int64_t strideB,
                  double *C, int64_t ldc, int64_t strideC, int64_t batch, int nthreads) {
    gemm_ctx g = {transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB, C, ldc, strideC, 1};
    run_gemm(&g, batch, nthreads);
}

void ref_gemm_bf16(int transA, int transB, int64_t M, int64_t N, int64_t K,
                   const uint16_t *A, int64_t lda, int64_t strideA,
                   const uint16_t *B, int64_t ldb, int64_t strideB,
                   void *C, int out_bf16, int64_t ldc, int64_t strideC, int64_t batch,
                   int nthreads) {
    gemm_ctx g = {transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB, C, ldc, strideC,
                  out_bf16 ? 3 : 2};
    run_gemm(&g, batch, nthreads);
}

/* ------------------------------------------------------------------ epilogue specs */

void ref_add_bias(float *Y, const float *bias, int64_t M, int64_t N) {
    /* src/nn/linear.rs:8-18: result[b * out + o] += bias[o] */
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) Y[m * N + n] = Y[m * N + n] + bias[n];
}

void ref_swiglu(const float *gate, const float *up, float *out, int64_t n) {
    /* src/shaders/elementwise.metal:107-113 */
    for (int64_t i = 0; i < n; ++i) {
        float g = gate[i];
        float sig = 1.0f / (1.0f + expf(-g));
        float silu = g * sig;
        out[i] = silu * up[i];
    }
}

void ref_swiglu_backward(const float *grad_out, const float *gate, const float *up,
                         float *grad_gate, float *grad_up, int64_t n) {
    /* src/shaders/backward/elementwise.metal:111-125 */
    for (int64_t i = 0; i < n; ++i) {
        float g = gate[i], u = up[i], go = grad_out[i];
        float sig = 1.0f / (1.0f + expf(-g));
        float silu = g * sig;
        grad_up[i] = go * silu;
        float d_silu = sig * (1.0f + g * (1.0f - sig));
        grad_gate[i] = go * u * d_silu;
    }
}

/* ------------------------------------------------------------------ softmax */

static void softmax_row(float *row, int64_t cols) {
    /* src/ops/attention.rs:580-588 */
    float mx = -INFINITY;
    for (int64_t c = 0; c < cols; ++c) mx = fmaxf(mx, row[c]);
    float sum = 0.0f;
    for (int64_t c = 0; c < cols; ++c) sum = sum + expf(row[c] - mx);
    for (int64_t c = 0; c < cols; ++c) row[c] = expf(row[c] - mx) / sum;
}

void ref_softmax_rows(float *X, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) softmax_row(X + r * cols, cols);
}

void ref_softmax_backward(const float *grad_y, const float *y, float *grad_x, int64_t rows,
                          int64_t cols) {
    /* src/shaders/backward/softmax.metal:29-44 */
    for (int64_t r = 0; r < rows; ++r) {
        const float *gy = grad_y + r * cols, *yy = y + r * cols;
        float dot = 0.0f;
        for (int64_t c = 0; c < cols; ++c) dot = dot + gy[c] * yy[c];
        for (int64_t c = 0; c < cols; ++c) grad_x[r * cols + c] = yy[c] * (gy[c] - dot);
    }
}

/* ------------------------------------------------------------------ attention */

typedef struct {
    const float *q, *k, *v;
    float *out, *P;
    int64_t seq, heads, head_dim;
    int64_t row_stride; /* elements between consecutive positions of one head */
    int64_t head_stride, batch_stride;
    float scale;
    int causal;
} attn_ctx;

/* One unit of work is one (batch, head) pair, as in reference_attention's outer loops. */
static void attn_units(void *vctx, int64_t u0, int64_t u1) {
    const attn_ctx *a = (const attn_ctx *)vctx;
    int64_t S = a->seq, D = a->head_dim;
    float *scores = (float *)malloc(sizeof(float) * (size_t)(S * S));
    if (!scores) abort();
    for (int64_t u = u0; u < u1; ++u) {
        int64_t b = u / a->heads, h = u % a->heads;
        int64_t base = b * a->batch_stride + h * a->head_stride;
        for (int64_t qp = 0; qp < S; ++qp)
            for (int64_t kp = 0; kp < S; ++kp) {
                float dot = 0.0f;
                for (int64_t d = 0; d < D; ++d) {
                    float prod = a->q[base + qp * a->row_stride + d] *
                                 a->k[base + kp * a->row_stride + d];
                    dot = dot + prod;
                }
                scores[qp * S + kp] = dot * a->scale;
            }
        if (a->causal)
            for (int64_t qp = 0; qp < S; ++qp)
                for (int64_t kp = qp + 1; kp < S; ++kp) scores[qp * S + kp] = -INFINITY;
        ref_softmax_rows(scores, S, S);
        if (a->P) memcpy(a->P + u * S * S, scores, sizeof(float) * (size_t)(S * S));
        for (int64_t qp = 0; qp < S; ++qp)
            for (int64_t d = 0; d < D; ++d) {
                float sum = 0.0f;
                for (int64_t kp = 0; kp < S; ++kp) {
                    float prod = scores[qp * S + kp] * a->v[base + kp * a->row_stride + d];
                    sum = sum + prod;
                }
                a->out[base + qp * a->row_stride + d] = sum;
            }
    }
    free(scores);
}

void ref_attention_bshd(const float *q, const float *k, const float *v, float *out,
                        int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, int causal,
                        int nthreads) {
    attn_ctx a = {q, k, v, out, NULL, seq, heads, head_dim,
                  heads * head_dim, head_dim, seq * heads * head_dim,
                  1.0f / sqrtf((float)head_dim), causal};
    parallel_rows(attn_units, &a, batch * heads, nthreads);
}

void ref_attention_fwd_bhsd(const float *q, const float *k, const float *v, float *out, float *P,
                            int64_t bh, int64_t seq, int64_t head_dim, float scale, int causal,
                            int nthreads) {
    attn_ctx a = {q, k, v, out, P, seq, 1, head_dim, head_dim, 0, seq * head_dim, scale, causal};
    parallel_rows(attn_units, &a, bh, nthreads);
}

void ref_attention_bwd_bhsd(const float *dO, const float *q, const float *k, const float *v,
                            float *dQ, float *dK, float *dV,
                            int64_t bh, int64_t seq, int64_t head_dim, float scale, int causal,
                            int nthreads) {
    /* src/train/helpers.rs:142-182, one matmul at a time on [BH,S,*] views. */
    int64_t S = seq, D = head_dim;
    size_t ss = (size_t)(bh * S * S);
    float *P = (float *)malloc(sizeof(float) * ss);
    float *dP = (float *)malloc(sizeof(float) * ss);
    float *dS = (float *)malloc(sizeof(float) * ss);
    if (!P || !dP || !dS) abort();
    /* scores = Q . K^T (NT), then scale, mask, softmax */
    ref_gemm_f32(0, 1, S, S, D, q, D, S * D, k, D, S * D, P, S, S * S, bh, nthreads);
    for (size_t i = 0; i < ss; ++i) P[i] = P[i] * scale;
    if (causal)
        for (int64_t u = 0; u < bh; ++u)
            for (int64_t r = 0; r < S; ++r)
                for (int64_t c = r + 1; c < S; ++c) P[u * S * S + r * S + c] = -INFINITY;
    ref_softmax_rows(P, bh * S, S);
    /* dV = P^T . dO (TN) */
    ref_gemm_f32(1, 0, S, D, S, P, S, S * S, dO, D, S * D, dV, D, S * D, bh, nthreads);
    /* dP = dO . V^T (NT) */
    ref_gemm_f32(0, 1, S, S, D, dO, D, S * D, v, D, S * D, dP, S, S * S, bh, nthreads);
    ref_softmax_backward(dP, P, dS, bh * S, S);
    /* dQ = (dS . K) * scale (NN) ; dK = (dS^T . Q) * scale (TN) */
    ref_gemm_f32(0, 0, S, D, S, dS, S, S * S, k, D, S * D, dQ, D, S * D, bh, nthreads);
    ref_gemm_f32(1, 0, S, D, S, dS, S, S * S, q, D, S * D, dK, D, S * D, bh, nthreads);
    for (int64_t i = 0; i < bh * S * D; ++i) {
        dQ[i] = dQ[i] * scale;
        dK[i] = dK[i] * scale;
    }
    free(P);
    free(dP);
    free(dS);
}

/* ------------------------------------------------------------------ attention helpers */

void ref_transpose_3d(const float *in, float *out, int64_t batch, int64_t m, int64_t n) {
    /* src/shaders/attention.metal:169-181: one output element per (b, j, i). */
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t j = 0; j < n; ++j)
            for (int64_t i = 0; i < m; ++i) out[b * n * m + j * m + i] = in[b * m * n + i * n + j];
}

void ref_causal_mask_3d(const float *in, float *out, int64_t batch, int64_t seq) {
    /* src/shaders/attention.metal:193-206 */
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t r = 0; r < seq; ++r)
            for (int64_t c = 0; c < seq; ++c) {
                const int64_t idx = b * seq * seq + r * seq + c;
                out[idx] = c > r ? -INFINITY : in[idx];
            }
}
