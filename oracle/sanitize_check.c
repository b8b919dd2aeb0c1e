/*
 * Exercises every function of the CPU oracle (ref.c, train_ref.c) once on small, ragged shapes,
 * with every buffer allocated at its exact size, for a build under AddressSanitizer and
 * UndefinedBehaviorSanitizer (make -C oracle sanitize). TEST INFRASTRUCTURE ONLY: a sanitizer
 * report or a failed consistency check ends the program with a non-zero status.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ref.h"

static uint64_t g_state = 0x9E3779B97F4A7C15ull;

static float rnd(void) {
    g_state ^= g_state << 13;
    g_state ^= g_state >> 7;
    g_state ^= g_state << 17;
    return (float)((g_state >> 11) * (1.0 / 9007199254740992.0)) * 2.0f - 1.0f;
}

static float *fbuf(int64_t n) {
    float *p = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    for (int64_t i = 0; i < n; ++i) p[i] = rnd();
    return p;
}

static int g_fail = 0;

static void check(int ok, const char *what) {
    if (!ok) {
        fprintf(stderr, "FAIL %s\n", what);
        g_fail = 1;
    }
}

static void gemm_layouts(int threads) {
    const int64_t M = 7, N = 5, K = 3, batch = 2;
    for (int ta = 0; ta < 2; ++ta)
        for (int tb = 0; tb < 2; ++tb) {
            const int64_t lda = ta ? M : K, ldb = tb ? K : N;
            float *A = fbuf(batch * M * K), *B = fbuf(batch * K * N), *C = fbuf(batch * M * N);
            double *D = (double *)malloc((size_t)(batch * M * N) * sizeof(double));
            ref_gemm_f32(ta, tb, M, N, K, A, lda, M * K, B, ldb, K * N, C, N, M * N, batch, threads);
            ref_gemm_f64(ta, tb, M, N, K, A, lda, M * K, B, ldb, K * N, D, N, M * N, batch, threads);
            for (int64_t i = 0; i < batch * M * N; ++i) check(fabs(C[i] - D[i]) < 1e-5, "gemm f32 vs f64");
            uint16_t *Ah = (uint16_t *)malloc((size_t)(batch * M * K) * 2), *Bh = (uint16_t *)malloc((size_t)(batch * K * N) * 2);
            ref_f32_to_bf16_n(A, Ah, batch * M * K);
            ref_f32_to_bf16_n(B, Bh, batch * K * N);
            uint16_t *Ch = (uint16_t *)malloc((size_t)(batch * M * N) * 2);
            ref_gemm_bf16(ta, tb, M, N, K, Ah, lda, M * K, Bh, ldb, K * N, C, 0, N, M * N, batch, threads);
            ref_gemm_bf16(ta, tb, M, N, K, Ah, lda, M * K, Bh, ldb, K * N, Ch, 1, N, M * N, batch, threads);
            float *Cw = fbuf(batch * M * N);
            ref_bf16_to_f32_n(Ch, Cw, batch * M * N);
            for (int64_t i = 0; i < batch * M * N; ++i) check(ref_f32_to_bf16(C[i]) == Ch[i], "gemm bf16 out is RNE of f32");
            free(A), free(B), free(C), free(D), free(Ah), free(Bh), free(Ch), free(Cw);
        }
}

int main(void) {
    check(ref_bf16_to_f32(ref_f32_to_bf16(1.5f)) == 1.5f, "bf16 round trip");
    gemm_layouts(1);
    gemm_layouts(3);

    const int64_t M = 6, N = 9;
    float *Y = fbuf(M * N), *bias = fbuf(N);
    ref_add_bias(Y, bias, M, N);
    float *g = fbuf(M * N), *u = fbuf(M * N), *h = fbuf(M * N), *dg = fbuf(M * N), *du = fbuf(M * N);
    ref_swiglu(g, u, h, M * N);
    ref_swiglu_backward(Y, g, u, dg, du, M * N);
    ref_softmax_rows(Y, M, N);
    for (int64_t r = 0; r < M; ++r) {
        double s = 0;
        for (int64_t c = 0; c < N; ++c) s += Y[r * N + c];
        check(fabs(s - 1.0) < 1e-5, "softmax rows sum to 1");
    }
    ref_softmax_backward(g, Y, h, M, N);

    const int64_t b = 2, s = 5, hh = 3, d = 4, bh = b * hh;
    float *q = fbuf(b * s * hh * d), *k = fbuf(b * s * hh * d), *v = fbuf(b * s * hh * d), *o = fbuf(b * s * hh * d);
    for (int causal = 0; causal < 2; ++causal) {
        ref_attention_bshd(q, k, v, o, b, s, hh, d, causal, 2);
        float *P = fbuf(bh * s * s), *o2 = fbuf(bh * s * d), *dq = fbuf(bh * s * d), *dk = fbuf(bh * s * d),
              *dv = fbuf(bh * s * d);
        ref_attention_fwd_bhsd(q, k, v, o2, P, bh, s, d, 0.5f, causal, 2);
        ref_attention_fwd_bhsd(q, k, v, o2, NULL, bh, s, d, 0.5f, causal, 1);
        ref_attention_bwd_bhsd(o, q, k, v, dq, dk, dv, bh, s, d, 0.5f, causal, 2);
        free(P), free(o2), free(dq), free(dk), free(dv);
    }
    check(ref_default_threads() >= 1, "default threads");

    const int64_t rows = 5, dim = 8;
    float *x = fbuf(rows * dim), *gamma = fbuf(dim), *y = fbuf(rows * dim), *dx = fbuf(rows * dim),
          *dgam = fbuf(dim);
    ref_rmsnorm_forward(x, gamma, y, rows, dim, 1e-5f);
    ref_rmsnorm_backward(y, x, gamma, dx, dgam, rows, dim, 1e-5f);
    float *qkv = fbuf(2 * 3 * (3 * 2 * 4));  /* batch 2, seq 3, row of 3 heads x 2 x dim 4 */
    ref_rope(qkv, 2, 3, 2, 4, 3 * 2 * 4, 10000.0f, 1, 0);
    ref_rope(qkv, 2, 3, 2, 4, 3 * 2 * 4, 10000.0f, 1, 1);
    const int64_t vocab = 7, ntok = 6;
    uint32_t ids[6] = {0, 6, 3, 3, 1, 6};
    float *table = fbuf(vocab * dim), *emb = fbuf(ntok * dim), *dw = fbuf(vocab * dim);
    ref_embedding_forward(table, ids, emb, ntok, dim);
    ref_embedding_backward(emb, ids, dw, ntok, dim, vocab);
    float *logits = fbuf(ntok * vocab), *losses = fbuf(ntok), *grad = fbuf(ntok * vocab);
    const float loss = ref_cross_entropy(logits, ids, losses, grad, ntok, vocab);
    check(loss > 0.0f && isfinite(loss), "cross entropy");
    float *w = fbuf(vocab * dim), *m = fbuf(vocab * dim);
    ref_lion(w, m, dw, vocab * dim, 1e-3f, 0.9f, 0.99f, 0.1f, 0.5f);
    check(ref_sum_squares(w, vocab * dim) > 0.0, "sum of squares");
    int32_t tgt[6] = {0, 6, -100, 3, 1, 6};
    float *gh = fbuf(ntok * dim), *gw = fbuf(vocab * dim);
    ref_fused_linear_cross_entropy(emb, table, tgt, losses, gh, gw, ntok, dim, vocab);
    float *fo = fbuf(rows * vocab);
    ref_fused_rmsnorm_linear(x, gamma, table, fo, rows, dim, vocab, 1e-5f);
    float *t3 = fbuf(2 * 3 * 4), *t3o = fbuf(2 * 4 * 3), *sq = fbuf(2 * 4 * 4), *sqo = fbuf(2 * 4 * 4);
    ref_transpose_3d(t3, t3o, 2, 3, 4);
    ref_causal_mask_3d(sq, sqo, 2, 4);

    free(Y), free(bias), free(g), free(u), free(h), free(dg), free(du), free(q), free(k), free(v), free(o);
    free(x), free(gamma), free(y), free(dx), free(dgam), free(qkv), free(table), free(emb), free(dw);
    free(logits), free(losses), free(grad), free(w), free(m), free(gh), free(gw), free(fo), free(t3), free(t3o);
    free(sq), free(sqo);
    printf(g_fail ? "oracle sanitize check: FAILED\n" : "oracle sanitize check: ok\n");
    return g_fail;
}
