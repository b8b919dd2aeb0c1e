/*
 * CPU ORACLE for the training-step ops around the contractions -- test infrastructure only
 * (see ref.h). Plain-C restatements of the reference's Metal kernels, in their arithmetic order,
 * built -ffp-contract=off. Each function cites the reference it follows; tests/test_oracle_train.py
 * pins each with closed forms, identities and finite differences.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "ref.h"

/* RMSNorm forward, src/shaders/norm.metal:16-44 (rmsnorm_f32): per row, sum of squares in index
 * order, rms = sqrt(sum/n + eps), y = x * (1/rms) * gamma. */
void ref_rmsnorm_forward(const float *x, const float *gamma, float *y, int64_t rows, int64_t dim, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * dim;
        float ss = 0.0f;
        for (int64_t i = 0; i < dim; ++i) ss += xr[i] * xr[i];
        const float rms = sqrtf(ss / (float)dim + eps);
        const float inv = 1.0f / rms;
        for (int64_t i = 0; i < dim; ++i) y[r * dim + i] = xr[i] * inv * gamma[i];
    }
}

/* RMSNorm backward, src/shaders/backward/norm.metal:22-69: s = 1/rms, dot = sum dy*gamma*x,
 * dx = dy*gamma*s - (1/n)*s^3*x*dot, dgamma += dy*x*s over rows (in row order here; the
 * reference adds atomically). */
void ref_rmsnorm_backward(const float *dy, const float *x, const float *gamma, float *dx, float *dgamma,
                          int64_t rows, int64_t dim, float eps) {
    const float n = (float)dim;
    for (int64_t i = 0; i < dim; ++i) dgamma[i] = 0.0f;
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * dim, *gr = dy + r * dim;
        float ss = 0.0f;
        for (int64_t i = 0; i < dim; ++i) ss += xr[i] * xr[i];
        const float rms = sqrtf(ss / n + eps);
        const float s = 1.0f / rms, s3 = s * s * s;
        float dot = 0.0f;
        for (int64_t i = 0; i < dim; ++i) dot += gr[i] * gamma[i] * xr[i];
        for (int64_t i = 0; i < dim; ++i) {
            dx[r * dim + i] = gr[i] * gamma[i] * s - (1.0f / n) * s3 * xr[i] * dot;
            dgamma[i] += gr[i] * xr[i] * s;
        }
    }
}

/* RoPE, src/shaders/rope.metal:22-62 (forward) and src/shaders/backward/rope.metal:25-62
 * (backward, the transposed rotation). x is [batch, seq, heads, head_dim] with row stride
 * `row_stride` elements between consecutive (batch, seq) positions (heads*head_dim when
 * contiguous); pairs (2i, 2i+1), theta_i = 1 / base^(2i/d), angle = (pos + offset) * theta_i. */
void ref_rope(float *x, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, int64_t row_stride,
              float base, int64_t offset, int backward) {
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t s = 0; s < seq; ++s)
            for (int64_t h = 0; h < heads; ++h)
                for (int64_t i = 0; i < head_dim / 2; ++i) {
                    const float theta = 1.0f / powf(base, (float)(i * 2) / (float)head_dim);
                    const float angle = (float)(s + offset) * theta;
                    const float c = cosf(angle), sn = sinf(angle);
                    float *p = x + (b * seq + s) * row_stride + h * head_dim + 2 * i;
                    const float x0 = p[0], x1 = p[1];
                    if (!backward) {
                        p[0] = x0 * c - x1 * sn;
                        p[1] = x0 * sn + x1 * c;
                    } else {
                        p[0] = x0 * c + x1 * sn;
                        p[1] = -x0 * sn + x1 * c;
                    }
                }
}

/* Embedding, src/shaders/embedding.metal:15-33 (gather) and the backward scatter-add
 * (src/shaders/embedding.metal:35-..., src/ops/backward/embedding.rs:21-61): rows of dY added into
 * dW[ids[i]] in index order. */
void ref_embedding_forward(const float *table, const uint32_t *ids, float *out, int64_t n, int64_t dim) {
    for (int64_t i = 0; i < n; ++i) memcpy(out + i * dim, table + (int64_t)ids[i] * dim, sizeof(float) * dim);
}

void ref_embedding_backward(const float *dy, const uint32_t *ids, float *dw, int64_t n, int64_t dim, int64_t vocab) {
    memset(dw, 0, sizeof(float) * (size_t)(vocab * dim));
    for (int64_t i = 0; i < n; ++i)
        for (int64_t j = 0; j < dim; ++j) dw[(int64_t)ids[i] * dim + j] += dy[i * dim + j];
}

/* Fused cross entropy, src/shaders/loss.metal:91-131 with the mean of src/ops/backward/loss.rs:
 * per row max, exp(x - max) summed in order, loss = -x[t] + max + log(sum), grad = (softmax -
 * onehot) * (1/rows); returns the mean loss (sum of row losses in order / rows). */
float ref_cross_entropy(const float *logits, const uint32_t *targets, float *losses, float *grad, int64_t rows,
                        int64_t vocab) {
    const float gs = 1.0f / (float)rows;
    float total = 0.0f;
    for (int64_t r = 0; r < rows; ++r) {
        const float *x = logits + r * vocab;
        float *g = grad + r * vocab;
        float mx = x[0];
        for (int64_t i = 1; i < vocab; ++i) mx = fmaxf(mx, x[i]);
        float sum = 0.0f;
        for (int64_t i = 0; i < vocab; ++i) {
            const float e = expf(x[i] - mx);
            g[i] = e;
            sum += e;
        }
        losses[r] = -x[targets[r]] + (mx + logf(sum));
        const float inv = 1.0f / sum;
        for (int64_t i = 0; i < vocab; ++i) g[i] = (g[i] * inv - (i == (int64_t)targets[r] ? 1.0f : 0.0f)) * gs;
        total += losses[r];
    }
    return total / (float)rows;
}

/* Lion, src/shaders/lion.metal (lion_step_f32): direction sign(beta2*m + (1-beta2)*g) (sign(0)=0),
 * momentum m = beta1*m + (1-beta1)*g, w = w - lr*dir - lr*wd*w. `scale` multiplies g first (the
 * trainer's gradient clipping, src/train/trainer/train_step.rs:405-414). */
void ref_lion(float *w, float *m, const float *g, int64_t n, float lr, float beta1, float beta2, float wd,
              float scale) {
    for (int64_t i = 0; i < n; ++i) {
        const float gi = g[i] * scale;
        const float u = beta2 * m[i] + (1.0f - beta2) * gi;
        const float dir = u > 0.0f ? 1.0f : (u < 0.0f ? -1.0f : 0.0f);
        m[i] = beta1 * m[i] + (1.0f - beta1) * gi;
        w[i] = w[i] - lr * dir - lr * wd * w[i];
    }
}

/* Global gradient L2 norm over several buffers (total_l2_norm_gpu, src/ops/reduction.rs), summed in
 * double to give an order-independent reference. */
double ref_sum_squares(const float *x, int64_t n) {
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) s += (double)x[i] * (double)x[i];
    return s;
}

/* Fused RMSNorm + projection, src/shaders/fused_rmsnorm_linear.metal:42-114: per row, sum of squares
 * in index order, inv = 1 / sqrt(sum/n + eps); out[o] = (sum_j (x_j * gamma_j) * W[o][j], j in order)
 * * inv. (The reference's own test compares against rmsnorm then matmul,
 * src/ops/fused_rmsnorm_linear.rs:214-245; the same value up to rounding.) */
void ref_fused_rmsnorm_linear(const float *x, const float *gamma, const float *w, float *out, int64_t rows,
                              int64_t hidden, int64_t out_features, float eps) {
    float *xg = (float *)malloc(sizeof(float) * (size_t)(hidden > 0 ? hidden : 1));
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * hidden;
        float ss = 0.0f;
        for (int64_t j = 0; j < hidden; ++j) {
            ss += xr[j] * xr[j];
            xg[j] = xr[j] * gamma[j];
        }
        const float rms = sqrtf(ss / (float)hidden + eps);
        const float inv = 1.0f / rms;
        for (int64_t o = 0; o < out_features; ++o) {
            const float *wo = w + o * hidden;
            float sum = 0.0f;
            for (int64_t j = 0; j < hidden; ++j) sum += xg[j] * wo[j];
            out[r * out_features + o] = sum * inv;
        }
    }
    free(xg);
}

/* Fused linear + cross entropy, src/shaders/fused_linear_cross_entropy.metal:189-280 (per token:
 * logits h.w_v in index order, max, sum of exp(logit - max), lse = max + log(sum), loss = lse -
 * logit[target], grad_h = (-w_target + sum_v exp(logit_v - lse) w_v) * grad_scale) and :119-185
 * (grad_weight[v][d] = sum over valid tokens in order of (p_tv - [v == target_t]) h_td, with no
 * grad_scale: the reference leaves the weight gradient unscaled). Targets outside [0, vocab) (-100
 * by convention) are ignored: zero loss and zero grad_h; grad_scale = 1 / valid count
 * (src/ops/fused_linear_cross_entropy.rs:131-133). Returns the mean loss over valid rows (summed in
 * row order, src/ops/fused_linear_cross_entropy.rs:196-208). grad_weight may be NULL. */
static float dot_seq(const float *a, const float *b, int64_t n) {
    float s = 0.0f;
    for (int64_t d = 0; d < n; ++d) s += a[d] * b[d];
    return s;
}

float ref_fused_linear_cross_entropy(const float *hidden, const float *weight, const int32_t *targets, float *losses,
                                     float *grad_hidden, float *grad_weight, int64_t rows, int64_t hd,
                                     int64_t vocab) {
    int64_t valid = 0;
    for (int64_t t = 0; t < rows; ++t) valid += targets[t] >= 0 && targets[t] < vocab;
    const float scale = valid > 0 ? 1.0f / (float)valid : 0.0f;
    float *lse = (float *)malloc(sizeof(float) * (size_t)(rows > 0 ? rows : 1));
    float total = 0.0f;
    for (int64_t t = 0; t < rows; ++t) {
        const float *h = hidden + t * hd;
        float *gh = grad_hidden + t * hd;
        const int32_t tg = targets[t];
        if (tg < 0 || tg >= vocab) {
            losses[t] = 0.0f;
            for (int64_t d = 0; d < hd; ++d) gh[d] = 0.0f;
            lse[t] = 0.0f;
            continue;
        }
        float mx = -INFINITY;
        for (int64_t v = 0; v < vocab; ++v) mx = fmaxf(mx, dot_seq(h, weight + v * hd, hd));
        float sum = 0.0f, tl = 0.0f;
        for (int64_t v = 0; v < vocab; ++v) {
            const float lg = dot_seq(h, weight + v * hd, hd);
            sum += expf(lg - mx);
            if (v == tg) tl = lg;
        }
        lse[t] = mx + logf(sum);
        losses[t] = lse[t] - tl;
        total += losses[t];
        for (int64_t d = 0; d < hd; ++d) gh[d] = -weight[(int64_t)tg * hd + d];
        for (int64_t v = 0; v < vocab; ++v) {
            const float *w = weight + v * hd;
            const float prob = expf(dot_seq(h, w, hd) - lse[t]);
            for (int64_t d = 0; d < hd; ++d) gh[d] += prob * w[d];
        }
        for (int64_t d = 0; d < hd; ++d) gh[d] *= scale;
    }
    if (grad_weight) {
        /* each grad_weight[v][d] sums its tokens in order, as the reference's per-(v, d) loop does */
        for (int64_t v = 0; v < vocab; ++v) {
            float *gw = grad_weight + v * hd;
            for (int64_t d = 0; d < hd; ++d) gw[d] = 0.0f;
            for (int64_t t = 0; t < rows; ++t) {
                const int32_t tg = targets[t];
                if (tg < 0 || tg >= vocab) continue;
                const float *h = hidden + t * hd;
                float gl = expf(dot_seq(h, weight + v * hd, hd) - lse[t]);
                if (tg == v) gl -= 1.0f;
                for (int64_t d = 0; d < hd; ++d) gw[d] += gl * h[d];
            }
        }
    }
    free(lse);
    return valid > 0 ? total / (float)valid : 0.0f;
}
